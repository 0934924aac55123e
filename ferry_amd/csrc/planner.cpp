// Host placement planner at world = 1.
//
// Reference: ferry/policy.py:130-194 (plan_layer), :109-127 (_choose_slot), :197-205
// (layer_slots), :36-46 (_admission_capacity) and the quota check of ferry/quota.py:63.
// At world = 1 both the FERRY and the RANDOM policy assign every miss to rank 0 (the quota
// table row is [m] and randint(0, 1) is 0), so only the capacity check, the slot choice and
// the state update remain.  The eviction key is the lexicographic minimum of
// (fp32 score of the key's own layer, last-use tick, key) over slots that do not hold an
// expert the current layer needs; the first empty slot wins outright.
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/ferry_amd.h"

namespace ferry {
void set_error(const char* fmt, ...);
void clear_error();
}  // namespace ferry

extern "C" int64_t ferry_choose_slot(int64_t layer, const uint8_t* active, const int64_t* slots,
                                     int64_t cap, const int64_t* last, const float* scores,
                                     int64_t experts) {
  // same initial key as the reference: (inf, 2^60, 2^60); scores widen exactly to double
  int64_t best = -1;
  double best_score = __builtin_inf();
  int64_t best_used = (int64_t)1 << 60, best_key = (int64_t)1 << 60;
  for (int64_t i = 0; i < cap; ++i) {
    const int64_t key = slots[i];
    if (key < 0) return i;
    if (key / experts == layer && active[key % experts]) continue;  // needed by this layer
    const double score = scores[key];
    const int64_t used = last[key];
    if (score < best_score ||
        (score == best_score && (used < best_used || (used == best_used && key < best_key)))) {
      best = i;
      best_score = score;
      best_used = used;
      best_key = key;
    }
  }
  return best;
}

extern "C" int64_t ferry_plan_layer(int64_t event, int64_t layer, const int64_t* selected,
                                    int64_t tokens, int64_t topk, const float* gate_scores,
                                    int64_t* slots, int64_t cap, int64_t* owner, int64_t* last,
                                    float* scores, int64_t experts, int64_t* fetches_out,
                                    int64_t* destinations_out) {
  ferry::clear_error();
  if (experts <= 0 || topk <= 0 || tokens < 0 || cap < 0 || layer < 0) {
    ferry::set_error("plan_layer: bad sizes");
    return -1;
  }
  // validate the routing before any state changes: every ID in [0, E), none repeated within
  // a token (the reference's demand count and layout assume both)
  std::vector<int64_t> seen((size_t)experts, -1);
  for (int64_t t = 0; t < tokens; ++t) {
    for (int64_t j = 0; j < topk; ++j) {
      const int64_t e = selected[t * topk + j];
      if (e < 0 || e >= experts) {
        ferry::set_error("plan_layer: expert id %lld of token %lld is out of range [0, %lld)",
                         (long long)e, (long long)t, (long long)experts);
        return -3;
      }
      if (seen[(size_t)e] == t) {
        ferry::set_error("plan_layer: expert id %lld repeated in token %lld", (long long)e,
                         (long long)t);
        return -3;
      }
      seen[(size_t)e] = t;
    }
  }
  const int64_t base = layer * experts;
  std::memcpy(scores + base, gate_scores, (size_t)experts * sizeof(float));
  std::vector<uint8_t> active((size_t)experts, 0);
  for (int64_t i = 0; i < tokens * topk; ++i) active[(size_t)selected[i]] = 1;
  std::vector<int64_t> misses;
  misses.reserve((size_t)experts);
  for (int64_t e = 0; e < experts; ++e)
    if (active[(size_t)e] && owner[base + e] < 0) misses.push_back(e);
  int64_t admissible = 0;
  for (int64_t i = 0; i < cap; ++i) {
    const int64_t key = slots[i];
    if (key < 0 || !(key / experts == layer && active[(size_t)(key % experts)])) ++admissible;
  }
  const int64_t m = (int64_t)misses.size();
  if (m > admissible) {
    ferry::set_error("missing experts exceed the total admission capacity (%lld > %lld)",
                     (long long)m, (long long)admissible);
    return -1;
  }
  for (int64_t i = 0; i < m; ++i) {
    const int64_t key = base + misses[(size_t)i];
    const int64_t slot =
        ferry_choose_slot(layer, active.data(), slots, cap, last, scores, experts);
    if (slot < 0) {
      ferry::set_error("no evictable cache slot for key %lld", (long long)key);
      return -1;
    }
    const int64_t victim = slots[slot];
    if (victim >= 0) owner[victim] = -1;
    slots[slot] = key;
    owner[key] = 0;
    fetches_out[3 * i + 0] = 0;
    fetches_out[3 * i + 1] = key;
    fetches_out[3 * i + 2] = slot;
  }
  for (int64_t e = 0; e < experts; ++e)
    if (active[(size_t)e]) last[base + e] = event + 1;
  if (destinations_out)
    for (int64_t i = 0; i < tokens * topk; ++i) destinations_out[i] = owner[base + selected[i]];
  return m;
}

extern "C" void ferry_layer_slots(const int64_t* slots, int64_t cap, int64_t layer,
                                  int64_t experts, int64_t* lookup) {
  for (int64_t e = 0; e < experts; ++e) lookup[e] = -1;
  for (int64_t i = 0; i < cap; ++i) {
    const int64_t key = slots[i];
    if (key >= 0 && key / experts == layer) lookup[key % experts] = i;
  }
}

extern "C" int64_t ferry_plan_fetch(int64_t event, int64_t layer, const uint8_t* ids,
                                    int64_t tokens, int64_t topk, const float* gate_scores,
                                    int64_t* slots, int64_t cap, int64_t* owner, int64_t* last,
                                    float* scores, int64_t experts, int64_t* fetches_out,
                                    int64_t* destinations_out, ferry_h2d* h2d) {
  if (tokens < 0 || topk <= 0) {
    ferry::clear_error();
    ferry::set_error("plan_fetch: bad sizes");
    return -1;
  }
  std::vector<int64_t> sel((size_t)(tokens * topk));
  for (size_t i = 0; i < sel.size(); ++i) sel[i] = ids[i];
  const int64_t m = ferry_plan_layer(event, layer, sel.data(), tokens, topk, gate_scores, slots,
                                     cap, owner, last, scores, experts, fetches_out,
                                     destinations_out);
  if (m <= 0 || !h2d) return m;
  std::vector<int64_t> fs((size_t)m), fk((size_t)m);
  for (int64_t j = 0; j < m; ++j) {
    fk[(size_t)j] = fetches_out[3 * j + 1];
    fs[(size_t)j] = fetches_out[3 * j + 2];
  }
  return ferry_h2d_fetch(h2d, fs.data(), fk.data(), m) == 0 ? m : -2;
}
