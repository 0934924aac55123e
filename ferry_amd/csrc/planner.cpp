// Host placement planner at world = 1.
//
// Reference: ferry/policy.py:130-194 (plan_layer), :109-127 (_choose_slot), :197-205
// (layer_slots), :36-46 (_admission_capacity) and the quota check of ferry/quota.py:63.
// At world = 1 both the FERRY and the RANDOM policy assign every miss to rank 0 (the quota
// table row is [m] and randint(0, 1) is 0), so only the capacity check, the slot choice and
// the state update remain.  The eviction key is the lexicographic minimum of
// (fp32 score of the key's own layer, last-use tick, key) over slots that do not hold an
// expert the current layer needs; the first empty slot wins outright.  ferry_choose_slot is
// that rule for one miss; a layer call applies it to all of its misses through one partial
// sort of the slots (the same choices, see plan_core).  The call's routing IDs are scanned
// once, which validates them and counts each expert's demand (returned by ferry_plan_fetch).
#include <algorithm>
#include <cmath>
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

namespace {

// plan_layer over routing IDs of type T (int64 from the Python API, uint8 from the mapped
// staging buffer).  One pass over the IDs validates them (every ID in [0, E), none repeated
// within a token: the reference's demand count and layout assume both) and counts each
// expert's demand, before any state changes; the misses, slot choices and state updates then
// work on the E demand counts.
template <typename T>
int64_t plan_core(int64_t event, int64_t layer, const T* ids, int64_t tokens, int64_t topk,
                  const float* gate_scores, int64_t* slots, int64_t cap, int64_t* owner,
                  int64_t* last, float* scores, int64_t experts, int64_t* fetches_out,
                  int64_t* destinations_out, int64_t* demand_out, const char* who) {
  ferry::clear_error();
  if (experts <= 0 || topk <= 0 || tokens < 0 || cap < 0 || layer < 0) {
    ferry::set_error("%s: bad sizes", who);
    return -1;
  }
  // Four demand histograms, by token mod 4, so that consecutive tokens naming the same expert
  // do not chain their increments through one memory word; a token's repeated IDs are found
  // with a per-expert last-token array.
  std::vector<int64_t> hist((size_t)(4 * experts), 0);
  std::vector<int32_t> seen((size_t)experts, -1);
  for (int64_t t = 0; t < tokens; ++t) {
    const T* row = ids + t * topk;
    int64_t* h = hist.data() + (t & 3) * experts;
    const int32_t tt = (int32_t)t;
    for (int64_t j = 0; j < topk; ++j) {
      const int64_t e = (int64_t)row[j];
      if (e < 0 || e >= experts) {
        ferry::set_error("%s: expert id %lld of token %lld is out of range [0, %lld)", who,
                         (long long)e, (long long)t, (long long)experts);
        return -3;
      }
      const bool repeated = seen[(size_t)e] == tt;
      seen[(size_t)e] = tt;
      if (repeated) {
        ferry::set_error("%s: expert id %lld repeated in token %lld", who, (long long)e,
                         (long long)t);
        return -3;
      }
      ++h[e];
    }
  }
  std::vector<int64_t> demand((size_t)experts);
  for (int64_t e = 0; e < experts; ++e)
    demand[(size_t)e] = hist[(size_t)e] + hist[(size_t)(experts + e)] +
                        hist[(size_t)(2 * experts + e)] + hist[(size_t)(3 * experts + e)];
  const int64_t base = layer * experts;
  std::memcpy(scores + base, gate_scores, (size_t)experts * sizeof(float));
  std::vector<uint8_t> active((size_t)experts, 0);
  for (int64_t e = 0; e < experts; ++e) active[(size_t)e] = demand[(size_t)e] > 0;
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
  // Repeated ferry_choose_slot calls, one per miss, pick the slots in one fixed order: a slot
  // that receives a miss then holds an expert this layer needs (never chosen again), and no
  // other slot's key, score or last-use tick changes during the call.  So the misses take the
  // first m admissible slots in that order: the empty slots by index, then the others by
  // (score of the key's own layer, last-use tick, key) -- O(cap + m log cap) instead of O(m cap).
  std::vector<int64_t> order;
  order.reserve((size_t)cap);
  int64_t empties = 0;
  for (int64_t i = 0; i < cap; ++i)
    if (slots[i] < 0) {
      order.push_back(i);
      ++empties;
    }
  if (empties < m) {
    // a key whose score is NaN never compares below the running best, so the scan never
    // picks its slot: such slots are no candidates
    for (int64_t i = 0; i < cap; ++i) {
      const int64_t key = slots[i];
      if (key >= 0 && !(key / experts == layer && active[(size_t)(key % experts)]) &&
          !std::isnan(scores[key]))
        order.push_back(i);
    }
    if ((int64_t)order.size() < m) {
      ferry::set_error("no evictable cache slot for key %lld",
                       (long long)(base + misses[order.size()]));
      return -1;
    }
    auto before = [&](int64_t a, int64_t b) {
      const int64_t ka = slots[a], kb = slots[b];
      const double sa = scores[ka], sb = scores[kb];
      if (sa != sb) return sa < sb;
      if (last[ka] != last[kb]) return last[ka] < last[kb];
      return ka < kb;
    };
    const auto first = order.begin() + empties;
    const auto upto = order.begin() + m;
    std::partial_sort(first, upto, order.end(), before);
  }
  for (int64_t i = 0; i < m; ++i) {
    const int64_t key = base + misses[(size_t)i];
    const int64_t slot = order[(size_t)i];
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
    for (int64_t i = 0; i < tokens * topk; ++i)
      destinations_out[i] = owner[base + (int64_t)ids[i]];
  if (demand_out) std::memcpy(demand_out, demand.data(), (size_t)experts * sizeof(int64_t));
  return m;
}

}  // namespace

extern "C" int64_t ferry_plan_layer(int64_t event, int64_t layer, const int64_t* selected,
                                    int64_t tokens, int64_t topk, const float* gate_scores,
                                    int64_t* slots, int64_t cap, int64_t* owner, int64_t* last,
                                    float* scores, int64_t experts, int64_t* fetches_out,
                                    int64_t* destinations_out) {
  return plan_core(event, layer, selected, tokens, topk, gate_scores, slots, cap, owner, last,
                   scores, experts, fetches_out, destinations_out, nullptr, "plan_layer");
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
                                    int64_t* destinations_out, int64_t* demand_out,
                                    ferry_h2d* h2d) {
  const int64_t m = plan_core(event, layer, ids, tokens, topk, gate_scores, slots, cap, owner,
                              last, scores, experts, fetches_out, destinations_out, demand_out,
                              "plan_fetch");
  if (m <= 0 || !h2d) return m;
  std::vector<int64_t> fs((size_t)m), fk((size_t)m);
  for (int64_t j = 0; j < m; ++j) {
    fk[(size_t)j] = fetches_out[3 * j + 1];
    fs[(size_t)j] = fetches_out[3 * j + 2];
  }
  return ferry_h2d_fetch(h2d, fs.data(), fk.data(), m) == 0 ? m : -2;
}
