// Host side of the packed expert rows (the format is described in pack_format.h): choosing each
// row's exponent windows and writing its packed form, over a pool of rows on several threads.
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/ferry_amd.h"
#include "pack_format.h"

namespace ferry {
void set_error(const char* fmt, ...);
void clear_error();

// Most populated window of `width` exponents in hist: its first exponent and its population.
static void best_window(const int64_t* hist, int width, uint32_t* base, int64_t* in_window) {
  int64_t in = 0, best = -1;
  uint32_t b_best = 0;
  for (int e = 0; e < width; ++e) in += hist[e];
  for (int b = 0; b + width <= 256; ++b) {
    if (b > 0) in += hist[b + width - 1] - hist[b - 1];
    if (in > best) {
      best = in;
      b_best = (uint32_t)b;
    }
  }
  *base = b_best;
  *in_window = best;
}

// The kPackTable most populated exponents of hist (ties: the smaller exponent first), their
// population, and hist with them taken out.
static int64_t take_table(int64_t* hist, uint8_t* table) {
  int64_t in = 0;
  for (int j = 0; j < kPackTable; ++j) {
    int best = 0;
    for (int e = 1; e < 256; ++e)
      if (hist[e] > hist[best]) best = e;
    table[j] = (uint8_t)best;
    in += hist[best];
    hist[best] = -1;   // taken (a later pick never matches it again)
  }
  for (int j = 0; j < kPackTable; ++j) hist[table[j]] = 0;
  return in;
}

// The exponent tables of one row of n bf16 values and its escape counts.
void pack_plan(const uint16_t* v, int64_t n, PackPlan* plan) {
  int64_t hist[256] = {};
  for (int64_t i = 0; i < n; ++i) ++hist[(v[i] >> 7) & 0xFF];
  const int64_t in1 = take_table(hist, plan->t1);
  const int64_t in2 = take_table(hist, plan->t2);
  uint32_t base3;
  int64_t in3;
  best_window(hist, kPackWindow3, &base3, &in3);
  plan->base3 = (uint8_t)base3;
  plan->esc1 = n - in1;
  plan->esc2 = plan->esc1 - in2;
  plan->esc3 = plan->esc2 - in3;
}

int64_t plan_bytes(int64_t n, const PackPlan& plan) {
  return packed_bytes(n, plan.esc1, plan.esc2, plan.esc3);
}

// index of e in a table of kPackTable exponents (the first match), or kPackTable
static inline uint32_t table_code(const uint8_t* t, uint32_t e) {
  for (int j = 0; j < kPackTable; ++j)
    if (t[j] == e) return (uint32_t)j;
  return kPackTable;
}

// Writes the packed row (plan_bytes(n, plan) bytes) of a row planned by pack_plan.
void pack_write(const uint16_t* v, int64_t n, const PackPlan& plan, uint8_t* dst) {
  const PackOffsets o = pack_offsets(n, plan.esc1, plan.esc2, plan.esc3);
  const int64_t bytes = plan_bytes(n, plan);
  PackHeader hd;
  std::memset(&hd, 0, sizeof(hd));
  hd.magic = kPackMagic;
  std::memcpy(hd.t1, plan.t1, kPackTable);
  std::memcpy(hd.t2, plan.t2, kPackTable);
  hd.base3 = plan.base3;
  hd.values = (uint64_t)n;
  hd.esc1 = (uint64_t)plan.esc1;
  hd.esc2 = (uint64_t)plan.esc2;
  hd.esc3 = (uint64_t)plan.esc3;
  hd.bytes = (uint64_t)bytes;
  std::memcpy(dst, &hd, sizeof(hd));
  std::memset(dst + o.c2, 0, (size_t)(bytes - o.c2));   // code streams, list, tail
  uint8_t* pa = dst + o.a;
  uint8_t* b0 = dst + o.b0;
  uint8_t* b1 = dst + o.b1;
  uint32_t* pre = reinterpret_cast<uint32_t*>(dst + o.p);
  uint8_t* c2s = dst + o.c2;
  uint8_t* c3s = dst + o.c3;
  uint32_t* lidx = reinterpret_cast<uint32_t*>(dst + o.l_idx);
  uint8_t* lexp = dst + o.l_exp;
  int64_t k1 = 0, k2 = 0, k3 = 0;   // escapes of each level so far
  for (int64_t i = 0; i < n; i += 8) {
    if (i % kPackBlock == 0) {
      pre[3 * (i / kPackBlock)] = (uint32_t)k1;
      pre[3 * (i / kPackBlock) + 1] = (uint32_t)k2;
      pre[3 * (i / kPackBlock) + 2] = (uint32_t)k3;
    }
    uint32_t p0 = 0, p1 = 0;
    for (int q = 0; q < 8; ++q) {
      const uint16_t x = v[i + q];
      const uint32_t e = (x >> 7) & 0xFF;
      pa[i + q] = (uint8_t)(((x >> 8) & 0x80) | (x & 0x7F));
      const uint32_t c = table_code(plan.t1, e);
      if (c == (uint32_t)kPackTable) {
        const uint32_t c2 = table_code(plan.t2, e);
        c2s[k1 >> 2] |= (uint8_t)(c2 << (2 * (k1 & 3)));
        ++k1;
        if (c2 == (uint32_t)kPackTable) {
          uint32_t c3 = e - plan.base3;   // wraps for e < base3
          if (c3 >= (uint32_t)kPackWindow3) {
            c3 = kPackWindow3;
            lidx[k3] = (uint32_t)(i + q);
            lexp[k3] = (uint8_t)e;
            ++k3;
          }
          c3s[k2 >> 1] |= (uint8_t)(c3 << (4 * (k2 & 1)));
          ++k2;
        }
      }
      p0 |= (c & 1u) << q;
      p1 |= ((c >> 1) & 1u) << q;
    }
    b0[i / 8] = (uint8_t)p0;
    b1[i / 8] = (uint8_t)p1;
  }
  const int64_t nb = (n + kPackBlock - 1) / kPackBlock;
  pre[3 * nb] = (uint32_t)k1;
  pre[3 * nb + 1] = (uint32_t)k2;
  pre[3 * nb + 2] = (uint32_t)k3;
}

// Run f(i) for i in [0, n) on `threads` threads.
template <typename F>
void parallel_rows(int64_t n, int threads, F f) {
  if (threads < 1) threads = 1;
  if (threads > n) threads = (int)(n > 0 ? n : 1);
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&, t] {
      for (int64_t i = t; i < n; i += threads) f(i);
    });
  for (auto& th : pool) th.join();
}

// Plans of `rows` rows of n values, on `threads` threads.
void pack_plan_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads, PackPlan* plan) {
  parallel_rows(rows, threads, [&](int64_t i) { pack_plan(pool + i * n, n, &plan[i]); });
}

// Packed rows written at dst + off[i] for every row with off[i] >= 0.
void pack_write_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads,
                     const PackPlan* plan, const int64_t* off, uint8_t* dst) {
  parallel_rows(rows, threads, [&](int64_t i) {
    if (off[i] >= 0) pack_write(pool + i * n, n, plan[i], dst + off[i]);
  });
}

}  // namespace ferry

// Packs one row of n bf16 values (n a multiple of 32) into dst (capacity cap bytes; null to
// query the size).  *bytes_out receives the packed size; returns 0, or 1 when the packed form
// is not smaller than the row (the row then stays raw and dst is untouched), 2 on bad arguments.
extern "C" int ferry_pack_row(const void* src, int64_t n, void* dst, int64_t cap,
                              int64_t* bytes_out) {
  ferry::clear_error();
  if (!src || n <= 0 || n % 32 != 0 || n >= ((int64_t)1 << 32) || !bytes_out) {
    ferry::set_error("pack_row: n must be a positive multiple of 32 below 2^32");
    return 2;
  }
  ferry::PackPlan plan;
  ferry::pack_plan((const uint16_t*)src, n, &plan);
  const int64_t bytes = ferry::plan_bytes(n, plan);
  *bytes_out = bytes;
  if (bytes >= 2 * n) return 1;
  if (!dst) return 0;
  if (cap < bytes) {
    ferry::set_error("pack_row: %lld bytes needed, %lld given", (long long)bytes, (long long)cap);
    return 2;
  }
  ferry::pack_write((const uint16_t*)src, n, plan, (uint8_t*)dst);
  return 0;
}
