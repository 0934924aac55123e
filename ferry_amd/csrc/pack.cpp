// Host side of the packed expert rows (the format is described in pack_format.h): choosing each
// row's exponent window and writing its packed form, over a pool of rows on several threads.
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/ferry_amd.h"
#include "pack_format.h"

namespace ferry {
void set_error(const char* fmt, ...);
void clear_error();

// Window base and escape count of one row of n bf16 values.
void pack_plan(const uint16_t* v, int64_t n, uint32_t* base, int64_t* escapes) {
  int64_t hist[256] = {};
  for (int64_t i = 0; i < n; ++i) ++hist[(v[i] >> 7) & 0xFF];
  int64_t best = -1, in = 0;
  uint32_t b_best = 0;
  for (int e = 0; e < kPackWindow; ++e) in += hist[e];
  for (int b = 0; b + kPackWindow <= 256; ++b) {
    if (b > 0) in += hist[b + kPackWindow - 1] - hist[b - 1];
    if (in > best) {
      best = in;
      b_best = (uint32_t)b;
    }
  }
  *base = b_best;
  *escapes = n - best;
}

// Writes the packed row (packed_bytes(n, escapes) bytes) of a row planned by pack_plan.
void pack_write(const uint16_t* v, int64_t n, uint32_t base, int64_t escapes, uint8_t* dst) {
  PackHeader hd;
  std::memset(&hd, 0, sizeof(hd));
  hd.magic = kPackMagic;
  hd.base = base;
  hd.values = (uint64_t)n;
  hd.escapes = (uint64_t)escapes;
  hd.bytes = (uint64_t)packed_bytes(n, escapes);
  std::memcpy(dst, &hd, sizeof(hd));
  uint8_t* pa = dst + kPackHeaderBytes;
  uint8_t* pb = pa + n;
  uint32_t* eidx = reinterpret_cast<uint32_t*>(pb + n / 2);
  uint8_t* eexp = reinterpret_cast<uint8_t*>(eidx + escapes);
  int64_t k = 0;
  for (int64_t i = 0; i < n; i += 2) {
    uint8_t codes = 0;
    for (int q = 0; q < 2; ++q) {
      const uint16_t x = v[i + q];
      const uint32_t e = (x >> 7) & 0xFF;
      pa[i + q] = (uint8_t)(((x >> 8) & 0x80) | (x & 0x7F));
      uint32_t c = e - base;  // wraps for e < base
      if (c >= (uint32_t)(kPackWindow)) {
        c = kPackWindow;
        eidx[k] = (uint32_t)(i + q);
        eexp[k] = (uint8_t)e;
        ++k;
      }
      codes |= (uint8_t)(c << (4 * q));
    }
    pb[i / 2] = codes;
  }
  const int64_t end = kPackHeaderBytes + n + n / 2 + 5 * escapes;
  std::memset(dst + end, 0, (size_t)(hd.bytes - end));
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

// Window bases and escape counts of `rows` rows of n values, on `threads` threads.
void pack_plan_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads, uint32_t* base,
                    int64_t* escapes) {
  parallel_rows(rows, threads, [&](int64_t i) { pack_plan(pool + i * n, n, &base[i], &escapes[i]); });
}

// Packed rows written at dst + off[i] for every row with off[i] >= 0.
void pack_write_rows(const uint16_t* pool, int64_t rows, int64_t n, int threads,
                     const uint32_t* base, const int64_t* escapes, const int64_t* off,
                     uint8_t* dst) {
  parallel_rows(rows, threads, [&](int64_t i) {
    if (off[i] >= 0) pack_write(pool + i * n, n, base[i], escapes[i], dst + off[i]);
  });
}

}  // namespace ferry

// Packs one row of n bf16 values (n a multiple of 16) into dst (capacity cap bytes; null to
// query the size).  *bytes_out receives the packed size; returns 0, or 1 when the packed form
// is not smaller than the row (the row then stays raw and dst is untouched), 2 on bad arguments.
extern "C" int ferry_pack_row(const void* src, int64_t n, void* dst, int64_t cap,
                              int64_t* bytes_out) {
  ferry::clear_error();
  if (!src || n <= 0 || n % 16 != 0 || n >= ((int64_t)1 << 32) || !bytes_out) {
    ferry::set_error("pack_row: n must be a positive multiple of 16 below 2^32");
    return 2;
  }
  uint32_t base;
  int64_t esc;
  ferry::pack_plan((const uint16_t*)src, n, &base, &esc);
  const int64_t bytes = ferry::packed_bytes(n, esc);
  *bytes_out = bytes;
  if (bytes >= 2 * n) return 1;
  if (!dst) return 0;
  if (cap < bytes) {
    ferry::set_error("pack_row: %lld bytes needed, %lld given", (long long)bytes, (long long)cap);
    return 2;
  }
  ferry::pack_write((const uint16_t*)src, n, base, esc, (uint8_t*)dst);
  return 0;
}
