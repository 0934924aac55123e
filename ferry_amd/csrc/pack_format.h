// Packed expert rows for the H2D link: a lossless format for bf16 rows.
//
// A bf16 value is sign (1 bit) | exponent (8) | mantissa (7).  Sign and mantissa are close to
// random in trained (and in Gaussian) weights; the exponent takes few values (the weights of a
// row span a few binades).  A packed row keeps, per value, one byte sign | mantissa and a 4-bit
// exponent code: exponent = base + code for code < 15, where [base, base + 14] is the row's
// most populated window of 15 exponents; code 15 marks an escape, whose exponent is stored in a
// list sorted by value index.  12 bits per value instead of 16, plus 5 bytes per escape.
//
// Layout (byte offsets from the row start; n = values per row, a multiple of 16):
//   [0, 64)                      PackHeader
//   [64, 64 + n)                 plane A: byte i = (sign << 7) | mantissa of value i
//   [64 + n, 64 + 3n/2)          plane B: nibble i (low nibble first) = exponent code of value i
//   [64 + 3n/2, + 4 escapes)     escape indices (uint32, ascending)
//   [.., + escapes)              escape exponents (uint8)
// The row's size is rounded up to 256 bytes.
#pragma once
#include <cstdint>

namespace ferry {

constexpr uint32_t kPackMagic = 0x4b504146u;  // "FAPK"
constexpr int64_t kPackHeaderBytes = 64;
constexpr int kPackWindow = 15;

struct PackHeader {
  uint32_t magic;
  uint32_t base;       // first exponent of the window
  uint64_t values;     // n
  uint64_t escapes;
  uint64_t bytes;      // packed size (rounded)
  uint64_t pad[4];
};
static_assert(sizeof(PackHeader) == kPackHeaderBytes, "header size");

constexpr int kUnpackRows = 64;   // rows per unpack launch

// kernel argument of one unpack launch
struct UnpackList {
  const uint8_t* src[kUnpackRows];  // packed rows (device staging buffers)
  uint16_t* dst[kUnpackRows];       // cache slots
  int32_t n_rows;
};

inline int64_t packed_bytes(int64_t n, int64_t escapes) {
  const int64_t b = kPackHeaderBytes + n + n / 2 + 4 * escapes + escapes;
  return (b + 255) / 256 * 256;
}

}  // namespace ferry
