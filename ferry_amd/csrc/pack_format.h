// Packed expert rows for the H2D link: a lossless format for bf16 rows.
//
// A bf16 value is sign (1 bit) | exponent (8) | mantissa (7).  Sign and mantissa are close to
// random in trained (and in Gaussian) weights; the exponent takes few values (the weights of a
// row span a few binades, most of them in a handful).  A packed row keeps, per value, one byte
// sign | mantissa and a 3-bit exponent code: exponent = base1 + code for code < 7, where
// [base1, base1 + 6] is the row's most populated window of 7 exponents.  Code 7 marks an escape;
// the escapes' exponents follow in value order as 4-bit codes against a second window
// [base2, base2 + 14] (the most populated among the escapes), and code 15 there sends the
// exponent to a third level, a list of (value index, exponent) sorted by index.  A prefix table
// gives, for each block of 8192 values, the escapes and the third-level entries before it, so a
// block decodes on its own: it counts its escapes' ranks within the block and reads its slice of
// the level-2 codes and of the third-level list.  About 11.1 bits per value for the
// Gaussian-like rows of expert weights, instead of 16.
//
// Layout (byte offsets from the row start; n = values per row, a multiple of 32):
//   [0, 64)                       PackHeader
//   A   n bytes                   byte i = (sign << 7) | mantissa of value i
//   B0, B1, B2  n / 8 bytes each  bit (i % 8) of byte i / 8: bit 0 / 1 / 2 of the code of value i
//   P   8 * (nb + 1) bytes        nb = ceil(n / 8192) blocks; uint32 pairs: P[2b] = escapes
//                                 among values [0, 8192 b), P[2b + 1] = third-level entries
//                                 among them (b = nb: the totals)
//   C   ceil(esc1 / 2) bytes      nibble k (low nibble first) = level-2 code of escape k
//   L   4 * esc2 + esc2 bytes     uint32 value indices (ascending), then uint8 exponents
// The row's size is rounded up to 256 bytes.
#pragma once
#include <cstdint>

namespace ferry {

constexpr uint32_t kPackMagic = 0x3250414bu;  // "KAP2"
constexpr int64_t kPackHeaderBytes = 64;
constexpr int64_t kPackBlock = 8192;     // values per prefix-table entry
constexpr int kPackWindow1 = 7;          // 3-bit codes 0..6, 7 = escape
constexpr int kPackWindow2 = 15;         // 4-bit codes 0..14, 15 = third level

struct PackHeader {
  uint32_t magic;
  uint32_t base1;      // first exponent of the 3-bit window
  uint32_t base2;      // first exponent of the level-2 window
  uint32_t pad0;
  uint64_t values;     // n
  uint64_t esc1;       // values with code 7
  uint64_t esc2;       // escapes with level-2 code 15 (third-level list)
  uint64_t bytes;      // packed size (rounded)
  uint64_t pad[2];
};
static_assert(sizeof(PackHeader) == kPackHeaderBytes, "header size");

struct PackOffsets {
  int64_t a, b0, b1, b2, p, c, l_idx, l_exp, end;
};

// Exponent windows and escape counts chosen for one row.
struct PackPlan {
  uint32_t base1, base2;
  int64_t esc1, esc2;
};

constexpr PackOffsets pack_offsets(int64_t n, int64_t esc1, int64_t esc2) {
  PackOffsets o{};
  o.a = kPackHeaderBytes;
  o.b0 = o.a + n;
  o.b1 = o.b0 + n / 8;
  o.b2 = o.b1 + n / 8;
  o.p = o.b2 + n / 8;
  o.c = o.p + 8 * ((n + kPackBlock - 1) / kPackBlock + 1);
  o.l_idx = o.c + (esc1 + 1) / 2;
  o.l_idx = (o.l_idx + 3) / 4 * 4;   // aligned uint32 indices
  o.l_exp = o.l_idx + 4 * esc2;
  o.end = o.l_exp + esc2;
  return o;
}

constexpr int64_t packed_bytes(int64_t n, int64_t esc1, int64_t esc2) {
  return (pack_offsets(n, esc1, esc2).end + 255) / 256 * 256;
}

constexpr int kUnpackRows = 64;   // rows per unpack launch

// kernel argument of one unpack launch
struct UnpackList {
  const uint8_t* src[kUnpackRows];  // packed rows: device staging buffers, or the packed pool
                                    // itself through its device mapping (read over the link)
  uint16_t* dst[kUnpackRows];       // cache slots
  uint8_t raw[kUnpackRows];         // 1: src holds the row's bf16 values as they are
  int32_t n_rows;
};

}  // namespace ferry
