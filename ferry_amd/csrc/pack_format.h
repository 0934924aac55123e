// Packed expert rows for the H2D link: a lossless format for bf16 rows.
//
// A bf16 value is sign (1 bit) | exponent (8) | mantissa (7).  Sign and mantissa are close to
// random in trained (and in Gaussian) weights; the exponent takes few values: the weights of a
// row span a few binades, most of them in a handful.  A packed row keeps, per value, one byte
// sign | mantissa and a 2-bit exponent code: codes 0-2 name the row's three most populated
// exponents (table T1), code 3 is an escape.  The escapes' exponents follow in value order as a
// second 2-bit code against the three most populated exponents among the escapes (table T2),
// whose code 3 sends the exponent on to a 4-bit code against a window [base3, base3 + 14] (the
// most populated window among what is left), whose code 15 sends it to a list of (value index,
// exponent) sorted by index.  A prefix table gives, for each block of 8192 values, the
// escapes of each level before it, so a block decodes on its own: two block-wide prefix sums
// rank its escapes of the first two levels, and it reads its slices of the level-2 and level-3
// codes and of the list.  About 10.7 bits per value for the Gaussian-like rows of expert
// weights, instead of 16 (the exponents' entropy bounds it at about 10.5).
//
// Layout (byte offsets from the row start; n = values per row, a multiple of 32):
//   [0, 64)                        PackHeader
//   A    n bytes                   byte i = (sign << 7) | mantissa of value i
//   B0, B1  n / 8 bytes each       bit (i % 8) of byte i / 8: bit 0 / 1 of the code of value i
//   P    12 * (nb + 1) bytes       nb = ceil(n / 8192) blocks; uint32 triples: P[3b + l] = the
//                                  level-(l + 1) escapes among values [0, 8192 b) (b = nb: totals)
//   C2   4 * ceil(esc1 / 16) bytes 2-bit code k (bits 2k, 2k + 1 of the little-endian stream) =
//                                  level-2 code of escape k
//   C3   4 * ceil(esc2 / 8) bytes  4-bit code k (nibble k, low nibble first) = level-3 code of
//                                  the k-th level-2 escape
//   L    4 * esc3 + esc3 bytes     uint32 value indices (ascending), then uint8 exponents
// The row's size is rounded up to 256 bytes.  The code streams are whole 32-bit words, so that a
// reader may fetch them a word at a time without leaving their region.
#pragma once
#include <cstdint>

namespace ferry {

constexpr uint32_t kPackMagic = 0x3350414bu;  // "KAP3"
constexpr int64_t kPackHeaderBytes = 64;
constexpr int64_t kPackBlock = 8192;     // values per prefix-table entry
constexpr int kPackTable = 3;            // 2-bit codes 0..2 name table entries, 3 = escape
constexpr int kPackWindow3 = 15;         // 4-bit codes 0..14, 15 = list

struct PackHeader {
  uint32_t magic;
  uint8_t t1[kPackTable];   // level-1 exponents
  uint8_t t2[kPackTable];   // level-2 exponents
  uint8_t base3;            // first exponent of the level-3 window
  uint8_t pad0;
  uint32_t pad1;
  uint64_t values;     // n
  uint64_t esc1;       // values with level-1 code 3
  uint64_t esc2;       // of those, with level-2 code 3
  uint64_t esc3;       // of those, with level-3 code 15 (list entries)
  uint64_t bytes;      // packed size (rounded)
  uint64_t pad2;
};
static_assert(sizeof(PackHeader) == kPackHeaderBytes, "header size");

struct PackOffsets {
  int64_t a, b0, b1, p, c2, c3, l_idx, l_exp, end;
};

// Exponent tables and escape counts chosen for one row.
struct PackPlan {
  uint8_t t1[kPackTable], t2[kPackTable];
  uint8_t base3;
  int64_t esc1, esc2, esc3;
};

constexpr PackOffsets pack_offsets(int64_t n, int64_t esc1, int64_t esc2, int64_t esc3) {
  PackOffsets o{};
  o.a = kPackHeaderBytes;
  o.b0 = o.a + n;
  o.b1 = o.b0 + n / 8;
  o.p = o.b1 + n / 8;
  o.c2 = o.p + 12 * ((n + kPackBlock - 1) / kPackBlock + 1);
  o.c3 = o.c2 + 4 * ((esc1 + 15) / 16);
  o.l_idx = o.c3 + 4 * ((esc2 + 7) / 8);
  o.l_exp = o.l_idx + 4 * esc3;
  o.end = o.l_exp + esc3;
  return o;
}

constexpr int64_t packed_bytes(int64_t n, int64_t esc1, int64_t esc2, int64_t esc3) {
  return (pack_offsets(n, esc1, esc2, esc3).end + 255) / 256 * 256;
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
