// Grouped SwiGLU expert FFN over cache slots (bf16 in, fp32 accumulate, bf16 out).
//
// Reference: ferry/csrc/expert_ops.cpp:13-45 (execute_experts) and expert_ops.cu:6-25
// (silu_mul).  For each expert e with rows p in [starts[e], starts[e+1]):
//   x = in[rows[p]];  g = bf16(x Wg^T);  u = bf16(x Wu^T);  a = bf16(silu(g) * u) (fp32 math)
//   y = bf16(a Wd^T);  out = bf16(y * w[rows[p], cols[p]])
// with cache[slot] = [Wg (I x H) | Wu (I x H) | Wd (H x I)], all row-major bf16.  Both GEMMs
// are "NT" (both operands contiguous along K), which is the native operand order of the
// CDNA4 MFMA instructions used here.  The bf16 rounding points of the reference are kept.
//
// Three kernel schemes, selected per expert by its row count n_e:
//  * skinny (n_e <= 16, decode): bandwidth-bound.  A workgroup owns 16 (phase 1) or 64
//    (phase 2) weight rows and splits K over its four wavefronts; the partial sums meet in
//    LDS.  The weights are loaded 8 rows x 128 B per instruction and turned into MFMA B
//    fragments through a small per-wavefront LDS tile; x rows come from L2.
//    v_mfma_f32_16x16x32_bf16.  For the decode shapes (H = 2048 up, I = 768 down) the K walk
//    is software-pipelined with inline-asm loads: the next batch is in flight while the
//    current one is multiplied.
//  * mid (16 < n_e <= 64, prefill): bandwidth-bound.  A workgroup owns 64 output columns over
//    the full K; the expert's token rows are staged once per workgroup in LDS, the weights
//    stream into MFMA B registers.  Launched together with the skinny experts of a list.
//  * tiled (n_e > 64, prefill): MFMA-bound.  Persistent workgroups walk a device-computed
//    list of 256x256 output tiles; A (gathered x rows / activation rows) and B (weight rows)
//    tiles of 64 along K are staged by direct global->LDS loads into a swizzled,
//    double-buffered LDS layout.  v_mfma_f32_32x32x16_bf16, eight wavefronts of 128x64.
// Phase 1 ("up") computes the gate and up projections together and applies silu(g)*u in the
// epilogue; phase 2 ("down") applies the routing weight in the epilogue and writes the
// per-(token, expert) row that the combine kernel sums.

#include "common.h"

#include <atomic>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

namespace ferry {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kListMax = 256;   // experts per launch (longer lists are split by the host)
constexpr int kSkinnyMax = 64;  // rows handled by the skinny and mid kernels (4 tiles of 16)

struct ExpertList {
  int32_t n;
  int32_t n_mid;   // small-expert up launch: the first n_mid entries take 64-column workgroups
  int16_t expert[kListMax];
  int32_t slot[kListMax];
};

struct FfnArgs {
  const bf16_t* cache;
  const bf16_t* x;        // [R, H]
  const bf16_t* w;        // [R, k] routing weights in sorted-ID order
  const int64_t* starts;  // [E+1]
  const int64_t* rows;    // [R*k]
  const int64_t* cols;    // [R*k]
  bf16_t* act;            // [R*k, I]
  bf16_t* out;            // [R*k, H]
  int64_t H, I, k;
  int32_t out_mode;
  ExpertList list;
};


__device__ __forceinline__ float silu_mul(float g, float u) {
  // silu(g) * u in fp32 on the bf16-rounded GEMM outputs: g * u / (1 + e^-g) with the
  // hardware exp2 and reciprocal (relative error ~1e-6, far below the bf16 rounding that
  // follows); a large negative g gives e^-g = inf and a zero result, the exact formula's limit
  return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// two floats rounded to bf16 (round to nearest even, as f32_to_bf16) in one instruction,
// packed as lo | hi << 16
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, b16x2));
}

__device__ __forceinline__ bf16x8 load8(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// Activation rows of the one-launch decode kernel (ffn_skinny_fused) are written by one
// workgroup and read by others, on any XCD, inside one launch.  With COH their stores and loads
// are agent-coherent (relaxed agent-scope atomic accesses: sc1), so that no L2 write-back or
// invalidate is needed between the two phases; the other kernels use plain accesses.
template <bool COH>
__device__ __forceinline__ void store_act(bf16_t* p, bf16_t v) {
  if constexpr (COH)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}
template <bool COH>
__device__ __forceinline__ bf16x8 load_act8(const bf16_t* p) {
  if constexpr (COH) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    struct { uint64_t a, b; } both = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  } else {
    return load8(p);
  }
}

// =============================================================================================
// Memory helpers shared by the kernels below
// =============================================================================================

// a wave-uniform pointer moved to scalar registers
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
// 16-byte global->LDS direct load of each lane: global address sbase + voff (wave-uniform base
// in scalar registers, 32-bit lane byte offset), LDS byte address lds + 16 * lane.  Issued as
// inline asm so that the address keeps this form wherever the load is scheduled; the compiler
// does not track these loads, their completion is awaited with wait_vmcnt0.  The asm writes
// m0 (the LDS base of the direct load); nothing else in these kernels uses m0.  An LDS direct
// load needs one wait state between the SALU write of m0 and its issue (the s_nop), which the
// compiler's hazard pass would add for its own instructions but cannot see inside the asm.
__device__ __forceinline__ void dma16(const char* sbase, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory", "m0");
}
// wait until at most N of this wavefront's vector-memory operations are outstanding
__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_char*)p;
}
// LDS fragment read issued as inline asm: the compiler cannot see that it reads memory that
// the in-flight direct loads write, so it does not insert a vmcnt(0) drain in front of it.
// Completion is awaited explicitly with lds_wait, which also ties the fragment registers.
template <int OFF>
__device__ __forceinline__ void ds_read16(bf16x8& v, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
}
__device__ __forceinline__ void lds_wait(bf16x8 (&a)[4], bf16x8 (&b)[2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1])
               :
               : "memory");
}
// workgroup barrier without the release/acquire fence of __syncthreads (which would drain
// the direct loads of the later stages); LDS visibility is established by the explicit waits
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// =============================================================================================
// Skinny kernels
// =============================================================================================

// Skinny kernels (experts with at most 16 rows: decode, and the smallest experts of a prefill).
// They are bound by the weight bytes.  The four wavefronts of a workgroup split K into
// contiguous ranges of 32-element steps; their partial sums are added in LDS in a fixed order.
// up_skinny / down_skinny below load the weights in MFMA fragment order (each lane 16 bytes
// straight into B-operand registers, the loads of UNR K steps issued before their MFMAs); they
// serve shapes whose per-wavefront K range is not a multiple of 64.  up_skinny_t /
// down_skinny_t load 128 bytes of a row per 8 lanes instead, which the memory system serves
// at a higher rate (every 128-byte line fetched by one instruction, not two), and reorder the
// data into fragments through LDS.

template <int U, int MT, int NB, bool COH = false>
__device__ __forceinline__ void skinny_batch(const bf16_t* const (&pb)[NB], const bf16_t* const (&px)[MT],
                                             const bool (&okx)[MT], int k0,
                                             floatx4 (&acc)[MT][NB]) {
  const bf16x8 zero8 = {};
  bf16x8 b[NB][U], ax[MT][U];
#pragma unroll
  for (int s = 0; s < U; ++s)
#pragma unroll
    for (int j = 0; j < NB; ++j) b[j][s] = load8(pb[j] + k0 + s * 32);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < U; ++s) ax[mt][s] = okx[mt] ? load_act8<COH>(px[mt] + k0 + s * 32) : zero8;
#pragma unroll
  for (int s = 0; s < U; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[mt][s], b[j][s], acc[mt][j], 0, 0, 0);
}
// K steps [k0, kend) (multiples of 32) in batches of U, then of 2 and 1 for the remainder
template <int U, int MT, int NB, bool COH = false>
__device__ __forceinline__ void skinny_k_range(const bf16_t* const (&pb)[NB], const bf16_t* const (&px)[MT],
                                               const bool (&okx)[MT], int k0, int kend,
                                               floatx4 (&acc)[MT][NB]) {
  for (; k0 + U * 32 <= kend; k0 += U * 32) skinny_batch<U, MT, NB, COH>(pb, px, okx, k0, acc);
  for (; k0 + 2 * 32 <= kend; k0 += 2 * 32) skinny_batch<2, MT, NB, COH>(pb, px, okx, k0, acc);
  if (k0 < kend) skinny_batch<1, MT, NB, COH>(pb, px, okx, k0, acc);
}
// the fixed-order K reduction over the KS wavefronts of a column group nt, through the LDS
// buffer red (KS*NT*MT*NB*64 entries); the wavefront with ks = 0 returns true with the sums
template <int KS, int NT, int MT, int NB>
__device__ __forceinline__ bool skinny_reduce(floatx4 (&acc)[MT][NB], int ks, int nt, int lane,
                                              floatx4* red) {
  if constexpr (KS == 1) return true;
  auto at = [&](int q, int mt, int j) -> floatx4& {
    return red[(((q * NT + nt) * MT + mt) * NB + j) * 64 + lane];
  };
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NB; ++j) at(ks, mt, j) = acc[mt][j];
  __syncthreads();
  if (ks != 0) return false;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[mt][j] = at(0, mt, j);
#pragma unroll
      for (int q = 1; q < KS; ++q) acc[mt][j] += at(q, mt, j);
    }
  return true;
}

// Phase 1, skinny: one workgroup = (expert, 16*NT*NC intermediate columns): NT column groups of
// NC tiles, each group's K split over KS = 4/NT wavefronts.  MT = number of 16-row M tiles
// (rows of the expert, <= 16*MT).  B operands j < NC: gate tiles, j >= NC: up tiles.
template <int NT, int NC, int MT, bool COH = false>
__device__ __forceinline__ void up_skinny(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                          floatx4* red) {
  constexpr int KS = 4 / NT;
  constexpr int UNR = NC == 1 && MT == 1 ? 8 : 4;
  const int H = (int)a.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nt = wave % NT, ks = wave / NT;
  const int i0 = (bx * NT + nt) * 16 * NC;
  const bf16_t* wg = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I;
  const bf16_t* wu = wg + a.H * a.I;
  const int r16 = lane & 15, kg = (lane >> 4) * 8;
  const bf16_t* pb[2 * NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    pb[c] = wg + (int64_t)(i0 + 16 * c + r16) * H + kg;
    pb[NC + c] = wu + (int64_t)(i0 + 16 * c + r16) * H + kg;
  }
  const bf16_t* px[MT];
  bool okx[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 16 + r16;
    okx[mt] = r < n;
    const int64_t t = okx[mt] ? a.rows[start + r] : 0;
    px[mt] = a.x + t * a.H + kg;
  }
  floatx4 acc[MT][2 * NC];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2 * NC; ++j) acc[mt][j] = floatx4{0, 0, 0, 0};
  const int steps = H / 32;
  skinny_k_range<UNR>(pb, px, okx, ks * steps / KS * 32, (ks + 1) * steps / KS * 32, acc);
  if (!skinny_reduce<KS, NT>(acc, ks, nt, lane, red)) return;
  // 16x16 accumulator layout: column = lane & 15, rows (lane >> 4) * 4 + [0, 4)
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = i0 + 16 * c + (lane & 15);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = mt * 16 + (lane >> 4) * 4 + q;
        if (r < n) {
          const float g = bf16r(acc[mt][c][q]), u = bf16r(acc[mt][NC + c][q]);
          store_act<COH>(&a.act[(start + r) * a.I + col], f32_to_bf16(silu_mul(g, u)));
        }
      }
    }
  }
}
// Phase 1, skinny, at most 16 rows (decode): one workgroup = (expert, 16 intermediate columns),
// K split over the four wavefronts as above, but the weights are loaded 128 bytes of a row per
// lane group (8 rows x 128 B per instruction, every 128-byte line fetched by one instruction)
// rather than in the MFMA fragment order (16 rows x 64 B, each line fetched by two).  Each
// wavefront turns them into B fragments through its own 4 KiB LDS tile, one K chunk of 64 at a
// time: 32 rows (gate 0-15, up 16-31) x 128 B, chunk c of row r at slot c ^ ((r >> 1) & 7), which
// keeps the fragment reads free of bank conflicts.  NCH chunks of loads are in flight.
template <int NCH, bool COH = false>
__device__ __forceinline__ void up_skinny_t(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                            floatx4* red, char* tile) {
  const int H = (int)a.H;
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int i0 = bx * 16;
  const bf16_t* wg = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I;
  const bf16_t* wu = wg + a.H * a.I;
  const int lr = lane >> 3, lc = lane & 7, r16 = lane & 15, kg = (lane >> 4) * 8;
  // row group g: rows 8g + lr of the tile (g = 0, 1 gate, 2, 3 up)
  const bf16_t* prow[4];
  uint32_t woff[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    prow[g] = (g < 2 ? wg : wu) + (int64_t)(i0 + 8 * (g & 1) + lr) * H + lc * 8;
    const int row = 8 * g + lr;
    woff[g] = (uint32_t)(row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
  }
  // fragment reads, K step s of a chunk: row r16 (gate) or 16 + r16 (up), chunk 4s + lane/16
  uint32_t roff[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 16 * j + r16;
      roff[st][j] = (uint32_t)(row * 128 + (((4 * st + (lane >> 4)) ^ ((row >> 1) & 7)) << 4));
    }
  const bool okx = r16 < n;
  const bf16_t* px = a.x + (okx ? a.rows[start + r16] : 0) * a.H + kg;
  floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
  const bf16x8 zero8 = {};
  auto batch = [&](int k0, auto nch) {
    constexpr int N = decltype(nch)::value;
    u32x4 w[N][4];
#pragma unroll
    for (int ch = 0; ch < N; ++ch)
#pragma unroll
      for (int g = 0; g < 4; ++g) w[ch][g] = *reinterpret_cast<const u32x4*>(prow[g] + k0 + 64 * ch);
    bf16x8 xa[2 * N];
#pragma unroll
    for (int st = 0; st < 2 * N; ++st) xa[st] = okx ? load8(px + k0 + 32 * st) : zero8;
#pragma unroll
    for (int ch = 0; ch < N; ++ch) {
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<u32x4*>(tile + woff[g]) = w[ch][g];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const bf16x8 bg = *reinterpret_cast<const bf16x8*>(tile + roff[st][0]);
        const bf16x8 bu = *reinterpret_cast<const bf16x8*>(tile + roff[st][1]);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], bg, acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], bu, acc[1], 0, 0, 0);
      }
    }
  };
  const int kb = ks * (H / 4), ke = kb + H / 4;   // H / 4 is a multiple of 64
  int k0 = kb;
  for (; k0 + 64 * NCH <= ke; k0 += 64 * NCH) batch(k0, std::integral_constant<int, NCH>{});
  for (; k0 < ke; k0 += 64) batch(k0, std::integral_constant<int, 1>{});
  floatx4 accm[1][2] = {{acc[0], acc[1]}};
  if (!skinny_reduce<4, 1>(accm, ks, 0, lane, red)) return;
  const int col = i0 + (lane & 15);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (lane >> 4) * 4 + q;
    if (r < n) {
      const float g = bf16r(accm[0][0][q]), u = bf16r(accm[0][1][q]);
      store_act<COH>(&a.act[(start + r) * a.I + col], f32_to_bf16(silu_mul(g, u)));
    }
  }
}

// Phase 2, skinny: one workgroup = (expert, 16*NT*NC hidden rows), laid out as phase 1.
template <int NT, int NC, int MT, bool COH = false>
__device__ __forceinline__ void down_skinny(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                            floatx4* red) {
  constexpr int KS = 4 / NT;
  constexpr int UNR = NC == 1 ? 8 : 4;
  const int I = (int)a.I;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nt = wave % NT, ks = wave / NT;
  const int h0 = (bx * NT + nt) * 16 * NC;
  const bf16_t* wd = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I + 2 * a.H * a.I;
  const int r16 = lane & 15, kg = (lane >> 4) * 8;
  const bf16_t* pb[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) pb[c] = wd + (int64_t)(h0 + 16 * c + r16) * I + kg;
  const bf16_t* pa[MT];
  bool oka[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 16 + r16;
    oka[mt] = r < n;
    pa[mt] = a.act + (start + (oka[mt] ? r : 0)) * a.I + kg;
  }
  floatx4 acc[MT][NC];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[mt][c] = floatx4{0, 0, 0, 0};
  const int steps = I / 32;
  skinny_k_range<UNR, MT, NC, COH>(pb, pa, oka, ks * steps / KS * 32, (ks + 1) * steps / KS * 32,
                                   acc);
  if (!skinny_reduce<KS, NT>(acc, ks, nt, lane, red)) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = mt * 16 + (lane >> 4) * 4 + q;
      if (r < n) {
        const int64_t p = start + r;
        const int64_t t = a.rows[p], j = a.cols[p];
        const float wt = bf16_to_f32(a.w[t * a.k + j]);
        const int64_t orow = a.out_mode == 0 ? t * a.k + j : p;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          a.out[orow * a.H + h0 + 16 * c + (lane & 15)] = f32_to_bf16(bf16r(acc[mt][c][q]) * wt);
      }
    }
  }
}
// Phase 2, skinny, at most 16 rows (decode): one workgroup = (expert, 64 hidden rows), K split
// over the four wavefronts; the weights go through the wavefront's LDS tile as in up_skinny_t,
// 32 rows (two 16-row column tiles) at a time.
template <int NCH, bool COH = false>
__device__ __forceinline__ void down_skinny_t(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                              floatx4* red, char* tile) {
  const int I = (int)a.I;
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int h0 = bx * 64;
  const bf16_t* wd = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I + 2 * a.H * a.I;
  const int lr = lane >> 3, lc = lane & 7, r16 = lane & 15, kg = (lane >> 4) * 8;
  // row group g (< 8): rows h0 + 8g + lr, at p0 + g * gstride; tile row (8g + lr) % 32
  const bf16_t* p0 = wd + (int64_t)(h0 + lr) * I + lc * 8;
  const int64_t gstride = (int64_t)8 * I;
  uint32_t woff[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int row = 8 * g + lr;
    woff[g] = (uint32_t)(row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
  }
  uint32_t roff[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 16 * j + r16;
      roff[st][j] = (uint32_t)(row * 128 + (((4 * st + (lane >> 4)) ^ ((row >> 1) & 7)) << 4));
    }
  const bool oka = r16 < n;
  const bf16_t* pa = a.act + (start + (oka ? r16 : 0)) * a.I + kg;
  // the token and slot index of the expert's row lane % 16, loaded ahead of the weights by the
  // wavefront that writes the output (the epilogue takes them from that lane by a shuffle)
  int32_t row_t = 0, row_j = 0;
  if (ks == 0) {
    const int64_t p = start + (r16 < n ? r16 : 0);
    row_t = (int32_t)a.rows[p];
    row_j = (int32_t)a.cols[p];
  }
  floatx4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = floatx4{0, 0, 0, 0};
  const bf16x8 zero8 = {};
  auto batch = [&](int k0, auto nch) {
    constexpr int N = decltype(nch)::value;
    u32x4 w[N][8];
#pragma unroll
    for (int ch = 0; ch < N; ++ch)
#pragma unroll
      for (int g = 0; g < 8; ++g) w[ch][g] = *reinterpret_cast<const u32x4*>(p0 + g * gstride + k0 + 64 * ch);
    bf16x8 xa[2 * N];
#pragma unroll
    for (int st = 0; st < 2 * N; ++st) xa[st] = oka ? load_act8<COH>(pa + k0 + 32 * st) : zero8;
#pragma unroll
    for (int ch = 0; ch < N; ++ch) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<u32x4*>(tile + woff[g]) = w[ch][4 * h + g];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(tile + roff[st][0]);
          const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(tile + roff[st][1]);
          acc[2 * h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], b0, acc[2 * h], 0, 0, 0);
          acc[2 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], b1, acc[2 * h + 1], 0, 0, 0);
        }
      }
    }
  };
  const int kb = ks * (I / 4), ke = kb + I / 4;   // I / 4 is a multiple of 64
  int k0 = kb;
  for (; k0 + 64 * NCH <= ke; k0 += 64 * NCH) batch(k0, std::integral_constant<int, NCH>{});
  for (; k0 < ke; k0 += 64) batch(k0, std::integral_constant<int, 1>{});
  floatx4 accm[1][4] = {{acc[0], acc[1], acc[2], acc[3]}};
  // the routing weight of each output row, loaded before the K reduction (whose barrier waits
  // for the other wavefronts)
  int32_t lane_orow = 0;
  float lane_wt = 0.0f;
  if (ks == 0) {
    const int64_t tj = (int64_t)row_t * a.k + row_j;
    lane_wt = bf16_to_f32(a.w[tj]);
    lane_orow = a.out_mode == 0 ? (int32_t)tj : (int32_t)(start + (r16 < n ? r16 : 0));
  }
  if (!skinny_reduce<4, 1>(accm, ks, 0, lane, red)) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (lane >> 4) * 4 + q;
    const int64_t orow = __shfl(lane_orow, r);
    const float wt = __shfl(lane_wt, r);
    if (r < n) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        a.out[orow * a.H + h0 + 16 * c + (lane & 15)] = f32_to_bf16(bf16r(accm[0][c][q]) * wt);
    }
  }
}

// 16-byte global load into registers (saddr + 32-bit lane byte offset) as inline asm: the
// compiler does not track it, so the registers are read only after vmcnt_tie names them.
__device__ __forceinline__ void gload16(bf16x8& v, const void* sbase, uint32_t voff) {
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(voff), "s"(sbase) : "memory");
}
// wait until at most N vector loads are outstanding; the registers named are those loads'
// destinations, tied so that no use of them is scheduled before the wait
template <int N>
__device__ __forceinline__ void vmcnt_tie(bf16x8 (&r)[8]) {
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]),
                 "+v"(r[6]), "+v"(r[7])
               : "n"(N)
               : "memory");
}
template <int N>
__device__ __forceinline__ void vmcnt_tie(bf16x8 (&r)[2]) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(r[0]), "+v"(r[1]) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void vmcnt_tie(bf16x8 (&r)[4]) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]) : "n"(N) : "memory");
}

// f(integral_constant<int, i>) for i = B .. E - 1, unrolled at compile time
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}
template <int OFF>
__device__ __forceinline__ void gload16o(bf16x8& v, const void* sbase, uint32_t voff) {
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3"
               : "=v"(v)
               : "v"(voff), "s"(sbase), "n"(OFF)
               : "memory");
}
// gload16o for activation rows: agent-coherent (sc1) under COH, see store_act
template <int OFF, bool COH>
__device__ __forceinline__ void gload16o_act(bf16x8& v, const void* sbase, uint32_t voff) {
  if constexpr (COH)
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3 sc1"
                 : "=v"(v)
                 : "v"(voff), "s"(sbase), "n"(OFF)
                 : "memory");
  else
    gload16o<OFF>(v, sbase, voff);
}

// Phase 1, skinny, at most 16 rows, H = 512 * NB: up_skinny_t's tile scheme with the K range of
// each wavefront walked in NB batches of two 64-element chunks, software-pipelined -- the loads
// of batch b + 1 are issued before batch b goes through the tile and the matrix cores, so that a
// wavefront always has a batch in flight.  All loads are inline asm (saddr + 32-bit lane offset:
// two registers per batch set instead of a 64-bit address per load), 12 per batch in a fixed
// order (8 weight loads, then 4 token-row loads; padding rows load token row 0 and are zeroed
// after the wait), so each wait has a fixed count of younger loads.  The batch loop is fully
// unrolled: no loop-carried register holds a load in flight.
template <int NB, bool COH = false>
__device__ __forceinline__ void up_skinny_p(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                            floatx4* red, char* tile) {
  static_assert(NB >= 2 && NB % 2 == 0, "an even number of batches");
  constexpr int H = 512 * NB;
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int i0 = bx * 16;
  const bf16_t* wg = uniform_ptr(a.cache + (int64_t)a.list.slot[li] * 3 * H * a.I);
  const bf16_t* xs = uniform_ptr(a.x);
  const int lr = lane >> 3, lc = lane & 7, r16 = lane & 15, kg = (lane >> 4) * 8;
  // byte offsets of the wavefront's K range: row group g = rows 8 (g & 1) + lr of the gate
  // (g < 2) or up (g >= 2) projection; the group offsets are wavefront-uniform
  const int kb = ks * (H / 4);
  const uint32_t wrow = (uint32_t)(((i0 + lr) * H + lc * 8 + kb) * 2);
  const uint32_t gup = (uint32_t)(H * a.I * 2);
  uint32_t woff[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int row = 8 * g + lr;
    woff[g] = (uint32_t)(row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
  }
  uint32_t roff[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 16 * j + r16;
      roff[st][j] = (uint32_t)(row * 128 + (((4 * st + (lane >> 4)) ^ ((row >> 1) & 7)) << 4));
    }
  const bool okx = r16 < n;
  floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
  const bf16x8 zero8 = {};
  // batch b: weights w[4 ch + g] (chunk ch of row group g), token rows xa[st] (K step st)
  uint32_t xrow;
  auto load_w = [&](auto b, bf16x8 (&w)[8]) {
    constexpr uint32_t kbyte = decltype(b)::value * 256;
    gload16o<0>(w[0], wg, wrow + kbyte);
    gload16o<0>(w[1], wg, wrow + kbyte + 16 * H);
    gload16o<0>(w[2], wg, wrow + kbyte + gup);
    gload16o<0>(w[3], wg, wrow + kbyte + gup + 16 * H);
    gload16o<128>(w[4], wg, wrow + kbyte);
    gload16o<128>(w[5], wg, wrow + kbyte + 16 * H);
    gload16o<128>(w[6], wg, wrow + kbyte + gup);
    gload16o<128>(w[7], wg, wrow + kbyte + gup + 16 * H);
  };
  auto load_x = [&](auto b, bf16x8 (&xa)[4]) {
    constexpr uint32_t kbyte = decltype(b)::value * 256;
    gload16o<0>(xa[0], xs, xrow + kbyte);
    gload16o<64>(xa[1], xs, xrow + kbyte);
    gload16o<128>(xa[2], xs, xrow + kbyte);
    gload16o<192>(xa[3], xs, xrow + kbyte);
  };
  auto mma = [&](bf16x8 (&w)[8], bf16x8 (&xa)[4]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) xa[st] = okx ? xa[st] : zero8;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<bf16x8*>(tile + woff[g]) = w[4 * ch + g];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const bf16x8 bg = *reinterpret_cast<const bf16x8*>(tile + roff[st][0]);
        const bf16x8 bu = *reinterpret_cast<const bf16x8*>(tile + roff[st][1]);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], bg, acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[2 * ch + st], bu, acc[1], 0, 0, 0);
      }
    }
  };
  auto load = [&](auto b, bf16x8 (&w)[8], bf16x8 (&xa)[4]) {
    load_w(b, w);
    load_x(b, xa);
  };
  // the token row of each lane (padding rows: row 0) is loaded ahead of the first weights and
  // awaited behind them, so the first batch keeps the fixed order of 8 weight and 4 row loads
  // (the low word suffices: token indices times H stay below 2^31)
  uint32_t trow;
  asm volatile("global_load_dword %0, %1, %2"
               : "=v"(trow)
               : "v"((uint32_t)((okx ? r16 : 0) * 8)), "s"(uniform_ptr(a.rows + start))
               : "memory");
  bf16x8 wA[8], wB[8], xA[4], xB[4];
  load_w(std::integral_constant<int, 0>{}, wA);
  asm volatile("s_waitcnt vmcnt(8)" : "+v"(trow) : : "memory");
  xrow = (trow * H + kg + kb) * 2;
  load_x(std::integral_constant<int, 0>{}, xA);
  static_for<0, NB / 2 - 1>([&](auto j) {
    load(std::integral_constant<int, 2 * decltype(j)::value + 1>{}, wB, xB);
    vmcnt_tie<12>(wA);
    vmcnt_tie<12>(xA);
    mma(wA, xA);
    load(std::integral_constant<int, 2 * decltype(j)::value + 2>{}, wA, xA);
    vmcnt_tie<12>(wB);
    vmcnt_tie<12>(xB);
    mma(wB, xB);
  });
  load(std::integral_constant<int, NB - 1>{}, wB, xB);
  vmcnt_tie<12>(wA);
  vmcnt_tie<12>(xA);
  mma(wA, xA);
  vmcnt_tie<0>(wB);
  vmcnt_tie<0>(xB);
  mma(wB, xB);
  floatx4 accm[1][2] = {{acc[0], acc[1]}};
  if (!skinny_reduce<4, 1>(accm, ks, 0, lane, red)) return;
  const int col = i0 + (lane & 15);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (lane >> 4) * 4 + q;
    if (r < n) {
      const float g = bf16r(accm[0][0][q]), u = bf16r(accm[0][1][q]);
      store_act<COH>(&a.act[(start + r) * a.I + col], f32_to_bf16(silu_mul(g, u)));
    }
  }
}

// Phase 2, skinny, at most 16 rows, I = 256 * NC: down_skinny_t's tile scheme with each
// wavefront's K range walked one 64-element chunk at a time, software-pipelined over two register
// sets -- chunk c + 1 is loaded while chunk c goes through the tile and the matrix cores.  Ten
// asm loads per chunk in a fixed order (eight 8-row weight groups, then two activation loads;
// padding rows load the expert's first row and are zeroed after the wait).  Fully unrolled.
template <int NC, bool COH = false>
__device__ __forceinline__ void down_skinny_p(const FfnArgs& a, int li, int64_t start, int n, int bx,
                                              floatx4* red, char* tile) {
  constexpr int I = 256 * NC;
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int h0 = bx * 64;
  const bf16_t* wd =
      uniform_ptr(a.cache + (int64_t)a.list.slot[li] * 3 * a.H * I + 2 * a.H * I);
  const bf16_t* as = uniform_ptr(a.act + start * I);
  const int lr = lane >> 3, lc = lane & 7, r16 = lane & 15, kg = (lane >> 4) * 8;
  const int kb = ks * (I / 4);
  // row group g (< 8): rows h0 + 8g + lr, byte offset wrow + g * 16 I; tile row (8g + lr) % 32
  const uint32_t wrow = (uint32_t)(((h0 + lr) * I + lc * 8 + kb) * 2);
  uint32_t woff[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int row = 8 * g + lr;
    woff[g] = (uint32_t)(row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
  }
  uint32_t roff[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 16 * j + r16;
      roff[st][j] = (uint32_t)(row * 128 + (((4 * st + (lane >> 4)) ^ ((row >> 1) & 7)) << 4));
    }
  const bool oka = r16 < n;
  const uint32_t arow = (uint32_t)(((oka ? r16 : 0) * I + kg + kb) * 2);
  floatx4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = floatx4{0, 0, 0, 0};
  const bf16x8 zero8 = {};
  auto load = [&](auto c, bf16x8 (&w)[8], bf16x8 (&xa)[2]) {
    constexpr uint32_t kbyte = decltype(c)::value * 128;
#pragma unroll
    for (int g = 0; g < 8; ++g) gload16o<0>(w[g], wd, wrow + kbyte + g * 16 * I);
    gload16o_act<0, COH>(xa[0], as, arow + kbyte);
    gload16o_act<64, COH>(xa[1], as, arow + kbyte);
  };
  auto mma = [&](bf16x8 (&w)[8], bf16x8 (&xa)[2]) {
#pragma unroll
    for (int st = 0; st < 2; ++st) xa[st] = oka ? xa[st] : zero8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<bf16x8*>(tile + woff[g]) = w[4 * h + g];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(tile + roff[st][0]);
        const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(tile + roff[st][1]);
        acc[2 * h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[st], b0, acc[2 * h], 0, 0, 0);
        acc[2 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[st], b1, acc[2 * h + 1], 0, 0, 0);
      }
    }
  };
  // the token and slot index of the expert's row lane % 16, loaded ahead of the weights by the
  // wavefront that writes the output (the epilogue takes them from that lane by a shuffle)
  int32_t row_t = 0, row_j = 0;
  if (ks == 0) {
    const int64_t p = start + (r16 < n ? r16 : 0);
    row_t = (int32_t)a.rows[p];
    row_j = (int32_t)a.cols[p];
  }
  bf16x8 wA[8], wB[8], xA[2], xB[2];
  load(std::integral_constant<int, 0>{}, wA, xA);
  static_for<0, NC>([&](auto c) {
    constexpr int C = decltype(c)::value;
    auto& wc = (C % 2 == 0) ? wA : wB;
    auto& xc = (C % 2 == 0) ? xA : xB;
    auto& wn = (C % 2 == 0) ? wB : wA;
    auto& xn = (C % 2 == 0) ? xB : xA;
    if constexpr (C + 1 < NC) {
      load(std::integral_constant<int, C + 1>{}, wn, xn);
      vmcnt_tie<10>(wc);
      vmcnt_tie<10>(xc);
    } else {
      vmcnt_tie<0>(wc);
      vmcnt_tie<0>(xc);
    }
    mma(wc, xc);
  });
  floatx4 accm[1][4] = {{acc[0], acc[1], acc[2], acc[3]}};
  // the routing weight of each output row, loaded before the K reduction (whose barrier waits
  // for the other wavefronts)
  int32_t lane_orow = 0;
  float lane_wt = 0.0f;
  if (ks == 0) {
    const int64_t tj = (int64_t)row_t * a.k + row_j;
    lane_wt = bf16_to_f32(a.w[tj]);
    lane_orow = a.out_mode == 0 ? (int32_t)tj : (int32_t)(start + (r16 < n ? r16 : 0));
  }
  if (!skinny_reduce<4, 1>(accm, ks, 0, lane, red)) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (lane >> 4) * 4 + q;
    const int64_t orow = __shfl(lane_orow, r);
    const float wt = __shfl(lane_wt, r);
    if (r < n) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        a.out[orow * a.H + h0 + 16 * c + (lane & 15)] = f32_to_bf16(bf16r(accm[0][c][q]) * wt);
    }
  }
}

// =============================================================================================
// Mid kernels
// =============================================================================================

// Mid scheme (experts with 17-64 rows, prefill).  The skinny kernels read an expert's token rows
// once per 16 output columns, which at 64 rows is twice the weight bytes; here a workgroup covers
// 64 columns and reads them once.  One workgroup = (expert, 64 output columns), four wavefronts,
// each a 16-column group over the full K (phase 1: its 16 gate and 16 up columns).  Rows are held
// in 16-row M tiles (MT of them).  K is walked in chunks of 64:
//  * the token rows go through a ring of three 8 KiB LDS buffers, staged by direct loads (8 rows
//    x 128 B each, XD per wavefront) two chunks ahead; 128-byte rows, chunk j of row r at slot
//    j ^ ((r >> 1) & 7), so that the A-fragment reads are free of bank conflicts;
//  * the weights, read exactly once, are loaded 8 rows x 128 B per instruction (every 128-byte
//    line fetched by one instruction) into a ring of three register sets three chunks ahead, and
//    each chunk goes through the wavefront's 2 KiB LDS tile (16 rows x 128 B) into B fragments.
// Per wavefront and chunk the loads are issued in a fixed order -- XD token-row loads at the top
// of the chunk, NW weight loads after the tile writes -- so every wait has a fixed count of
// younger loads.
constexpr int kMidXBuf = 64 * 128;                    // token-row ring buffer (64 rows x 128 B)
constexpr int kMidLds = 3 * kMidXBuf + 4 * 2048;      // ring + four wavefront tiles: 32 KiB

template <int N>
__device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory"); }

template <int MODE, int MT>
__device__ __forceinline__ void ffn_mid_body_t(const FfnArgs& a, int li, int64_t start, int n,
                                               int bx, char* sm) {
  static_assert(MT == 1 || MT == 2 || MT == 4, "MT 16-row tiles");
  // token-row direct loads per wavefront and chunk (MT = 1 stages 32 rows, of which 16 are used)
  constexpr int XD = MT >= 2 ? MT / 2 : 1;
  constexpr int NB = MODE == 0 ? 2 : 1;
  constexpr int NW = 2 * NB;                 // weight loads per wavefront and chunk
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = (int)(MODE == 0 ? a.H : a.I);
  const int C = K / 64;
  const int lr = lane >> 3, lc = lane & 7, r16 = lane & 15;
  const uint32_t lds0 = lds_addr(sm);
  char* tile = sm + 3 * kMidXBuf + wave * 2048;
  // token rows: direct load i of this wavefront moves rows 8 (XD wave + i) + lr
  const char* xbase = reinterpret_cast<const char*>(MODE == 0 ? a.x : a.act);
  uint32_t xoff[XD];
#pragma unroll
  for (int i = 0; i < XD; ++i) {
    const int r = 8 * (XD * wave + i) + lr;
    const int rr = r < n ? r : 0;   // rows past the expert's last load a valid row
    const uint32_t t = MODE == 0 ? (uint32_t)a.rows[start + rr] : (uint32_t)(start + rr);
    xoff[i] = t * (uint32_t)(K * 2) + (uint32_t)((lc ^ ((r >> 1) & 7)) << 4);
  }
  auto stage = [&](int c) {   // chunks past the last restage it into a buffer nobody reads
    const int cc = c < C ? c : C - 1;
    const uint32_t dst = lds0 + (uint32_t)((c % 3) * kMidXBuf + XD * wave * 1024);
#pragma unroll
    for (int i = 0; i < XD; ++i) dma16(xbase + cc * 128, xoff[i], dst + (uint32_t)(i * 1024));
  };
  // weights: row group g (< NW) = rows 8 (g & 1) + lr of gate (g < 2) or up / down, 128 B of
  // the chunk per lane group
  const int col0 = bx * 64 + wave * 16;
  const bf16_t* slot = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I;
  const bf16_t* wbase = uniform_ptr(slot + (MODE == 0 ? (int64_t)col0 * a.H
                                                      : 2 * a.H * a.I + (int64_t)col0 * a.I));
  uint32_t woff[NW];
#pragma unroll
  for (int g = 0; g < NW; ++g)
    woff[g] = (uint32_t)(((g >= 2 ? a.H * a.I : 0) + (int64_t)(8 * (g & 1) + lr) * K + lc * 8) * 2);
  bf16x8 wb[3][NW];
  auto wload = [&](int c, bf16x8 (&w)[NW]) {   // chunks past the last reload it
    const int cc = c < C ? c : C - 1;
    const char* b = reinterpret_cast<const char*>(wbase) + cc * 128;
#pragma unroll
    for (int g = 0; g < NW; ++g) gload16(w[g], b, woff[g]);
  };
  // tile rows: write row group g2 (< 2) at rows 8 g2 + lr; fragment read of K step st: row r16,
  // chunk 4 st + lane / 16
  uint32_t twoff[2], troff[2], aoff[2];
#pragma unroll
  for (int g2 = 0; g2 < 2; ++g2) {
    const int row = 8 * g2 + lr;
    twoff[g2] = (uint32_t)(row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
  }
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    troff[st] = (uint32_t)(r16 * 128 + (((4 * st + (lane >> 4)) ^ ((r16 >> 1) & 7)) << 4));
    aoff[st] = troff[st];   // token-row fragments: the same layout, rows mt*16 + r16
  }
  floatx4 acc[MT][NB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[mt][j] = floatx4{0, 0, 0, 0};
  auto chunk = [&](int c, auto par) {
    constexpr int P = decltype(par)::value;   // c % 3
    wg_barrier();             // chunk c staged by every wavefront; chunk c-1's buffer free
    stage(c + 2);
    // this chunk's weights: older than x(c), w(c+1), x(c+1), w(c+2), x(c+2)
    vmcnt_tie<3 * XD + 2 * NW>(wb[P]);
    bf16x8 bfr[NB][2];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) *reinterpret_cast<bf16x8*>(tile + twoff[g2]) = wb[P][2 * j + g2];
#pragma unroll
      for (int st = 0; st < 2; ++st) bfr[j][st] = *reinterpret_cast<const bf16x8*>(tile + troff[st]);
    }
    wload(c + 3, wb[P]);
    const char* xb = sm + P * kMidXBuf;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      bf16x8 xa[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xa[mt] = *reinterpret_cast<const bf16x8*>(xb + mt * 16 * 128 + aoff[st]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mt], bfr[j][st], acc[mt][j], 0, 0, 0);
    }
    // token rows of chunk c+1 landed: older than w(c+2), x(c+2), w(c+3)
    wait_vmcnt<2 * NW + XD>();
  };
  // phase 2: lane l loads the token and slot index of the expert's row l ahead of the weights,
  // so that after the K loop only the routing weight's load (which depends on them) is left;
  // the epilogue takes each row's output offset and weight from its lane by a shuffle
  int32_t row_t = 0, row_j = 0;
  if (MODE == 1) {
    const int64_t p = start + (lane < n ? lane : 0);
    row_t = (int32_t)a.rows[p];
    row_j = (int32_t)a.cols[p];
  }
  // prologue in the steady-state order: w(0), x(0), w(1), x(1), w(2)
  wload(0, wb[0]);
  stage(0);
  wload(1, wb[1]);
  stage(1);
  wload(2, wb[2]);
  wait_vmcnt<2 * NW + XD>();   // x(0) landed
  for (int c = 0; c < C; c += 3) {
    chunk(c, std::integral_constant<int, 0>{});
    if (c + 1 < C) chunk(c + 1, std::integral_constant<int, 1>{});
    if (c + 2 < C) chunk(c + 2, std::integral_constant<int, 2>{});
  }
  // the loads past the last chunk are never used: hold their registers (and the LDS) until
  // they landed
  wait_vmcnt<0>();
  vmcnt_tie<0>(wb[0]);
  vmcnt_tie<0>(wb[1]);
  vmcnt_tie<0>(wb[2]);
  // 16x16 accumulator layout: column = lane & 15, rows (lane >> 4) * 4 + [0, 4)
  const int col = col0 + (lane & 15);
  int32_t lane_orow = 0;
  float lane_wt = 0.0f;
  if (MODE == 1) {
    const int64_t tj = (int64_t)row_t * a.k + row_j;
    lane_wt = bf16_to_f32(a.w[tj]);
    lane_orow = a.out_mode == 0 ? (int32_t)tj : (int32_t)(start + (lane < n ? lane : 0));
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = mt * 16 + (lane >> 4) * 4 + q;
      if (MODE == 0) {
        if (r < n) {
          const float g = bf16r(acc[mt][0][q]), u = bf16r(acc[mt][NB - 1][q]);
          a.act[(start + r) * a.I + col] = f32_to_bf16(silu_mul(g, u));
        }
      } else {
        const int64_t orow = __shfl(lane_orow, r);
        const float wt = __shfl(lane_wt, r);
        if (r < n) a.out[orow * a.H + col] = f32_to_bf16(bf16r(acc[mt][0][q]) * wt);
      }
    }
  }
}

// Small experts (at most 64 rows), one launch for a list of mixed sizes so that together they
// fill the GPU: up to 16 rows the skinny scheme, 17-64 rows the mid scheme.  MTMAX = 1 when no
// expert of the list has more than 16 rows: then only the skinny scheme is compiled in and a
// phase-1 workgroup covers 16 intermediate columns (grid (I / 16, list)).  Otherwise the grid
// is one-dimensional: the list's first n_mid entries (those the host knows to have 17-64 rows)
// take I / 64 workgroups of 64 columns each, the rest I / 16 workgroups of 16 columns each, so
// that the larger workgroups are dispatched first.  A workgroup whose expert turns out to have
// the other scheme's row count still covers its columns: a 64-column workgroup of an expert with
// at most 16 rows runs four 16-column skinny passes (a one-tile mid workgroup when H is not a
// multiple of 256); of the four 16-column workgroups of a 64-column block of an expert with more
// than 16 rows, the first runs the block's mid workgroup and the others return.  Phase 2: 64
// hidden rows per workgroup in both schemes (grid (H / 64, list)).
template <int MTMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void ffn_up_skinny(FfnArgs a) {
  // MTMAX = 1: the K-reduction buffer (8 KiB) and four 4 KiB weight tiles
  __shared__ __attribute__((aligned(1024))) char sm[MTMAX > 1 ? kMidLds : 8192 + 4 * 4096];
  int li = blockIdx.y, bx = blockIdx.x;
  bool wide = false;   // a 64-column workgroup
  if (MTMAX > 1) {
    const int per_mid = (int)(a.I / 64), per_sk = (int)(a.I / 16);
    const int mid_wgs = a.list.n_mid * per_mid;
    const int b = blockIdx.x;
    wide = b < mid_wgs;
    li = wide ? b / per_mid : a.list.n_mid + (b - mid_wgs) / per_sk;
    bx = wide ? b % per_mid : (b - mid_wgs) % per_sk;
  }
  if (li >= a.list.n) return;
  const int e = a.list.expert[li];
  const int64_t start = a.starts[e];
  const int n = (int)(a.starts[e + 1] - start);
  if (n == 0 || n > 16 * MTMAX) return;
  if (MTMAX == 1 || (!wide && n <= 16)) {
    if (a.H == 2048)
      up_skinny_p<4>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                  sm + 8192 + (threadIdx.x >> 6) * 4096);
    else if (a.H % 256 == 0)
      up_skinny_t<4>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                     sm + 8192 + (threadIdx.x >> 6) * 4096);
    else
      up_skinny<1, 1, 1>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm));
    return;
  }
  if constexpr (MTMAX > 1) {
    if (!wide) {   // 16-column workgroup of an expert with more than 16 rows
      if (bx % 4 != 0) return;
      bx /= 4;
    }
    if (n > 32) {
      ffn_mid_body_t<0, 4>(a, li, start, n, bx, sm);
    } else if (n > 16) {
      ffn_mid_body_t<0, 2>(a, li, start, n, bx, sm);
    } else if (a.H % 256 == 0) {
#pragma unroll 1
      for (int j = 0; j < 4; ++j) {
        up_skinny_t<2>(a, li, start, n, bx * 4 + j, reinterpret_cast<floatx4*>(sm),
                       sm + 8192 + (threadIdx.x >> 6) * 4096);
        __syncthreads();   // the K-reduction buffer is free again
      }
    } else {
      ffn_mid_body_t<0, 1>(a, li, start, n, bx, sm);
    }
  }
}
template <int MTMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void ffn_down_skinny(FfnArgs a) {
  // the K-reduction buffer (16 KiB) and four 4 KiB weight tiles
  __shared__ __attribute__((aligned(1024))) char sm[MTMAX > 1 ? kMidLds : 16384 + 4 * 4096];
  const int li = blockIdx.y;
  if (li >= a.list.n) return;
  const int e = a.list.expert[li];
  const int64_t start = a.starts[e];
  const int n = (int)(a.starts[e + 1] - start);
  if (n == 0 || n > 16 * MTMAX) return;
  if (MTMAX == 1 || n <= 16) {
    if (a.I == 768)
      down_skinny_p<3>(a, li, start, n, blockIdx.x, reinterpret_cast<floatx4*>(sm),
                       sm + 16384 + (threadIdx.x >> 6) * 4096);
    else if (a.I % 256 == 0)
      down_skinny_t<2>(a, li, start, n, blockIdx.x, reinterpret_cast<floatx4*>(sm),
                       sm + 16384 + (threadIdx.x >> 6) * 4096);
    else
      down_skinny<1, 4, 1>(a, li, start, n, blockIdx.x, reinterpret_cast<floatx4*>(sm));
    return;
  }
  if constexpr (MTMAX > 1) {
    if (n > 32)
      ffn_mid_body_t<1, 4>(a, li, start, n, blockIdx.x, sm);
    else
      ffn_mid_body_t<1, 2>(a, li, start, n, blockIdx.x, sm);
  }
}

// =============================================================================================
// Decode: both phases of every expert (at most 16 rows each) in one launch
// =============================================================================================

// The workgroups of ffn_up_skinny<1> (I/16 per expert) come first in the grid, those of
// ffn_down_skinny<1> (H/64 per expert) after them.  A down workgroup needs every intermediate
// column of its expert's activation rows, so it waits for all of that expert's up workgroups:
// each up workgroup, once its rows are stored, sets its arrival flag; a down workgroup's first
// wavefront waits for all flags of its expert.  The L2s of the XCDs are not coherent with
// each other, and a release / acquire pair would write back and invalidate a whole L2 for every
// workgroup (measured: 550 us per launch instead of 30): instead the activation rows themselves
// are stored and loaded agent-coherently (sc1, see store_act), each wavefront waits for its
// stores to complete before the workgroup arrives, and the flags are relaxed agent-scope
// atomic words.  Workgroups are dispatched in index order, so every producer a down
// workgroup waits for has been dispatched before it: the wait ends.  It is still bounded
// (kSyncSpinLimit sleeps, about a second); a down workgroup that runs out counts a timeout and
// skips its expert rather than read unfinished rows.  The count lives in device memory
// (g_sync_timeouts); the history kernel copies it into the caller's mapped host buffer at the
// start of every layer call, so that the runtime raises on the next call's routing readback
// instead of returning unwritten rows as output.
//
// Arrival flags: one 32-bit word per up workgroup, holding the epoch (a number unique to the
// call) once that workgroup's rows are stored.  A down workgroup's first wavefront checks all
// flags of its expert at once (one lane per flag) until every one holds the call's epoch.  Flags
// from earlier calls hold older epochs, so nothing is ever cleared, and no word is written by
// two workgroups (no read-modify-write contention).  The flags live in a static per-device ring
// of kSyncSets sets (set = epoch % kSyncSets); calls that run at the same time on one GPU use
// different sets unless kSyncSets of them overlap.
constexpr int kSyncSets = 8;
constexpr int kMaxUpWgs = 128;   // up workgroups per expert (I / 16): I <= 2048
constexpr int kSyncSpinLimit = 1 << 21;
static __device__ __align__(256) uint32_t g_sync[kSyncSets][kListMax][kMaxUpWgs];
static __device__ int32_t g_sync_timeouts;

struct FusedSync {
  uint32_t* flags;   // the call's flag set (device address of g_sync[epoch % kSyncSets])
  int32_t* timeouts;
  uint32_t epoch;
  int32_t up_wgs;    // up workgroups per expert (I / 16)
  int32_t down_wgs;  // down workgroups per expert (H / 64)
  int32_t spin_limit;  // polls before a down workgroup gives up (0: gives up at once)
};

__device__ __forceinline__ void sync_arrive(const FusedSync& fs, int li, int bx) {
  __hip_atomic_store(fs.flags + li * kMaxUpWgs + bx, fs.epoch, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// wavefront 0 of a down workgroup: true once every up workgroup of list entry li has arrived,
// false on timeout
__device__ __forceinline__ bool sync_wait(const FusedSync& fs, int li) {
  const int lane = threadIdx.x & 63;
  const uint32_t* f = fs.flags + li * kMaxUpWgs;
  for (int spins = 0;; ++spins) {
    if (spins >= fs.spin_limit) {
      if (lane == 0) atomicAdd(fs.timeouts, 1);
      return false;
    }
    bool mine = true;
    for (int j = lane; j < fs.up_wgs; j += 64)
      mine &= __hip_atomic_load(f + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == fs.epoch;
    if (__all(mine)) return true;
    __builtin_amdgcn_s_sleep(8);
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void ffn_skinny_fused(
    FfnArgs a, FusedSync fs) {
  // phase 2's K-reduction buffer (16 KiB; phase 1 uses 8) and four 4 KiB weight tiles
  __shared__ __attribute__((aligned(1024))) char sm[16384 + 4 * 4096];
  __shared__ int ok_s;
  const int nup = fs.up_wgs * a.list.n;
  const bool up = (int)blockIdx.x < nup;
  const int b = up ? (int)blockIdx.x : (int)blockIdx.x - nup;
  const int per = up ? fs.up_wgs : fs.down_wgs;
  const int li = b / per, bx = b % per;
  const int e = a.list.expert[li];
  const int64_t start = a.starts[e];
  const int n = (int)(a.starts[e + 1] - start);
  if (n == 0 || n > 16) return;   // up and down workgroups of such an expert both skip it
  if (up) {
    if (a.H == 2048)
      up_skinny_p<4, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                     sm + 16384 + (threadIdx.x >> 6) * 4096);
    else if (a.H % 256 == 0)
      up_skinny_t<4, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                     sm + 16384 + (threadIdx.x >> 6) * 4096);
    else
      up_skinny<1, 1, 1, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm));
    // the agent-coherent activation stores of every wavefront complete before the arrival
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) sync_arrive(fs, li, bx);
    return;
  }
  if (threadIdx.x < 64) {
    const bool ok = sync_wait(fs, li);
    if (threadIdx.x == 0) ok_s = ok ? 1 : 0;
  }
  __syncthreads();
  if (!ok_s) return;
  if (a.I == 768)
    down_skinny_p<3, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                     sm + 16384 + (threadIdx.x >> 6) * 4096);
  else if (a.I % 256 == 0)
    down_skinny_t<2, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm),
                     sm + 16384 + (threadIdx.x >> 6) * 4096);
  else
    down_skinny<1, 4, 1, true>(a, li, start, n, bx, reinterpret_cast<floatx4*>(sm));
}

// =============================================================================================
// Tiled kernels
// =============================================================================================

// Output tile 256 x 256 per workgroup (the wavefront layout is described at ffn_tiled).
// Phase 1's 256 B rows are 128 gate rows and the 128 up rows of the same intermediate columns,
// so every wavefront owns matching gate/up accumulators and the SwiGLU runs in registers.
//
// Operand staging: global -> LDS direct loads (global_load_lds_dwordx4, no VGPR round trip).
// A stage holds BK = 64 columns of K: 256 A rows and 256 B rows of 128 bytes.  One direct
// load moves 8 full rows (64 lanes x 16 B, lane l -> row l / 8, LDS slot l % 8), which keeps
// the global side fully coalesced.  Inside a row the 16-byte chunk c is stored at slot
// c ^ ((row >> 1) & 7): the MFMA fragment read (32 rows x one chunk per half-wavefront) then
// touches 16 distinct 16-byte bank groups in every 16 lanes, i.e. no LDS bank conflicts.
// Two stages (2 x 64 KiB): the loads of stage kt+1 run while stage kt is multiplied.
constexpr int BM = 256, BN = 256, BK = 64, STAGES = 2;
constexpr int kRowBytes = BK * 2;                                // 128
constexpr int kOperandBytes = 256 * kRowBytes;                   // 32 KiB per operand tile
constexpr int kStageBytes = 2 * kOperandBytes;                   // A then B
constexpr int kTileLds = STAGES * kStageBytes / 2;               // bf16 elements (128 KiB)

struct TileTable {
  int32_t cum[kListMax + 1];  // cumulative M tiles over list entries
  int32_t total;
  int64_t start[kListMax];    // per list entry: its expert's first grouped row, and row count
  int32_t rows[kListMax];
};

// Wavefront 0 builds the cumulative M-tile counts of the big experts of the list.
__device__ void build_tile_table(const FfnArgs& a, TileTable& tt) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int cnt[4];
    int local = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int li = lane * 4 + q;
      int c = 0;
      if (li < a.list.n) {
        const int e = a.list.expert[li];
        const int64_t s0 = a.starts[e];
        const int64_t n = a.starts[e + 1] - s0;
        c = n > kSkinnyMax ? (int)((n + BM - 1) / BM) : 0;
        tt.start[li] = s0;
        tt.rows[li] = (int32_t)n;
      }
      cnt[q] = c;
      local += c;
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    int run = incl - local;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      tt.cum[lane * 4 + q] = run;
      run += cnt[q];
    }
    if (lane == 63) {
      tt.cum[kListMax] = incl;
      tt.total = incl;
    }
  }
  __syncthreads();
}

// largest li with cum[li] <= m (cum is non-decreasing)
__device__ __forceinline__ int find_entry(const TileTable& tt, int m) {
  int lo = 0, hi = kListMax;  // cum[lo] <= m < cum[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tt.cum[mid] <= m)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// MODE 0: A = gathered x rows (K = H); B rows 0..127 = Wg[i0 ..], 128..255 = Wu[i0 ..];
//         epilogue act[p, i0 + c] = bf16(silu(bf16(g)) * bf16(u)).
// MODE 1: A = activation rows (K = I); B rows = Wd[h0 ..];
//         epilogue out[row(p), h0 + c] = bf16(bf16(y) * w(p)).
//
// Eight wavefronts, two per SIMD: wavefront (wm, wn) = (w / 4, w % 4) computes rows
// 128 wm .. +128 of the tile and a quarter of its columns (MODE 0: gate and up columns
// 32 wn .. +32, MODE 1: columns 64 wn .. +64), 4 x 2 tiles of 32x32 (128 accumulators).
// A wavefront that stalls -- issuing its direct loads while the address unit drains the
// others', or waiting for LDS fragments -- leaves its SIMD to the other wavefront's MFMAs.
constexpr int kTiledThreads = 512;
template <int MODE>
__global__ __launch_bounds__(kTiledThreads, 1) void ffn_tiled(FfnArgs a) {
  __shared__ TileTable tt;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[kTileLds];
  __shared__ int64_t orow_s[BM];   // phase 2: byte offset of each tile row's output row
  __shared__ float wt_s[BM];
  build_tile_table(a, tt);
  const int64_t K = MODE == 0 ? a.H : a.I;
  const int ntn = MODE == 0 ? (int)(a.I / 128) : (int)(a.H / BN);
  const int total = tt.total * ntn;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int KT = (int)(K / BK);
  const int l32 = lane & 31;

  // XCD-aware order: workgroup b runs on XCD b % 8 (round-robin dispatch), so in each round
  // of gridDim tiles the workgroups of one XCD take a contiguous run of tiles.  Tiles of one
  // expert are consecutive with N fastest, so a run covers a compact block of M x N tiles whose
  // A and B slices are shared in that XCD's L2.
  const int per_xcd = gridDim.x % 8 == 0 ? (int)gridDim.x / 8 : 0;
  const int lslot = per_xcd ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  for (int tile = lslot; tile < total; tile += gridDim.x) {
    const int mt_global = tile / ntn, ntile = tile % ntn;
    const int li = find_entry(tt, mt_global);
    const int64_t start = tt.start[li];
    const int n = tt.rows[li];
    const int m0 = (mt_global - tt.cum[li]) * BM;
    const bf16_t* slot = a.cache + (int64_t)a.list.slot[li] * 3 * a.H * a.I;

    // Direct loads: this wavefront moves tile rows 32*wave + 8*q + lane/8 (q < 4) of A and of
    // B, lane slot lane % 8 holding chunk (lane % 8) ^ ((row >> 1) & 7).  Rows past the
    // expert's last row load a valid row instead: each output row depends only on its own A
    // row, and those rows are never stored.
    const int r8 = lane >> 3, slot8 = lane & 7;
    // byte offsets of this lane's A rows (+ chunk) from abase: < 2^32 (host-checked sizes)
    uint32_t aoff[4];
    const char* abase = reinterpret_cast<const char*>(MODE == 0 ? a.x : a.act);
    const uint32_t lda = (uint32_t)(MODE == 0 ? a.H : a.I);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 32 * wave + 8 * q + r8;
      const int chunk = slot8 ^ ((row >> 1) & 7);
      const int r = m0 + row;
      const bool ok = r < n;
      const uint32_t t = MODE == 0 ? (uint32_t)a.rows[start + (ok ? r : 0)]
                                   : (uint32_t)(start + (ok ? r : 0));
      aoff[q] = (t * lda + (uint32_t)(chunk * 8)) * 2u;
    }
    // B rows of this wavefront: 32*wave .. +32 (MODE 0: waves 0-3 gate rows, 4-7 up rows)
    const int64_t ldb = MODE == 0 ? a.H : a.I;
    const int brow0 = 32 * wave;
    const char* bbase = reinterpret_cast<const char*>(uniform_ptr(
        MODE == 0 ? slot + (brow0 < 128 ? (int64_t)(ntile * 128 + brow0) * a.H
                                        : a.H * a.I + (int64_t)(ntile * 128 + brow0 - 128) * a.H)
                  : slot + 2 * a.H * a.I + (int64_t)(ntile * BN + brow0) * a.I));
    uint32_t boff[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = brow0 + 8 * q + r8;
      boff[q] = (uint32_t)(((8 * q + r8) * ldb + (slot8 ^ ((row >> 1) & 7)) * 8) * 2);
    }
    const uint32_t lds_smem = lds_addr(smem);
    // Rows past the expert's last one (the partial last M tile of an expert) are not computed:
    // in such a tile the A direct loads of 8-row groups that lie wholly past it are skipped,
    // and so are the MFMAs of 32-row blocks that do.  Their LDS rows then hold stale data, which
    // only reaches output rows that are never stored.  Full tiles run a copy of the loop
    // without these tests.
    const int vrows = n - m0;                                          // > 0
    const int nfa = __builtin_amdgcn_readfirstlane(
        vrows >= wm * 128 + 128 ? 4 : (vrows > wm * 128 ? (vrows - wm * 128 + 31) / 32 : 0));
    // per-row output row and routing weight for the phase-2 epilogue; run after the first
    // stage's direct loads are issued, so that its dependent loads overlap them
    auto row_meta = [&]() {
      if (MODE == 1) {
        for (int r = tid; r < BM; r += kTiledThreads) {
          const int rr = m0 + r;
          int64_t orow = 0;
          float wt = 0.f;
          if (rr < n) {
            const int64_t p = start + rr;
            const int64_t t = a.rows[p], j = a.cols[p];
            wt = bf16_to_f32(a.w[t * a.k + j]);
            orow = (a.out_mode == 0 ? t * a.k + j : p) * a.H * 2;   // byte offset of the row
          }
          orow_s[r] = orow;
          wt_s[r] = wt;
        }
      }
    };

    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // Fragment addresses.  Lane l reads row (first row of the fragment) + l % 32, chunk
    // 2*sub + l / 32, at byte row*128 + ((chunk ^ ((row >> 1) & 7)) << 4); fragment rows are
    // multiples of 32 apart, so the swizzle term only depends on the lane and the sub-step.
    // A fragments i: rows wm*128 + 32 i.  B fragments j: MODE 0 gate rows 32 wn (j = 0) and
    // up rows 128 + 32 wn (j = 1); MODE 1 rows 64 wn + 32 j.
    const uint32_t smem_base = lds_addr(smem);
    const int swz = (l32 >> 1) & 7, half = lane >> 5;
    uint32_t a_addr[4], b_addr[4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const uint32_t slotb = (uint32_t)((((2 * sub + half) ^ swz)) << 4);
      a_addr[sub] = smem_base + (uint32_t)((wm * 128 + l32) * kRowBytes) + slotb;
      b_addr[sub] = smem_base + kOperandBytes + (uint32_t)(((MODE == 0 ? wn * 32 : wn * 64) + l32) * kRowBytes) + slotb;
    }
    auto rd = [&](int kt, int sub, bf16x8 (&fa)[4], bf16x8 (&fb)[2]) {
      const uint32_t so = (uint32_t)((kt % STAGES) * kStageBytes);
      const uint32_t ab = a_addr[sub] + so, bb = b_addr[sub] + so;
      ds_read16<0 * 4096>(fa[0], ab);
      ds_read16<1 * 4096>(fa[1], ab);
      ds_read16<2 * 4096>(fa[2], ab);
      ds_read16<3 * 4096>(fa[3], ab);
      ds_read16<0>(fb[0], bb);
      ds_read16<MODE == 0 ? 16384 : 4096>(fb[1], bb);
    };
    auto pipeline = [&](auto part) {
    constexpr bool PARTIAL = decltype(part)::value;
    // direct load n (< 8) of stage kt: A rows 32 wave + 8n of this wavefront for n < 4, B rows
    // 32 wave + 8 (n - 4) for n >= 4
    auto dma = [&](int kt, int n) {
      const uint32_t st = lds_smem + (uint32_t)((kt % STAGES) * kStageBytes + 32 * wave * kRowBytes);
      const int q = n & 3;
      if (n < 4) {
        if (!PARTIAL || 32 * wave + 8 * q < vrows)
          dma16(abase + kt * BK * 2, aoff[q], st + (uint32_t)(8 * q * kRowBytes));
      } else {
        dma16(bbase + kt * BK * 2, boff[q], st + (uint32_t)(kOperandBytes + 8 * q * kRowBytes));
      }
    };
    auto issue = [&](int kt) {
#pragma unroll
      for (int n = 0; n < 8; ++n) dma(kt, n);
    };
    auto mma = [&](const bf16x8 (&fa)[4], const bf16x8 (&fb)[2]) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!PARTIAL || i < nfa) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      __builtin_amdgcn_sched_barrier(0);
    };
    // pipeline: stage kt+1 streams in while stage kt is multiplied; the fragments of the next
    // sub-step are read while the MFMAs of the current one run
    bf16x8 f0a[4], f0b[2], f1a[4], f1b[2];
    issue(0);
    row_meta();
    wait_vmcnt0();
    wg_barrier();
    if (1 < KT) issue(1);
    rd(0, 0, f0a, f0b);
    lds_wait(f0a, f0b);
    for (int kt = 0; kt < KT; ++kt) {
      rd(kt, 1, f1a, f1b);
      mma(f0a, f0b);
      lds_wait(f1a, f1b);
      rd(kt, 2, f0a, f0b);
      mma(f1a, f1b);
      lds_wait(f0a, f0b);
      rd(kt, 3, f1a, f1b);
      mma(f0a, f0b);
      lds_wait(f1a, f1b);  // stage kt fully read by this wavefront
      const bool more = kt + 1 < KT;
      if (more) {
        wait_vmcnt0();   // this wavefront's loads of stage kt+1 landed
        wg_barrier();    // ... everyone's; and stage kt is no longer read by anyone
        // stage kt+2 into the buffer stage kt just freed.  The two wavefronts of a SIMD (wm 0
        // and 1) issue their direct loads one MFMA group apart, so that one runs its MFMAs
        // while the other waits for the address unit to take its loads.
        if (kt + 2 < KT && wm == 0) issue(kt + 2);
        rd(kt + 1, 0, f0a, f0b);
      }
      mma(f1a, f1b);
      if (more) {
        if (kt + 2 < KT && wm == 1) issue(kt + 2);
        lds_wait(f0a, f0b);
      }
    }
    };
    if (vrows >= BM)
      pipeline(std::false_type{});
    else
      pipeline(std::true_type{});
    // 32x32 accumulator layout: column = lane & 31, row(v) = (v / 4) * 8 + (lane / 32) * 4 + v % 4.
    if constexpr (MODE == 1) {
      // phase-2 epilogue, straight from the accumulators: for each pair of rows (v, v + 1) a
      // lane rounds both of its column's values at once (v_cvt_pk_bf16_f32), applies the rows'
      // routing weights and rounds again into one packed word (row v low, row v + 1 high),
      // swaps that word with its neighbour lane (DPP quad_perm [1,0,3,2]) and picks two adjacent
      // columns of one row with one byte permute -- the even lane row v (its own low half, the
      // neighbour's low half), the odd lane row v + 1 (the neighbour's high half, its own high
      // half) -- stored as 4 bytes.  This is the issue-bound part of a phase-2 tile (all eight
      // wavefronts run it at once), so each row pair costs one address and about nine VALU
      // instructions per 32-column block.  No LDS staging and no barrier before the stores;
      // the barrier after them keeps the row table until every wavefront has read it.
      const bool odd = lane & 1;
      const uint32_t pick = odd ? 0x03020706u : 0x05040100u;
      char* const obase = reinterpret_cast<char*>(a.out) +
                          ((int64_t)ntile * BN + wn * 64 + (l32 & ~1)) * 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int vp = 0; vp < 8; ++vp) {
          const int v0 = 2 * vp;
          const int r0 = wm * 128 + i * 32 + (v0 >> 2) * 8 + (lane >> 5) * 4 + (v0 & 3);  // even
          const float w0 = wt_s[r0], w1 = wt_s[r0 + 1];
          const int r = odd ? r0 + 1 : r0;
          char* const rowp = obase + orow_s[r];
          const bool ok = m0 + r < n;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t g = pk_bf16(acc[i][j][v0], acc[i][j][v0 + 1]);
            const uint32_t y = pk_bf16(__uint_as_float(g << 16) * w0,
                                       __uint_as_float(g & 0xffff0000u) * w1);
            const uint32_t yn =
                (uint32_t)__builtin_amdgcn_update_dpp((int)y, (int)y, 0xB1, 0xf, 0xf, false);
            if (ok)
              *reinterpret_cast<uint32_t*>(rowp + j * 64) = __builtin_amdgcn_perm(yn, y, pick);
          }
        }
      }
      wg_barrier();
      continue;
    }
    __syncthreads();  // all fragment reads done before the staging area is reused

    // phase-1 epilogue: act[p, i0 + c] = bf16(silu(bf16 g) * bf16 u), the bf16 tile staged in
    // LDS (128 columns), then 16-byte row stores.  g and u are rounded by one packed
    // conversion; the results of rows (v, v + 1) of a column are packed likewise, swapped with
    // the neighbour lane and byte-permuted into two adjacent columns of one row (as in the
    // phase-2 epilogue), so that each LDS write carries two outputs.
    constexpr int OC = 128, OLD = OC + 8, CPR = OC / 8;   // CPR: 16-byte chunks per row
    bf16_t* os = smem;
    const bool odd = lane & 1;
    const uint32_t pick = odd ? 0x03020706u : 0x05040100u;
    const int col = wn * 32 + (l32 & ~1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int vp = 0; vp < 8; ++vp) {
        const int v0 = 2 * vp;
        const int r0 = wm * 128 + i * 32 + (v0 >> 2) * 8 + (lane >> 5) * 4 + (v0 & 3);  // even
        const uint32_t gu0 = pk_bf16(acc[i][0][v0], acc[i][1][v0]);
        const uint32_t gu1 = pk_bf16(acc[i][0][v0 + 1], acc[i][1][v0 + 1]);
        const float s0 = silu_mul(__uint_as_float(gu0 << 16), __uint_as_float(gu0 & 0xffff0000u));
        const float s1 = silu_mul(__uint_as_float(gu1 << 16), __uint_as_float(gu1 & 0xffff0000u));
        const uint32_t y = pk_bf16(s0, s1);
        const uint32_t yn =
            (uint32_t)__builtin_amdgcn_update_dpp((int)y, (int)y, 0xB1, 0xf, 0xf, false);
        const int r = odd ? r0 + 1 : r0;
        *reinterpret_cast<uint32_t*>(&os[r * OLD + col]) = __builtin_amdgcn_perm(yn, y, pick);
      }
    }
    __syncthreads();
    for (int c = tid; c < BM * CPR; c += kTiledThreads) {
      const int r = c / CPR, cc = (c % CPR) * 8;
      if (m0 + r >= n) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&os[r * OLD + cc]);
      *reinterpret_cast<u32x4*>(&a.act[(start + m0 + r) * a.I + ntile * 128 + cc]) = v;
    }
    // the staging reads are complete (their values are in the stores); the stores stay in
    // flight across the barrier (__syncthreads would wait for them)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wg_barrier();
  }
}

int g_num_cus = 0;

// Device addresses of g_sync / g_sync_timeouts on each device (resolved on first use there).
constexpr int kMaxDevices = 64;
std::mutex g_sync_mu;
uint32_t* g_sync_dev[kMaxDevices];
int32_t* g_timeouts_dev[kMaxDevices];
std::atomic<uint32_t> g_epoch{0};
std::atomic<int32_t> g_spin_limit{kSyncSpinLimit};

int sync_addresses(uint32_t** sync, int32_t** timeouts) {
  int dev = -1;
  FERRY_HIP(hipGetDevice(&dev));
  FERRY_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_sync_mu);
  if (g_sync_dev[dev] == nullptr) {
    void* ps = nullptr;
    void* pt = nullptr;
    FERRY_HIP(hipGetSymbolAddress(&ps, HIP_SYMBOL(g_sync)));
    FERRY_HIP(hipGetSymbolAddress(&pt, HIP_SYMBOL(g_sync_timeouts)));
    g_sync_dev[dev] = (uint32_t*)ps;
    g_timeouts_dev[dev] = (int32_t*)pt;
  }
  *sync = g_sync_dev[dev];
  *timeouts = g_timeouts_dev[dev];
  return 0;
}

}  // namespace

// device address of the fused decode kernel's timeout counter on the current device (for the
// history kernel's copy of it)
int ffn_timeouts_address(int32_t** timeouts) {
  uint32_t* sync = nullptr;
  return sync_addresses(&sync, timeouts);
}

}  // namespace ferry

using namespace ferry;

static int ffn_launch_list(FfnArgs& args, const int32_t* expert_list, const int32_t* slot_of,
                           int32_t n_list, int32_t n_mid, int64_t maxn, int64_t min_rows,
                           int64_t pairs, int32_t phases, int64_t hidden, int64_t inter,
                           hipStream_t s);

extern "C" int ferry_expert_ffn(const void* cache, int64_t cache_rows, int64_t hidden,
                                int64_t inter, const void* x, int64_t rows_in, int64_t topk,
                                const void* w_sorted, const int64_t* starts, const int64_t* rows,
                                const int64_t* cols, const int32_t* expert_list, int32_t n_list,
                                const int32_t* slot_of, int64_t experts,
                                int64_t max_rows_per_expert, int64_t min_rows_per_expert,
                                const int32_t* list_rows, void* act, void* out,
                                int32_t out_mode, int32_t phases, void* stream) {
  clear_error();
  FERRY_CHECK_ARG(phases >= 1 && phases <= 3, "phases must be 1 (up), 2 (down) or 3 (both)");
  FERRY_CHECK_ARG(hidden > 0 && hidden % 128 == 0, "hidden must be a positive multiple of 128");
  FERRY_CHECK_ARG(inter > 0 && inter % 128 == 0, "intermediate must be a positive multiple of 128");
  FERRY_CHECK_ARG(topk >= 1 && rows_in >= 0 && n_list >= 0 && max_rows_per_expert >= 0,
                  "bad sizes");
  FERRY_CHECK_ARG(min_rows_per_expert >= 0 && min_rows_per_expert <= max_rows_per_expert,
                  "min_rows_per_expert must be in [0, max_rows_per_expert]");
  FERRY_CHECK_ARG(experts >= 1 && experts <= FERRY_MAX_EXPERTS, "experts must be in [1, %d]",
                  FERRY_MAX_EXPERTS);
  FERRY_CHECK_ARG(out_mode == 0 || out_mode == 1, "out_mode must be 0 or 1");
  // the tiled down projection covers the hidden dimension in 256-column tiles
  FERRY_CHECK_ARG(hidden % 256 == 0 || max_rows_per_expert <= kSkinnyMax,
                  "hidden must be a multiple of 256 when an expert has more than %d rows",
                  kSkinnyMax);
  FERRY_CHECK_ARG(rows_in * topk < (int64_t)1 << 31, "rows*topk must be < 2^31");
  // the kernels address weights with 32-bit byte offsets from the expert's cache row
  FERRY_CHECK_ARG(3 * hidden * inter * 2 < ((int64_t)1 << 32),
                  "an expert's cache row (3 * hidden * intermediate bf16) must be under 4 GiB");
  // the tiled kernels address A rows with 32-bit byte offsets
  FERRY_CHECK_ARG(rows_in * hidden < ((int64_t)1 << 31) &&
                      rows_in * topk * inter < ((int64_t)1 << 31),
                  "x / act must hold fewer than 2^31 elements");
  if (n_list == 0 || rows_in == 0) return 0;
  FERRY_CHECK_ARG(cache && x && w_sorted && starts && rows && cols && expert_list && slot_of &&
                      act && out,
                  "null pointer argument");
  for (int32_t i = 0; i < n_list; ++i) {
    const int32_t e = expert_list[i];
    FERRY_CHECK_ARG(e >= 0 && e < experts, "expert_list[%d] = %d out of range", i, e);
    const int32_t s = slot_of[e];
    FERRY_CHECK_ARG(s >= 0 && s < cache_rows, "expert %d is not cached (slot %d)", e, s);
    if (list_rows)
      FERRY_CHECK_ARG(list_rows[i] >= min_rows_per_expert && list_rows[i] <= max_rows_per_expert,
                      "list_rows[%d] = %d outside [min_rows_per_expert, max_rows_per_expert]", i,
                      list_rows[i]);
  }
  if (g_num_cus == 0) {
    int dev = 0, cus = 0;
    FERRY_HIP(hipGetDevice(&dev));
    FERRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    g_num_cus = cus > 0 ? cus : 256;
  }
  hipStream_t s = (hipStream_t)stream;
  FfnArgs args;
  args.cache = (const bf16_t*)cache;
  args.x = (const bf16_t*)x;
  args.w = (const bf16_t*)w_sorted;
  args.starts = starts;
  args.rows = rows;
  args.cols = cols;
  args.act = (bf16_t*)act;
  args.out = (bf16_t*)out;
  args.H = hidden;
  args.I = inter;
  args.k = topk;
  args.out_mode = out_mode;
  // max_rows_per_expert must bound every n_e from above (rows_in does for a layout from
  // ferry_layout) and min_rows_per_expert from below (0 when unknown); the kernels size their
  // work from the device starts, the bounds only select and gate the launches.  With the
  // entries' row counts (list_rows) the list is issued as two lists with exact bounds: the
  // small experts (1-64 rows; those with 17-64 rows first), then the tiled ones (the small
  // launches measured slower after the tiled ones, whose output writes they then meet); experts
  // without rows are left out.
  if (!list_rows)
    return ffn_launch_list(args, expert_list, slot_of, n_list, n_list, max_rows_per_expert,
                           min_rows_per_expert, rows_in * topk, phases, hidden, inter, s);
  std::vector<int32_t> small, big;
  int32_t n_mid = 0;
  int64_t small_max = 0, small_min = kSkinnyMax, big_max = 0, big_min = INT64_MAX;
  for (int pass = 0; pass < 2; ++pass)   // 17-64 rows, then 1-16 rows
    for (int32_t i = 0; i < n_list; ++i) {
      const int64_t r = list_rows[i];
      if (r > 16 && r <= kSkinnyMax && pass == 0) small.push_back(expert_list[i]), ++n_mid;
      if (r >= 1 && r <= 16 && pass == 1) small.push_back(expert_list[i]);
      if (r >= 1 && r <= kSkinnyMax && pass == 0) {
        small_max = r > small_max ? r : small_max;
        small_min = r < small_min ? r : small_min;
      }
      if (r > kSkinnyMax && pass == 0) {
        big.push_back(expert_list[i]);
        big_max = r > big_max ? r : big_max;
        big_min = r < big_min ? r : big_min;
      }
    }
  if (!small.empty()) {
    const int rc = ffn_launch_list(args, small.data(), slot_of, (int32_t)small.size(), n_mid,
                                   small_max, small_min, rows_in * topk, phases, hidden, inter, s);
    if (rc != 0) return rc;
  }
  if (!big.empty())
    return ffn_launch_list(args, big.data(), slot_of, (int32_t)big.size(), 0, big_max, big_min,
                           rows_in * topk, phases, hidden, inter, s);
  return 0;
}

// The launches of one list: n_mid of its leading entries are known to hold 17-64 rows (the
// small-expert up launch gives them 64-column workgroups; the others get 16-column ones unless
// the bounds allow no expert of more than 16 rows, n_mid = n_list when unknown).
static int ffn_launch_list(FfnArgs& args, const int32_t* expert_list, const int32_t* slot_of,
                           int32_t n_list, int32_t n_mid, int64_t maxn, int64_t min_rows,
                           int64_t pairs, int32_t phases, int64_t hidden, int64_t inter,
                           hipStream_t s) {
  const bool any_small = min_rows <= kSkinnyMax;
  for (int32_t off = 0; off < n_list; off += kListMax) {
    const int32_t cnt = (n_list - off) < kListMax ? (n_list - off) : kListMax;
    args.list.n = cnt;
    const int32_t mid_left = n_mid - off;
    args.list.n_mid = mid_left < 0 ? 0 : (mid_left < cnt ? mid_left : cnt);
    for (int32_t i = 0; i < kListMax; ++i) {
      args.list.expert[i] = (int16_t)(i < cnt ? expert_list[off + i] : 0);
      args.list.slot[i] = i < cnt ? slot_of[expert_list[off + i]] : 0;
    }
    const bool any_big = maxn > kSkinnyMax;
    // M tiles over experts with > 64 rows: sum ceil(n/BM) <= pairs/BM + (experts with > 64 rows)
    const int64_t tile_bound = pairs / BM + pairs / (kSkinnyMax + 1) + 1;  // and those are <= pairs/65
    const int64_t grid_cap = (int64_t)g_num_cus;  // one 256x256 workgroup per CU
    if (phases == 3 && any_small && !any_big && maxn <= 16 && inter / 16 <= kMaxUpWgs) {
      // decode: both phases in one launch, each expert's down projection as soon as its up
      // projection is stored
      FusedSync fs;
      uint32_t* sync = nullptr;
      const int rc = sync_addresses(&sync, &fs.timeouts);
      if (rc != 0) return rc;
      uint32_t epoch = ++g_epoch;
      if (epoch == 0) epoch = ++g_epoch;   // epoch 0 would match never-used words
      fs.epoch = epoch;
      fs.flags = sync + (int64_t)(epoch % kSyncSets) * kListMax * kMaxUpWgs;
      fs.up_wgs = (int32_t)(inter / 16);
      fs.down_wgs = (int32_t)(hidden / 64);
      fs.spin_limit = g_spin_limit.load();
      launch("ffn_skinny_fused", ffn_skinny_fused,
             dim3((unsigned)((fs.up_wgs + fs.down_wgs) * cnt)), dim3(256), 0, s, args, fs);
      FERRY_LAUNCHED("ffn_skinny_fused");
      continue;
    }
    if (phases & 1) {
      // 16 intermediate columns per workgroup, K split over the four wavefronts
      if (any_small) {
        const dim3 g1((unsigned)(inter / 16), cnt);
        const int64_t wgs = args.list.n_mid * (inter / 64) + (cnt - args.list.n_mid) * (inter / 16);
        if (maxn <= 16)
          launch("ffn_up_skinny", ffn_up_skinny<1>, g1, dim3(256), 0, s, args);
        else
          launch("ffn_up_skinny", ffn_up_skinny<4>, dim3((unsigned)wgs), dim3(256), 0, s, args);
        FERRY_LAUNCHED("ffn_up_skinny");
      }
      if (any_big) {
        const int64_t t1 = tile_bound * (inter / 128);
        launch("ffn_tiled_up", ffn_tiled<0>, dim3((unsigned)(t1 < grid_cap ? t1 : grid_cap)),
                           dim3(kTiledThreads), 0, s, args);
        FERRY_LAUNCHED("ffn_tiled<up>");
      }
    }
    if (phases & 2) {
      // 64 hidden rows per workgroup
      if (any_small) {
        const dim3 g2((unsigned)(hidden / 64), cnt);
        if (maxn <= 16)
          launch("ffn_down_skinny", ffn_down_skinny<1>, g2, dim3(256), 0, s, args);
        else
          launch("ffn_down_skinny", ffn_down_skinny<4>, g2, dim3(256), 0, s, args);
        FERRY_LAUNCHED("ffn_down_skinny");
      }
      if (any_big) {
        const int64_t t2 = tile_bound * (hidden / BN);
        launch("ffn_tiled_down", ffn_tiled<1>, dim3((unsigned)(t2 < grid_cap ? t2 : grid_cap)),
                           dim3(kTiledThreads), 0, s, args);
        FERRY_LAUNCHED("ffn_tiled<down>");
      }
    }
  }
  return 0;
}

// Number of fused decode launches whose down phase gave up waiting for its up phase (each such
// workgroup left its rows unwritten); 0 unless workgroups were not dispatched in index order.
extern "C" int ferry_expert_ffn_sync_timeouts(int64_t* count) {
  clear_error();
  FERRY_CHECK_ARG(count, "null pointer argument");
  uint32_t* sync = nullptr;
  int32_t* timeouts = nullptr;
  const int rc = sync_addresses(&sync, &timeouts);
  if (rc != 0) return rc;
  int32_t v = 0;
  FERRY_HIP(hipMemcpy(&v, timeouts, sizeof(v), hipMemcpyDeviceToHost));
  *count = v;
  return 0;
}

// How many times a fused decode launch's down workgroup polls its up workgroups' flags before
// giving up (limit < 0: the default, about a second of polling; 0: it gives up without polling,
// so that a caller can check how a timeout is reported).  Applies to launches made after it.
extern "C" int ferry_expert_ffn_set_sync_spin_limit(int64_t limit) {
  clear_error();
  FERRY_CHECK_ARG(limit < ((int64_t)1 << 30), "spin limit must be below 2^30");
  g_spin_limit.store(limit < 0 ? kSyncSpinLimit : (int32_t)limit);
  return 0;
}
