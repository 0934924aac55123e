// Combine: gate-weighted expert outputs summed per token in fp32, cast to bf16.
//
// Reference: ferry/csrc/expert_ops.cpp:75-92.  reduce_partials builds an fp32 [R, H] zero
// tensor, index_add_s every expert's bf16 output (already multiplied by its routing weight)
// in ascending expert order and casts to bf16; at world = 1 scatter_returned is an fp32
// round trip of that bf16 tensor, i.e. the identity.  A token's k entries are stored in
// ascending-ID order, so summing j = 0..k-1 reproduces the reference order exactly.
//
// DeepSeek-V2 adds the shared experts' bf16 output to the routed bf16 output
// (transformers modeling_deepseek_v2.py:136, `hidden_states + self.shared_experts(residuals)`):
// with `addend` the bf16 combine result is added to it in fp32 and rounded again, which is
// torch's bf16 addition.
//
// One block per token row chunk: each thread owns 8 consecutive hidden elements (one 16-byte
// load per entry), so a token row of H = 2048 is one 256-thread block.
#include "common.h"

namespace ferry {
namespace {

constexpr int kThreads = 256;
constexpr int kVec = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void combine_kernel(const bf16_t* __restrict__ part,
                                                           const int32_t* __restrict__ pair_pos,
                                                           const bf16_t* __restrict__ addend,
                                                           int64_t tokens, int k, int64_t H,
                                                           bf16_t* __restrict__ out) {
  const int64_t chunks_per_row = H / kVec;
  const int64_t total = tokens * chunks_per_row;
  for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * kThreads) {
    const int64_t t = c / chunks_per_row;
    const int64_t h0 = (c % chunks_per_row) * kVec;
    float acc[kVec];
#pragma unroll
    for (int i = 0; i < kVec; ++i) acc[i] = 0.f;
    for (int j = 0; j < k; ++j) {
      const int64_t src = pair_pos ? (int64_t)pair_pos[t * k + j] : t * k + j;
      if (src < 0) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(part + src * H + h0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf16_to_f32((bf16_t)(v[i] & 0xffffu));
        acc[2 * i + 1] += bf16_to_f32((bf16_t)(v[i] >> 16));
      }
    }
    if (addend) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(addend + t * H + h0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = bf16r(acc[2 * i]) + bf16_to_f32((bf16_t)(v[i] & 0xffffu));
        acc[2 * i + 1] = bf16r(acc[2 * i + 1]) + bf16_to_f32((bf16_t)(v[i] >> 16));
      }
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = (uint32_t)f32_to_bf16(acc[2 * i]) | ((uint32_t)f32_to_bf16(acc[2 * i + 1]) << 16);
    *reinterpret_cast<u32x4*>(out + t * H + h0) = o;
  }
}

}  // namespace
}  // namespace ferry

using namespace ferry;

namespace {
int combine_impl(const void* part, const int32_t* pair_pos, int64_t tokens, int64_t topk,
                 int64_t hidden, const void* addend, void* out, void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0 && topk >= 1, "bad sizes");
  FERRY_CHECK_ARG(hidden > 0 && hidden % kVec == 0, "hidden must be a positive multiple of %d",
                  kVec);
  FERRY_CHECK_ARG(tokens == 0 || (part && out), "null pointer argument");
  FERRY_CHECK_ARG(((uintptr_t)part % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                      ((uintptr_t)addend % 16) == 0,
                  "part/addend/out must be 16-byte aligned");
  if (tokens == 0) return 0;
  const int64_t work = tokens * (hidden / kVec);
  int64_t grid = ceil_div(work, kThreads);
  if (grid > 65536) grid = 65536;
  launch("combine_kernel", combine_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)part, pair_pos, (const bf16_t*)addend, tokens, (int)topk, hidden,
                     (bf16_t*)out);
  FERRY_LAUNCHED("combine_kernel");
  return 0;
}
}  // namespace

extern "C" int ferry_combine(const void* part, const int32_t* pair_pos, int64_t tokens,
                             int64_t topk, int64_t hidden, void* out, void* stream) {
  return combine_impl(part, pair_pos, tokens, topk, hidden, nullptr, out, stream);
}

extern "C" int ferry_combine_add(const void* part, const int32_t* pair_pos, int64_t tokens,
                                 int64_t topk, int64_t hidden, const void* addend, void* out,
                                 void* stream) {
  if (!addend && tokens > 0) {
    clear_error();
    FERRY_CHECK_ARG(false, "addend must not be null");
  }
  return combine_impl(part, pair_pos, tokens, topk, hidden, addend, out, stream);
}
