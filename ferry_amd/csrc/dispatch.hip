// Dispatch packets: the byte format of the reference's token exchange.
//
// Reference: ferry/csrc/expert_ops.cpp:88-111 (pack_dispatch / unpack_dispatch), called by
// Transport.dispatch (ferry/transport.py:22-29).  A packet row is
//   [ hidden[send_idx[i]] (2H bytes) | packet weights (2k bytes, bf16) | expert IDs (k bytes) ]
// where packet weight j is the token's routing weight of expert send_ids[i, j]: the reference
// scatters the bf16 weights into a dense fp32 [T, E] row (scatter_add_, so repeated IDs add),
// casts it to bf16 and gathers it at send_ids (clamped at 0) times the validity mask
// send_ids >= 0.  IDs are stored as send_ids cast to uint8 (two's complement: -1 -> 255).
//
// At world = 1 the packets never leave the GPU (the fused path reads the routing weights in
// sorted-ID order straight from the layout kernel); these entry points give callers of the
// reference's Transport the same bytes.  One workgroup per packet row: 16-byte copies of the
// hidden row where the row pitch allows, byte copies otherwise.
#include "common.h"

namespace ferry {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 64;

__global__ __launch_bounds__(kThreads) void pack_dispatch_kernel(
    const uint8_t* __restrict__ hidden, int64_t tokens, int64_t hbytes,
    const int64_t* __restrict__ selected,
    const bf16_t* __restrict__ weights, int ksel, const int64_t* __restrict__ send_idx,
    const int64_t* __restrict__ send_ids, int k, int64_t experts, uint8_t* __restrict__ payload,
    int64_t pitch, int vec16) {
  const int64_t i = blockIdx.x;
  const int64_t t = send_idx[i];
  if (t < 0 || t >= tokens) return;   // not a token of this call: the row is left unwritten
  const uint8_t* src = hidden + t * hbytes;
  uint8_t* dst = payload + i * pitch;
  if (vec16) {
    const int64_t n16 = hbytes >> 4;
    for (int64_t c = threadIdx.x; c < n16; c += kThreads)
      reinterpret_cast<uint4*>(dst)[c] = reinterpret_cast<const uint4*>(src)[c];
  } else {
    for (int64_t c = threadIdx.x; c < hbytes; c += kThreads) dst[c] = src[c];
  }
  if (threadIdx.x < k) {
    const int j = threadIdx.x;
    const int64_t id = send_ids[i * k + j];
    const int64_t e = id < 0 ? 0 : id;   // clamp_min(0)
    // dense[t, e] = bf16(sum over the token's entries equal to e of fp32(weight)); an ID past
    // the dense row's width reads 0
    float acc = 0.f;
    for (int q = 0; q < ksel; ++q)
      if (selected[t * ksel + q] == e && e < experts) acc += bf16_to_f32(weights[t * ksel + q]);
    const float dense = bf16r(acc);
    const bf16_t w = f32_to_bf16(dense * (id >= 0 ? 1.f : 0.f));   // * valid, a bf16 product
    uint8_t* wdst = dst + hbytes + 2 * j;
    wdst[0] = (uint8_t)(w & 0xFF);
    wdst[1] = (uint8_t)(w >> 8);
    dst[hbytes + 2 * k + j] = (uint8_t)id;
  }
}

}  // namespace
}  // namespace ferry

using namespace ferry;

extern "C" int ferry_pack_dispatch(const void* hidden, int64_t tokens, int64_t hidden_size,
                                   const int64_t* selected, const void* weights_bf16,
                                   int64_t topk_selected, const int64_t* send_idx,
                                   const int64_t* send_ids, int64_t packets, int64_t topk,
                                   int64_t experts, void* payload, void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0 && packets >= 0 && hidden_size >= 1 && experts >= 1, "bad sizes");
  FERRY_CHECK_ARG(topk >= 1 && topk <= kMaxK && topk_selected >= 1,
                  "topk must be in [1, %d]", kMaxK);
  FERRY_CHECK_ARG(packets < (1LL << 31), "too many packets");
  if (packets == 0) return 0;
  FERRY_CHECK_ARG(hidden && selected && weights_bf16 && send_idx && send_ids && payload,
                  "null pointer argument");
  const int64_t hbytes = 2 * hidden_size, pitch = hbytes + 3 * topk;
  // 16-byte copies need 16-byte aligned rows on both sides
  const int vec16 = ((((uintptr_t)hidden | (uintptr_t)payload) & 15) == 0 &&
                     ((hbytes | pitch) & 15) == 0);
  launch("pack_dispatch_kernel", pack_dispatch_kernel, dim3((unsigned)packets), dim3(kThreads), 0,
         (hipStream_t)stream, (const uint8_t*)hidden, tokens, hbytes, selected,
         (const bf16_t*)weights_bf16, (int)topk_selected, send_idx, send_ids, (int)topk, experts,
         (uint8_t*)payload, pitch, vec16);
  FERRY_LAUNCHED("pack_dispatch_kernel");
  return 0;
}

extern "C" int ferry_unpack_dispatch(const void* payload, int64_t packets, int64_t hidden_size,
                                     int64_t topk, void* hidden_out, void* weights_out,
                                     void* stream) {
  clear_error();
  FERRY_CHECK_ARG(packets >= 0 && hidden_size >= 1 && topk >= 1, "bad sizes");
  if (packets == 0) return 0;
  FERRY_CHECK_ARG(payload && hidden_out && weights_out, "null pointer argument");
  const size_t pitch = (size_t)(2 * hidden_size + 3 * topk);
  hipStream_t s = (hipStream_t)stream;
  FERRY_HIP(hipMemcpy2DAsync(hidden_out, (size_t)(2 * hidden_size), payload, pitch,
                             (size_t)(2 * hidden_size), (size_t)packets, hipMemcpyDeviceToDevice,
                             s));
  FERRY_HIP(hipMemcpy2DAsync(weights_out, (size_t)(2 * topk),
                             (const uint8_t*)payload + 2 * hidden_size, pitch, (size_t)(2 * topk),
                             (size_t)packets, hipMemcpyDeviceToDevice, s));
  return 0;
}
