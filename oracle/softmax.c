/*
 * CPU oracle (test infrastructure only): torch's CPU softmax and short last-dim sum, the two
 * float computations of the reference router (ferry/model.py:142-145: softmax(logits, fp32),
 * topk, w / w.sum(-1)), restated rounding step for rounding step so that the probabilities --
 * whose equalities decide torch.topk's ties -- and the renormalised weights can be reproduced
 * bit for bit.  Pinned by the tests against torch.softmax / torch.sum themselves.
 *
 *  oracle_expf       SLEEF's expf_u10 (xexpf, sleefsimdsp.c of SLEEF 3), the exp of torch's
 *                    Vectorized<float> (ATen/cpu/vec/vec512/vec512_float.h:307-309): Cody-Waite
 *                    reduction by ln 2 in two parts, a degree-6 Horner polynomial with fused
 *                    multiply-adds, scaling by 2^q in two steps.
 *  oracle_softmax    torch's vectorized last-dim softmax on 16-lane vectors: max, exp(x - max),
 *                    sum in vec::reduce_all order (ATen/cpu/vec/functional_base.h:185-203 and
 *                    the AVX-512 VecReduceAllSIMD at :78-98), 1 / sum, multiply.
 *  oracle_weight_sum torch's CPU sum over a contiguous last dim of k <= 32 (its 8-lane
 *                    reduction kernel): k < 8 -- four interleaved scalar partial sums, the tail
 *                    into partial 0, then 0 + 1 + 2 + 3; k >= 8 -- 8 lane sums over the full
 *                    vectors, and the scalar tail summed first, then the 8 lanes in order.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float pow2i(int q) {
  uint32_t u = (uint32_t)(q + 0x7f) << 23;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_expf(float d) {
  if (d != d) return d;
  if (d < -104.f) return 0.f;
  if (d > 100.f) return INFINITY;
  const float rln2 = 1.442695040888963407359924681001892137f;
  const float l2u = 0.693145751953125f, l2l = 1.428606765330187045e-06f;
  const int q = (int)rintf(d * rln2);
  float s = fmaf((float)q, -l2u, d);
  s = fmaf((float)q, -l2l, s);
  float u = 0.000198527617612853646278381f;
  u = fmaf(u, s, 0.00139304355252534151077271f);
  u = fmaf(u, s, 0.00833336077630519866943359f);
  u = fmaf(u, s, 0.0416664853692054748535156f);
  u = fmaf(u, s, 0.166666671633720397949219f);
  u = fmaf(u, s, 0.5f);
  u = 1.0f + fmaf(s * s, u, s);
  return u * pow2i(q >> 1) * pow2i(q - (q >> 1));
}

void oracle_softmax(const float* x, int64_t rows, int64_t n, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * n;
    float* out = y + r * n;
    float m = in[0];
    int nan = in[0] != in[0];
    for (int64_t i = 1; i < n; ++i) {
      nan |= in[i] != in[i];
      if (in[i] > m) m = in[i];
    }
    if (nan) m = NAN;   /* vec::maximum propagates NaN */
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_expf(in[i] - m);
    float sum;
    if (n < 16) {
      sum = out[0];
      for (int64_t i = 1; i < n; ++i) sum += out[i];
    } else {
      float acc[16];
      for (int l = 0; l < 16; ++l) acc[l] = out[l];
      const int64_t full = n - n % 16;
      for (int64_t c = 16; c < full; c += 16)
        for (int l = 0; l < 16; ++l) acc[l] += out[c + l];
      for (int64_t l = 0; l < n - full; ++l) acc[l] += out[full + l];
      for (int h = 8; h >= 1; h >>= 1)
        for (int l = 0; l < h; ++l) acc[l] += acc[l + h];
      sum = acc[0];
    }
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; ++i) out[i] *= inv;
  }
}

void oracle_weight_sum(const float* w, int64_t rows, int64_t k, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = w + r * k;
    if (k < 8) {
      float p[4] = {0.f, 0.f, 0.f, 0.f};
      int64_t i = 0;
      if (k >= 4)
        for (; i < 4; ++i) p[i] += v[i];
      for (; i < k; ++i) p[0] += v[i];
      out[r] = ((p[0] + p[1]) + p[2]) + p[3];
      continue;
    }
    const int64_t nv = k / 8;
    float acc = 0.f;
    for (int64_t i = 8 * nv; i < k; ++i) acc += v[i];
    for (int l = 0; l < 8; ++l) {
      float lane = v[l];
      for (int64_t j = 1; j < nv; ++j) lane += v[8 * j + l];
      acc += lane;
    }
    out[r] = acc;
  }
}
