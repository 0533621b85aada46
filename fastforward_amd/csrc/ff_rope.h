// Per-head q/k RMSNorm + rotate-half rotary (qk_pair's row arithmetic), shared
// by the q/k/v post-processing kernel and the QKV GEMM epilogue.
#pragma once

#include "ff_common.h"

namespace ff {

constexpr int kHeadDim = 128;

// One 16-lane group per (token, head) row of 128: lane j holds elements
// [8j, 8j+8); its rotate-half partner block sits in lane j ^ 8. wv is the lane's
// 8 norm weights, cs / sn its 8 cos / sin values (bf16) of the row's token, loaded
// by the caller so that a loop over rows can issue all its global loads first.
__device__ __forceinline__ void rope_row_pre(const bf16_t* __restrict__ src, const float (&wv)[8], float eps,
                                             const u32x4 cs, const u32x4 sn, bf16_t* __restrict__ dst, int j,
                                             bool valid) {
  float x[8], c[8], s[8];
  if (valid) {
    unpack8(*reinterpret_cast<const u32x4*>(src + 8 * j), x);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  // 16-lane sum on DPP (each step adds a commutative pair, so all 16 lanes end
  // with the same bits)
  ss += dpp<kDppXor1>(ss);
  ss += dpp<kDppXor2>(ss);
  ss += dpp<kDppHalfMirror>(ss);
  ss += dpp<kDppRowMirror>(ss);
  const float inv = rsqrt_rn(ss / (float)kHeadDim + eps);
  float xn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) xn[e] = round_bf16(round_bf16(x[e] * inv) * wv[e]);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = dpp<kDppRowRor8>(xn[e]);  // lane j ^ 8 of the 16-lane row
    r[e] = j < 8 ? -p : p;
  }
  if (!valid) return;
  unpack8(cs, c);
  unpack8(sn, s);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf16(xn[e] * c[e]) + round_bf16(r[e] * s[e]);
  *reinterpret_cast<u32x4*>(dst + 8 * j) = pack8(y);
}

__device__ __forceinline__ void rope_row(const bf16_t* __restrict__ src, const bf16_t* __restrict__ w,
                                         float eps, const bf16_t* __restrict__ cs,
                                         const bf16_t* __restrict__ sn, bf16_t* __restrict__ dst,
                                         int j, bool valid) {
  float wv[8];
  unpack8(*reinterpret_cast<const u32x4*>(w + 8 * j), wv);
  rope_row_pre(src, wv, eps, *reinterpret_cast<const u32x4*>(cs + 8 * j), *reinterpret_cast<const u32x4*>(sn + 8 * j),
               dst, j, valid);
}

}  // namespace ff
