// Per-head q/k RMSNorm + rotate-half rotary (qk_pair's row arithmetic), shared
// by the q/k/v post-processing kernel and the QKV GEMM epilogue.
#pragma once

#include "ff_common.h"

namespace ff {

constexpr int kHeadDim = 128;

// One 16-lane group per (token, head) row of 128: lane j holds elements
// [8j, 8j+8); its rotate-half partner block sits in lane j ^ 8.
__device__ __forceinline__ void rope_row(const bf16_t* __restrict__ src, const bf16_t* __restrict__ w,
                                         float eps, const bf16_t* __restrict__ cs,
                                         const bf16_t* __restrict__ sn, bf16_t* __restrict__ dst,
                                         int j, bool valid) {
  float x[8], wv[8], c[8], s[8];
  if (valid) {
    unpack8(*reinterpret_cast<const u32x4*>(src + 8 * j), x);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = rsqrt_rn(ss / (float)kHeadDim + eps);
  unpack8(*reinterpret_cast<const u32x4*>(w + 8 * j), wv);
  float xn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) xn[e] = round_bf16(round_bf16(x[e] * inv) * wv[e]);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = __shfl_xor(xn[e], 8, 64);
    r[e] = j < 8 ? -p : p;
  }
  if (!valid) return;
  unpack8(*reinterpret_cast<const u32x4*>(cs + 8 * j), c);
  unpack8(*reinterpret_cast<const u32x4*>(sn + 8 * j), s);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf16(xn[e] * c[e]) + round_bf16(r[e] * s[e]);
  *reinterpret_cast<u32x4*>(dst + 8 * j) = pack8(y);
}

}  // namespace ff
