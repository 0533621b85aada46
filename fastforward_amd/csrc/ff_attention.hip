// Attention path for gfx950: per-head q/k RMSNorm + M-RoPE (qk_pair), the
// transposed-V producer, and causal GQA flash attention on bf16 MFMA.
//
// Attention computes S^T = K Q^T and O^T = V^T P^T with
// v_mfma_f32_16x16x32_bf16 so that every accumulator a lane holds belongs to
// one query (the lane's column): the online-softmax statistics then live in
// registers of that lane and P^T leaves the S^T accumulator directly in the
// B-operand layout of the P.V product, with no LDS round trip. The key order
// inside each 32-key chunk is chosen so that lane group g = l/16 owns keys
// 8g..8g+7 in both products; V^T (keys contiguous per d) is produced once per
// layer by the q/k/v post-processing kernel.
#include "ff_common.h"

using namespace ff;

namespace {

constexpr int kThreads = 256;
constexpr int D = 128;

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// ---------------------------------------------------------------- q/k norm + rope

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
  const float inv = rsqrt_rn(ss / (float)D + eps);
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

// Grid: [q rows / 16 | k rows / 16 | v tiles (hk * t_pad/64)].
__global__ __launch_bounds__(kThreads) void qkv_post_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    int64_t row_stride, int64_t v_hs, const bf16_t* __restrict__ wq, const bf16_t* __restrict__ wk,
    float eps_q, float eps_k, const bf16_t* __restrict__ cs, const bf16_t* __restrict__ sn,
    int64_t cos_ts, int64_t sin_ts, bf16_t* __restrict__ yq, bf16_t* __restrict__ yk,
    bf16_t* __restrict__ vt, int t, int t_pad, int hq, int hk, int nq_blocks, int nk_blocks) {
  __shared__ bf16_t tile[D][64 + 8];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  if (b < nq_blocks + nk_blocks) {
    const bool isq = b < nq_blocks;
    const int heads = isq ? hq : hk;
    const int row = (isq ? b : b - nq_blocks) * 16 + (tid >> 4);
    const int j = tid & 15;
    const bool valid = row < t * heads;
    const int rr = valid ? row : 0;
    const int token = rr / heads, head = rr % heads;
    rope_row((isq ? q : k) + (int64_t)token * row_stride + head * D, isq ? wq : wk, isq ? eps_q : eps_k,
             cs + (int64_t)token * cos_ts, sn + (int64_t)token * sin_ts,
             (isq ? yq : yk) + ((int64_t)head * t + token) * D, j, valid);
    return;
  }
  // V^T tile: 64 keys x 128 d of one kv head.
  const int vb = b - nq_blocks - nk_blocks;
  const int tiles_per_head = t_pad / 64;
  const int head = vb / tiles_per_head, key0 = (vb % tiles_per_head) * 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + i * kThreads;  // 64 keys x 16 chunks
    const int key = c >> 4, d0 = (c & 15) * 8;
    float f[8];
    if (key0 + key < t) {
      unpack8(*reinterpret_cast<const u32x4*>(v + (int64_t)(key0 + key) * row_stride + head * v_hs + d0), f);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[d0 + e][key] = (bf16_t)f32_to_bf16(f[e]);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + i * kThreads;  // 128 d rows x 8 chunks of 8 keys
    const int d = c >> 3, k0 = (c & 7) * 8;
    u32x4 o;
    o.x = tile[d][k0] | ((uint32_t)tile[d][k0 + 1] << 16);
    o.y = tile[d][k0 + 2] | ((uint32_t)tile[d][k0 + 3] << 16);
    o.z = tile[d][k0 + 4] | ((uint32_t)tile[d][k0 + 5] << 16);
    o.w = tile[d][k0 + 6] | ((uint32_t)tile[d][k0 + 7] << 16);
    *reinterpret_cast<u32x4*>(vt + ((int64_t)head * D + d) * t_pad + key0 + k0) = o;
  }
}

// ---------------------------------------------------------------- attention

// S^T tile pair for one 32-key chunk starting at kc: lane (r16, g) gets the
// scaled scores of keys kc + 8g + jj (jj = 0..7) for its query, with keys past
// the query's position (or past t) at -inf. A-row i of tile tt is key
// kc + 8*(i/4) + 4*tt + (i%4), so both products see the same key order.
__device__ __forceinline__ void score_chunk(const bf16_t* __restrict__ kp, const u32x4* qf, int kc, int t,
                                            int pos, float scale, int r16, int g, float* sc) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    int key = kc + 8 * (r16 >> 2) + 4 * tt + (r16 & 3);
    key = min(key, t - 1);
    const bf16_t* kr = kp + (int64_t)key * D;
    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) a = mfma_bf16(*reinterpret_cast<const u32x4*>(kr + 32 * st + 8 * g), qf[st], a);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kk = kc + 8 * g + 4 * tt + r;
      sc[4 * tt + r] = (kk > pos || kk >= t) ? -INFINITY : a[r] * scale;
    }
  }
}

// Grid (ceil(s/64), hq); 4 waves, each owns 16 queries of one head. Keys are
// consumed in 64-key blocks aligned at key 0 with one running-max update per
// block, as the reference kernel does (BN = 64): s = (q.k)*scale in fp32,
// p = exp(s - max), den = den*alpha + sum(p), acc = acc*alpha + bf16(p).V,
// out = acc/den.
__global__ __launch_bounds__(kThreads) void attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ vt,
    const int64_t* __restrict__ positions, int gather_q, bf16_t* __restrict__ y, int s_len, int t,
    int t_pad, int hq, int hk, float scale) {
  const int head = blockIdx.y;
  const int kvh = head / (hq / hk);
  const int qblock = gridDim.x - 1 - blockIdx.x;  // heaviest (latest) query blocks first
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q0 = qblock * 64 + wave * 16;
  if (q0 >= s_len) return;
  const int r16 = lane & 15, g = lane >> 4;
  const int qi = q0 + r16;
  const bool qvalid = qi < s_len;
  const int qrow = qvalid ? qi : s_len - 1;
  const int pos = positions ? (int)positions[qrow] : qrow;
  int kend = pos + 1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) kend = max(kend, __shfl_xor(kend, o, 64));
  kend = min(kend, t);

  const int64_t qsrc = gather_q ? min(max(pos, 0), t - 1) : qrow;
  const bf16_t* qp = q + ((int64_t)head * (gather_q ? t : s_len) + qsrc) * D;
  u32x4 qf[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) qf[st] = *reinterpret_cast<const u32x4*>(qp + 32 * st + 8 * g);

  const bf16_t* kp = k + (int64_t)kvh * t * D;
  const bf16_t* vp = vt + (int64_t)kvh * D * t_pad;

  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, den = 0.f;

  for (int kb = 0; kb < kend; kb += 64) {
    const bool two = kb + 32 < kend;  // wave-uniform: second chunk has a visible key
    float sc[16];
    score_chunk(kp, qf, kb, t, pos, scale, r16, g, sc);
    if (two) {
      score_chunk(kp, qf, kb + 32, t, pos, scale, r16, g, sc + 8);
    } else {
#pragma unroll
      for (int jj = 8; jj < 16; ++jj) sc[jj] = -INFINITY;
    }
    float bmax = sc[0];
#pragma unroll
    for (int jj = 1; jj < 16; ++jj) bmax = fmaxf(bmax, sc[jj]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(m, bmax);
    const float alpha = expf(m - mnew);
    float p[16], psum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      p[jj] = expf(sc[jj] - mnew);
      psum += p[jj];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    den = den * alpha + psum;
    m = mnew;
    u32x4 pf0, pf1;
    pf0.x = pack_bf16x2(p[0], p[1]);
    pf0.y = pack_bf16x2(p[2], p[3]);
    pf0.z = pack_bf16x2(p[4], p[5]);
    pf0.w = pack_bf16x2(p[6], p[7]);
    pf1.x = pack_bf16x2(p[8], p[9]);
    pf1.y = pack_bf16x2(p[10], p[11]);
    pf1.z = pack_bf16x2(p[12], p[13]);
    pf1.w = pack_bf16x2(p[14], p[15]);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const bf16_t* vr = vp + (int64_t)(16 * dt + r16) * t_pad + kb + 8 * g;
      f32x4 acc = o[dt] * alpha;
      acc = mfma_bf16(*reinterpret_cast<const u32x4*>(vr), pf0, acc);
      if (two) acc = mfma_bf16(*reinterpret_cast<const u32x4*>(vr + 32), pf1, acc);
      o[dt] = acc;
    }
  }
  if (!qvalid) return;
  bf16_t* yp = y + ((int64_t)qi * hq + head) * D;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    u32x2 w2;
    w2.x = pack_bf16x2(o[dt][0] / den, o[dt][1] / den);
    w2.y = pack_bf16x2(o[dt][2] / den, o[dt][3] / den);
    *reinterpret_cast<u32x2*>(yp + 16 * dt + 4 * g) = w2;
  }
}

}  // namespace

extern "C" int ff_qkv_post(const void* q, const void* k, const void* v, int64_t row_stride,
                           const void* wq, const void* wk, float eps_q, float eps_k, const void* cos,
                           const void* sin, void* yq, void* yk, void* vt, int64_t t, int64_t t_pad,
                           int64_t hq, int64_t hk, int64_t d, ff_stream_t stream) {
  FF_REQUIRE(d == D, "ff_qkv_post: head_dim %lld unsupported (128 only)", (long long)d);
  FF_REQUIRE(q && k && wq && wk && cos && sin && yq && yk, "ff_qkv_post: null pointer");
  FF_REQUIRE(t > 0 && hq > 0 && hk > 0 && row_stride % 8 == 0, "ff_qkv_post: bad sizes");
  FF_REQUIRE(!vt || (v && t_pad >= t && t_pad % 64 == 0), "ff_qkv_post: v/t_pad");
  FF_REQUIRE(ff_aligned(q, 16) && ff_aligned(k, 16) && ff_aligned(yq, 16) && ff_aligned(yk, 16) &&
                 ff_aligned(cos, 16) && ff_aligned(sin, 16) && (!vt || (ff_aligned(v, 16) && ff_aligned(vt, 16))),
             "ff_qkv_post: alignment");
  const int nq = (int)((t * hq + 15) / 16), nk = (int)((t * hk + 15) / 16);
  const int nv = vt ? (int)(hk * (t_pad / 64)) : 0;
  hipLaunchKernelGGL(qkv_post_kernel, dim3(nq + nk + nv), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, row_stride, (int64_t)D,
                     (const bf16_t*)wq, (const bf16_t*)wk, eps_q, eps_k, (const bf16_t*)cos,
                     (const bf16_t*)sin, (int64_t)D, (int64_t)D, (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)vt,
                     (int)t, (int)t_pad, (int)hq, (int)hk, nq, nk);
  FF_LAUNCH_CHECK("ff_qkv_post");
  return FF_OK;
}

extern "C" int ff_qk_pair(const void* q, const void* k, int64_t row_stride, const void* wq,
                          const void* wk, float eps_q, float eps_k, const void* cos, const void* sin,
                          int64_t cos_ts, int64_t cos_ds, int64_t sin_ts, int64_t sin_ds, void* yq,
                          void* yk, int64_t t, int64_t hq, int64_t hk, int64_t d, ff_stream_t stream) {
  FF_REQUIRE(d == D, "ff_qk_pair: head_dim %lld unsupported (128 only)", (long long)d);
  FF_REQUIRE(cos_ds == 1 && sin_ds == 1 && cos_ts % 8 == 0 && sin_ts % 8 == 0,
             "ff_qk_pair: cos/sin must be contiguous along d");
  FF_REQUIRE(q && k && wq && wk && cos && sin && yq && yk, "ff_qk_pair: null pointer");
  FF_REQUIRE(t > 0 && hq > 0 && hk > 0 && row_stride % 8 == 0, "ff_qk_pair: bad sizes");
  FF_REQUIRE(ff_aligned(q, 16) && ff_aligned(k, 16) && ff_aligned(yq, 16) && ff_aligned(yk, 16) &&
                 ff_aligned(cos, 16) && ff_aligned(sin, 16),
             "ff_qk_pair: alignment");
  const int nq = (int)((t * hq + 15) / 16), nk = (int)((t * hk + 15) / 16);
  hipLaunchKernelGGL(qkv_post_kernel, dim3(nq + nk), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)nullptr, row_stride, (int64_t)0,
                     (const bf16_t*)wq, (const bf16_t*)wk, eps_q, eps_k, (const bf16_t*)cos,
                     (const bf16_t*)sin, cos_ts, sin_ts, (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)nullptr,
                     (int)t, 64, (int)hq, (int)hk, nq, nk);
  FF_LAUNCH_CHECK("ff_qk_pair");
  return FF_OK;
}

extern "C" int ff_v_transpose(const void* v, int64_t v_ts, int64_t v_hs, void* vt, int64_t t,
                              int64_t t_pad, int64_t hk, int64_t d, ff_stream_t stream) {
  FF_REQUIRE(d == D, "ff_v_transpose: head_dim %lld unsupported (128 only)", (long long)d);
  FF_REQUIRE(v && vt && t > 0 && t_pad >= t && t_pad % 64 == 0 && hk > 0, "ff_v_transpose: bad arguments");
  FF_REQUIRE(v_ts % 8 == 0 && v_hs % 8 == 0 && ff_aligned(v, 16) && ff_aligned(vt, 16),
             "ff_v_transpose: alignment");
  const int nv = (int)(hk * (t_pad / 64));
  hipLaunchKernelGGL(qkv_post_kernel, dim3(nv), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)nullptr, (const bf16_t*)nullptr, (const bf16_t*)v, v_ts, v_hs,
                     (const bf16_t*)nullptr, (const bf16_t*)nullptr, 0.f, 0.f, (const bf16_t*)nullptr,
                     (const bf16_t*)nullptr, (int64_t)0, (int64_t)0, (bf16_t*)nullptr, (bf16_t*)nullptr,
                     (bf16_t*)vt, (int)t, (int)t_pad, 1, (int)hk, 0, 0);
  FF_LAUNCH_CHECK("ff_v_transpose");
  return FF_OK;
}

extern "C" int ff_attention_vt(const void* q, const void* k, const void* vt, const int64_t* positions,
                               int gather_q, void* y, int64_t s, int64_t t, int64_t t_pad, int64_t hq,
                               int64_t hk, int64_t d, float scale, ff_stream_t stream) {
  FF_REQUIRE(d == D, "ff_attention_vt: head_dim %lld unsupported (128 only)", (long long)d);
  FF_REQUIRE(q && k && vt && y, "ff_attention_vt: null pointer");
  FF_REQUIRE(s > 0 && t > 0 && t_pad >= t && t_pad % 64 == 0 && hq > 0 && hk > 0 && hq % hk == 0,
             "ff_attention_vt: bad sizes s=%lld t=%lld t_pad=%lld hq=%lld hk=%lld", (long long)s,
             (long long)t, (long long)t_pad, (long long)hq, (long long)hk);
  FF_REQUIRE(positions || s <= t, "ff_attention_vt: without positions s must be <= t");
  FF_REQUIRE(!gather_q || positions, "ff_attention_vt: gather_q needs positions");
  FF_REQUIRE(ff_aligned(q, 16) && ff_aligned(k, 16) && ff_aligned(vt, 16) && ff_aligned(y, 8),
             "ff_attention_vt: alignment");
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)((s + 63) / 64), (unsigned)hq), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)vt, positions,
                     gather_q, (bf16_t*)y, (int)s, (int)t, (int)t_pad, (int)hq, (int)hk, scale);
  FF_LAUNCH_CHECK("ff_attention_vt");
  return FF_OK;
}
