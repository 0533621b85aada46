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
#include <stdlib.h>

#include "ff_common.h"
#include "ff_rope.h"

using namespace ff;

namespace {

constexpr int kThreads = 256;
constexpr int D = 128;

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// ---------------------------------------------------------------- q/k norm + rope


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
//
// Both attention kernels keep the reference kernel's schedule (BN = 64): keys
// are consumed in 64-key blocks aligned at key 0 with one running-max update
// per block; s = q.k * scale in fp32, p = exp(s - max), den = den*alpha +
// sum(p), acc = acc*alpha + bf16(p).V, out = acc/den. exp is the hardware
// exp2 of (s - max) * log2(e), as tl.exp lowers on the reference's GPUs.
// Both kernels share the per-block softmax below, so they produce identical
// bits for the same query.

// One 64-key block of the online softmax for a 16-query tile held as S^T
// accumulators: s[2c + tt][r] = q.k of key kb + 32c + 8g + 4tt + r for the
// lane's query (lane (r16, g) = (query, key group)). Keys whose offset
// 32c + 4tt + r exceeds lim = min(position, t-1) - kb - 8g are masked when
// `masked` (blocks entirely visible to the tile skip it). Returns alpha and P^T
// as bf16 B-operand fragments (keys kb + 32c + 8g .. +7 in pf[c]); den is this
// lane's partial denominator over its key groups (reduced with sum_rows at the
// end); m is the running max of q.k (the scale is positive, so max commutes
// with it).
__device__ __forceinline__ float softmax_block(f32x4 (&s)[4], bool masked, int lim, float c2, float& m,
                                               float& den, u32x4 (&pf)[2]) {
  if (masked) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (32 * (i >> 1) + 4 * (i & 1) + r > lim) s[i][r] = -INFINITY;
  }
  float bmax = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
#pragma unroll
  for (int i = 1; i < 4; ++i) bmax = fmaxf(bmax, fmaxf(fmaxf(s[i][0], s[i][1]), fmaxf(s[i][2], s[i][3])));
  const float mnew = fmaxf(m, max_rows(bmax));
  const float mref = mnew == -INFINITY ? 0.f : mnew;  // a fully masked query keeps p = 0, alpha = 0
  const float alpha = __builtin_amdgcn_exp2f((m - mref) * c2);
  float p[16], psum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = __builtin_amdgcn_exp2f((s[i][r] - mref) * c2);
      p[4 * i + r] = e;
      psum += e;
    }
  den = den * alpha + psum;
  m = mnew;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    pf[c].x = pack_bf16x2(p[8 * c + 0], p[8 * c + 1]);
    pf[c].y = pack_bf16x2(p[8 * c + 2], p[8 * c + 3]);
    pf[c].z = pack_bf16x2(p[8 * c + 4], p[8 * c + 5]);
    pf[c].w = pack_bf16x2(p[8 * c + 6], p[8 * c + 7]);
  }
  return alpha;
}

// acc *= alpha (its first DTN 16-column tiles), skipped when no query of the
// wave changed its max (alpha == 1 exactly leaves acc unchanged).
template <int DTN = 8>
__device__ __forceinline__ void rescale(f32x4 (&o)[8], float alpha) {
  if (__ballot(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt) o[dt] = o[dt] * alpha;
  }
}

// Output row of one (query, head): o / den as bf16, the first DOUT of the 128
// head dims (DOUT % 4 == 0; the columns past it are the zero padding of a
// narrower head).
template <int DOUT = D>
__device__ __forceinline__ void store_rows(bf16_t* __restrict__ yp, const f32x4 (&o)[8], float den, int g) {
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    if (16 * dt + 4 * g >= DOUT) continue;
    u32x2 w2;
    w2.x = pack_bf16x2(o[dt][0] / den, o[dt][1] / den);
    w2.y = pack_bf16x2(o[dt][2] / den, o[dt][3] / den);
    *reinterpret_cast<u32x2*>(yp + 16 * dt + 4 * g) = w2;
  }
}

// The same output row quantised with a static calibrated multiplier instead of
// stored: e4m3(clamp(bf16(o / den) * inv, +-448)), i.e. the bf16 attention
// output the reference writes, then its runtime-scale cast, 4 bytes per dt.
__device__ __forceinline__ void store_rows_q(uint8_t* __restrict__ yp, const f32x4 (&o)[8], float den, int g,
                                             float inv) {
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    *reinterpret_cast<uint32_t*>(yp + 16 * dt + 4 * g) =
        quant4_static(round_bf16(o[dt][0] / den), round_bf16(o[dt][1] / den), round_bf16(o[dt][2] / den),
                      round_bf16(o[dt][3] / den), inv);
  }
}

// S^T tiles of one 32-key chunk starting at kc read straight from global
// memory: A-row i of tile tt is key kc + 8*(i/4) + 4*tt + (i%4), so lane group
// g of the result holds keys kc + 8g + 4tt + r.
__device__ __forceinline__ void score_chunk(const bf16_t* __restrict__ kp, const u32x4* qf, int kc, int t,
                                            int r16, int g, f32x4& s0, f32x4& s1) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    int key = kc + 8 * (r16 >> 2) + 4 * tt + (r16 & 3);
    key = min(key, t - 1);
    const bf16_t* kr = kp + (int64_t)key * D;
    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) a = mfma_bf16(*reinterpret_cast<const u32x4*>(kr + 32 * st + 8 * g), qf[st], a);
    (tt ? s1 : s0) = a;
  }
}

// Per-head kernel, used for selected query positions (the pick-only tail) and
// head groups the grouped kernel does not cover. Grid (ceil(s/64), hq);
// 4 waves, each owns 16 queries of one head; K and V^T are read from global
// memory (L2) directly.
__global__ __launch_bounds__(kThreads) void attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ vt,
    const int64_t* __restrict__ positions, int gather_q, bf16_t* __restrict__ y, int s_len, int t,
    int t_pad, int hq, int hk, float c2) {
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
  const int plim = min(pos, t - 1);

  for (int kb = 0; kb < kend; kb += 64) {
    const bool two = kb + 32 < kend;  // wave-uniform: the second chunk has a visible key
    f32x4 sc[4];
    score_chunk(kp, qf, kb, t, r16, g, sc[0], sc[1]);
    if (two) {
      score_chunk(kp, qf, kb + 32, t, r16, g, sc[2], sc[3]);
    } else {
      sc[2] = sc[3] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    u32x4 pf[2];
    const float alpha = softmax_block(sc, true, plim - kb - 8 * g, c2, m, den, pf);
    rescale(o, alpha);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const bf16_t* vr = vp + (int64_t)(16 * dt + r16) * t_pad + kb + 8 * g;
      o[dt] = mfma_bf16(*reinterpret_cast<const u32x4*>(vr), pf[0], o[dt]);
      if (two) o[dt] = mfma_bf16(*reinterpret_cast<const u32x4*>(vr + 32), pf[1], o[dt]);
    }
  }
  den = sum_rows(den);
  if (!qvalid) return;
  store_rows(y + ((int64_t)qi * hq + head) * D, o, den, g);
}

// Selected rows, split over keys: for at most 16 queries (the pick-only tail
// scores one), one workgroup per head runs 8 waves over interleaved 64-key
// blocks (wave w takes blocks w, w + 8, ...) and keeps the reference's
// sequential schedule bit for bit in P:
//   pass 1: every wave computes its blocks' scores and each block's max per
//           query into LDS; the running max after block b of the sequential
//           walk is the prefix max pm[b] = max(bmax[0..b]), one scan per query;
//   pass 2: every wave forms p = exp(s - pm[b]) for its blocks with the
//           running max the sequential walk would hold at block b, so bf16(p)
//           -- the rounding the output depends on -- is identical. Its partial
//           den and acc = sum bf16(p).V are kept in the frame of its latest pm
//           and rescaled as pm grows, like the one-pass kernels' alpha.
// The waves' partials are merged in LDS in the frame of the final max
// M = pm[last]: den = sum_w den_w 2^((pm_w - M) log2e scale), acc likewise,
// out = acc / den. Only the fp32 order of the rescales differs from the
// one-pass kernels (a factor 2^((pm_b - M) c2) per wave instead of a product of
// per-block alphas).
//
// The kernel is a chain of dependent memory latencies, so its loads are issued
// as early as their addresses allow: the K fragments of a wave's first two
// blocks (all of them up to 1024 keys) at entry, beside the positions and
// before q, whose address may depend on the positions; their V^T fragments
// before the prefix-max scan. Those blocks keep their scores in registers
// from pass 1 to pass 2; blocks past the first two (t > 1024) recompute them
// from K in pass 2 with the same instructions, hence the same bits.
constexpr int kDecodeWaves = 8;
constexpr int kDecodeMaxBlocks = 256;  // 64-key blocks the LDS block maxima hold (t <= 16384)

// Maximum over the 16 lanes of each row of 16: quad_perm swaps (lane ^ 1,
// lane ^ 2), then row_half_mirror (lane i with 7 - i of each half row) and
// row_mirror (lane i with 15 - i).
__device__ __forceinline__ int max_row16(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));
  return max(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false));
}

// The 16 K fragments of 64-key block kb in the order the S MFMAs take them:
// kf[4 * (2c + tt) + st] is what score_chunk reads for chunk kb + 32c, tile tt,
// step st.
__device__ __forceinline__ void load_block_k(const bf16_t* __restrict__ kp, int kb, int t, int r16, int g,
                                             u32x4 (&kf)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = min(kb + 32 * (i >> 1) + 8 * (r16 >> 2) + 4 * (i & 1) + (r16 & 3), t - 1);
    const bf16_t* kr = kp + (int64_t)key * D;
#pragma unroll
    for (int st = 0; st < 4; ++st) kf[4 * i + st] = *reinterpret_cast<const u32x4*>(kr + 32 * st + 8 * g);
  }
}

// V^T fragments of block kb: vf[c][dt] feeds the P.V MFMA of chunk c, d tile dt
// (keys kb + 32c + 8g .. +7 of d row 16 dt + r16; t_pad >= kb + 64 keeps both
// chunks in bounds).
__device__ __forceinline__ void load_block_v(const bf16_t* __restrict__ vp, int kb, int t_pad, int r16, int g,
                                             u32x4 (&vf)[2][8]) {
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      vf[c][dt] = *reinterpret_cast<const u32x4*>(vp + (int64_t)(16 * dt + r16) * t_pad + kb + 32 * c + 8 * g);
}

// Scores of one 64-key block (kb) for the lane's query from its K fragments
// (score_chunk's arithmetic), the second 32-key chunk dropped when no visible
// key reaches it, masked past lim (the routine of softmax_block's mask); returns
// the block max over the tile's rows of this lane's query (reduced over the 4
// key groups).
__device__ __forceinline__ float decode_scores(const u32x4 (&kf)[16], const u32x4 (&qf)[4], int kb, int kend,
                                               int lim, f32x4 (&sc)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) a = mfma_bf16(kf[4 * i + st], qf[st], a);
    sc[i] = a;
  }
  if (!(kb + 32 < kend)) sc[2] = sc[3] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (32 * (i >> 1) + 4 * (i & 1) + r > lim) sc[i][r] = -INFINITY;
  float bmax = fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3]));
#pragma unroll
  for (int i = 1; i < 4; ++i) bmax = fmaxf(bmax, fmaxf(fmaxf(sc[i][0], sc[i][1]), fmaxf(sc[i][2], sc[i][3])));
  return max_rows(bmax);
}

// Pass 2 for one block: P against the sequential running max mnew of the
// block, this wave's den and acc rescaled into that frame, acc += bf16(P).V.
__device__ __forceinline__ void decode_accumulate(const f32x4 (&sc)[4], const u32x4 (&vf)[2][8], bool two,
                                                  float mnew, float c2, float& m, float& den, f32x4 (&o)[8]) {
  const float mref = mnew == -INFINITY ? 0.f : mnew;  // a fully masked query keeps p = 0
  const float alpha = __builtin_amdgcn_exp2f((m - mref) * c2);
  float p[16], psum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = __builtin_amdgcn_exp2f((sc[i][r] - mref) * c2);
      p[4 * i + r] = e;
      psum += e;
    }
  den = den * alpha + psum;
  m = mnew;
  u32x4 pf[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    pf[c].x = pack_bf16x2(p[8 * c + 0], p[8 * c + 1]);
    pf[c].y = pack_bf16x2(p[8 * c + 2], p[8 * c + 3]);
    pf[c].z = pack_bf16x2(p[8 * c + 4], p[8 * c + 5]);
    pf[c].w = pack_bf16x2(p[8 * c + 6], p[8 * c + 7]);
  }
  rescale(o, alpha);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    o[dt] = mfma_bf16(vf[0][dt], pf[0], o[dt]);
    if (two) o[dt] = mfma_bf16(vf[1][dt], pf[1], o[dt]);
  }
}

__global__ __launch_bounds__(kDecodeWaves * 64) void attention_decode_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ vt,
    const int64_t* __restrict__ positions, int gather_q, bf16_t* __restrict__ y, int s_len, int t, int t_pad,
    int hq, int hk, float c2) {
  __shared__ float pm[kDecodeMaxBlocks][16];
  __shared__ float sm[kDecodeWaves][16];
  __shared__ float sden[kDecodeWaves][16];
  __shared__ float so[kDecodeWaves][16][D + 1];
  const int head = blockIdx.x;
  const int kvh = head / (hq / hk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const bf16_t* kp = k + (int64_t)kvh * t * D;
  const bf16_t* vp = vt + (int64_t)kvh * D * t_pad;
  // The lane's query position, then the K of blocks b0 = wave and
  // b1 = wave + 8, then the visible key range: the maximum of
  // the positions over the 16 lanes of a row (every row holds the same ones).
  const bool qvalid = r16 < s_len;
  const int qrow = qvalid ? r16 : s_len - 1;
  const int pos = (int)positions[qrow];
  const int kb0 = wave * 64, kb1 = (wave + kDecodeWaves) * 64;
  u32x4 kf0[16], kf1[16];  // unconditional (keys clamp to t - 1): no branch splits the loads from the wait
  load_block_k(kp, kb0, t, r16, g, kf0);
  load_block_k(kp, kb1, t, r16, g, kf1);
  const int kend = min(__builtin_amdgcn_readfirstlane(max_row16(pos + 1)), t);
  const int nb = (kend + 63) / 64;  // <= kDecodeMaxBlocks (checked at launch)
  const int64_t qsrc = gather_q ? min(max(pos, 0), t - 1) : qrow;
  const bf16_t* qp = q + ((int64_t)head * (gather_q ? t : s_len) + qsrc) * D;
  u32x4 qf[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) qf[st] = *reinterpret_cast<const u32x4*>(qp + 32 * st + 8 * g);
  const int plim = min(pos, t - 1);

  // pass 1: block maxima (scores of the first two blocks kept), then the V^T
  // loads of those blocks, then the running max of the sequential walk
  f32x4 sc0[4], sc1[4];
  const bool has0 = kb0 < kend, has1 = kb1 < kend;  // wave-uniform
  if (has0) {
    const float bmax = decode_scores(kf0, qf, kb0, kend, plim - kb0 - 8 * g, sc0);
    if (g == 0) pm[wave][r16] = bmax;
  }
  if (has1) {
    const float bmax = decode_scores(kf1, qf, kb1, kend, plim - kb1 - 8 * g, sc1);
    if (g == 0) pm[wave + kDecodeWaves][r16] = bmax;
  }
  for (int kb = kb1 + kDecodeWaves * 64; kb < kend; kb += kDecodeWaves * 64) {
    u32x4 kf[16];
    load_block_k(kp, kb, t, r16, g, kf);
    f32x4 sc[4];
    const float bmax = decode_scores(kf, qf, kb, kend, plim - kb - 8 * g, sc);
    if (g == 0) pm[kb / 64][r16] = bmax;
  }
  u32x4 vf0[2][8], vf1[2][8];
  if (has0) load_block_v(vp, kb0, t_pad, r16, g, vf0);
  if (has1) load_block_v(vp, kb1, t_pad, r16, g, vf1);
  barrier_lds();  // block maxima written (the V^T loads stay in flight)
  // prefix max over the blocks, 16 blocks at a time per query
  if (threadIdx.x < 16) {
    float run = -INFINITY;
    for (int b0 = 0; b0 < nb; b0 += 16) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = b0 + j < nb ? pm[b0 + j][threadIdx.x] : -INFINITY;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        run = fmaxf(run, v[j]);
        if (b0 + j < nb) pm[b0 + j][threadIdx.x] = run;
      }
    }
  }
  barrier_lds();

  // pass 2: P against the sequential running max of each block
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, den = 0.f;  // the frame (a prefix max) of this wave's partials
  if (has0) decode_accumulate(sc0, vf0, kb0 + 32 < kend, pm[wave][r16], c2, m, den, o);
  if (has1) decode_accumulate(sc1, vf1, kb1 + 32 < kend, pm[wave + kDecodeWaves][r16], c2, m, den, o);
  for (int kb = kb1 + kDecodeWaves * 64; kb < kend; kb += kDecodeWaves * 64) {
    u32x4 kf[16];
    u32x4 vf[2][8];
    load_block_k(kp, kb, t, r16, g, kf);
    load_block_v(vp, kb, t_pad, r16, g, vf);
    f32x4 sc[4];
    decode_scores(kf, qf, kb, kend, plim - kb - 8 * g, sc);
    decode_accumulate(sc, vf, kb + 32 < kend, pm[kb / 64][r16], c2, m, den, o);
  }
  den = sum_rows(den);
  if (g == 0) {
    sm[wave][r16] = m;
    sden[wave][r16] = den;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) so[wave][r16][16 * dt + 4 * g + r] = o[dt][r];
  __syncthreads();
  // merge: thread -> (query, 4 consecutive d), in the frame of the final running max
  for (int e = threadIdx.x; e < 16 * (D / 4); e += kDecodeWaves * 64) {
    const int qi = e / (D / 4), d0 = (e % (D / 4)) * 4;
    if (qi >= s_len) continue;
    const float mx = nb > 0 ? pm[nb - 1][qi] : -INFINITY;
    const float mref = mx == -INFINITY ? 0.f : mx;
    float dsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      if (w * 64 >= kend) continue;  // a wave without blocks holds nothing
      const float wt = __builtin_amdgcn_exp2f((sm[w][qi] - mref) * c2);
      dsum += sden[w][qi] * wt;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += so[w][qi][d0 + r] * wt;
    }
    u32x2 w2;
    w2.x = pack_bf16x2(acc[0] / dsum, acc[1] / dsum);
    w2.y = pack_bf16x2(acc[2] / dsum, acc[3] / dsum);
    *reinterpret_cast<u32x2*>(y + ((int64_t)qi * hq + head) * D + d0) = w2;
  }
}

// ---------------------------------------------------------------- grouped prefill attention
//
// A workgroup owns one 64-key-block walk for HPW query heads that share a kv
// head (HPW = 4, 2 or 1 for GQA groups that are multiples of 4, 2 or 1) and
// QB = 16*QT*(4/HPW) consecutive queries: wave w takes head w % HPW and QT
// tiles of 16 queries from row set w / HPW. Each 64-key block of K
// (64 x 256 B) and V^T (128 x 128 B) is fetched once per workgroup into LDS
// with global_load_lds_dwordx4 (one 1 KB instruction = 8 rows x 128 B, whole
// cache lines), NS stages deep with NS-1 in flight (NS = 3: one workgroup per
// CU, 96 KB LDS; NS = 2: two per CU, 64 KB each), and every fragment read
// from LDS feeds QT MFMAs.
//
// LDS stage layout (32 KB): K at [0, 16 KB), V^T at [16 KB, 32 KB), each as
// sixteen 1 KB blocks of 8 rows x 128 B. K row `key` (0..63 within the block)
// half h sits in block 2*(key/8) + h, row key%8; V^T row d in block d/8, row
// d%8. Inside a 128 B row the 16 B chunk c is stored at slot c ^ swz with
// swz = ((key>>1)&1) | ((key>>2)&6) for K and (d>>1)&7 for V^T, which makes
// every MFMA fragment read (16 lanes per LDS cycle) hit 16 distinct bank
// groups.
//
// Grid: one dimension, heaviest query blocks first across all groups; the
// group is blockIdx % (hq/HPW), so with 8 XCDs taking workgroups round-robin
// the groups of one kv head stay on one XCD (and its L2).
//
// CAUSAL = false: every query sees all t keys (bidirectional attention of the
// vision tower); only the keys past t in the last block are masked. DOUT: the
// head dim stored per (query, head) of y, which is (s, hq, DOUT); heads
// narrower than 128 are zero-padded to 128 in q, k and V^T, which leaves every
// score and every stored output column exact.
template <int QT, int HPW, int NS, bool CAUSAL = true, int DOUT = D, bool QOUT = false>
__global__ __launch_bounds__(kThreads, NS == 2 ? 2 : 1) void attention_prefill_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ vt,
    bf16_t* __restrict__ y, int s_len, int t, int t_pad, int hq, int hk, float c2, int nqb, float qinv) {
  constexpr int QB = 16 * QT * (4 / HPW);
  constexpr int STAGE = 32 * 1024;
  static_assert(NS == 2 || NS == 3, "two or three K/V stages");
  __shared__ __align__(1024) uint8_t smem[NS * STAGE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int ngroups = hq / HPW;
  const int grp = (int)blockIdx.x % ngroups;
  const int qb = nqb - 1 - (int)blockIdx.x / ngroups;
  const int head = grp * HPW + wave % HPW;
  const int kvh = head / (hq / hk);
  const int q0 = qb * QB;
  const int wq0 = q0 + (wave / HPW) * 16 * QT;  // first query of this wave
  const int kend = CAUSAL ? min(t, min(s_len, q0 + QB)) : t;  // keys [0, kend) are visible to some query
  const int nblocks = (kend + 63) / 64;

  // Load sources of this lane: blocks wave + 4i, i = 0..7 (0..15 K, 16..31 V^T).
  const bf16_t* kbase = k + (int64_t)kvh * t * D;
  const bf16_t* vbase = vt + (int64_t)kvh * D * t_pad;
  int k_key[4], k_col[4];
  int64_t v_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int bi = wave + 4 * i;  // K block
    const int key = 8 * (bi >> 1) + (lane >> 3);
    const int swz = ((key >> 1) & 1) | ((key >> 2) & 6);
    k_key[i] = key;
    k_col[i] = 64 * (bi & 1) + 8 * ((lane & 7) ^ swz);
    const int d = 8 * bi + (lane >> 3);  // V^T block bi
    v_off[i] = (int64_t)d * t_pad + 8 * ((lane & 7) ^ ((d >> 1) & 7));
  }
  const uint32_t lds0 = lds_addr(smem) + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024;
  auto issue = [&](int kb, int buf) {
    const uint32_t st = lds0 + buf * STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = min(kb + k_key[i], t - 1);
      lds_dma16(kbase + (int64_t)key * D + k_col[i], st + 4 * i * 1024);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) lds_dma16(vbase + v_off[i] + kb, st + 16 * 1024 + 4 * i * 1024);
  };

  // Fragment read offsets (bytes within a stage). K fragment (c, tt, st):
  // key = 32c + 8(r16>>2) + 4tt + (r16&3), d chunk 4st + g, swz = r16>>1.
  // V^T fragment (dt, c): d = 16dt + r16, key chunk 4c + g, swz = (r16>>1)&7.
  const int sw = r16 >> 1;
  auto koff = [&](int c, int tt, int st) {
    return ((4 * c + (r16 >> 2)) * 2 + (st >> 1)) * 1024 + (4 * tt + (r16 & 3)) * 128 +
           16 * ((4 * (st & 1) + g) ^ sw);
  };
  auto voff = [&](int dt, int c) {
    return 16 * 1024 + (2 * dt + (r16 >> 3)) * 1024 + (r16 & 7) * 128 + 16 * ((4 * c + g) ^ sw);
  };

  f32x4 o[QT][8];
  float m[QT], den[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = -INFINITY;
    den[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // The first NS-1 key blocks and the queries load together. The queries are
  // waited for before the loop: a compiler-placed wait for them inside the
  // loop would also wait for the prefetches issued there.
  issue(0, 0);
  if (NS == 3 && nblocks > 1) issue(64, 1);
  // Head dims past DOUT are zero in q, k and V^T: only the first KST 32-dim
  // steps of q.k and the first DTN 16-dim tiles of P.V are computed.
  constexpr int KST = (DOUT + 31) / 32, DTN = (DOUT + 15) / 16;
  u32x4 qf[QT][4];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qrow = min(wq0 + 16 * qt + r16, s_len - 1);
    const bf16_t* qp = q + ((int64_t)head * s_len + qrow) * D;
#pragma unroll
    for (int st = 0; st < KST; ++st) qf[qt][st] = *reinterpret_cast<const u32x4*>(qp + 32 * st + 8 * g);
  }
  // consuming the registers here makes the compiler wait for the loads now
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int st = 0; st < KST; ++st)
      asm volatile("" : : "v"(qf[qt][st].x), "v"(qf[qt][st].y), "v"(qf[qt][st].z), "v"(qf[qt][st].w));
  for (int ib = 0; ib < nblocks; ++ib) {
    if (NS == 3 && ib + 1 < nblocks) wait_vmcnt<8>();
    else wait_vmcnt<0>();
    barrier_lds();  // block ib landed for every wave; block ib-1 fully consumed
    if (ib + NS - 1 < nblocks) issue((ib + NS - 1) * 64, (ib + NS - 1) % NS);
    const int kb = ib * 64;
    if (CAUSAL && (kb >= s_len || kb > wq0 + 16 * QT - 1)) continue;  // wave-uniform: no query of the wave sees it
    const uint8_t* st_base = smem + (ib % NS) * STAGE;

    // Every K fragment of the block is read before the first S MFMA, and every
    // V^T fragment right after the last one, so that these LDS reads are in
    // flight together (one latency per group, the V^T reads under the softmax)
    // instead of a few at a time ahead of each MFMA. The scheduling barriers
    // keep the compiler from sinking the reads back to their uses. QT = 4 has
    // no registers for that and reads each fragment ahead of its MFMAs.
    constexpr bool BATCH = QT <= 2;
    u32x4 kf[KST][4], vf[2][DTN];
    if constexpr (BATCH) {
#pragma unroll
      for (int st = 0; st < KST; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) kf[st][i] = *reinterpret_cast<const u32x4*>(st_base + koff(i >> 1, i & 1, st));
      __builtin_amdgcn_sched_barrier(0);
    }
    f32x4 sc[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[qt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KST; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (!BATCH) kf[st][i] = *reinterpret_cast<const u32x4*>(st_base + koff(i >> 1, i & 1, st));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) sc[qt][i] = mfma_bf16(kf[st][i], qf[qt][st], sc[qt][i]);
      }
    if constexpr (BATCH) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt) vf[c][dt] = *reinterpret_cast<const u32x4*>(st_base + voff(dt, c));
      __builtin_amdgcn_sched_barrier(0);
    }
    u32x4 pf[QT][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int tq0 = wq0 + 16 * qt;  // first query of the tile
      const bool masked = CAUSAL ? (kb + 63 > tq0 || kb + 63 >= t) : kb + 63 >= t;
      const int lim = (CAUSAL ? min(tq0 + r16, t - 1) : t - 1) - kb - 8 * g;
      const float alpha = softmax_block(sc[qt], masked, lim, c2, m[qt], den[qt], pf[qt]);
      rescale<DTN>(o[qt], alpha);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) {
        if constexpr (!BATCH) vf[c][dt] = *reinterpret_cast<const u32x4*>(st_base + voff(dt, c));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][dt] = mfma_bf16(vf[c][dt], pf[qt][c], o[qt][dt]);
      }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float dsum = sum_rows(den[qt]);
    const int qi = wq0 + 16 * qt + r16;
    if (qi >= s_len) continue;
    if constexpr (QOUT)
      store_rows_q(reinterpret_cast<uint8_t*>(y) + ((int64_t)qi * hq + head) * D, o[qt], dsum, g, qinv);
    else
      store_rows<DOUT>(y + ((int64_t)qi * hq + head) * DOUT, o[qt], dsum, g);
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

// y: bf16 output (s, hq, 128); or, with yq, the e4m3 codes of it under the
// static multiplier qinv (grouped prefill only).
static int attention_vt(const void* q, const void* k, const void* vt, const int64_t* positions, int gather_q,
                        void* y, void* yq, float qinv, int64_t s, int64_t t, int64_t t_pad, int64_t hq, int64_t hk,
                        int64_t d, float scale, ff_stream_t stream) {
  FF_REQUIRE(d == D, "ff_attention_vt: head_dim %lld unsupported (128 only)", (long long)d);
  FF_REQUIRE(q && k && vt && (y || yq), "ff_attention_vt: null pointer");
  FF_REQUIRE(s > 0 && t > 0 && t_pad >= t && t_pad % 64 == 0 && hq > 0 && hk > 0 && hq % hk == 0,
             "ff_attention_vt: bad sizes s=%lld t=%lld t_pad=%lld hq=%lld hk=%lld", (long long)s,
             (long long)t, (long long)t_pad, (long long)hq, (long long)hk);
  FF_REQUIRE(positions || s <= t, "ff_attention_vt: without positions s must be <= t");
  FF_REQUIRE(!gather_q || positions, "ff_attention_vt: gather_q needs positions");
  FF_REQUIRE(ff_aligned(q, 16) && ff_aligned(k, 16) && ff_aligned(vt, 16) && ff_aligned(y ? y : yq, 8),
             "ff_attention_vt: alignment");
  const float c2 = (float)((double)scale * 1.4426950408889634);  // scale * log2(e)
  const int group = (int)(hq / hk);
  const int hpw = group % 4 == 0 ? 4 : (group == 2 ? 2 : (group == 1 ? 1 : 0));
  hipStream_t st = (hipStream_t)stream;
  if (!positions && s == t && hpw) {
    // ff_set_tuning(FF_TUNE_ATTN_QT, 1 | 2 | 4) overrides the query tiles per wave.
    const int qt_env = ff_tuning(FF_TUNE_ATTN_QT);
    // One query tile per wave while the grid at one tile stays under 1024
    // workgroups: 32/8 heads at 1040 / 1536 tokens take 22.6 / 37.0 us with one
    // tile and 28.6 / 41.9 us with two; at 2048 tokens (1024 workgroups) two
    // tiles are ahead, 57.4 against 59.6 us (88.5 against 104.2 with 64/8 heads).
    const int64_t wg1 = (s + 64 / hpw - 1) / (64 / hpw) * (hq / hpw);  // 16 (4 / hpw) queries x hpw heads each
    const int qt = (qt_env == 1 || qt_env == 2 || qt_env == 4)
                       ? qt_env
                       : (s <= 1024 || (s <= 2048 && wg1 < 1024) ? 1 : (s <= 2048 ? 2 : 4));
    // ff_set_tuning(FF_TUNE_ATTN_NS, 2 | 3) overrides the number of K/V LDS stages.
    const int ns_env = ff_tuning(FF_TUNE_ATTN_NS);
    // Two stages run at two workgroups per CU, which fits the registers of
    // QT <= 2 only (QT = 4 would spill); at QT = 1 the 8B prefill (576 tokens,
    // 32/8 heads) takes 12.9 us with two stages and 15.2 us with three.
    const int ns = qt <= 2 && ns_env != 3 ? 2 : 3;
    const int qb = 16 * qt * (4 / hpw);
    const int nqb = (int)((s + qb - 1) / qb);
    const dim3 grid((unsigned)(nqb * (hq / hpw))), block(kThreads);
#define FF_PREFILL(QT, HPW, NS)                                                                              \
  if (qt == QT && hpw == HPW && ns == NS) {                                                                  \
    if (yq)                                                                                                   \
      hipLaunchKernelGGL((attention_prefill_kernel<QT, HPW, NS, true, D, true>), grid, block, 0, st,         \
                         (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)vt, (bf16_t*)yq, (int)s, (int)t,   \
                         (int)t_pad, (int)hq, (int)hk, c2, nqb, qinv);                                        \
    else                                                                                                      \
      hipLaunchKernelGGL((attention_prefill_kernel<QT, HPW, NS>), grid, block, 0, st, (const bf16_t*)q,      \
                         (const bf16_t*)k, (const bf16_t*)vt, (bf16_t*)y, (int)s, (int)t, (int)t_pad,        \
                         (int)hq, (int)hk, c2, nqb, 0.f);                                                     \
  }
#define FF_PREFILL_NS(QT, HPW) FF_PREFILL(QT, HPW, 2) FF_PREFILL(QT, HPW, 3)
    FF_PREFILL_NS(1, 4) FF_PREFILL_NS(2, 4) FF_PREFILL(4, 4, 3)
    FF_PREFILL_NS(1, 2) FF_PREFILL_NS(2, 2) FF_PREFILL(4, 2, 3)
    FF_PREFILL_NS(1, 1) FF_PREFILL_NS(2, 1) FF_PREFILL(4, 1, 3)
#undef FF_PREFILL_NS
#undef FF_PREFILL
    FF_LAUNCH_CHECK("ff_attention_vt");
    return FF_OK;
  }
  FF_REQUIRE(!yq, "ff_attention_vt_q: quantised output only for causal prefill (s == t, no positions, hq/hk in "
                  "{1, 2} or a multiple of 4)");
  if (positions && s <= 16 && (t + 63) / 64 <= kDecodeMaxBlocks) {
    hipLaunchKernelGGL(attention_decode_kernel, dim3((unsigned)hq), dim3(kDecodeWaves * 64), 0, st,
                       (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)vt, positions, gather_q, (bf16_t*)y,
                       (int)s, (int)t, (int)t_pad, (int)hq, (int)hk, c2);
    FF_LAUNCH_CHECK("ff_attention_vt");
    return FF_OK;
  }
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)((s + 63) / 64), (unsigned)hq), dim3(kThreads), 0, st,
                     (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)vt, positions, gather_q, (bf16_t*)y,
                     (int)s, (int)t, (int)t_pad, (int)hq, (int)hk, c2);
  FF_LAUNCH_CHECK("ff_attention_vt");
  return FF_OK;
}

extern "C" int ff_attention_vt(const void* q, const void* k, const void* vt, const int64_t* positions,
                               int gather_q, void* y, int64_t s, int64_t t, int64_t t_pad, int64_t hq,
                               int64_t hk, int64_t d, float scale, ff_stream_t stream) {
  return attention_vt(q, k, vt, positions, gather_q, y, nullptr, 0.f, s, t, t_pad, hq, hk, d, scale, stream);
}

extern "C" int ff_attention_vt_q(const void* q, const void* k, const void* vt, void* yq, float inv, int64_t s,
                                 int64_t t, int64_t t_pad, int64_t hq, int64_t hk, int64_t d, float scale,
                                 ff_stream_t stream) {
  FF_REQUIRE(yq, "ff_attention_vt_q: null output");
  return attention_vt(q, k, vt, nullptr, 0, nullptr, yq, inv, s, t, t_pad, hq, hk, d, scale, stream);
}

extern "C" int ff_attention_full(const void* q, const void* k, const void* vt, void* y, int64_t t, int64_t t_pad,
                                 int64_t heads, int64_t d_out, float scale, ff_stream_t stream) {
  FF_REQUIRE(q && k && vt && y, "ff_attention_full: null pointer");
  FF_REQUIRE(t > 0 && t_pad >= t && t_pad % 64 == 0 && heads > 0, "ff_attention_full: bad sizes t=%lld t_pad=%lld",
             (long long)t, (long long)t_pad);
  FF_REQUIRE(d_out == 64 || d_out == 72 || d_out == 128,
             "ff_attention_full: output head dim %lld unsupported (64, 72, 128)",
             (long long)d_out);
  FF_REQUIRE(ff_aligned(q, 16) && ff_aligned(k, 16) && ff_aligned(vt, 16) && ff_aligned(y, 8),
             "ff_attention_full: alignment");
  const float c2 = (float)((double)scale * 1.4426950408889634);  // scale * log2(e)
  // One query tile per wave while that grid fits two workgroups per CU (512;
  // the 8B tower at 2048 patches, 16 heads: 512 workgroups, tower step 5.97
  // -> 5.87 ms against two tiles at 256, same bits), else two.
  // ff_set_tuning(FF_TUNE_ATTN_QT, 1 | 2) overrides the query tiles per wave.
  const int qt_env = ff_tuning(FF_TUNE_ATTN_QT);
  const int qt = qt_env == 1 || qt_env == 2 ? qt_env : ((t + 63) / 64 * heads <= 512 ? 1 : 2);
  const int qb = 16 * qt * 4;  // one head per workgroup: 4 waves x QT tiles of 16 queries
  const int nqb = (int)((t + qb - 1) / qb);
  const dim3 grid((unsigned)(nqb * heads)), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
#define FF_FULL(QT, DO)                                                                                    \
  if (qt == QT && d_out == DO)                                                                             \
    hipLaunchKernelGGL((attention_prefill_kernel<QT, 1, 2, false, DO>), grid, block, 0, st, (const bf16_t*)q, \
                       (const bf16_t*)k, (const bf16_t*)vt, (bf16_t*)y, (int)t, (int)t, (int)t_pad, (int)heads, \
                       (int)heads, c2, nqb, 0.f);
  FF_FULL(1, 64) FF_FULL(2, 64) FF_FULL(1, 72) FF_FULL(2, 72) FF_FULL(1, 128) FF_FULL(2, 128)
#undef FF_FULL
  FF_LAUNCH_CHECK("ff_attention_full");
  return FF_OK;
}
