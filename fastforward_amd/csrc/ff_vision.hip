// Vision-tower kernels for gfx950: pixel packing, LayerNorm, the bf16 linear
// layers (bias, GELU and residual epilogues), the 2-D vision rotary and the
// zero-padded head layouts the attention kernel reads.
//
// The tower is the reference's NativeNormVision.core (scaled_qwen_runtime.py:42-55):
// patch embedding + interpolated position embedding, then per block
// h += proj(attn(rope(qkv(LN1(h))))), h += fc2(gelu(fc1(LN2(h)))), DeepStack
// mergers after the listed blocks and the final patch merger. Every module is
// a bf16 torch module there, so each kernel rounds to bf16 where that module
// returns.
#include <math.h>

#include <stdlib.h>
#include <string.h>

#include "ff_common.h"

using namespace ff;

namespace {

constexpr int kThreads = 256;
constexpr int kXcds = 8;
constexpr int kPatchElems = 1536;  // 3 channels x 2 frames x 16 x 16

// ---------------------------------------------------------------- pixel packing
//
// rgb (height, width, 3) uint8 -> patches (n, 1536) bf16 in the order the
// image processor emits them: patch p of the 2 x 2 merge-block walk (blocks
// row-major over the (height/32, width/32) grid, the four 16 x 16 patches of a
// block row-major), element d = (c, frame, y, x) with both frames the same
// image; value (u8 - 127.5) / 127.5 (pack_rectangle, _family/depth_runtime.py:18-25).
// One thread per 8 consecutive elements (8 pixels of one row of one channel).
__global__ __launch_bounds__(kThreads) void pack_pixels_kernel(const uint8_t* __restrict__ rgb,
                                                               bf16_t* __restrict__ out, int width, int64_t chunks) {
  const int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (i >= chunks) return;
  const int64_t p = i / (kPatchElems / 8);
  const int d = (int)(i % (kPatchElems / 8)) * 8;
  const int c = d / 512, y0 = (d % 256) / 16, x0 = d % 16;
  const int gw = width / 16;
  const int64_t gy = p / (gw / 2 * 4);
  const int gx = (int)((p / 4) % (gw / 2)), my = (int)(p % 4) / 2, mx = (int)(p % 2);
  const int64_t y = gy * 32 + my * 16 + y0;
  const int x = gx * 32 + mx * 16 + x0;
  const uint8_t* src = rgb + (y * width + x) * 3 + c;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = ((float)src[3 * e] - 127.5f) / 127.5f;
  *reinterpret_cast<u32x4*>(out + p * kPatchElems + d) = pack8(v);
}

// ---------------------------------------------------------------- LayerNorm
//
// y = bf16((x - mean) * rstd * w + b) per row, mean and variance in fp32 over
// the bf16 inputs (two passes over registers), rstd = 1/sqrt(var + eps).
// One workgroup per row, h % 8 == 0, h <= 8 * 256 * kLnChunks.
constexpr int kLnChunks = 3;

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = sum_rows(v);
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += red[w];
  return t;
}

// Columns [col, col + 8) of row `row` of a k-split GEMM's output: the S fp32
// partial rows added in split order, then bf16(sum + bias) and, with a
// residual row r, bf16(r + that): the epilogue of gemm_bf16_kernel (no
// activation) on the split sums. The results are bf16 values held as floats.
__device__ __forceinline__ void split_row8(const float* __restrict__ part, int splits, int64_t mp, int n, int64_t row,
                                           int col, const bf16_t* __restrict__ bias, const bf16_t* r, float (&v)[8]) {
  const float* src = part + row * n + col;
  f32x4 s0 = *reinterpret_cast<const f32x4*>(src), s1 = *reinterpret_cast<const f32x4*>(src + 4);
  for (int sp = 1; sp < splits; ++sp) {
    const f32x4 t0 = *reinterpret_cast<const f32x4*>(src + sp * mp * n);
    const f32x4 t1 = *reinterpret_cast<const f32x4*>(src + sp * mp * n + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s0[e] += t0[e];
      s1[e] += t1[e];
    }
  }
  float bv[8];
  unpack8(*reinterpret_cast<const u32x4*>(bias + col), bv);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = round_bf16(s0[e] + bv[e]);
    v[4 + e] = round_bf16(s1[e] + bv[4 + e]);
  }
  if (r) {
    float rv[8];
    unpack8(*reinterpret_cast<const u32x4*>(r + col), rv);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = round_bf16(rv[e] + v[e]);
  }
}

// PART: the row is first formed from the S fp32 partial rows of a k-split
// GEMM (added in split order) as that GEMM's epilogue would: y = bf16(r +
// bf16(sum + bias)) with the residual r; y is stored (yres, which may be r
// itself: each element is read and written by one thread) and normalised.
// x is unused then.
template <bool PART = false>
__global__ __launch_bounds__(kThreads) void layer_norm_kernel(const bf16_t* __restrict__ x, int64_t x_rs,
                                                              const bf16_t* __restrict__ w,
                                                              const bf16_t* __restrict__ b, bf16_t* __restrict__ y,
                                                              int64_t y_rs, int h, float eps,
                                                              const float* __restrict__ part = nullptr,
                                                              int splits = 0, int64_t mp = 0,
                                                              const bf16_t* __restrict__ bias = nullptr,
                                                              const bf16_t* resid = nullptr, int64_t ldr = 0,
                                                              bf16_t* yres = nullptr, int64_t ldyres = 0) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const bf16_t* xr = x + row * x_rs;
  float v[kLnChunks][8];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kLnChunks; ++c) {
    const int col = 8 * (threadIdx.x + kThreads * c);
    if (col < h) {
      if constexpr (PART) {
        split_row8(part, splits, mp, h, row, col, bias, resid ? resid + row * ldr : nullptr, v[c]);
        *reinterpret_cast<u32x4*>(yres + row * ldyres + col) = pack8(v[c]);
      } else {
        unpack8(*reinterpret_cast<const u32x4*>(xr + col), v[c]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[c][e];
    }
  }
  const float mean = block_sum(s, red) / (float)h;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < kLnChunks; ++c) {
    const int col = 8 * (threadIdx.x + kThreads * c);
    if (col < h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dlt = v[c][e] - mean;
        q += dlt * dlt;
      }
    }
  }
  const float var = block_sum(q, red) / (float)h;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int c = 0; c < kLnChunks; ++c) {
    const int col = 8 * (threadIdx.x + kThreads * c);
    if (col < h) {
      float wv[8], bv[8], o[8];
      unpack8(*reinterpret_cast<const u32x4*>(w + col), wv);
      unpack8(*reinterpret_cast<const u32x4*>(b + col), bv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[c][e] - mean) * rstd * wv[e] + bv[e];
      *reinterpret_cast<u32x4*>(y + row * y_rs + col) = pack8(o);
    }
  }
}

// ---------------------------------------------------------------- bf16 GEMM
//
// y[m, n] = epilogue(sum_k a[m, k] w[n, k]) with a (M, K) and w (N, K) bf16,
// both K-contiguous (torch Linear weights). A workgroup of 4 waves (2 x 2)
// owns a BM x BN tile; each wave (BM/2) x (BN/2) as 16 x 16 tiles of
// v_mfma_f32_16x16x32_bf16. K advances 64 elements (128 bytes) per stage:
// both operands go global -> LDS with global_load_lds_dwordx4 (8 rows x 128 B
// per instruction, XOR-swizzled 16-byte chunks), S stages with S - 1 in
// flight, one barrier per stage. Lane l (row l % 16, g = l / 16) reads chunks
// 2g and 2g + 1 of its row for the two MFMAs of a stage: k [16 g, 16 g + 8)
// and [16 g + 8, 16 g + 16) of the 64, the same k for A and B.
//
// Epilogue (the bf16 module boundaries of the reference): v = bf16(acc + bias);
// kGeluTanh: v = bf16(gelu_tanh(v)); kGeluErf: v = bf16(gelu(v)); with a
// residual r: y = bf16(r + v) (r may be y itself: each element is read and
// written by one thread).
constexpr int kActNone = 0, kGeluTanh = 1, kGeluErf = 2;

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// GELU with the tanh approximation, as torch computes it in fp32 for bf16
// tensors: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k_beta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float inner = k_beta * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// Exact GELU: x / 2 (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float gelu_erf(float x) { return x * 0.5f * (1.0f + erff(x * 0.7071067811865476f)); }

template <int BM, int BN, int S>
struct GemmCfg {
  static constexpr int RA = BM / 16, RB = BN / 16;
  static constexpr int BLOCKS = 2 * (RA + RB);  // 1 KB blocks per stage
  static constexpr int STAGE = BLOCKS * 1024;
  static constexpr int WI = RA / 2, WJ = RB / 2;
  static constexpr int SMEM = S * STAGE;
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(RA % 2 == 0 && RB % 2 == 0 && BLOCKS % 4 == 0, "2 x 2 waves");
};

template <int BM, int BN, int S, int OCC, int ACT, bool RESID>
__global__ __launch_bounds__(kThreads, OCC) void gemm_bf16_kernel(
    const bf16_t* __restrict__ a, int64_t lda, const bf16_t* __restrict__ w, const bf16_t* __restrict__ bias,
    bf16_t* y, int64_t ldy, const bf16_t* resid, int64_t ldr, int M, int N, int K, int tiles_m, int tiles_n) {
  using C = GemmCfg<BM, BN, S>;
  __shared__ __align__(1024) uint8_t smem[C::SMEM];
  __shared__ __align__(16) bf16_t sbias[BN];  // the tile's bias columns
  static_assert(BN == 128, "one wave's dword DMA carries the tile's bias");
  const int nblk = tiles_m * tiles_n;
  const int blk_id = blockIdx.x;
  int logical = blk_id;
  if (nblk % kXcds == 0) logical = (blk_id % kXcds) * (nblk / kXcds) + blk_id / kXcds;
  const int tm = logical % tiles_m, tn = logical / tiles_m;  // M fastest: an XCD's tiles share weight slabs
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  // Sources of this lane for each 1 KB block it loads (k offset 0); rows past
  // M / N are clamped (in bounds; masked at the store).
  constexpr int PER_WAVE = C::BLOCKS / 4;
  const uint8_t* src[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int blk = wave + 4 * i, h = blk & 1;
    const int rr = 8 * h + (lane >> 3);
    const int ch = (lane & 7) ^ (rr >> 1);
    if (blk < 2 * C::RA) {
      const int row = min(m0 + (blk >> 1) * 16 + rr, M - 1);
      src[i] = reinterpret_cast<const uint8_t*>(a + (int64_t)row * lda) + 16 * ch;
    } else {
      const int row = min(n0 + ((blk - 2 * C::RA) >> 1) * 16 + rr, N - 1);
      src[i] = reinterpret_cast<const uint8_t*>(w + (int64_t)row * K) + 16 * ch;
    }
  }
  const uint32_t lds0 = lds_addr(smem) + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024;
  auto issue = [&](int kt, int buf) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) lds_dma16(src[i] + (int64_t)kt * 128, lds0 + buf * C::STAGE + 4 * i * 1024);
  };

  f32x4 acc[C::WI][C::WJ];
#pragma unroll
  for (int i = 0; i < C::WI; ++i)
#pragma unroll
    for (int j = 0; j < C::WJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / 64;
  // Wave 0 copies the tile's bias into LDS ahead of the first stage (one
  // dword DMA: two columns a lane, the address clamped in bounds past N);
  // issued before the stages, it has landed when the loop's first wait for
  // stage 0 returns, and that iteration's barrier publishes it.
  if (wave == 0) lds_dma4(bias + min(n0 + 2 * lane, N - 2), lds_addr(sbias));
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < KT) issue(st, st);
  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int c0 = 16 * ((2 * g) ^ (r16 >> 1)), c1 = 16 * ((2 * g + 1) ^ (r16 >> 1));
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + S - 2 < KT) wait_vmcnt<(S - 2) * PER_WAVE>();
    else wait_vmcnt<0>();
    barrier_lds();  // every wave's loads for stage kt landed; stage kt - 1 fully consumed
    if (kt + S - 1 < KT) issue(kt + S - 1, (kt + S - 1) % S);
    const uint8_t* st = smem + (kt % S) * C::STAGE + frag;
    u32x4 a0[C::WI], a1[C::WI];
#pragma unroll
    for (int i = 0; i < C::WI; ++i) {
      const uint8_t* p = st + 2 * (wm * C::WI + i) * 1024;
      a0[i] = *reinterpret_cast<const u32x4*>(p + c0);
      a1[i] = *reinterpret_cast<const u32x4*>(p + c1);
    }
#pragma unroll
    for (int j = 0; j < C::WJ; ++j) {
      const uint8_t* p = st + (2 * C::RA + 2 * (wn * C::WJ + j)) * 1024;
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(p + c0);
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(p + c1);
#pragma unroll
      for (int i = 0; i < C::WI; ++i) acc[i][j] = mfma_bf16(b1, a1[i], mfma_bf16(b0, a0[i], acc[i][j]));
    }
  }

  // The weight fragment is the MFMA's first operand, so lane (r16, g) of tile
  // (i, j) holds row m0 + wm BM/2 + 16 i + r16, columns n0 + wn BN/2 + 16 j + 4 g .. + 3.
#pragma unroll
  for (int i = 0; i < C::WI; ++i) {
    const int m = m0 + wm * (BM / 2) + 16 * i + r16;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < C::WJ; ++j) {
      const int n = n0 + wn * (BN / 2) + 16 * j + 4 * g;
      if (n >= N) continue;  // N % 4 == 0: a 4-column group is all in or all out
      const u32x2 bb = *reinterpret_cast<const u32x2*>(sbias + n - n0);
      float v[4] = {bf16_to_f32(bb.x & 0xFFFFu), bf16_to_f32(bb.x >> 16), bf16_to_f32(bb.y & 0xFFFFu),
                    bf16_to_f32(bb.y >> 16)};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = round_bf16(acc[i][j][r] + v[r]);
        if constexpr (ACT == kGeluTanh) t = round_bf16(gelu_tanh(t));
        if constexpr (ACT == kGeluErf) t = round_bf16(gelu_erf(t));
        v[r] = t;
      }
      if constexpr (RESID) {
        const u32x2 rr = *reinterpret_cast<const u32x2*>(resid + (int64_t)m * ldr + n);
        v[0] += bf16_to_f32(rr.x & 0xFFFFu);
        v[1] += bf16_to_f32(rr.x >> 16);
        v[2] += bf16_to_f32(rr.y & 0xFFFFu);
        v[3] += bf16_to_f32(rr.y >> 16);
      }
      *reinterpret_cast<u32x2*>(y + (int64_t)m * ldy + n) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
}

// ---------------------------------------------------------------- packed-weight bf16 GEMM
//
// The product and epilogue of gemm_bf16_kernel with the weight read from a
// setup-time copy in MFMA operand order (ff_pack_weight_bf16) straight into
// registers, so that only the activations go through LDS. A workgroup of 4
// waves owns BM rows x BN = 4 CW columns; wave w owns columns [w CW, (w + 1)
// CW) and all BM rows, so each weight fragment feeds BM / 16 MFMAs and each
// activation fragment read from LDS CW / 16. A step is 128 k (256 bytes of an
// activation row, halves h = 0, 1); its four MFMAs per (i, j), sub = 2 h + s,
// take k 128 kt + 64 h + 16 g + 8 s .. + 8 for lane (r, g): the k partition
// and order of gemm_bf16_kernel's two MFMAs per 64-k stage, so the
// accumulators and y are bit-identical to it.
//
// Activations: two LDS stages of BM rows x 256 bytes, written from registers
// loaded a step ahead (16-byte chunk c of row r at half c / 8, 1 KB block r / 8,
// row r % 8, slot (c % 8) ^ ((r % 16) / 2)). Weights: fragment (f, kt) is the 4
// KB at (kt N / 16 + f) 4096; its sub-block `sub` (1 KB) holds for lane 16 g + r
// the 16 bytes of row 16 f + r at k 128 kt + 64 (sub / 2) + 16 g + 8 (sub % 2).
// Each lane holds two steps of fragments in registers; fragment (j, sub) of
// step kt is reloaded with step kt + 2's right after its MFMAs issue.
constexpr int kBfStep = 128;  // k per step of the packed kernel

// PART (k split): workgroup (tile, split) runs k steps [split KT / S, (split
// + 1) KT / S) and stores its fp32 sums, row-major over the rows padded to
// whole tiles, at part[(split tiles_m BM + row) N + col] instead of y; the
// launch that follows adds the S partials in split order and applies the
// epilogue (bf16_split_reduce_kernel, or layer_norm_kernel<true>).
template <int BM, int CW, int ACT, bool RESID, bool PART = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_pk_kernel(
    const bf16_t* __restrict__ a, int64_t lda, const uint8_t* __restrict__ wp, const bf16_t* __restrict__ bias,
    bf16_t* y, int64_t ldy, const bf16_t* resid, int64_t ldr, int M, int N, int K, int tiles_m, int tiles_n,
    int splits = 1, float* __restrict__ part = nullptr) {
  constexpr int RA = BM / 16, TJ = CW / 16;
  constexpr int A_CHUNKS = BM * 16;  // 16-byte chunks of one stage
  constexpr int FULL = A_CHUNKS / kThreads, REM = A_CHUNKS % kThreads;
  constexpr int NA = FULL + (REM ? 1 : 0);
  constexpr int HALF = BM * 128, STAGE = 2 * HALF;
  static_assert(A_CHUNKS >= kThreads, "at least one full activation round");
  __shared__ __align__(1024) uint8_t smem[2 * STAGE];
  __shared__ __align__(16) float sbias[PART ? 1 : 4 * CW];  // the tile's bias columns, as fp32
  // The residual tile (RESID): wave w's BM x CW columns at sres + w BM CW,
  // row-major, copied in by 16-byte LDS DMA after the prologue's loads so that
  // the epilogue reads it from LDS. Needs 16-byte aligned rows (resid and ldr);
  // otherwise the epilogue reads it from global memory.
  constexpr bool RT = RESID && !PART;
  constexpr int RCH = CW / 8, RQ = BM * RCH / 64;  // chunks per slab row, DMAs per wave
  static_assert(BM * RCH % 64 == 0, "whole DMA instructions per slab");
  __shared__ __align__(16) bf16_t sres[RT ? BM * 4 * CW : 1];

  const int S = PART ? splits : 1;
  const int nblk = tiles_m * tiles_n * S;
  int logical = blockIdx.x;
  if (nblk % kXcds == 0) logical = (blockIdx.x % kXcds) * (nblk / kXcds) + blockIdx.x / kXcds;
  const int tm = logical % tiles_m, rest = logical / tiles_m;  // M fastest: an XCD's tiles share weight slabs
  const int split = rest % S, tn = rest / S;
  const int m0 = tm * BM, n0 = tn * 4 * CW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int KT = K / kBfStep;
  const int kt0 = split * KT / S, kt1 = (split + 1) * KT / S;  // S <= KT: every split has a step

  // Activations: chunk c = tid + 256 i is row c / 16, chunk c % 16 (a partial
  // last round is moved back over the last 256 chunks, writing the overlap
  // twice with the same bytes); rows past M are clamped (masked at the store).
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(a, (uint32_t)((int64_t)M * lda * 2));
  uint32_t voffA[NA];
  int dstA[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = i < FULL ? tid + kThreads * i : A_CHUNKS - kThreads + tid;
    const int row = c >> 4, ch = c & 15;
    voffA[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)(2 * lda) + 16 * ch;
    dstA[i] = (ch >> 3) * HALF + (row >> 3) * 1024 + 128 * (row & 7) + 16 * ((ch & 7) ^ ((row & 15) >> 1));
  }
  i32x4v ast[NA];
  auto loadA = [&](int kt) {
#pragma unroll
    for (int i = 0; i < NA; ++i) ast[i] = bload16(rA, voffA[i], (uint32_t)kt * 256u);
  };
  auto writeA = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) *reinterpret_cast<i32x4v*>(smem + buf * STAGE + dstA[i]) = ast[i];
  };

  const __amdgpu_buffer_rsrc_t rB = make_rsrc(wp, (uint32_t)((int64_t)N * K * 2));
  const uint32_t kstride = (uint32_t)N * 256u;  // bytes per step: N / 16 fragments of 4 KB
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t sB[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) sB[j] = (uint32_t)((n0 + wave_s * CW + 16 * j) / 16) * 4096u;
  const uint32_t voffB = 16u * (uint32_t)lane;
  i32x4v bq[2][TJ][4];
  auto loadB1 = [&](int kt, int slot, int j, int sub) {
    bq[slot][j][sub] = bload16(rB, voffB + 1024u * (uint32_t)sub, sB[j] + (uint32_t)kt * kstride);
  };
  auto loadB = [&](int kt, int slot) {
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) loadB1(kt, slot, j, sub);
  };

  f32x4 acc[RA][TJ];
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The bias is read ahead of the first step (its latency then passes under
  // the prologue's loads) and kept in LDS for the epilogue.
  uint32_t braw = 0;
  if constexpr (!PART)
    if (tid < 4 * CW) braw = bias[n0 + tid];
  loadA(kt0);
  loadB(kt0, 0);
  writeA(0);
  if constexpr (!PART)
    if (tid < 4 * CW) sbias[tid] = bf16_to_f32(braw);
  loadA(min(kt0 + 1, kt1 - 1));
  loadB(min(kt0 + 1, kt1 - 1), 1);
  const bool rdma = RT && ((uintptr_t)resid & 15) == 0 && (ldr & 7) == 0;
  if constexpr (RT) {
    if (rdma) {
      const uint32_t slab = lds_addr(sres) + (uint32_t)wave_s * (BM * CW * 2);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int c = 64 * q + lane, row = c / RCH, ch = c % RCH;
        lds_dma16(resid + (int64_t)min(m0 + row, M - 1) * ldr + n0 + wave * CW + 8 * ch, slab + 1024u * q);
      }
    }
  }

  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int cA[2] = {16 * ((2 * g) ^ (r16 >> 1)), 16 * ((2 * g + 1) ^ (r16 >> 1))};
  // A fragments of the current substep (af[sub & 1]); a step's first substep is
  // read at the start of the previous step's last substep (the first step's here).
  i32x4v af[2][RA];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RA; ++i) af[0][i] = *reinterpret_cast<const i32x4v*>(smem + frag + 2 * i * 1024 + cA[0]);
  for (int kb = kt0; kb < kt1; kb += 2) {
    static_for<0, 2>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      const int kt = kb + u;
      if (kt < kt1) {  // uniform: an odd step count ends on u = 0
        // Stage u was written during the previous step and made visible by its
        // barrier; stage u ^ 1, read in the previous step before that barrier,
        // is written here for step kt + 1. This step's one barrier comes before
        // its last substep, which reads step kt + 1's first substep into af[0].
        const int kta = min(kt + 2, kt1 - 1);
        writeA(u ^ 1);
        loadA(kta);
        const uint8_t* st = smem + u * STAGE + frag;
        static_for<0, 4>([&](auto S_) {
          constexpr int sub = decltype(S_)::value;
          if constexpr (sub < 3) {
#pragma unroll
            for (int i = 0; i < RA; ++i)
              af[(sub + 1) & 1][i] =
                  *reinterpret_cast<const i32x4v*>(st + ((sub + 1) >> 1) * HALF + 2 * i * 1024 + cA[(sub + 1) & 1]);
          } else {
            __syncthreads();  // every wave's writes of stage u ^ 1 are done
            const uint8_t* stn = smem + (u ^ 1) * STAGE + frag;
#pragma unroll
            for (int i = 0; i < RA; ++i) af[0][i] = *reinterpret_cast<const i32x4v*>(stn + 2 * i * 1024 + cA[0]);
          }
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            const u32x4 b = __builtin_bit_cast(u32x4, bq[u][j][sub]);
#pragma unroll
            for (int i = 0; i < RA; ++i) acc[i][j] = mfma_bf16(b, __builtin_bit_cast(u32x4, af[sub & 1][i]), acc[i][j]);
            loadB1(kta, u, j, sub);
          }
        });
      }
    });
  }

  // lane (r16, g) of fragment (i, j): row m0 + 16 i + r16, columns
  // n0 + wave CW + 16 j + 4 g .. + 3; the epilogue of gemm_bf16_kernel
  if constexpr (PART) {
    float* dst = part + ((int64_t)split * tiles_m * BM + m0 + r16) * N + n0 + wave * CW + 4 * g;
#pragma unroll
    for (int i = 0; i < RA; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) *reinterpret_cast<f32x4*>(dst + (int64_t)16 * i * N + 16 * j) = acc[i][j];
    return;
  }
  if constexpr (RT)
    if (rdma) {
      wait_vmcnt<0>();  // this wave's residual DMAs have landed (each wave reads only its own slab)
      asm volatile("" : : : "memory");
    }
#pragma unroll
  for (int i = 0; i < RA; ++i) {
    const int m = m0 + 16 * i + r16;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + wave * CW + 16 * j + 4 * g;
      const f32x4 bv = *reinterpret_cast<const f32x4*>(sbias + n - n0);
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = round_bf16(acc[i][j][r] + bv[r]);
        if constexpr (ACT == kGeluTanh) t = round_bf16(gelu_tanh(t));
        if constexpr (ACT == kGeluErf) t = round_bf16(gelu_erf(t));
        v[r] = t;
      }
      if constexpr (RESID) {
        const u32x2 rr = rdma ? *reinterpret_cast<const u32x2*>(sres + (wave * BM + 16 * i + r16) * CW + 16 * j + 4 * g)
                              : *reinterpret_cast<const u32x2*>(resid + (int64_t)m * ldr + n);
        v[0] += bf16_to_f32(rr.x & 0xFFFFu);
        v[1] += bf16_to_f32(rr.x >> 16);
        v[2] += bf16_to_f32(rr.y & 0xFFFFu);
        v[3] += bf16_to_f32(rr.y >> 16);
      }
      *reinterpret_cast<u32x2*>(y + (int64_t)m * ldy + n) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
}

// The epilogue of gemm_bf16_kernel on a k-split launch's S fp32 partial rows
// (added in split order): y = bf16(sum + bias), then the activation, then the
// residual add; one thread per 8 columns.
template <int ACT, bool RESID>
__global__ __launch_bounds__(kThreads) void bf16_split_reduce_kernel(const float* __restrict__ part, int splits,
                                                                     int64_t mp, const bf16_t* __restrict__ bias,
                                                                     bf16_t* y, int64_t ldy, const bf16_t* resid,
                                                                     int64_t ldr, int M, int N) {
  const int nc = N / 8;
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= (int64_t)M * nc) return;
  const int64_t m = e / nc;
  const int col = (int)(e % nc) * 8;
  float v[8];
  split_row8(part, splits, mp, N, m, col, bias, nullptr, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (ACT == kGeluTanh) v[i] = round_bf16(gelu_tanh(v[i]));
    if constexpr (ACT == kGeluErf) v[i] = round_bf16(gelu_erf(v[i]));
  }
  if constexpr (RESID) {
    float rv[8];
    unpack8(*reinterpret_cast<const u32x4*>(resid + m * ldr + col), rv);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_bf16(rv[i] + v[i]);
  }
  *reinterpret_cast<u32x4*>(y + m * ldy + col) = pack8(v);
}

// Weight copy in the packed kernel's operand order: one thread per 16-byte
// piece ((kt N/16 + f) 4 + sub) 64 + lane of the output.
__global__ __launch_bounds__(kThreads) void pack_bf16_kernel(const bf16_t* __restrict__ w, uint8_t* __restrict__ dst,
                                                             int64_t n, int64_t k) {
  const int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (i >= n * k / 8) return;
  const int lane = (int)(i & 63), sub = (int)((i >> 6) & 3);
  const int64_t rest = i >> 8, nf = n / 16;
  const int64_t f = rest % nf, kt = rest / nf;
  const int64_t row = 16 * f + (lane & 15);
  const int64_t kk = kBfStep * kt + 64 * (sub >> 1) + 16 * (lane >> 4) + 8 * (sub & 1);
  *reinterpret_cast<u32x4*>(dst + i * 16) = *reinterpret_cast<const u32x4*>(w + row * k + kk);
}

// ---------------------------------------------------------------- vision rotary
//
// y = bf16(x * cos + rotate_half(x) * sin) in fp32 for q and k of every
// (token, head), cos / sin (n, hd) fp32 (vision_rope, _legacy/search_kernels.py:111-134;
// apply_rotary_pos_emb_vision in transformers). Inputs have token stride
// x_ts and head stride x_hs; outputs y_ts / y_hs, with columns [hd, dpad) of
// each output head written as zeros. One thread per 4 columns of one
// (token, head) of q or of k; hd % 8 == 0 so the rotation partner (hd / 2 away)
// is a whole 4-column group.
__device__ __forceinline__ void vision_rope_block(
    int64_t blk, const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, int64_t x_ts, int64_t x_hs,
    const float* __restrict__ cos, const float* __restrict__ sin, bf16_t* __restrict__ yq, bf16_t* __restrict__ yk,
    int64_t y_ts, int64_t y_hs, int n, int heads, int hd, int dpad) {
  const int gpr = dpad / 4;  // 4-column groups per output head row
  const int64_t i = blk * kThreads + threadIdx.x;
  const int64_t per = (int64_t)n * heads * gpr;
  if (i >= 2 * per) return;
  const bool isk = i >= per;
  const int64_t r = isk ? i - per : i;
  const int c = (int)(r % gpr) * 4;
  const int64_t th = r / gpr;
  const int head = (int)(th % heads);
  const int64_t tok = th / heads;
  bf16_t* dst = (isk ? yk : yq) + tok * y_ts + head * y_hs + c;
  if (c >= hd) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{0u, 0u};
    return;
  }
  const bf16_t* xr = (isk ? k : q) + tok * x_ts + head * x_hs;
  const int half = hd / 2;
  const int pc = c < half ? c + half : c - half;
  const u32x2 xv = *reinterpret_cast<const u32x2*>(xr + c);
  const u32x2 pv = *reinterpret_cast<const u32x2*>(xr + pc);
  const float4 cv = *reinterpret_cast<const float4*>(cos + tok * hd + c);
  const float4 sv = *reinterpret_cast<const float4*>(sin + tok * hd + c);
  const float x4[4] = {bf16_to_f32(xv.x & 0xFFFFu), bf16_to_f32(xv.x >> 16), bf16_to_f32(xv.y & 0xFFFFu),
                       bf16_to_f32(xv.y >> 16)};
  float p4[4] = {bf16_to_f32(pv.x & 0xFFFFu), bf16_to_f32(pv.x >> 16), bf16_to_f32(pv.y & 0xFFFFu),
                 bf16_to_f32(pv.y >> 16)};
  if (c < half) {
#pragma unroll
    for (int e = 0; e < 4; ++e) p4[e] = -p4[e];
  }
  const float c4[4] = {cv.x, cv.y, cv.z, cv.w}, s4[4] = {sv.x, sv.y, sv.z, sv.w};
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = x4[e] * c4[e] + p4[e] * s4[e];
  *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
}

__global__ __launch_bounds__(kThreads) void vision_rope_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, int64_t x_ts, int64_t x_hs,
    const float* __restrict__ cos, const float* __restrict__ sin, bf16_t* __restrict__ yq, bf16_t* __restrict__ yk,
    int64_t y_ts, int64_t y_hs, int n, int heads, int hd, int dpad) {
  vision_rope_block(blockIdx.x, q, k, x_ts, x_hs, cos, sin, yq, yk, y_ts, y_hs, n, heads, hd, dpad);
}

// V^T with zero padding: v (token stride v_ts, head stride v_hs, hd columns)
// -> vt (heads, 128, t_pad), rows [hd, 128) and tokens [n, t_pad) zero. One
// workgroup per (head, 64 tokens): the 64 x hd block is staged in LDS as raw
// bf16 (17 KB, so that a launch that also runs other workgroups keeps eight
// workgroups per CU), then each thread writes 8 consecutive tokens of one d row.
constexpr int kVtPitch = 136;  // bf16 per staged token row (128 + 8: 8-byte aligned rows)
__device__ __forceinline__ void vision_vt_block(int blk, uint16_t (&tile)[64][kVtPitch], const bf16_t* __restrict__ v,
                                                int64_t v_ts, int64_t v_hs, bf16_t* __restrict__ vt, int n, int t_pad,
                                                int heads, int hd) {
  const int head = blk % heads, t0 = (blk / heads) * 64;
  for (int c = threadIdx.x; c < 64 * 32; c += kThreads) {
    const int tt = c / 32, d = (c % 32) * 4;
    const int tok = t0 + tt;
    u32x2 x{0u, 0u};
    if (tok < n && d < hd) x = *reinterpret_cast<const u32x2*>(v + (int64_t)tok * v_ts + (int64_t)head * v_hs + d);
    *reinterpret_cast<u32x2*>(&tile[tt][d]) = x;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 128 * 8; c += kThreads) {
    const int d = c % 128, tb = (c / 128) * 8;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = (uint32_t)tile[tb + 2 * e][d] | ((uint32_t)tile[tb + 2 * e + 1][d] << 16);
    *reinterpret_cast<u32x4*>(vt + ((int64_t)head * 128 + d) * t_pad + t0 + tb) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

__global__ __launch_bounds__(kThreads) void vision_vt_kernel(const bf16_t* __restrict__ v, int64_t v_ts,
                                                             int64_t v_hs, bf16_t* __restrict__ vt, int n, int t_pad,
                                                             int heads, int hd) {
  __shared__ __align__(16) uint16_t tile[64][kVtPitch];
  vision_vt_block(blockIdx.x, tile, v, v_ts, v_hs, vt, n, t_pad, heads, hd);
}

// The rotary of vision_rope_block for the packed qkv output, two 8-column
// groups (two 16-byte stores) per thread: thread -> (q or k, token, head,
// group pair c and c + 64 of the 128-column output row, c in 0, 8, .., 56);
// the partners (hd / 2 away, hd % 8 == 0 so each 4-column half of a group
// lies on one side of hd / 2) come as two 8-byte loads, cos / sin as two
// 16-byte loads each; both groups' loads are issued before either's
// arithmetic. The same two fp32 products and sum per element, rounded once.
__device__ __forceinline__ void vision_rope8_block(int64_t blk, const bf16_t* __restrict__ qkv, int64_t ts,
                                                   const float* __restrict__ cos, const float* __restrict__ sin,
                                                   bf16_t* __restrict__ yq, bf16_t* __restrict__ yk, int n,
                                                   int heads, int hd) {
  const int64_t i = blk * kThreads + threadIdx.x;
  const int64_t per = (int64_t)n * heads * 8;
  if (i >= 2 * per) return;
  const bool isk = i >= per;
  const int64_t r = isk ? i - per : i;
  const int64_t th = r >> 3;
  const int head = (int)(th % heads);
  const int64_t tok = th / heads;
  bf16_t* row = (isk ? yk : yq) + ((int64_t)head * n + tok) * 128;
  const bf16_t* xr = qkv + tok * ts + (int64_t)(isk ? heads + head : head) * hd;
  const int half = hd / 2;
  u32x4 xv[2];
  u32x2 pv[2][2];
  float4 cv[2][2], sv[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = (int)(r & 7) * 8 + 64 * u;
    if (c < hd) {
      xv[u] = *reinterpret_cast<const u32x4*>(xr + c);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int cc = c + 4 * h;
        pv[u][h] = *reinterpret_cast<const u32x2*>(xr + (cc < half ? cc + half : cc - half));
        cv[u][h] = *reinterpret_cast<const float4*>(cos + tok * hd + cc);
        sv[u][h] = *reinterpret_cast<const float4*>(sin + tok * hd + cc);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = (int)(r & 7) * 8 + 64 * u;
    if (c >= hd) {
      *reinterpret_cast<u32x4*>(row + c) = u32x4{0u, 0u, 0u, 0u};
      continue;
    }
    float x8[8], p8[8], c8[8], s8[8];
    unpack8(xv[u], x8);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool lo = c + 4 * h < half;
      const float pf[4] = {bf16_to_f32(pv[u][h].x & 0xFFFFu), bf16_to_f32(pv[u][h].x >> 16),
                           bf16_to_f32(pv[u][h].y & 0xFFFFu), bf16_to_f32(pv[u][h].y >> 16)};
#pragma unroll
      for (int e = 0; e < 4; ++e) p8[4 * h + e] = lo ? -pf[e] : pf[e];
      c8[4 * h] = cv[u][h].x; c8[4 * h + 1] = cv[u][h].y; c8[4 * h + 2] = cv[u][h].z; c8[4 * h + 3] = cv[u][h].w;
      s8[4 * h] = sv[u][h].x; s8[4 * h + 1] = sv[u][h].y; s8[4 * h + 2] = sv[u][h].z; s8[4 * h + 3] = sv[u][h].w;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = x8[e] * c8[e] + p8[e] * s8[e];
    *reinterpret_cast<u32x4*>(row + c) = pack8(o);
  }
}

// Both of the above for the packed qkv output (n, 3, heads, hd) in one launch:
// workgroups [0, nrope) rotate q and k into the zero-padded head-major layout
// (heads, n, 128), the rest write the padded V^T (heads, 128, t_pad).
__global__ __launch_bounds__(kThreads) void vision_qkv_kernel(const bf16_t* __restrict__ qkv,
                                                              const float* __restrict__ cos,
                                                              const float* __restrict__ sin, bf16_t* __restrict__ yq,
                                                              bf16_t* __restrict__ yk, bf16_t* __restrict__ vt, int n,
                                                              int t_pad, int heads, int hd, int nrope) {
  __shared__ __align__(16) uint16_t tile[64][kVtPitch];
  const int64_t ts = 3 * (int64_t)heads * hd;
  if ((int)blockIdx.x < nrope) {
    vision_rope8_block(blockIdx.x, qkv, ts, cos, sin, yq, yk, n, heads, hd);
  } else {
    vision_vt_block((int)blockIdx.x - nrope, tile, qkv + 2 * (int64_t)heads * hd, ts, hd, vt, n, t_pad, heads, hd);
  }
}

// Interpolated position embedding: out[p, :] = bf16(sum_t table[idx[p, t], :] *
// wt[p, t]) with the products and the sum in fp32, taps in order
// (fast_pos_embed_interpolate, transformers modeling_qwen3_vl.py:664-679).
// Indices are clamped to the table's rows. One thread per 8 channels of one
// patch.
__global__ __launch_bounds__(kThreads) void pos_interp_kernel(const bf16_t* __restrict__ table,
                                                              const int64_t* __restrict__ idx,
                                                              const float* __restrict__ wt, bf16_t* __restrict__ out,
                                                              int n, int taps, int hidden, int64_t rows) {
  const int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  const int cpr = hidden / 8;
  if (i >= (int64_t)n * cpr) return;
  const int64_t p = i / cpr;
  const int c = (int)(i % cpr) * 8;
  float acc[8];
  for (int t = 0; t < taps; ++t) {
    float e[8];
    const int64_t r = min(max(idx[p * taps + t], (int64_t)0), rows - 1);
    unpack8(*reinterpret_cast<const u32x4*>(table + r * hidden + c), e);
    const float wv = wt[p * taps + t];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = t == 0 ? e[q] * wv : acc[q] + e[q] * wv;
  }
  *reinterpret_cast<u32x4*>(out + p * hidden + c) = pack8(acc);
}

template <int BM, int BN, int S, int OCC>
int launch_gemm(const void* a, int64_t lda, const void* w, const void* bias, void* y, int64_t ldy, const void* resid,
                int64_t ldr, int64_t m, int64_t n, int64_t k, int act, hipStream_t st) {
  const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)((n + BN - 1) / BN);
  const dim3 grid((unsigned)(tiles_m * tiles_n)), block(kThreads);
#define FF_G(ACT, RES)                                                                                          \
  if (act == ACT && (resid != nullptr) == RES)                                                                  \
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, S, OCC, ACT, RES>), grid, block, 0, st, (const bf16_t*)a, lda, \
                       (const bf16_t*)w, (const bf16_t*)bias, (bf16_t*)y, ldy, (const bf16_t*)resid, ldr, (int)m, \
                       (int)n, (int)k, tiles_m, tiles_n);
  FF_G(kActNone, false) FF_G(kActNone, true) FF_G(kGeluTanh, false) FF_G(kGeluErf, false)
#undef FF_G
  return FF_OK;
}

// Tile of the packed kernel for an m x n GEMM: the first (BM, CW) of
// (128, 48), (64, 64), (64, 48), (64, 32) whose BN = 4 CW divides n and whose
// grid of 192 .. 256 workgroups runs in one round at one workgroup per CU; 0
// if none (the LDS-staged kernel then runs). Grids past one round lose to it:
// the tower's qkv (288 tiles of 128 x 192) took 43.7 us against 28.5, fc1
// (544 of 64 x 256) 69.2 against 51.0; one-round grids win: proj / fc2 (192
// of 64 x 192) 30.1 against 32.9 us, the merger's fc1 50.8 against 57.1 and
// fc2 (256 of 64 x 128) 33.4 against 37.2. (128, 64) would spill: two steps
// of its weight fragments, two sets of activation fragments and the staging
// registers exceed the 256 VGPRs.
int bf16pk_tile(int64_t m, int64_t n) {
  constexpr int cand[4][2] = {{128, 48}, {64, 64}, {64, 48}, {64, 32}};
  for (int c = 0; c < 4; ++c) {
    if (n % (4 * cand[c][1])) continue;
    const int64_t tiles = (m + cand[c][0] - 1) / cand[c][0] * (n / (4 * cand[c][1]));
    if (tiles >= 192 && tiles <= 256) return c + 1;
  }
  return 0;
}

template <int BM, int CW>
void launch_gemm_pk(const void* a, int64_t lda, const void* wp, const void* bias, void* y, int64_t ldy,
                    const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, int act, hipStream_t st) {
  const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)(n / (4 * CW));
  const dim3 grid((unsigned)(tiles_m * tiles_n)), block(kThreads);
#define FF_G(ACT, RES)                                                                                         \
  if (act == ACT && (resid != nullptr) == RES)                                                                 \
    hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, CW, ACT, RES>), grid, block, 0, st, (const bf16_t*)a, lda,     \
                       (const uint8_t*)wp, (const bf16_t*)bias, (bf16_t*)y, ldy, (const bf16_t*)resid, ldr,    \
                       (int)m, (int)n, (int)k, tiles_m, tiles_n);
  FF_G(kActNone, false) FF_G(kActNone, true) FF_G(kGeluTanh, false) FF_G(kGeluErf, false)
#undef FF_G
}

// k split of the packed GEMM for grids with no one-round tile (bf16pk_tile 0)
// whose unsplit fallback, 64 x 128 tiles, fills less than half the GPU (the
// tower at short patch counts, e.g. 400 patches: proj and fc2 have 63 such
// tiles, the mergers 72; its qkv, 189, runs unsplit: 13.9 us against 15.0 +
// 4.9 us split 2 ways): the (BM, CW) tile and split count S in {2, 3, 4, 8}
// whose grid of tiles x S workgroups lies in 192 .. 256 (one round at one per
// CU) with the least work per workgroup (k steps per split x BM x CW); s = 0
// when none. ff_set_tuning(FF_TUNE_BF16_PK_SPLIT, 1) turns splits off, 2 .. 8
// forces the split count.
struct Bf16Split {
  int bm = 0, cw = 0, s = 0;
};
Bf16Split bf16pk_split(int64_t m, int64_t n, int64_t k) {
  Bf16Split p;
  const int forced = ff_tuning(FF_TUNE_BF16_PK_SPLIT);
  if (forced == 1 || m <= 0 || k % kBfStep || bf16pk_tile(m, n)) return p;
  if (!forced && (m + 63) / 64 * ((n + 127) / 128) >= 128) return p;
  const int64_t kt = k / kBfStep;
  constexpr int cand[4][2] = {{64, 32}, {64, 48}, {64, 64}, {128, 48}};
  constexpr int spl[4] = {2, 3, 4, 8};
  int64_t best = 0;
  for (const auto& c : cand) {
    if (n % (4 * c[1])) continue;
    const int64_t t = (m + c[0] - 1) / c[0] * (n / (4 * c[1]));
    for (const int sp : spl) {
      if ((forced && sp != forced) || sp > kt || t * sp < 192 || t * sp > 256) continue;
      const int64_t cost = (kt + sp - 1) / sp * c[0] * c[1];
      if (p.s == 0 || cost < best) {
        p = Bf16Split{c[0], c[1], sp};
        best = cost;
      }
    }
  }
  return p;
}

int64_t bf16pk_split_bytes(const Bf16Split& p, int64_t m, int64_t n) {
  return p.s < 2 ? 0 : (m + p.bm - 1) / p.bm * p.bm * n * p.s * 4;
}

template <int BM, int CW>
void launch_gemm_pk_part(const void* a, int64_t lda, const void* wp, int64_t m, int64_t n, int64_t k, int splits,
                         void* part, hipStream_t st) {
  const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)(n / (4 * CW));
  hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, CW, kActNone, false, true>), dim3((unsigned)(tiles_m * tiles_n * splits)),
                     dim3(kThreads), 0, st, (const bf16_t*)a, lda, (const uint8_t*)wp, nullptr, nullptr, 0, nullptr, 0,
                     (int)m, (int)n, (int)k, tiles_m, tiles_n, splits, (float*)part);
}

// The split GEMM's partials for plan p (the packed kernel's conditions and the
// workspace already checked).
void launch_split_part(const Bf16Split& p, const void* a, int64_t lda, const void* wp, int64_t m, int64_t n, int64_t k,
                       void* part, hipStream_t st) {
  if (p.bm == 64 && p.cw == 32) launch_gemm_pk_part<64, 32>(a, lda, wp, m, n, k, p.s, part, st);
  else if (p.bm == 64 && p.cw == 48) launch_gemm_pk_part<64, 48>(a, lda, wp, m, n, k, p.s, part, st);
  else if (p.bm == 64 && p.cw == 64) launch_gemm_pk_part<64, 64>(a, lda, wp, m, n, k, p.s, part, st);
  else launch_gemm_pk_part<128, 48>(a, lda, wp, m, n, k, p.s, part, st);
}

// Whether a call can take the k split: the packed kernel's operand limits and
// the 16-byte accesses of the split epilogue.
bool bf16_split_ok(const void* a, int64_t lda, const void* w_packed, const void* bias, const void* y, int64_t ldy,
                   const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k) {
  return w_packed && a && bias && y && m > 0 && lda >= k && lda % 8 == 0 && ldy >= n && ldy % 8 == 0 &&
         (!resid || (ldr >= n && ldr % 8 == 0 && ff_aligned(resid, 16))) && ff_aligned(w_packed, 16) &&
         ff_aligned(a, 16) && ff_aligned(bias, 16) && ff_aligned(y, 16) && m * lda * 2 < (int64_t(1) << 31) &&
         n * k * 2 < (int64_t(1) << 31);
}

}  // namespace

extern "C" int ff_pack_pixels(const void* rgb, void* out, int64_t height, int64_t width, ff_stream_t stream) {
  FF_REQUIRE(rgb && out, "ff_pack_pixels: null pointer");
  FF_REQUIRE(height > 0 && width > 0 && height % 32 == 0 && width % 32 == 0,
             "ff_pack_pixels: height and width must be multiples of 32 (got %lld x %lld)", (long long)height,
             (long long)width);
  FF_REQUIRE(ff_aligned(out, 16), "ff_pack_pixels: alignment");
  const int64_t chunks = (height / 16) * (width / 16) * (kPatchElems / 8);
  hipLaunchKernelGGL(pack_pixels_kernel, dim3((unsigned)((chunks + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)rgb, (bf16_t*)out, (int)width, chunks);
  FF_LAUNCH_CHECK("ff_pack_pixels");
  return FF_OK;
}

extern "C" int ff_layer_norm(const void* x, int64_t x_rs, const void* w, const void* b, void* y, int64_t y_rs,
                             int64_t rows, int64_t h, float eps, ff_stream_t stream) {
  FF_REQUIRE(x && w && b && y, "ff_layer_norm: null pointer");
  FF_REQUIRE(rows >= 0 && h > 0 && h % 8 == 0 && h <= 8 * kThreads * kLnChunks && x_rs >= h && y_rs >= h &&
                 x_rs % 8 == 0 && y_rs % 8 == 0,
             "ff_layer_norm: bad sizes rows=%lld h=%lld", (long long)rows, (long long)h);
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(w, 16) && ff_aligned(b, 16) && ff_aligned(y, 16),
             "ff_layer_norm: alignment");
  if (rows == 0) return FF_OK;
  hipLaunchKernelGGL(layer_norm_kernel<false>, dim3((unsigned)rows), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)x, x_rs, (const bf16_t*)w, (const bf16_t*)b, (bf16_t*)y, y_rs, (int)h, eps);
  FF_LAUNCH_CHECK("ff_layer_norm");
  return FF_OK;
}

extern "C" int ff_gemm_bf16(const void* a, int64_t lda, const void* w, const void* bias, void* y, int64_t ldy,
                            const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, int act,
                            ff_stream_t stream) {
  FF_REQUIRE(a && w && bias && y, "ff_gemm_bf16: null pointer");
  FF_REQUIRE(m > 0 && n > 0 && n % 4 == 0 && k > 0 && k % 64 == 0 && lda >= k && ldy >= n && lda % 8 == 0 &&
                 ldy % 4 == 0 && (!resid || (ldr >= n && ldr % 4 == 0)) && m * lda < (int64_t(1) << 40),
             "ff_gemm_bf16: bad sizes m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  FF_REQUIRE(act == kActNone || act == kGeluTanh || act == kGeluErf, "ff_gemm_bf16: act %d unknown", act);
  FF_REQUIRE(!resid || act == kActNone, "ff_gemm_bf16: a residual add takes no activation");
  FF_REQUIRE(ff_aligned(a, 16) && ff_aligned(w, 16) && ff_aligned(bias, 8) && ff_aligned(y, 8) &&
                 (!resid || ff_aligned(resid, 8)),
             "ff_gemm_bf16: alignment");
  hipStream_t st = (hipStream_t)stream;
  const int64_t big = ((m + 127) / 128) * ((n + 127) / 128);
  // ff_set_tuning(FF_TUNE_GEMM_BF16_TILE, 1..3) forces 64x128 | 128x128 | 64x128 at three per CU.
  const int forced = ff_tuning(FF_TUNE_GEMM_BF16_TILE) - 1;
  // 128 x 128 tiles at two workgroups per CU when they fill at least three
  // quarters of the 512 slots, else 64 x 128 tiles (more workgroups for the
  // narrow projections). The GELU-tanh MLP input projection (the tower's fc1,
  // 2048 x 1152 -> 4352 at 2048 patches) runs 64 x 128 tiles at three per CU
  // instead: 42.7 us against 51.5 (128 x 128) and 50.3 (64 x 128, two per CU),
  // its VALU-heavy epilogue overlapping the other workgroups' main loops.
  const int tile = forced >= 0 ? forced : (big >= 384 ? (act == kGeluTanh ? 2 : 1) : 0);
  if (tile == 1)
    launch_gemm<128, 128, 2, 2>(a, lda, w, bias, y, ldy, resid, ldr, m, n, k, act, st);
  else if (tile == 2)
    launch_gemm<64, 128, 2, 3>(a, lda, w, bias, y, ldy, resid, ldr, m, n, k, act, st);
  else
    launch_gemm<64, 128, 3, 2>(a, lda, w, bias, y, ldy, resid, ldr, m, n, k, act, st);
  FF_LAUNCH_CHECK("ff_gemm_bf16");
  return FF_OK;
}

extern "C" int ff_pack_weight_bf16(const void* w, void* packed, int64_t n, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(w && packed, "ff_pack_weight_bf16: null pointer");
  FF_REQUIRE(n > 0 && k > 0 && n % 16 == 0 && k % kBfStep == 0, "ff_pack_weight_bf16: n %% 16, k %% 128 (n=%lld k=%lld)",
             (long long)n, (long long)k);
  FF_REQUIRE(ff_aligned(w, 16) && ff_aligned(packed, 16), "ff_pack_weight_bf16: alignment");
  const int64_t pieces = n * k / 8;
  hipLaunchKernelGGL(pack_bf16_kernel, dim3((unsigned)((pieces + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)w, (uint8_t*)packed, n, k);
  FF_LAUNCH_CHECK("ff_pack_weight_bf16");
  return FF_OK;
}

extern "C" int ff_gemm_bf16_pk(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias,
                               void* y, int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k,
                               int act, ff_stream_t stream) {
  const int tile = w_packed && k % kBfStep == 0 && ff_aligned(w_packed, 16) && ff_aligned(a, 16) &&
                           m * lda * 2 < (int64_t(1) << 31) && n * k * 2 < (int64_t(1) << 31)
                       ? bf16pk_tile(m, n)
                       : 0;
  if (tile == 0) return ff_gemm_bf16(a, lda, w, bias, y, ldy, resid, ldr, m, n, k, act, stream);
  FF_REQUIRE(a && w && bias && y, "ff_gemm_bf16_pk: null pointer");
  FF_REQUIRE(m > 0 && lda >= k && ldy >= n && lda % 8 == 0 && ldy % 4 == 0 && (!resid || (ldr >= n && ldr % 4 == 0)),
             "ff_gemm_bf16_pk: bad sizes m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  FF_REQUIRE(act == kActNone || act == kGeluTanh || act == kGeluErf, "ff_gemm_bf16_pk: act %d unknown", act);
  FF_REQUIRE(!resid || act == kActNone, "ff_gemm_bf16_pk: a residual add takes no activation");
  FF_REQUIRE(ff_aligned(bias, 8) && ff_aligned(y, 8) && (!resid || ff_aligned(resid, 8)), "ff_gemm_bf16_pk: alignment");
  hipStream_t st = (hipStream_t)stream;
  if (tile == 1)
    launch_gemm_pk<128, 48>(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k, act, st);
  else if (tile == 2)
    launch_gemm_pk<64, 64>(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k, act, st);
  else if (tile == 3)
    launch_gemm_pk<64, 48>(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k, act, st);
  else
    launch_gemm_pk<64, 32>(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k, act, st);
  FF_LAUNCH_CHECK("ff_gemm_bf16_pk");
  return FF_OK;
}

extern "C" int ff_gemm_bf16_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes) {
  FF_REQUIRE(bytes && m >= 0 && n >= 0 && k >= 0, "ff_gemm_bf16_pk_workspace: bad arguments");
  *bytes = bf16pk_split_bytes(bf16pk_split(m, n, k), m, n);
  return FF_OK;
}

extern "C" int ff_gemm_bf16_pk_ws(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias,
                                  void* y, int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k,
                                  int act, void* workspace, int64_t workspace_bytes, ff_stream_t stream) {
  const Bf16Split p = bf16_split_ok(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k) ? bf16pk_split(m, n, k)
                                                                                          : Bf16Split{};
  if (p.s < 2) return ff_gemm_bf16_pk(a, lda, w, w_packed, bias, y, ldy, resid, ldr, m, n, k, act, stream);
  FF_REQUIRE(act == kActNone || act == kGeluTanh || act == kGeluErf, "ff_gemm_bf16_pk_ws: act %d unknown", act);
  FF_REQUIRE(!resid || act == kActNone, "ff_gemm_bf16_pk_ws: a residual add takes no activation");
  const int64_t need = bf16pk_split_bytes(p, m, n);
  FF_REQUIRE(workspace && workspace_bytes >= need && ff_aligned(workspace, 16),
             "ff_gemm_bf16_pk_ws: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  hipStream_t st = (hipStream_t)stream;
  launch_split_part(p, a, lda, w_packed, m, n, k, workspace, st);
  const int64_t mp = (m + p.bm - 1) / p.bm * p.bm;
  const unsigned blocks = (unsigned)((m * (n / 8) + kThreads - 1) / kThreads);
#define FF_R(ACT, RES)                                                                                            \
  if (act == ACT && (resid != nullptr) == RES)                                                                    \
    hipLaunchKernelGGL((bf16_split_reduce_kernel<ACT, RES>), dim3(blocks), dim3(kThreads), 0, st,                \
                       (const float*)workspace, p.s, mp, (const bf16_t*)bias, (bf16_t*)y, ldy, (const bf16_t*)resid, \
                       ldr, (int)m, (int)n);
  FF_R(kActNone, false) FF_R(kActNone, true) FF_R(kGeluTanh, false) FF_R(kGeluErf, false)
#undef FF_R
  FF_LAUNCH_CHECK("ff_gemm_bf16_pk_ws");
  return FF_OK;
}

extern "C" int ff_gemm_bf16_pk_ln(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias,
                                  void* y, int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k,
                                  void* workspace, int64_t workspace_bytes, const void* ln_w, const void* ln_b,
                                  float eps, void* ln_out, int64_t ln_ld, ff_stream_t stream) {
  FF_REQUIRE(resid, "ff_gemm_bf16_pk_ln: the residual is required");
  FF_REQUIRE(!ln_w || (ln_b && ln_out && ln_ld >= n && ln_ld % 8 == 0 && n % 8 == 0 && n <= 8 * kThreads * kLnChunks &&
                       ff_aligned(ln_w, 16) && ff_aligned(ln_b, 16) && ff_aligned(ln_out, 16)),
             "ff_gemm_bf16_pk_ln: LayerNorm arguments (n %% 8, n <= %d, 16-byte alignment)", 8 * kThreads * kLnChunks);
  const Bf16Split p = bf16_split_ok(a, lda, w_packed, bias, y, ldy, resid, ldr, m, n, k) ? bf16pk_split(m, n, k)
                                                                                          : Bf16Split{};
  if (p.s < 2) {
    const int rc = ff_gemm_bf16_pk(a, lda, w, w_packed, bias, y, ldy, resid, ldr, m, n, k, kActNone, stream);
    if (rc != FF_OK || !ln_w) return rc;
    return ff_layer_norm(y, ldy, ln_w, ln_b, ln_out, ln_ld, m, n, eps, stream);
  }
  const int64_t need = bf16pk_split_bytes(p, m, n);
  FF_REQUIRE(workspace && workspace_bytes >= need && ff_aligned(workspace, 16),
             "ff_gemm_bf16_pk_ln: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  hipStream_t st = (hipStream_t)stream;
  launch_split_part(p, a, lda, w_packed, m, n, k, workspace, st);
  const int64_t mp = (m + p.bm - 1) / p.bm * p.bm;
  if (ln_w)
    hipLaunchKernelGGL(layer_norm_kernel<true>, dim3((unsigned)m), dim3(kThreads), 0, st, (const bf16_t*)y, ldy,
                       (const bf16_t*)ln_w, (const bf16_t*)ln_b, (bf16_t*)ln_out, ln_ld, (int)n, eps,
                       (const float*)workspace, p.s, mp, (const bf16_t*)bias, (const bf16_t*)resid, ldr, (bf16_t*)y,
                       ldy);
  else
    hipLaunchKernelGGL((bf16_split_reduce_kernel<kActNone, true>), dim3((unsigned)((m * (n / 8) + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, st, (const float*)workspace, p.s, mp, (const bf16_t*)bias, (bf16_t*)y, ldy,
                       (const bf16_t*)resid, ldr, (int)m, (int)n);
  FF_LAUNCH_CHECK("ff_gemm_bf16_pk_ln");
  return FF_OK;
}

extern "C" int ff_vision_rope(const void* q, const void* k, int64_t x_ts, int64_t x_hs, const float* cos,
                              const float* sin, void* yq, void* yk, int64_t y_ts, int64_t y_hs, int64_t n,
                              int64_t heads, int64_t hd, int64_t dpad, ff_stream_t stream) {
  FF_REQUIRE(q && k && cos && sin && yq && yk, "ff_vision_rope: null pointer");
  FF_REQUIRE(n > 0 && heads > 0 && hd > 0 && hd % 8 == 0 && dpad >= hd && dpad % 4 == 0 && x_ts % 4 == 0 &&
                 x_hs % 4 == 0 && y_ts % 4 == 0 && y_hs % 4 == 0,
             "ff_vision_rope: bad sizes n=%lld heads=%lld hd=%lld dpad=%lld", (long long)n, (long long)heads,
             (long long)hd, (long long)dpad);
  FF_REQUIRE(ff_aligned(q, 8) && ff_aligned(k, 8) && ff_aligned(cos, 16) && ff_aligned(sin, 16) &&
                 ff_aligned(yq, 8) && ff_aligned(yk, 8),
             "ff_vision_rope: alignment");
  const int64_t threads = 2 * n * heads * (dpad / 4);
  hipLaunchKernelGGL(vision_rope_kernel, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)q, (const bf16_t*)k, x_ts, x_hs, cos, sin, (bf16_t*)yq,
                     (bf16_t*)yk, y_ts, y_hs, (int)n, (int)heads, (int)hd, (int)dpad);
  FF_LAUNCH_CHECK("ff_vision_rope");
  return FF_OK;
}

extern "C" int ff_vision_vt(const void* v, int64_t v_ts, int64_t v_hs, void* vt, int64_t n, int64_t t_pad,
                            int64_t heads, int64_t hd, ff_stream_t stream) {
  FF_REQUIRE(v && vt, "ff_vision_vt: null pointer");
  FF_REQUIRE(n > 0 && t_pad >= n && t_pad % 64 == 0 && heads > 0 && hd > 0 && hd <= 128 && hd % 4 == 0 &&
                 v_ts % 4 == 0 && v_hs % 4 == 0,
             "ff_vision_vt: bad sizes");
  FF_REQUIRE(ff_aligned(v, 8) && ff_aligned(vt, 16), "ff_vision_vt: alignment");
  hipLaunchKernelGGL(vision_vt_kernel, dim3((unsigned)(heads * (t_pad / 64))), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)v, v_ts, v_hs, (bf16_t*)vt, (int)n, (int)t_pad, (int)heads,
                     (int)hd);
  FF_LAUNCH_CHECK("ff_vision_vt");
  return FF_OK;
}

extern "C" int ff_pos_interp(const void* table, const int64_t* idx, const float* wt, void* out, int64_t n,
                             int64_t taps, int64_t hidden, int64_t rows, ff_stream_t stream) {
  FF_REQUIRE(table && idx && wt && out, "ff_pos_interp: null pointer");
  FF_REQUIRE(n > 0 && taps > 0 && hidden > 0 && hidden % 8 == 0 && rows > 0, "ff_pos_interp: bad sizes");
  FF_REQUIRE(ff_aligned(table, 16) && ff_aligned(out, 16), "ff_pos_interp: alignment");
  const int64_t threads = n * (hidden / 8);
  hipLaunchKernelGGL(pos_interp_kernel, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)table, idx, wt, (bf16_t*)out, (int)n, (int)taps,
                     (int)hidden, rows);
  FF_LAUNCH_CHECK("ff_pos_interp");
  return FF_OK;
}

extern "C" int ff_vision_qkv(const void* qkv, const float* cos, const float* sin, void* yq, void* yk, void* vt,
                             int64_t n, int64_t t_pad, int64_t heads, int64_t hd, ff_stream_t stream) {
  FF_REQUIRE(qkv && cos && sin && yq && yk && vt, "ff_vision_qkv: null pointer");
  FF_REQUIRE(n > 0 && heads > 0 && hd > 0 && hd <= 128 && hd % 8 == 0 && t_pad >= n && t_pad % 64 == 0,
             "ff_vision_qkv: bad sizes n=%lld heads=%lld hd=%lld t_pad=%lld", (long long)n, (long long)heads,
             (long long)hd, (long long)t_pad);
  FF_REQUIRE(ff_aligned(qkv, 16) && ff_aligned(cos, 16) && ff_aligned(sin, 16) && ff_aligned(yq, 16) &&
                 ff_aligned(yk, 16) && ff_aligned(vt, 16),
             "ff_vision_qkv: alignment (16 bytes)");
  const int64_t rope_threads = 2 * n * heads * (128 / 16);
  const int nrope = (int)((rope_threads + kThreads - 1) / kThreads);
  const int nvt = (int)(heads * (t_pad / 64));
  hipLaunchKernelGGL(vision_qkv_kernel, dim3((unsigned)(nrope + nvt)), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)qkv, cos, sin, (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)vt, (int)n, (int)t_pad,
                     (int)heads, (int)hd, nrope);
  FF_LAUNCH_CHECK("ff_vision_qkv");
  return FF_OK;
}
