// FP8 (e4m3fn) GEMM for gfx950: y = bf16((sum_k qa[m,k] qw[n,k]) * sa * sw).
//
// Both operands are K-contiguous ("TN"): activations qa (M,K) and weights qw
// (N,K), as the reference stores FP8 weights (N,K) row-major. A workgroup of 4
// waves (2 x 2) owns a BM x BN tile; each wave owns (BM/2) x (BN/2) as 16 x 16
// tiles of v_mfma_f32_16x16x128_f8f6f4 with fp32 accumulators.
//
// K is consumed KS x 128 bytes per stage. Stages are filled with
// global_load_lds_dwordx4 (gfx950 direct-to-LDS loads: lane l's 16 bytes land at
// base + 16*l, no staging registers). Each load instruction covers 8 rows x 128
// bytes -- whole cache lines, which doubles the bytes per memory request over a
// 16-row pattern -- with the 16-byte chunk of row r stored at slot
// 8*(r%8) + (chunk ^ (r/2)) of its 1 KB block (r in 0..15 within a 16-row group;
// rows 0-7 in block 0, rows 8-15 in block 1). An MFMA operand for lane l
// (row l%16, g = l/16) is chunks 2g and 2g+1 of its row: the XOR places the 16
// rows a wave reads per ds_read_b128 pass in 16 distinct bank groups, and the
// operand is k in [32g, 32g+32), the same for A and B.
// S stages rotate through LDS with S-1 in flight; one barrier per stage.
//
// The accumulator of lane l holds D[4*(l/16) + r][l % 16]. The epilogue applies
// the scales, rounds to bf16 and stages the tile through LDS so global stores
// are 16-byte row chunks.
//
// Tiles are ordered XCD-aware: consecutive workgroups are dealt round-robin to
// the 8 XCDs, so the logical tile id gives each XCD a contiguous range of tiles
// walked M-fastest; tiles that share a weight slab then share an L2.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ff_common.h"
#include "ff_rope.h"

using namespace ff;

namespace {

constexpr int BK = 128;
constexpr int kThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  // scale operands 0 select the unscaled v_mfma_f32_16x16x128_f8f6f4; format 0 = e4m3.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Weight row of tile column r for the gate/up pairing: tile tn covers channels
// [64 tn, 64 tn + 64) of the gate rows [0, half) and of the up rows [half, 2 half).
__device__ __forceinline__ int weight_row_swiglu(int r, int tn, int half) {
  return r < 64 ? tn * 64 + r : half + tn * 64 + (r - 64);
}

template <int BM, int BN, int KS, int S>
struct Cfg {
  static constexpr int RA = BM / 16, RB = BN / 16;     // 16-row groups
  static constexpr int SUB = 2 * (RA + RB);            // 1 KB blocks per 128-byte k-substep
  static constexpr int BLOCKS = SUB * KS;              // 1 KB blocks per stage
  static constexpr int STAGE = BLOCKS * 1024;
  static constexpr int WI = RA / 2, WJ = RB / 2;       // MFMA tiles per wave (rows, cols)
  static constexpr int EPI_LD = BN + 8;                // bf16 row pitch of the epilogue tile
  static constexpr int SMEM = S * STAGE > BM * EPI_LD * 2 ? S * STAGE : BM * EPI_LD * 2;
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(RA % 2 == 0 && RB % 2 == 0, "tile must split over 2 x 2 waves");
  static_assert(BLOCKS % 4 == 0, "stage blocks must split over 4 waves");
};

// KS = 128-byte k-substeps per stage; S = LDS stages, S-1 in flight; OCC =
// workgroups per CU the register budget is sized for.
// EPI selects the epilogue: kPlain stores y (M, N); kSwiglu reads the weight as
// [gate (half rows); up (half rows)] and gives each workgroup BN/2 channels of
// both halves (gate in tile columns [0, BN/2), up in [BN/2, BN)), then stores
// y = bf16(bf16(silu(gate)) * up) (M, half) and the per-row max |y| of its
// channels in pmax[m * tiles_n + tile].
// kQkv: N = (hq + 2 hk) * 128 and BN = 128, so tile column block tn is one head
// of the packed QKV output: q/k heads get the per-head RMSNorm + rotary of
// qk_pair and are stored head-major (heads, M, 128); v heads are stored
// transposed, vt (hk, 128, t_pad), with zeros for tokens in [M, t_pad).
// kSwigluQ: kSwiglu whose output is the e4m3 code of h under a static
// multiplier, e4m3(clamp(h * qinv, +-448)) (y is then bytes, ldy in bytes),
// and no row maxima.
constexpr int kPlain = 0, kSwiglu = 1, kQkv = 2, kSwigluQ = 3;
constexpr bool is_swiglu(int epi) { return epi == kSwiglu || epi == kSwigluQ; }

struct QkvEpilogue {
  const bf16_t* qn;  // q_norm weight (128)
  const bf16_t* kn;  // k_norm weight (128)
  float eps_q, eps_k;
  const bf16_t* cos;  // (M, 128)
  const bf16_t* sin;
  bf16_t* yq;  // (hq, M, 128)
  bf16_t* yk;  // (hk, M, 128)
  bf16_t* vt;  // (hk, 128, t_pad)
  int hq, hk, t_pad;
};

template <int BM, int BN, int KS, int S, int OCC, int EPI>
__global__ __launch_bounds__(kThreads, OCC) void gemm_fp8_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, int sa_rows,
    const uint8_t* __restrict__ qw, const float* __restrict__ sw, int sw_cols,
    bf16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int tiles_m, int tiles_n, int half,
    float* __restrict__ pmax, QkvEpilogue qe, float qinv) {
  using C = Cfg<BM, BN, KS, S>;
  __shared__ __align__(16) uint8_t smem[C::SMEM];

  const int nblk = tiles_m * tiles_n;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical % tiles_m, tn = logical / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  // Source pointers of this lane for every block this wave loads (k offset 0).
  // Rows past M / N are clamped to the last row (in bounds; masked at the store).
  constexpr int PER_WAVE = C::BLOCKS / 4;
  const uint8_t* src[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int blk = wave + 4 * i;
    const int ks = blk / C::SUB, rem = blk % C::SUB, h = rem & 1;
    const int rr = 8 * h + (lane >> 3);             // row within the 16-row group
    const int ch = (lane & 7) ^ (rr >> 1);          // 16-byte chunk of the row
    if (rem < 2 * C::RA) {
      const int row = min(m0 + (rem >> 1) * 16 + rr, M - 1);
      src[i] = qa + (size_t)row * K + ks * 128 + 16 * ch;
    } else {
      const int r = ((rem - 2 * C::RA) >> 1) * 16 + rr;  // B row within the tile
      const int row = is_swiglu(EPI) ? weight_row_swiglu(r, tn, half) : min(n0 + r, N - 1);
      src[i] = qw + (size_t)row * K + ks * 128 + 16 * ch;
    }
  }
  const uint32_t lds0 = lds_addr(smem) + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024;
  auto issue = [&](int k0, int buf) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) lds_dma16(src[i] + k0, lds0 + buf * C::STAGE + 4 * i * 1024);
  };

  f32x4 acc[C::WI][C::WJ];
#pragma unroll
  for (int i = 0; i < C::WI; ++i)
#pragma unroll
    for (int j = 0; j < C::WJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / (BK * KS);
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < KT) issue(st * BK * KS, st);
  // fragment read offsets (within a k-substep): rows r16 of block pair blk, chunks 2g, 2g+1
  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int c0 = 16 * ((2 * g) ^ (r16 >> 1)), c1 = 16 * ((2 * g + 1) ^ (r16 >> 1));
  for (int kt = 0; kt < KT; ++kt) {
    // stage kt has landed once at most (stages issued after it) x PER_WAVE loads remain
    if (kt + S - 2 < KT) wait_vmcnt<(S - 2) * PER_WAVE>();
    else wait_vmcnt<0>();
    barrier_lds();  // every wave's loads for stage kt landed; stage kt-1 fully consumed
    if (kt + S - 1 < KT) issue((kt + S - 1) * BK * KS, (kt + S - 1) % S);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint8_t* st = smem + (kt % S) * C::STAGE + ks * C::SUB * 1024 + frag;
      i32x8 af[C::WI];
#pragma unroll
      for (int i = 0; i < C::WI; ++i) {
        const uint8_t* p = st + 2 * (wm * C::WI + i) * 1024;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + c0);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + c1);
        af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int j = 0; j < C::WJ; ++j) {
        const uint8_t* p = st + (2 * C::RA + 2 * (wn * C::WJ + j)) * 1024;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + c0);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + c1);
        const i32x8 bfr = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
        for (int i = 0; i < C::WI; ++i) acc[i][j] = mfma_fp8(af[i], bfr, acc[i][j]);
      }
    }
  }
  __syncthreads();  // all stages consumed before the epilogue reuses the LDS

  // QKV epilogue of a q/k head: issue its global loads (norm weights, the cos /
  // sin rows of this thread's tokens) now, so they land while the tile is staged.
  constexpr int kRopeRows = BM / (kThreads / 16);
  float rope_w[8];
  u32x4 rope_c[kRopeRows], rope_s[kRopeRows];
  if constexpr (EPI == kQkv) {
    if (tn < qe.hq + qe.hk) {
      const int j = tid & 15, grp = tid >> 4;
      unpack8(*reinterpret_cast<const u32x4*>((tn < qe.hq ? qe.qn : qe.kn) + 8 * j), rope_w);
#pragma unroll
      for (int p = 0; p < kRopeRows; ++p) {
        const int mm = min(m0 + grp + p * (kThreads / 16), M - 1);
        rope_c[p] = *reinterpret_cast<const u32x4*>(qe.cos + (size_t)mm * kHeadDim + 8 * j);
        rope_s[p] = *reinterpret_cast<const u32x4*>(qe.sin + (size_t)mm * kHeadDim + 8 * j);
      }
    }
  }

  // epilogue: y = bf16((acc * sa) * sw), staged through LDS as a row-major tile.
  bf16_t* tile = reinterpret_cast<bf16_t*>(smem);
#pragma unroll
  for (int j = 0; j < C::WJ; ++j) {
    const int cl = wn * (BN / 2) + j * 16 + r16;
    const int n = is_swiglu(EPI) ? weight_row_swiglu(cl, tn, half) : min(n0 + cl, N - 1);
    const float swv = sw[sw_cols ? n : 0];
#pragma unroll
    for (int i = 0; i < C::WI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rl = wm * (BM / 2) + i * 16 + 4 * g + r;
        const int m = min(m0 + rl, M - 1);
        const float sav = sa[sa_rows ? m : 0];
        tile[rl * C::EPI_LD + cl] = (bf16_t)f32_to_bf16((acc[i][j][r] * sav) * swv);
      }
  }
  __syncthreads();
  if constexpr (is_swiglu(EPI)) {
    // 8 channels per thread; the 8 threads of one row are 8 consecutive lanes.
    constexpr int CH = BN / 2, CPR = CH / 8;
    static_assert(CPR == 8, "row max reduces over 8 lanes");
    const int g0 = tn * CH;
#pragma unroll
    for (int c = tid; c < BM * CPR; c += kThreads) {
      const int rl = c / CPR, cc = (c % CPR) * 8;
      float gv[8], uv[8], hv[8];
      unpack8(*reinterpret_cast<const u32x4*>(tile + rl * C::EPI_LD + cc), gv);
      unpack8(*reinterpret_cast<const u32x4*>(tile + rl * C::EPI_LD + CH + cc), uv);
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hv[e] = round_bf16(round_bf16(silu(gv[e])) * uv[e]);
        mx = fmaxf(mx, fabsf(hv[e]));
      }
      mx = fmaxf(mx, dpp<kDppXor1>(mx));
      mx = fmaxf(mx, dpp<kDppXor2>(mx));
      mx = fmaxf(mx, dpp<kDppHalfMirror>(mx));
      const int m = m0 + rl;
      if constexpr (EPI == kSwigluQ) {
        if (m < M)
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(y) + (size_t)m * ldy + g0 + cc) =
              quant8_static(hv, qinv);
      } else if (m < M) {
        *reinterpret_cast<u32x4*>(y + (size_t)m * ldy + g0 + cc) = pack8(hv);
        if (cc == 0) pmax[(size_t)m * tiles_n + tn] = mx;
      }
    }
    return;
  }
  if constexpr (EPI == kQkv) {
    static_assert(BN == kHeadDim, "one head per tile column block");
    const int head = tn;
    if (head < qe.hq + qe.hk) {
      // q or k head: one 16-lane group per token row, as the qkv_post kernel does
      const bool isq = head < qe.hq;
      const int hh = isq ? head : head - qe.hq;
      const float eps = isq ? qe.eps_q : qe.eps_k;
      bf16_t* dst = (isq ? qe.yq : qe.yk) + (size_t)hh * M * kHeadDim;
      const int grp = tid >> 4, j = tid & 15;
#pragma unroll
      for (int p = 0; p < kRopeRows; ++p) {
        const int rl = grp + p * (kThreads / 16);
        const int m = m0 + rl;
        const bool valid = m < M;
        const int mm = valid ? m : M - 1;
        rope_row_pre(tile + rl * C::EPI_LD, rope_w, eps, rope_c[p], rope_s[p], dst + (size_t)mm * kHeadDim, j, valid);
      }
    } else {
      // v head: 8 consecutive tokens of one d row per thread (16-byte stores);
      // consecutive lanes take consecutive d, so each LDS read of a wave is one
      // 128-byte row segment (no bank conflicts)
      const int hv = head - qe.hq - qe.hk;
      for (int c = tid; c < kHeadDim * (BM / 8); c += kThreads) {
        const int d = c % kHeadDim, t0 = (c / kHeadDim) * 8;
        const int tok = m0 + t0;
        if (tok >= qe.t_pad) continue;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (tok + e < M) ? bf16_to_f32(tile[(t0 + e) * C::EPI_LD + d]) : 0.f;
        *reinterpret_cast<u32x4*>(qe.vt + ((size_t)hv * kHeadDim + d) * qe.t_pad + tok) = pack8(f);
      }
    }
    return;
  }
  constexpr int CHUNKS = BM * BN / 8;
#pragma unroll
  for (int c = tid; c < CHUNKS; c += kThreads) {
    const int rl = c / (BN / 8), cl = (c % (BN / 8)) * 8;
    const int m = m0 + rl, n = n0 + cl;
    if (m < M && n < N)
      *reinterpret_cast<u32x4*>(y + (size_t)m * ldy + n) = *reinterpret_cast<const u32x4*>(tile + rl * C::EPI_LD + cl);
  }
}

// ---------------------------------------------------------------- GEMV (m <= 4)
//
// For a handful of rows (the pick-only tail runs its linears on one token) the
// tile kernel leaves most of the machine idle; these kernels stream each weight
// row once instead: one wave per output row (or per gate/up channel pair),
// every lane 16-byte chunks of it, e4m3 decoded with v_cvt_pk_f32_fp8 and the
// exact products summed with fp32 FMAs, then a wave reduction. The sum is more
// accurate than the matrix-unit path (it does not truncate 32-product blocks).

constexpr int kGemvMaxM = 4;

__device__ __forceinline__ void decode_e4m3x16(const u32x4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], true);
    f[4 * q + 0] = lo[0];
    f[4 * q + 1] = lo[1];
    f[4 * q + 2] = hi[0];
    f[4 * q + 3] = hi[1];
  }
}

// acc[m] += sum over this lane's chunks of a[m, k] * w[row, k] for NR weight rows;
// chunks c = lane + 64 j, B chunks per lane in flight per row.
template <int MM, int NR, int B>
__device__ __forceinline__ void gemv_rows(const uint8_t* __restrict__ qa, const uint8_t* const* wrow, int K,
                                          int lane, float (&acc)[NR][MM]) {
  const int nchunk = K / 16;
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
  for (int c0 = lane; c0 < nchunk; c0 += 64 * B) {
    u32x4 wv[NR][B];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int c = c0 + 64 * u;
        wv[r][u] = c < nchunk ? *reinterpret_cast<const u32x4*>(wrow[r] + (size_t)c * 16) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int c = c0 + 64 * u;
      if (c >= nchunk) break;
      float af[MM][16];
#pragma unroll
      for (int m = 0; m < MM; ++m) decode_e4m3x16(*reinterpret_cast<const u32x4*>(qa + (size_t)m * K + (size_t)c * 16), af[m]);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float wf[16];
        decode_e4m3x16(wv[r][u], wf);
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[r][m] = __builtin_fmaf(af[m][e], wf[e], acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = wave_sum(acc[r][m]);
}

// y[m, n] = bf16((dot * sa) * sw): one wave per output row n, 4 rows per workgroup.
template <int MM>
__global__ __launch_bounds__(256) void gemv_fp8_kernel(const uint8_t* __restrict__ qa, const float* __restrict__ sa,
                                                       int sa_rows, const uint8_t* __restrict__ qw,
                                                       const float* __restrict__ sw, int sw_cols,
                                                       bf16_t* __restrict__ y, int64_t ldy, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // wave-uniform
  const uint8_t* wrow[1] = {qw + (size_t)n * K};
  float acc[1][MM];
  gemv_rows<MM, 1, 8>(qa, wrow, K, lane, acc);
  if (lane == 0) {
    const float swv = sw[sw_cols ? n : 0];
#pragma unroll
    for (int m = 0; m < MM; ++m) y[(size_t)m * ldy + n] = (bf16_t)f32_to_bf16((acc[0][m] * sa[sa_rows ? m : 0]) * swv);
  }
}

// SwiGLU GEMV: workgroup = 16 waves = 64 channels, 4 per wave; gate row c and
// up row half + c per channel; h = bf16(bf16(silu(g)) * u); pmax[m, block] = the
// block's max |h| (the 64-channel blocks of ff_gemm_fp8_swiglu). With hq, h is
// written as e4m3(clamp(h * qinv, +-448)) instead (static quantisation of the
// next GEMM's input) and no maxima. sa / sw per row / column or one value.
template <int MM>
__global__ __launch_bounds__(1024) void gemv_fp8_swiglu_kernel(const uint8_t* __restrict__ qa,
                                                              const float* __restrict__ sa, int sa_rows,
                                                              const uint8_t* __restrict__ qw,
                                                              const float* __restrict__ sw, int sw_cols,
                                                              bf16_t* __restrict__ h, int64_t ldh,
                                                              float* __restrict__ pmax, uint8_t* __restrict__ hq,
                                                              float qinv, int half, int K) {
  __shared__ float red[16][kGemvMaxM];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = (int)blockIdx.x * 64 + wave * 4;
  const uint8_t* wrow[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    wrow[2 * j] = qw + (size_t)(c0 + j) * K;
    wrow[2 * j + 1] = qw + (size_t)(half + c0 + j) * K;
  }
  float acc[8][MM];
  gemv_rows<MM, 8, 2>(qa, wrow, K, lane, acc);
  float mx[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    mx[m] = 0.f;
    const float sav = sa[sa_rows ? m : 0];
    float hv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g = round_bf16((acc[2 * j][m] * sav) * sw[sw_cols ? c0 + j : 0]);
      const float u = round_bf16((acc[2 * j + 1][m] * sav) * sw[sw_cols ? half + c0 + j : 0]);
      hv[j] = round_bf16(round_bf16(silu(g)) * u);
      mx[m] = fmaxf(mx[m], fabsf(hv[j]));
      if (lane == 0 && !hq) h[(size_t)m * ldh + c0 + j] = (bf16_t)f32_to_bf16(hv[j]);
    }
    if (lane == 0 && hq)
      *reinterpret_cast<uint32_t*>(hq + (size_t)m * ldh + c0) = quant4_static(hv[0], hv[1], hv[2], hv[3], qinv);
    if (lane == 0) red[wave][m] = mx[m];
  }
  if (hq) return;
  __syncthreads();
  if (threadIdx.x < MM) {
    float v = 0.f;
    for (int w = 0; w < 16; ++w) v = fmaxf(v, red[w][threadIdx.x]);
    pmax[(size_t)threadIdx.x * (half / 64) + blockIdx.x] = v;
  }
}

int launch_gemv(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw, int sw_cols,
                void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, hipStream_t s) {
  const dim3 grid((unsigned)((n + 3) / 4)), block(256);
#define FF_GEMV(MM)                                                                                       \
  case MM:                                                                                                \
    hipLaunchKernelGGL(gemv_fp8_kernel<MM>, grid, block, 0, s, (const uint8_t*)qa, sa, sa_rows,            \
                       (const uint8_t*)qw, sw, sw_cols, (bf16_t*)y, ldy, (int)n, (int)k);                  \
    break;
  switch (m) { FF_GEMV(1) FF_GEMV(2) FF_GEMV(3) FF_GEMV(4) }
#undef FF_GEMV
  return FF_OK;
}

int launch_gemv_swiglu(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw, int sw_cols,
                       void* h, int64_t ldh, float* pmax, uint8_t* hq, float qinv, int64_t m, int64_t i, int64_t k,
                       hipStream_t s) {
  const dim3 grid((unsigned)(i / 64)), block(1024);
#define FF_GEMVS(MM)                                                                                      \
  case MM:                                                                                                \
    hipLaunchKernelGGL(gemv_fp8_swiglu_kernel<MM>, grid, block, 0, s, (const uint8_t*)qa, sa, sa_rows,     \
                       (const uint8_t*)qw, sw, sw_cols, (bf16_t*)h, ldh, pmax, hq, qinv, (int)i, (int)k);  \
    break;
  switch (m) { FF_GEMVS(1) FF_GEMVS(2) FF_GEMVS(3) FF_GEMVS(4) }
#undef FF_GEMVS
  return FF_OK;
}

template <int BM, int BN, int KS, int S, int OCC, int EPI = kPlain>
int launch(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw, int sw_cols,
           void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, hipStream_t s, float* pmax = nullptr,
           QkvEpilogue qe = QkvEpilogue{}, float qinv = 0.f) {
  static_assert(OCC * Cfg<BM, BN, KS, S>::SMEM <= 160 * 1024, "LDS budget for the occupancy");
  // kSwiglu / kSwigluQ: n = 2 * half weight rows, BN/2 channels of each half per tile
  const int tiles_m = (int)((m + BM - 1) / BM);
  const int tiles_n = is_swiglu(EPI) ? (int)(n / BN) : (int)((n + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_fp8_kernel<BM, BN, KS, S, OCC, EPI>), dim3(tiles_m * tiles_n), dim3(kThreads), 0, s,
                     (const uint8_t*)qa, sa, sa_rows, (const uint8_t*)qw, sw, sw_cols, (bf16_t*)y, ldy, (int)m,
                     (int)n, (int)k, tiles_m, tiles_n, (int)(n / 2), pmax, qe, qinv);
  return FF_OK;
}

// Tile choice, measured at M = 576 with the weights streamed from HBM as in the
// step (each launch on a different weight matrix): 128 x 128 tiles with two
// stages and two workgroups per CU when there are at least two such tiles per
// CU; 128 x 128 tiles with four stages (three in flight), one workgroup per CU,
// when the tiles about fill the CUs once (the 8B QKV: 30.4 us in the step
// against 30.9 us for 64 x 128 tiles; with the weights resident in the last-level
// cache, as in a loop over a few weight copies, 64 x 128 looks 3 us faster);
// otherwise 64 x 128 tiles (three stages, two per CU), which double the
// workgroups at the price of more operand traffic.
enum Tile { k64x128, k128x128, k128x128Deep, k128x256 };

Tile pick_tile(int64_t m, int64_t n) {
  const int64_t tiles_128 = ((m + 127) / 128) * ((n + 127) / 128);
  if (tiles_128 >= 2 * 256) return k128x128;
  if (tiles_128 >= 192 && tiles_128 <= 256) return k128x128Deep;
  return k64x128;
}

// ff_set_tuning(FF_TUNE_GEMM_FP8_TILE, 1..4) forces a tile (measurement
// sweeps); 0 = the choice above.
int forced_tile() {
  switch (ff_tuning(FF_TUNE_GEMM_FP8_TILE)) {
    case 1: return k64x128;
    case 2: return k128x128;
    case 3: return k128x128Deep;
    case 4: return k128x256;
    default: return -1;
  }
}

}  // namespace

extern "C" int ff_gemm_fp8(const void* qa, const float* sa, int sa_rows, const void* qw,
                           const float* sw, int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n,
                           int64_t k, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && qw && sw && y, "ff_gemm_fp8: null pointer");
  FF_REQUIRE(m >= 0 && n > 0 && k > 0 && k % BK == 0, "ff_gemm_fp8: k=%lld must be a multiple of %d",
             (long long)k, BK);
  FF_REQUIRE(n % 8 == 0 && ldy >= n && ldy % 8 == 0 && m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
             "ff_gemm_fp8: bad sizes (n and ldy must be multiples of 8)");
  FF_REQUIRE(ff_aligned(qa, 16) && ff_aligned(qw, 16) && ff_aligned(y, 16),
             "ff_gemm_fp8: operands must be 16-byte aligned");
  if (m == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (m <= kGemvMaxM) {
    launch_gemv(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, s);
    FF_LAUNCH_CHECK("ff_gemm_fp8");
    return FF_OK;
  }
  const int forced = forced_tile();
  const int tile = forced >= 0 ? forced : pick_tile(m, n);
  if (tile == k128x256) launch<128, 256, 1, 3, 1>(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, s);
  else if (tile == k128x128) launch<128, 128, 1, 2, 2>(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, s);
  else if (tile == k128x128Deep) launch<128, 128, 1, 4, 1>(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, s);
  else launch<64, 128, 1, 3, 2>(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, s);
  FF_LAUNCH_CHECK("ff_gemm_fp8");
  return FF_OK;
}

extern "C" int ff_gemm_fp8_swiglu(const void* qa, const float* sa, const void* qw, const float* sw, void* h,
                                  int64_t ldh, float* pmax, int64_t m, int64_t i, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && qw && sw && h && pmax, "ff_gemm_fp8_swiglu: null pointer");
  FF_REQUIRE(m >= 0 && i > 0 && i % 64 == 0 && k > 0 && k % BK == 0 && ldh >= i && ldh % 8 == 0 &&
                 m < (1 << 30) && i < (1 << 29) && k < (1 << 30),
             "ff_gemm_fp8_swiglu: bad sizes (i %% 64, k %% 128, ldh %% 8)");
  FF_REQUIRE(ff_aligned(qa, 16) && ff_aligned(qw, 16) && ff_aligned(h, 16),
             "ff_gemm_fp8_swiglu: operands must be 16-byte aligned");
  if (m == 0) return FF_OK;
  if (m <= kGemvMaxM)
    launch_gemv_swiglu(qa, sa, 1, qw, sw, 1, h, ldh, pmax, nullptr, 0.f, m, i, k, (hipStream_t)stream);
  else
    launch<128, 128, 1, 2, 2, kSwiglu>(qa, sa, 1, qw, sw, 1, h, ldh, m, 2 * i, k, (hipStream_t)stream, pmax);
  FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu");
  return FF_OK;
}

namespace ff {

// Gate/up GEMM with the SwiGLU epilogue writing e4m3(clamp(h * inv, +-448)),
// per-tensor scales sa[0], sw[0]: the GEMV kernel for m <= 4 rows, else the
// row-major tile (the packed file's fallback for shapes its tile does not take).
int gemm_swiglu_static_rowmajor(const void* qa, const float* sa, const void* qw, const float* sw, void* hq,
                                int64_t ldh, float inv, int64_t m, int64_t i, int64_t k, hipStream_t s) {
  if (m == 0) return FF_OK;
  if (m <= kGemvMaxM)
    launch_gemv_swiglu(qa, sa, 0, qw, sw, 0, nullptr, ldh, nullptr, (uint8_t*)hq, inv, m, i, k, s);
  else
    launch<128, 128, 1, 2, 2, kSwigluQ>(qa, sa, 0, qw, sw, 0, hq, ldh, m, 2 * i, k, s, nullptr, QkvEpilogue{}, inv);
  FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu_static");
  return FF_OK;
}

}  // namespace ff

extern "C" int ff_gemm_fp8_qkv(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw,
                               int sw_cols, int64_t m, int64_t k, int64_t hq, int64_t hk, const void* q_norm,
                               const void* k_norm, float eps_q, float eps_k, const void* cos, const void* sin, void* yq,
                               void* yk, void* vt, int64_t t_pad, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && qw && sw && q_norm && k_norm && cos && sin && yq && yk && vt,
             "ff_gemm_fp8_qkv: null pointer");
  FF_REQUIRE(m > 0 && k > 0 && k % BK == 0 && hq > 0 && hk > 0 && hq % hk == 0 && t_pad >= m && t_pad % 64 == 0 &&
                 m < (1 << 30) && k < (1 << 30) && (hq + 2 * hk) * kHeadDim < (1 << 30),
             "ff_gemm_fp8_qkv: bad sizes m=%lld k=%lld hq=%lld hk=%lld t_pad=%lld", (long long)m, (long long)k,
             (long long)hq, (long long)hk, (long long)t_pad);
  FF_REQUIRE(ff_aligned(qa, 16) && ff_aligned(qw, 16) && ff_aligned(cos, 16) && ff_aligned(sin, 16) &&
                 ff_aligned(q_norm, 16) && ff_aligned(k_norm, 16) && ff_aligned(yq, 16) && ff_aligned(yk, 16) &&
                 ff_aligned(vt, 16),
             "ff_gemm_fp8_qkv: operands must be 16-byte aligned");
  const int64_t n = (hq + 2 * hk) * kHeadDim;
  QkvEpilogue qe{(const bf16_t*)q_norm, (const bf16_t*)k_norm, eps_q, eps_k, (const bf16_t*)cos,
                 (const bf16_t*)sin, (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)vt, (int)hq, (int)hk, (int)t_pad};
  hipStream_t s = (hipStream_t)stream;
  const int forced = forced_tile();
  const int tile = forced >= 0 && forced != k128x256 ? forced : pick_tile(m, n);
  if (tile == k128x128)
    launch<128, 128, 1, 2, 2, kQkv>(qa, sa, sa_rows, qw, sw, sw_cols, nullptr, 0, m, n, k, s, nullptr, qe);
  else if (tile == k128x128Deep)
    launch<128, 128, 1, 4, 1, kQkv>(qa, sa, sa_rows, qw, sw, sw_cols, nullptr, 0, m, n, k, s, nullptr, qe);
  else
    launch<64, 128, 1, 3, 2, kQkv>(qa, sa, sa_rows, qw, sw, sw_cols, nullptr, 0, m, n, k, s, nullptr, qe);
  FF_LAUNCH_CHECK("ff_gemm_fp8_qkv");
  return FF_OK;
}
