// FP8 (e4m3fn) GEMM for gfx950: y = bf16(sum_k qa[m,k] qw[n,k] * sa * sw).
//
// Both operands are K-contiguous ("TN"): activations qa (M,K) and weights qw
// (N,K), as the reference stores FP8 weights (N,K) row-major. A workgroup of
// 256 threads (4 waves, 2x2) computes a BM x BN = 128 x 128 tile; each wave owns
// 64 x 64 = 4 x 4 tiles of v_mfma_f32_16x16x128_f8f6f4 (fp32 accumulate). K is
// consumed in 128-byte steps staged through LDS with double buffering; 16-byte
// chunks are XOR-swizzled by row so the fragment reads of 16 consecutive rows
// spread over the LDS banks.
//
// MFMA operand layout used (any K permutation is valid as long as A and B use
// the same one): lane l supplies row (l % 16) of its 16-row A (or B) tile and
// the 32 bytes k in [32*(l/16), 32*(l/16)+32) of the 128-byte K step. The
// accumulator of lane l holds D[4*(l/16) + r][l % 16], r = 0..3.
//
// Tiles are ordered XCD-aware: consecutive workgroups are dealt round-robin to
// the 8 XCDs, so the logical tile id gives each XCD a contiguous range of tiles
// walked M-fastest; the few M-tiles that share a weight tile then hit the same
// L2, and the weights stream from HBM about once.
#include "ff_common.h"

using namespace ff;

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int kThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  // scale operands 0 select the unscaled v_mfma_f32_16x16x128_f8f6f4; format 0 = e4m3.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }

__global__ __launch_bounds__(kThreads, 2) void gemm_fp8_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, int sa_rows,
    const uint8_t* __restrict__ qw, const float* __restrict__ sw, int sw_cols,
    bf16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int tiles_m, int tiles_n) {
  __shared__ __align__(16) uint8_t smem[2][(BM + BN) * BK];

  // XCD-aware logical tile id.
  const int nblk = tiles_m * tiles_n;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical % tiles_m, tn = logical / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  // global -> register staging: 4 chunks of A and 4 of B per thread.
  u32x4 ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + i * kThreads, row = q >> 3, c = q & 7;
      const int m = m0 + row;
      if (m < M) ra[i] = *reinterpret_cast<const u32x4*>(qa + (size_t)m * K + k0 + c * 16);
      else ra[i] = u32x4{0, 0, 0, 0};
      const int n = n0 + row;
      if (n < N) rb[i] = *reinterpret_cast<const u32x4*>(qw + (size_t)n * K + k0 + c * 16);
      else rb[i] = u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* As = smem[buf];
    uint8_t* Bs = smem[buf] + BM * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + i * kThreads, row = q >> 3, c = q & 7;
      *reinterpret_cast<u32x4*>(As + swz(row, c)) = ra[i];
      *reinterpret_cast<u32x4*>(Bs + swz(row, c)) = rb[i];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
    const uint8_t* As = smem[buf];
    const uint8_t* Bs = smem[buf] + BM * BK;
    i32x8 af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wm * 64 + i * 16 + r16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(As + swz(row, 2 * g));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(As + swz(row, 2 * g + 1));
      af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 64 + j * 16 + r16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(Bs + swz(row, 2 * g));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(Bs + swz(row, 2 * g + 1));
      bfr[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma_fp8(af[i], bfr[j], acc[i][j]);
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: y = bf16((acc * sa) * sw)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + r16;
    if (n >= N) continue;
    const float swv = sw[sw_cols ? n : 0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + 4 * g + r;
        if (m < M) {
          const float sav = sa[sa_rows ? m : 0];
          y[(size_t)m * ldy + n] = (bf16_t)f32_to_bf16((acc[i][j][r] * sav) * swv);
        }
      }
    }
  }
}

}  // namespace

extern "C" int ff_gemm_fp8(const void* qa, const float* sa, int sa_rows, const void* qw,
                           const float* sw, int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n,
                           int64_t k, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && qw && sw && y, "ff_gemm_fp8: null pointer");
  FF_REQUIRE(m >= 0 && n > 0 && k > 0 && k % BK == 0, "ff_gemm_fp8: k=%lld must be a multiple of %d",
             (long long)k, BK);
  FF_REQUIRE(ldy >= n && m < (1 << 30) && n < (1 << 30) && k < (1 << 30), "ff_gemm_fp8: bad sizes");
  FF_REQUIRE(ff_aligned(qa, 16) && ff_aligned(qw, 16), "ff_gemm_fp8: operands must be 16-byte aligned");
  if (m == 0) return FF_OK;
  const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)((n + BN - 1) / BN);
  hipLaunchKernelGGL(gemm_fp8_kernel, dim3(tiles_m * tiles_n), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint8_t*)qa, sa, sa_rows, (const uint8_t*)qw, sw, sw_cols, (bf16_t*)y, ldy,
                     (int)m, (int)n, (int)k, tiles_m, tiles_n);
  FF_LAUNCH_CHECK("ff_gemm_fp8");
  return FF_OK;
}
