// W4A16 GEMM for gfx950: y = bf16(x @ dequant(W)^T), fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.
//
// W is stored as packed nibbles (N, K/2) -- even k in the high nibble -- with
// (scale, zero) bf16 pairs laid out [K/group, N, 2], the reference's Int4 layout
// before its library repack. Dequantisation w = bf16((q-8)*s + z) is fused into
// the B-operand staging: each thread loads 16 packed bytes (32 nibbles) from HBM,
// dequantises them once for the whole workgroup and writes the bf16 tile to LDS,
// so HBM sees 0.5 byte per weight. (q-8)*s is exact in fp32 (4-bit by 8-bit
// significands), so the single rounding of (q-8)*s + z matches the fp32
// dequantised weight the reference checks against, up to the bf16 operand cast.
//
// Tiles: 128 x 128 per workgroup (4 waves, 2x2, each 64 x 64 = 4 x 4 MFMA tiles),
// BK = 64 k per stage, LDS double buffered, 16-byte chunks XOR-swizzled by row.
// MFMA operand layout: lane l supplies row (l % 16) and k in [8*(l/16), +8) of
// each 32-k step; the accumulator of lane l holds D[4*(l/16) + r][l % 16].
#include "ff_common.h"

using namespace ff;

namespace {

constexpr int BM = 128, BN = 128, BK = 64;  // BK in k elements (128 bytes of bf16 per row)
constexpr int kThreads = 256;
constexpr int kXcds = 8;
constexpr int kRowBytes = BK * 2;

__device__ __forceinline__ int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ (row & 7)) << 4); }

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

__global__ __launch_bounds__(kThreads, 2) void gemm_w4a16_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ packed,
    const bf16_t* __restrict__ scales, int group, bf16_t* __restrict__ y, int64_t ldy, int M, int N,
    int K, int tiles_m, int tiles_n) {
  __shared__ __align__(16) uint8_t smem[2][(BM + BN) * kRowBytes];

  const int nblk = tiles_m * tiles_n;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical % tiles_m, tn = logical / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  // A staging: 128 rows x 8 chunks of 16 B -> 4 chunks per thread.
  // B staging: 128 rows x 32 packed bytes -> one 16-byte load (32 nibbles) per thread.
  u32x4 ra[4];
  u32x4 rbq;
  float bs = 0.f, bz = 0.f;
  const int brow = tid >> 1, bhalf = tid & 1;
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + i * kThreads, row = q >> 3, c = q & 7;
      const int m = m0 + row;
      if (m < M) ra[i] = *reinterpret_cast<const u32x4*>(x + (size_t)m * ldx + k0 + c * 8);
      else ra[i] = u32x4{0, 0, 0, 0};
    }
    const int n = n0 + brow;
    if (n < N) {
      rbq = *reinterpret_cast<const u32x4*>(packed + (size_t)n * (K / 2) + k0 / 2 + bhalf * 16);
      const int kk = k0 + bhalf * 32;  // the 32 k of this load share one group
      const uint32_t sz = *reinterpret_cast<const uint32_t*>(scales + ((size_t)(kk / group) * N + n) * 2);
      bs = bf16_to_f32(sz & 0xFFFFu);
      bz = bf16_to_f32(sz >> 16);
    } else {
      rbq = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      bs = 0.f;
      bz = 0.f;
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* As = smem[buf];
    uint8_t* Bs = smem[buf] + BM * kRowBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + i * kThreads, row = q >> 3, c = q & 7;
      *reinterpret_cast<u32x4*>(As + swz(row, c)) = ra[i];
    }
    // 32 nibbles -> 32 bf16 = 4 chunks (this thread's half of the row).
    const uint32_t words[4] = {rbq.x, rbq.y, rbq.z, rbq.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t wd = words[c];
      float f[8];
#pragma unroll
      for (int byte = 0; byte < 4; ++byte) {
        const uint32_t v = (wd >> (8 * byte)) & 0xFFu;
        f[2 * byte] = fmaf((float)((int)(v >> 4) - 8), bs, bz);
        f[2 * byte + 1] = fmaf((float)((int)(v & 15u) - 8), bs, bz);
      }
      *reinterpret_cast<u32x4*>(Bs + swz(brow, bhalf * 4 + c)) = pack8(f);
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
    const uint8_t* Bs = smem[buf] + BM * kRowBytes;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      u32x4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const u32x4*>(As + swz(wm * 64 + i * 16 + r16, 4 * s + g));
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = *reinterpret_cast<const u32x4*>(Bs + swz(wn * 64 + j * 16 + r16, 4 * s + g));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_bf16(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + r16;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + 4 * g + r;
        if (m < M) y[(size_t)m * ldy + n] = (bf16_t)f32_to_bf16(acc[i][j][r]);
      }
  }
}

}  // namespace

extern "C" int ff_gemm_w4a16(const void* x, int64_t ldx, const void* packed, const void* scales,
                             int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                             ff_stream_t stream) {
  FF_REQUIRE(x && packed && scales && y, "ff_gemm_w4a16: null pointer");
  FF_REQUIRE(k > 0 && k % BK == 0 && group >= 32 && group % 32 == 0 && k % group == 0,
             "ff_gemm_w4a16: k=%lld must be a multiple of %d and of group=%lld (group %% 32 == 0)",
             (long long)k, BK, (long long)group);
  FF_REQUIRE(m >= 0 && n > 0 && ldx >= k && ldx % 8 == 0 && ldy >= n, "ff_gemm_w4a16: bad sizes");
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(packed, 16) && ff_aligned(scales, 4),
             "ff_gemm_w4a16: alignment");
  if (m == 0) return FF_OK;
  const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)((n + BN - 1) / BN);
  hipLaunchKernelGGL(gemm_w4a16_kernel, dim3(tiles_m * tiles_n), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)x, ldx, (const uint8_t*)packed, (const bf16_t*)scales, (int)group,
                     (bf16_t*)y, ldy, (int)m, (int)n, (int)k, tiles_m, tiles_n);
  FF_LAUNCH_CHECK("ff_gemm_w4a16");
  return FF_OK;
}
