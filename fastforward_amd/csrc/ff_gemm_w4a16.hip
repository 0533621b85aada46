// W4A16 GEMM for gfx950: y = bf16(x @ dequant(W)^T), fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.
//
// W is stored as packed nibbles (N, K/2) -- even k in the high nibble -- with
// (scale, zero) bf16 pairs laid out [K/group, N, 2], the reference's Int4 layout
// before its library repack. The dequantised weight is w = bf16((q-8)*s + z):
// (q-8)*s is exact in fp32 (4-bit by 8-bit significands), so one rounding to fp32
// and one to bf16 give the value of the fp32 dequantised weight the reference
// checks against, cast to the bf16 MFMA operand.
//
// Work split: a workgroup owns BM rows x BN = 4*CW columns; wave w owns all BM
// rows of columns [w*CW, w*CW + CW). Each weight is therefore dequantised by
// exactly one wave, in registers, straight into the MFMA B operand -- the bf16
// weight never touches LDS. The activation tile, which all four waves read, is
// staged in LDS. Per 64-k stage the four waves issue global_load_lds_dwordx4
// (direct-to-LDS) for
//   * A: BM rows x 128 bytes, 16-byte chunk c of row r (r within its 16-row
//     group) at slot 8*(r%8) + (c ^ (r/2)) of the group's two 1 KB blocks --
//     the layout of the FP8 GEMM, conflict-free for the operand reads;
//   * B: the wave's CW rows x 32 packed bytes, 512 bytes per 16-column tile,
//     row-major;
//   * the wave's (s, z) pairs for the one or two groups the stage touches
//     (256 bytes per group).
// S stages rotate through LDS with S-1 in flight and one barrier per stage.
//
// MFMA k order: in step t (0, 1) of a stage, lane l (row l%16, g = l/16)
// supplies k = 16g + 8t + [0, 8) for both operands -- A chunk 2g+t of its row
// and packed bytes [8g + 4t, 8g + 4t + 4) of its weight row -- so one 8-byte LDS
// read gives the lane all 16 nibbles it needs per stage.
//
// Dequantisation per nibble is one v_cvt_f32_ubyte (after separating high and
// low nibbles into bytes), one fma with z8 = z - 8s and half a v_cvt_pk_bf16_f32.
// fma(q, s, z8) equals fma(q-8, s, z) whenever z8 is exact, i.e. unless z and 8s
// are more than 2^15 apart in magnitude; the stages where some lane's z8 is
// inexact take the two-operation form (q-8, then fma) instead.
//
// The accumulator of lane l holds D[4*(l/16) + r][l % 16]; the epilogue rounds
// to bf16 and stages the tile through LDS so global stores are 16-byte row
// chunks. Tiles are dealt to the 8 XCDs in contiguous ranges of the logical tile
// id, walked N-fastest, so an XCD's concurrent workgroups share few row tiles of
// the bf16 activations (4.7 MB at 576 x 4096 would not fit one XCD's L2).
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "ff_common.h"

using namespace ff;

namespace {

constexpr int KSTAGE = 64;  // k per stage
constexpr int kThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// 8 nibbles of one packed dword (k order: byte b high nibble, byte b low nibble,
// b = 0..3) -> 8 bf16 of bf16(q*s + z8), as the MFMA operand (pairs in k order).
__device__ __forceinline__ u32x4 dequant8(uint32_t w, float s, float z8) {
  uint32_t hi = (w >> 4) & 0x0F0F0F0Fu, lo = w & 0x0F0F0F0Fu;
  // Opaque to the optimiser, so each byte converts with one v_cvt_f32_ubyte{0..3}
  // instead of a bit-field extract per nibble followed by a conversion.
  asm("" : "+v"(hi));
  asm("" : "+v"(lo));
  u32x4 r;
  r.x = pack_bf16x2(fmaf((float)(hi & 0xFFu), s, z8), fmaf((float)(lo & 0xFFu), s, z8));
  r.y = pack_bf16x2(fmaf((float)((hi >> 8) & 0xFFu), s, z8), fmaf((float)((lo >> 8) & 0xFFu), s, z8));
  r.z = pack_bf16x2(fmaf((float)((hi >> 16) & 0xFFu), s, z8), fmaf((float)((lo >> 16) & 0xFFu), s, z8));
  r.w = pack_bf16x2(fmaf((float)(hi >> 24), s, z8), fmaf((float)(lo >> 24), s, z8));
  return r;
}

// Same values through (q-8) first: exact for every (s, z).
__device__ __forceinline__ u32x4 dequant8_exact(uint32_t w, float s, float z) {
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu, lo = w & 0x0F0F0F0Fu;
  auto v = [&](uint32_t q) { return fmaf((float)q - 8.f, s, z); };
  u32x4 r;
  r.x = pack_bf16x2(v(hi & 0xFFu), v(lo & 0xFFu));
  r.y = pack_bf16x2(v((hi >> 8) & 0xFFu), v((lo >> 8) & 0xFFu));
  r.z = pack_bf16x2(v((hi >> 16) & 0xFFu), v((lo >> 16) & 0xFFu));
  r.w = pack_bf16x2(v(hi >> 24), v(lo >> 24));
  return r;
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int BM, int CW, int S>
struct W4Cfg {
  static constexpr int BN = 4 * CW;
  static constexpr int RA = BM / 16;                 // A 16-row groups
  static constexpr int TJ = CW / 16;                 // column tiles per wave
  static constexpr int A_BYTES = BM * 128;           // A bytes per stage
  static constexpr int NDA = BM / 32;                // A DMA blocks (1 KB) per wave per stage
  static constexpr int NDB = (TJ + 1) / 2;           // B DMA blocks per wave per stage
  static constexpr int B_WAVE = NDB * 1024;          // B bytes per wave per stage
  static constexpr int SC_WAVE = 512;                // (s, z) bytes per wave per stage (two groups)
  static constexpr int STAGE = A_BYTES + 4 * (B_WAVE + SC_WAVE);
  static constexpr int ND = NDA + NDB + 1;           // DMA instructions per wave per stage
  static constexpr int EPI_LD = BN + 8;              // bf16 row pitch of the epilogue tile
  static constexpr int EPI32_LD = BN + 4;            // fp32 row pitch of a split-K partial tile
  static constexpr int SMEM = S * STAGE > BM * EPI_LD * 2 ? S * STAGE : BM * EPI_LD * 2;
  static constexpr bool kSplitK = BM * EPI32_LD * 4 <= SMEM;  // the fp32 partial tile fits the LDS
  static_assert(BM % 32 == 0 && CW % 16 == 0 && CW <= 64, "tile shape");
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert((S - 1) * ND < 64 && S >= 3, "vmcnt range; two stages resident");
};

template <int BM, int CW, int S, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void gemm_w4a16_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ packed,
    const bf16_t* __restrict__ scales, int group, bf16_t* __restrict__ y, int64_t ldy, int M, int N, int K,
    int tiles_m, int tiles_n, int splits, float* __restrict__ ws) {
  using C = W4Cfg<BM, CW, S>;
  __shared__ __align__(16) uint8_t smem[C::SMEM];

  const int nblk = tiles_m * tiles_n;
  const int split = blockIdx.x / nblk;
  const int b = blockIdx.x % nblk;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical / tiles_n, tn = logical % tiles_n;
  // Split-K: this workgroup's k range, in whole pairs of stages (the loop runs two per trip).
  const int kp = K / (2 * KSTAGE);
  const int kp0 = (int)((int64_t)kp * split / splits), kp1 = (int)((int64_t)kp * (split + 1) / splits);
  const int kbase = kp0 * 2 * KSTAGE;
  const int m0 = tm * BM, n0 = tn * C::BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int nw = n0 + wave * CW;  // first column of this wave

  // DMA sources at k = 0. A: block i of this wave is 1 KB block blk = wave + 4 i
  // of the stage (16-row group blk/2, rows 8*(blk%2) + lane/8).
  const uint8_t* srcA[C::NDA];
#pragma unroll
  for (int i = 0; i < C::NDA; ++i) {
    const int blk = wave + 4 * i, h = blk & 1;
    const int rr = 8 * h + (lane >> 3);
    const int ch = (lane & 7) ^ (rr >> 1);
    const int row = min(m0 + (blk >> 1) * 16 + rr, M - 1);
    srcA[i] = reinterpret_cast<const uint8_t*>(x + (size_t)row * ldx) + 16 * ch;
  }
  // B: block i covers tiles 2i, 2i+1 of the wave; lane p -> tile 2i + p/32, row (p%32)/2, 16-byte half p%2.
  const uint8_t* srcB[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) {
    const int j = 2 * i + (lane >> 5);
    const int n = min(nw + 16 * j + ((lane & 31) >> 1), N - 1);
    srcB[i] = packed + (size_t)n * (K / 2) + 16 * (lane & 1);
  }
  // (s, z): lane p -> group slot p/16 of the stage, columns [4 (p%16), +4) of the wave.
  const int sc_h = lane >> 4, sc_c = lane & 15;
  const bool sc_active = sc_c * 4 < CW && (group < KSTAGE ? sc_h < KSTAGE / group : sc_h == 0);
  const uint8_t* srcS =
      reinterpret_cast<const uint8_t*>(scales) + ((size_t)min(nw + 4 * sc_c, N - 4)) * 4 + (size_t)sc_h * N * 4;

  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsA = lds0 + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024;
  const uint32_t ldsB = lds0 + C::A_BYTES + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * C::B_WAVE;
  const uint32_t ldsS = lds0 + C::A_BYTES + 4 * C::B_WAVE + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * C::SC_WAVE;
  auto issue = [&](int kt, int buf) {
    const int k0 = kbase + kt * KSTAGE;
    const uint32_t off = buf * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::NDA; ++i) lds_dma16(srcA[i] + 2 * k0, ldsA + off + 4 * i * 1024);
#pragma unroll
    for (int i = 0; i < C::NDB; ++i) lds_dma16(srcB[i] + k0 / 2, ldsB + off + i * 1024);
    const size_t gi = (size_t)(k0 / group);
    if (sc_active) lds_dma16(srcS + gi * N * 4, ldsS + off);  // lane l lands at 16 l = 256 sc_h + 16 sc_c
  };

  f32x4 acc[C::RA][C::TJ];
#pragma unroll
  for (int i = 0; i < C::RA; ++i)
#pragma unroll
    for (int j = 0; j < C::TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = 2 * (kp1 - kp0);  // stages of this workgroup
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < KT) issue(st, st);
  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int c0 = 16 * ((2 * g) ^ (r16 >> 1)), c1 = 16 * ((2 * g + 1) ^ (r16 >> 1));
  const int sc_slot = group < KSTAGE ? (16 * g) / group : 0;  // group slot of this lane's 16 k

  // B operands of one stage (tile j, step t) in the exact form, from the stage's
  // LDS buffer (the rare path; see the file comment).
  auto dequant_exact_stage = [&](int kt, u32x4 (&bop)[C::TJ][2]) {
    const uint8_t* st = smem + (kt % S) * C::STAGE;
    const uint8_t* bw = st + C::A_BYTES + wave * C::B_WAVE;
    const uint8_t* sw = st + C::A_BYTES + 4 * C::B_WAVE + wave * C::SC_WAVE + 256 * sc_slot;
#pragma unroll
    for (int j = 0; j < C::TJ; ++j) {
      const u32x2 p = *reinterpret_cast<const u32x2*>(bw + (j >> 1) * 1024 + (j & 1) * 512 + r16 * 32 + 8 * g);
      const uint32_t sz = *reinterpret_cast<const uint32_t*>(sw + (j * 16 + r16) * 4);
      const float sv = bf16_to_f32(sz & 0xFFFFu), zv = bf16_to_f32(sz >> 16);
      bop[j][0] = dequant8_exact(p.x, sv, zv);
      bop[j][1] = dequant8_exact(p.y, sv, zv);
    }
  };
  // One pipelined step: the MFMAs of stage kt (A from LDS, B operands bcur)
  // interleaved with the z8-form dequantisation of stage ktn into bnext.
  // *bad_next reports whether some lane's z8 is inexact for stage ktn.
  constexpr int UNITS = 2 * C::TJ;                         // packed dwords per stage (8 nibbles each)
  constexpr int PER_I = (UNITS + C::RA - 1) / C::RA;       // dequant dwords per A tile
  auto step = [&](int kt, const u32x4 (&bcur)[C::TJ][2], int ktn, u32x4 (&bnext)[C::TJ][2], bool* bad_next) {
    const uint8_t* st = smem + (kt % S) * C::STAGE;
    const uint8_t* stn = smem + (ktn % S) * C::STAGE;
    const uint8_t* bw = stn + C::A_BYTES + wave * C::B_WAVE;
    const uint8_t* sw = stn + C::A_BYTES + 4 * C::B_WAVE + wave * C::SC_WAVE + 256 * sc_slot;
    uint32_t pk[UNITS];
    uint32_t sz[C::TJ];
#pragma unroll
    for (int j = 0; j < C::TJ; ++j) {
      const u32x2 p = *reinterpret_cast<const u32x2*>(bw + (j >> 1) * 1024 + (j & 1) * 512 + r16 * 32 + 8 * g);
      pk[2 * j] = p.x;
      pk[2 * j + 1] = p.y;
      sz[j] = *reinterpret_cast<const uint32_t*>(sw + (j * 16 + r16) * 4);
    }
    u32x4 a[2][2];
    {
      const uint8_t* p = st + frag;
      a[0][0] = *reinterpret_cast<const u32x4*>(p + c0);
      a[0][1] = *reinterpret_cast<const u32x4*>(p + c1);
    }
    float sv[C::TJ], z8[C::TJ];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < C::RA; ++i) {
      if (i + 1 < C::RA) {
        const uint8_t* p = st + 2 * (i + 1) * 1024 + frag;
        a[(i + 1) & 1][0] = *reinterpret_cast<const u32x4*>(p + c0);
        a[(i + 1) & 1][1] = *reinterpret_cast<const u32x4*>(p + c1);
      }
      if (i == 0) {
#pragma unroll
        for (int j = 0; j < C::TJ; ++j) {
          sv[j] = bf16_to_f32(sz[j] & 0xFFFFu);
          const float zv = bf16_to_f32(sz[j] >> 16);
          z8[j] = fmaf(-8.f, sv[j], zv);
          bad |= (z8[j] + 8.f * sv[j] != zv) || (zv - z8[j] != 8.f * sv[j]);
        }
      }
#pragma unroll
      for (int u = i * PER_I; u < (i + 1) * PER_I && u < UNITS; ++u)
        bnext[u >> 1][u & 1] = dequant8(pk[u], sv[u >> 1], z8[u >> 1]);
#pragma unroll
      for (int j = 0; j < C::TJ; ++j) {
        acc[i][j] = mfma_bf16(a[i & 1][0], bcur[j][0], acc[i][j]);
        acc[i][j] = mfma_bf16(a[i & 1][1], bcur[j][1], acc[i][j]);
      }
      // Keep the code of A tile i together: the reads of tile i+1 and this
      // tile's share of the dequantisation run under its MFMAs.
      __builtin_amdgcn_sched_barrier(0);
    }
    *bad_next = bad;
  };

  // Software pipeline: iteration kt runs the MFMAs of stage kt while it
  // dequantises stage kt+1 (so stage kt+1 must have landed at its top).
  u32x4 bop[2][C::TJ][2];
  bool inexact[2];
  wait_vmcnt<0>();
  barrier_lds();
  dequant_exact_stage(0, bop[0]);
  inexact[0] = false;
  for (int kb = 0; kb < KT; kb += 2) {
    static_for<0, 2>([&](auto U) {
      constexpr int u = decltype(U)::value;
      const int kt = kb + u;
      if (kt + S - 2 < KT) wait_vmcnt<(S - 3) * C::ND>();
      else wait_vmcnt<0>();
      barrier_lds();  // stages kt, kt+1 landed for every wave; stage kt-1 fully consumed
      if (kt + S - 1 < KT) issue(kt + S - 1, (kt + S - 1) % S);
      if (__builtin_amdgcn_ballot_w64(inexact[u]) != 0) dequant_exact_stage(kt, bop[u]);
      step(kt, bop[u], min(kt + 1, KT - 1), bop[u ^ 1], &inexact[u ^ 1]);
    });
  }
  __syncthreads();  // all stages consumed before the epilogue reuses the LDS

  if constexpr (C::kSplitK) {
   if (splits > 1) {
    // fp32 partial tile of this split, row-major (M, N) at ws + split * M * N
    float* tile32 = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int j = 0; j < C::TJ; ++j) {
      const int cl = wave * CW + j * 16 + r16;
#pragma unroll
      for (int i = 0; i < C::RA; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) tile32[(i * 16 + 4 * g + r) * C::EPI32_LD + cl] = acc[i][j][r];
    }
    __syncthreads();
    float* part = ws + (size_t)split * M * N;
    constexpr int CH4 = BM * C::BN / 4;
#pragma unroll
    for (int c = tid; c < CH4; c += kThreads) {
      const int rl = c / (C::BN / 4), cl = (c % (C::BN / 4)) * 4;
      const int m = m0 + rl, n = n0 + cl;
      if (m < M && n < N)
        *reinterpret_cast<f32x4*>(part + (size_t)m * N + n) = *reinterpret_cast<const f32x4*>(tile32 + rl * C::EPI32_LD + cl);
    }
    return;
   }
  }

  bf16_t* tile = reinterpret_cast<bf16_t*>(smem);
#pragma unroll
  for (int j = 0; j < C::TJ; ++j) {
    const int cl = wave * CW + j * 16 + r16;
#pragma unroll
    for (int i = 0; i < C::RA; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) tile[(i * 16 + 4 * g + r) * C::EPI_LD + cl] = (bf16_t)f32_to_bf16(acc[i][j][r]);
  }
  __syncthreads();
  constexpr int CHUNKS = BM * C::BN / 8;
#pragma unroll
  for (int c = tid; c < CHUNKS; c += kThreads) {
    const int rl = c / (C::BN / 8), cl = (c % (C::BN / 8)) * 8;
    const int m = m0 + rl, n = n0 + cl;
    if (m < M && n < N)
      *reinterpret_cast<u32x4*>(y + (size_t)m * ldy + n) = *reinterpret_cast<const u32x4*>(tile + rl * C::EPI_LD + cl);
  }
}

// y = bf16(sum over splits of the fp32 partials, in split order); 8 outputs per thread.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int splits, int M, int N,
                                                            bf16_t* __restrict__ y, int64_t ldy) {
  const int64_t per_row = N / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * per_row) return;
  const int m = (int)(i / per_row), n = (int)(i % per_row) * 8;
  const size_t off = (size_t)m * N + n;
  f32x4 a = *reinterpret_cast<const f32x4*>(ws + off), b = *reinterpret_cast<const f32x4*>(ws + off + 4);
  for (int s = 1; s < splits; ++s) {
    a += *reinterpret_cast<const f32x4*>(ws + (size_t)s * M * N + off);
    b += *reinterpret_cast<const f32x4*>(ws + (size_t)s * M * N + off + 4);
  }
  u32x4 o;
  o.x = pack_bf16x2(a[0], a[1]); o.y = pack_bf16x2(a[2], a[3]);
  o.z = pack_bf16x2(b[0], b[1]); o.w = pack_bf16x2(b[2], b[3]);
  *reinterpret_cast<u32x4*>(y + (size_t)m * ldy + n) = o;
}

enum W4Tile { kW64x256, kW192x192 };

template <int BM, int CW, int S, int OCC>
void launch_w4(const void* x, int64_t ldx, const void* packed, const void* scales, int group, void* y, int64_t ldy,
               int m, int n, int k, int splits, float* ws, hipStream_t stream) {
  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + 4 * CW - 1) / (4 * CW);
  hipLaunchKernelGGL((gemm_w4a16_kernel<BM, CW, S, OCC>), dim3(tiles_m * tiles_n * splits), dim3(kThreads), 0,
                     stream, (const bf16_t*)x, ldx, (const uint8_t*)packed, (const bf16_t*)scales, group,
                     (bf16_t*)y, ldy, m, n, k, tiles_m, tiles_n, splits, ws);
  if (splits > 1) {
    const int64_t items = (int64_t)m * (n / 8);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, stream, ws, splits,
                       m, n, (bf16_t*)y, ldy);
  }
}

// 192 x 192 tiles dequantise each weight for 192 rows (a third of the VALU work
// per MFMA of 64-row tiles) but need enough tiles to cover the 256 CUs; below
// that, 64 x 256 tiles at two workgroups per CU. ff_set_tuning(FF_TUNE_W4A16_TILE,
// 1 | 2) forces 64x256 | 192x192.
W4Tile pick_w4_tile(int64_t m, int64_t n) {
  if (const int f = ff_tuning(FF_TUNE_W4A16_TILE)) return f == 1 ? kW64x256 : kW192x192;
  const int64_t tiles192 = ((m + 191) / 192) * ((n + 191) / 192);
  return (m > 64 && tiles192 >= 256) ? kW192x192 : kW64x256;
}

// Split-K factor of the 64 x 256 tiles: grids below 256 workgroups leave CUs
// idle, so the k range is split until about two workgroups per CU (at most 8
// ways, at least one pair of stages each); the fp32 partials cost 8 bytes per
// output per split (written once, read once by the reduction).
// ff_set_tuning(FF_TUNE_W4A16_SPLITS, s) overrides the choice.
int pick_w4_splits(W4Tile t, int64_t m, int64_t n, int64_t k) {
  static_assert(W4Cfg<64, 64, 4>::kSplitK, "the 64 x 256 tile stages its fp32 partials in LDS");
  if (t != kW64x256) return 1;
  const int64_t pairs = k / (2 * KSTAGE);
  int64_t s;
  if (const int f = ff_tuning(FF_TUNE_W4A16_SPLITS)) {
    s = f;
  } else {
    const int64_t tiles = ((m + 63) / 64) * ((n + 255) / 256);
    s = tiles >= 256 ? 1 : 512 / tiles;
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>({s, 8, pairs}));
}

static int gemm_w4a16(const void* x, int64_t ldx, const void* packed, const void* scales, int64_t group, void* y,
                      int64_t ldy, int64_t m, int64_t n, int64_t k, void* ws, int64_t ws_bytes, ff_stream_t stream) {
  FF_REQUIRE(x && packed && scales && y, "ff_gemm_w4a16: null pointer");
  FF_REQUIRE(k > 0 && k % (2 * KSTAGE) == 0 && (group == 32 || group % 64 == 0) && k % group == 0,
             "ff_gemm_w4a16: k=%lld must be a multiple of %d and of group=%lld (group 32 or a multiple of 64)",
             (long long)k, 2 * KSTAGE, (long long)group);
  FF_REQUIRE(m >= 0 && n >= 8 && n % 8 == 0 && ldx >= k && ldx % 8 == 0 && ldy >= n && ldy % 8 == 0,
             "ff_gemm_w4a16: bad sizes (n %% 8 == 0, ldx and ldy multiples of 8)");
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(packed, 16) && ff_aligned(scales, 16) && ff_aligned(y, 16),
             "ff_gemm_w4a16: x, packed, scales and y must be 16-byte aligned");
  FF_REQUIRE(ws_bytes >= 0 && (ws_bytes == 0 || (ws && ff_aligned(ws, 16))),
             "ff_gemm_w4a16_ws: workspace must be 16-byte aligned");
  if (m == 0) return FF_OK;
  const hipStream_t s = (hipStream_t)stream;
  const W4Tile t = pick_w4_tile(m, n);
  int splits = pick_w4_splits(t, m, n, k);
  while (splits > 1 && (int64_t)splits * m * n * 4 > ws_bytes) --splits;
  switch (t) {
    case kW64x256:
      launch_w4<64, 64, 4, 2>(x, ldx, packed, scales, (int)group, y, ldy, (int)m, (int)n, (int)k, splits,
                              (float*)ws, s);
      break;
    case kW192x192:
      launch_w4<192, 48, 4, 1>(x, ldx, packed, scales, (int)group, y, ldy, (int)m, (int)n, (int)k, 1, nullptr, s);
      break;
  }
  FF_LAUNCH_CHECK("ff_gemm_w4a16");
  return FF_OK;
}

}  // namespace

extern "C" int ff_gemm_w4a16(const void* x, int64_t ldx, const void* packed, const void* scales,
                             int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                             ff_stream_t stream) {
  return gemm_w4a16(x, ldx, packed, scales, group, y, ldy, m, n, k, nullptr, 0, stream);
}

extern "C" int ff_gemm_w4a16_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes) {
  FF_REQUIRE(bytes && m >= 0 && n > 0 && k > 0, "ff_gemm_w4a16_workspace: bad arguments");
  const int splits = k % (2 * KSTAGE) == 0 ? pick_w4_splits(pick_w4_tile(m, n), m, n, k) : 1;
  *bytes = splits > 1 ? (int64_t)splits * m * n * 4 : 0;
  return FF_OK;
}

extern "C" int ff_gemm_w4a16_ws(const void* x, int64_t ldx, const void* packed, const void* scales, int64_t group,
                                void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, void* workspace,
                                int64_t workspace_bytes, ff_stream_t stream) {
  return gemm_w4a16(x, ldx, packed, scales, group, y, ldy, m, n, k, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------ allocation-free variant
//
// ff_gemm_w4a16_noalloc keeps the split-K partials in `scratch`, a file-scope
// device array of kScratchBytes: each GPU the library runs on holds its own copy
// until the process ends. The array's host-side name is not a device address;
// its address on a device comes from hipGetSymbolAddress, taken once per device
// on the first call made with that device current, and only that address is
// handed to kernels. Every split writes all of its partials before the reduction
// reads them, so nothing has to start at zero. All calls on one GPU share its
// array: calls that overlap in time on one GPU (two streams, two threads) race.

namespace {

constexpr int64_t kScratchBytes = int64_t(32) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of this device's `scratch` (taken once per device), or nullptr
// with the error set.
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    ff_set_error("ff_gemm_w4a16_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      ff_set_error("ff_gemm_w4a16_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                   hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int ff_gemm_w4a16_noalloc(const void* x, int64_t ldx, const void* packed, const void* scales,
                                     int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                                     ff_stream_t stream) {
  FF_REQUIRE(m >= 0 && n > 0 && k > 0, "ff_gemm_w4a16_noalloc: bad sizes");
  int64_t need = 0;
  if (k % (2 * KSTAGE) == 0) {
    const int splits = pick_w4_splits(pick_w4_tile(m, n), m, n, k);
    need = splits > 1 ? (int64_t)splits * m * n * 4 : 0;
  }
  FF_REQUIRE(need <= kScratchBytes,
             "ff_gemm_w4a16_noalloc: this %lld x %lld x %lld product needs %lld bytes of split-K scratch; the "
             "static scratch holds %lld (use ff_gemm_w4a16_ws with a workspace)",
             (long long)m, (long long)n, (long long)k, (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_on_current_device();
    if (!ws) return FF_EDEVICE;
  }
  return gemm_w4a16(x, ldx, packed, scales, group, y, ldy, m, n, k, ws, need, stream);
}
