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
#include "ff_rope.h"

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

// ------------------------------------------------------------------ packed-weight kernels
//
// The weight is repacked once (ff_pack_weight_int4) into MFMA fragment order:
// the 16 rows x 128 k of fragment (f, kt) are the 1 KB at (kt N/16 + f) 1024
// (k-step major: the fragments all workgroups load at one k step are
// contiguous, which streams weights from HBM faster than 32 KB-strided loads);
// lane l = 16 g + r holds row 16 f + r, the packed bytes of k = 128 kt + 64 h +
// 16 g + [0, 16) for h = 0, 1 (8 bytes each, source byte order, each nibble
// q stored as q ^ 8) at 16 l. One
// 16-byte buffer load per lane moves a fragment (1 KB of whole cache lines per
// instruction) straight into registers; dword 2 h + t of a lane feeds MFMA
// (h, t) of the step, k = 128 kt + 64 h + 16 g + 8 t + [0, 8) -- the k
// assignment and MFMA order of the LDS-staged kernel above, so that unsplit
// products are bit-identical between the two.
//
// A workgroup of 4 waves owns BM tokens x 4 CW weight rows and wave w owns all
// BM tokens x CW rows, so each weight is dequantised once per workgroup by the
// wave that owns it, in registers. The bf16 activations go global -> registers
// -> LDS: two 128-k stages and one barrier per step; each 256-byte row sits as
// two 128-byte halves, each half in the packed FP8 GEMM's swizzled layout (1 KB
// blocks of 8 rows, 16-byte chunk c of row r at slot c ^ (r % 8) ^ ((r / 8) % 2)).
// The weight fragment is the MFMA's first operand, so the accumulator holds the
// transposed tile: lane 16 g + r of fragment (i, j) holds token 16 i + r,
// weight rows 16 j + 4 g .. + 3, and the epilogues store 8-byte row pieces
// from registers. The (s, z) pairs come as fp32 (16 s, z) from the copy
// ff_pack_scales_int4 makes at setup ([K/group, N] order, one 8-byte load per
// lane, fragment and half step; group a power of two >= 32, so a lane's 16 k
// share a group).
// The fragments store each nibble q as q ^ 8, so that one v_cvt_off_f32_i4 per
// weight gives (q - 8) / 16 and one fma the exactly rounded (q - 8) s + z
// (dequant8_off): the same values as the kernel above, with no inexact-z8 case.

namespace {

constexpr int kPkStep = 128;  // k per step

// (q - 8) / 16 from the low 4 bits of byte B of x, read as a signed 4-bit value
// (the packed fragments store q ^ 8): v_cvt_off_f32_i4 maps 4-bit two's
// complement n to n / 16, exactly.
template <int B>
__device__ __forceinline__ float cvt_off_byte(uint32_t x) {
  float f;
  if constexpr (B == 0) asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(f) : "v"(x));
  if constexpr (B == 1) asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(f) : "v"(x));
  if constexpr (B == 2) asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(f) : "v"(x));
  if constexpr (B == 3) asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(f) : "v"(x));
  return f;
}

// 8 nibbles of one fragment dword (stored q ^ 8; k order: byte b high nibble,
// byte b low nibble) -> 8 bf16 of bf16((q - 8) s + z), as the MFMA operand.
// fma((q - 8) / 16, 16 s, z) forms the exact product (q - 8) s (4-bit by 8-bit
// significands) and rounds once: the value of dequant8_exact for every (s, z),
// at the cost of dequant8 and without its z8 condition. s16 = 16 s.
__device__ __forceinline__ u32x4 dequant8_off(uint32_t w, float s16, float z) {
  const uint32_t hi = w >> 4;
  u32x4 r;
  r.x = pack_bf16x2(fmaf(cvt_off_byte<0>(hi), s16, z), fmaf(cvt_off_byte<0>(w), s16, z));
  r.y = pack_bf16x2(fmaf(cvt_off_byte<1>(hi), s16, z), fmaf(cvt_off_byte<1>(w), s16, z));
  r.z = pack_bf16x2(fmaf(cvt_off_byte<2>(hi), s16, z), fmaf(cvt_off_byte<2>(w), s16, z));
  r.w = pack_bf16x2(fmaf(cvt_off_byte<3>(hi), s16, z), fmaf(cvt_off_byte<3>(w), s16, z));
  return r;
}

// dequant8_off in 7 pieces of 3 VALU instructions, to be spread between MFMAs
// (same operations, same values): w (fragment dword), s16 = 16 s and z set by
// the caller (the fp32 pair of ff_pack_scales_int4), r the result.
struct DqPieces {
  uint32_t w, hi;
  float s16, z;
  float f[8], y[8];
  u32x4 r;
  template <int P>
  __device__ __forceinline__ void piece() {
    if constexpr (P == 0) {
      hi = w >> 4;
      f[0] = cvt_off_byte<0>(hi);
      f[1] = cvt_off_byte<0>(w);
    } else if constexpr (P == 1) {
      y[0] = fmaf(f[0], s16, z);
      y[1] = fmaf(f[1], s16, z);
      f[2] = cvt_off_byte<1>(hi);
    } else if constexpr (P == 2) {
      f[3] = cvt_off_byte<1>(w);
      y[2] = fmaf(f[2], s16, z);
      y[3] = fmaf(f[3], s16, z);
    } else if constexpr (P == 3) {
      r.x = pack_bf16x2(y[0], y[1]);
      r.y = pack_bf16x2(y[2], y[3]);
      f[4] = cvt_off_byte<2>(hi);
    } else if constexpr (P == 4) {
      f[5] = cvt_off_byte<2>(w);
      y[4] = fmaf(f[4], s16, z);
      y[5] = fmaf(f[5], s16, z);
    } else if constexpr (P == 5) {
      f[6] = cvt_off_byte<3>(hi);
      f[7] = cvt_off_byte<3>(w);
      y[6] = fmaf(f[6], s16, z);
    } else {
      y[7] = fmaf(f[7], s16, z);
      r.z = pack_bf16x2(y[4], y[5]);
      r.w = pack_bf16x2(y[6], y[7]);
    }
  }
};

// acc += A . B for one 16 x 16 x 32 bf16 tile, accumulator tied in place in
// AGPRs (as the packed FP8 kernel: with the builtin the compiler moves every
// accumulator between AGPRs and VGPRs at the loop edge). The compiler does not
// see this asm as an MFMA, so it inserts none of the MFMA's wait states: the
// main loop places every VALU write of an A operand (the dequantised weights)
// at least two MFMAs, or a barrier, before the MFMA that reads it (2 wait
// states are needed), and the accumulator hazards are covered by s_nop at the
// loop's ends.
__device__ __forceinline__ void mfma_bf16_acc(f32x4& acc, const u32x4& a, const i32x4v& b) {
  const i32x4v av = __builtin_bit_cast(i32x4v, a);
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(av), "v"(b));
}

__global__ __launch_bounds__(kThreads) void pack_int4_kernel(const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst, int64_t n, int64_t k) {
  const int64_t kt_n = k / kPkStep;
  const int64_t lanes = (n / 16) * kt_n * 64;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < lanes; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t f = i >> 6;  // fragment f16 * kt_n + kt
    const int64_t kt = f % kt_n, f16 = f / kt_n;
    const int64_t row = f16 * 16 + (l & 15);
    const int64_t nf = n / 16;
    const uint8_t* s = src + row * (k / 2) + kt * 64 + 8 * (l >> 4);
    const u32x2 a = *reinterpret_cast<const u32x2*>(s), b = *reinterpret_cast<const u32x2*>(s + 32);
    constexpr uint32_t kFlip = 0x88888888u;  // nibble q stored as q ^ 8: its signed 4-bit value is q - 8
    *reinterpret_cast<u32x4*>(dst + (kt * nf + f16) * 1024 + 16 * l) =
        u32x4{a.x ^ kFlip, a.y ^ kFlip, b.x ^ kFlip, b.y ^ kFlip};
  }
}

// acc (BM x 4 CW tile, wave w owning all BM rows x CW weight rows, transposed
// layout) = sum over k steps [kt0, kt0 + nk) of A . B^T. sB[j]: byte offset of
// this wave's weight fragment row j at k step 0; colS[j]: the weight row whose
// (s, z) this lane reads for fragment j. nk even, kt0 even.
template <int BM, int CW, typename Pre>
__device__ __forceinline__ void w4pk_mainloop(f32x4 (&acc)[BM / 16][CW / 16], uint8_t* smem,
                                              const bf16_t* __restrict__ x, int64_t ldx, int M, int m0,
                                              const uint8_t* __restrict__ wp, uint32_t wbytes,
                                              const uint32_t (&sB)[CW / 16], const float* __restrict__ sz,
                                              uint32_t szbytes, const uint32_t (&colS)[CW / 16], int N, int gshift,
                                              int kt0, int nk, Pre&& pre) {
  constexpr int RA = BM / 16, TJ = CW / 16;
  constexpr int A_CHUNKS = BM * 16;  // 16-byte chunks of one A stage (BM rows x 256 bytes)
  constexpr int FULL = A_CHUNKS / kThreads, REM = A_CHUNKS % kThreads;
  constexpr int NA = FULL + (REM ? 1 : 0);
  constexpr int HALF = BM * 128;  // one 128-byte half of every row of a stage
  constexpr int STAGE = 2 * HALF;
  static_assert(A_CHUNKS >= kThreads, "at least one full activation round");
  static_assert(RA >= 9, "a group's MFMAs carry the next group's 7 dequantisation pieces, 2 MFMAs before its use");
  const int tid = threadIdx.x, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int kend = kt0 + nk;

  // Activations: chunk c = tid + 256 i is row c / 16, chunk c % 16 (a partial
  // last round is moved back over the last 256 chunks, loading and storing the
  // overlap twice with the same bytes, so nothing is predicated).
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(x, (uint32_t)((int64_t)M * ldx * 2));
  uint32_t voffA[NA];
  int dstA[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = i < FULL ? tid + kThreads * i : A_CHUNKS - kThreads + tid;
    const int row = c >> 4, ch = c & 15;
    voffA[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)(2 * ldx) + 16 * ch;
    dstA[i] = (ch >> 3) * HALF + (row >> 3) * 1024 + 128 * (row & 7) + 16 * ((ch & 7) ^ (row & 7) ^ ((row >> 3) & 1));
  }
  i32x4v ast[NA];
  auto loadA1 = [&](int kt, int i) { ast[i] = bload16(rA, voffA[i], (uint32_t)kt * 256u); };
  auto writeA1 = [&](int buf, int i) { *reinterpret_cast<i32x4v*>(smem + buf * STAGE + dstA[i]) = ast[i]; };
  auto loadA = [&](int kt) {
#pragma unroll
    for (int i = 0; i < NA; ++i) loadA1(kt, i);
  };
  auto writeA = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) writeA1(buf, i);
  };

  const __amdgpu_buffer_rsrc_t rB = make_rsrc(wp, wbytes);
  const __amdgpu_buffer_rsrc_t rS = make_rsrc(sz, szbytes);
  const uint32_t voffB = 16u * (uint32_t)lane;
  const uint32_t kstride = (uint32_t)N * 64u;  // bytes per k step: N / 16 fragments of 1 KB
  i32x4v bq[2][TJ];
  float sq[2][TJ][2][2];  // (16 s, z) of halves h = 0, 1
  auto loadB1 = [&](int kt, auto SLOT, int j) {
    constexpr int slot = decltype(SLOT)::value;
    bq[slot][j] = bload16(rB, voffB, sB[j] + (uint32_t)kt * kstride);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t gi = (uint32_t)(kPkStep * kt + 64 * h + 16 * g) >> gshift;
      const i32x2v v = bload8(rS, (gi * (uint32_t)N + colS[j]) * 8u, 0);
      sq[slot][j][h][0] = __int_as_float(v.x);
      sq[slot][j][h][1] = __int_as_float(v.y);
    }
  };
  auto loadB = [&](int kt, auto SLOT) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) loadB1(kt, SLOT, j);
  };

#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // W4_PIN: every accumulator through an asm barrier (each is zeroed before it).
  // W4_NOPS: wait states between VALU writes / MFMA results and their readers.
#define W4_PIN()                                      \
  do {                                                \
    _Pragma("unroll") for (int i_ = 0; i_ < RA; ++i_) \
    _Pragma("unroll") for (int j_ = 0; j_ < TJ; ++j_) \
      asm volatile("" : "+a"(acc[i_][j_]));           \
  } while (0)
#define W4_NOPS() asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc[RA - 1][TJ - 1]))
  W4_PIN();
  W4_NOPS();

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  loadA(kt0);
  loadB(kt0, I0{});
  __builtin_amdgcn_sched_barrier(0);
  pre();  // epilogue set-up that does not depend on the product, while the loads are in flight
  __builtin_amdgcn_sched_barrier(0);
  writeA(0);
  loadA(min(kt0 + 1, kend - 1));
  loadB(min(kt0 + 1, kend - 1), I1{});

  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int sw = (r16 & 7) ^ (r16 >> 3);
  const int cA[2] = {16 * ((2 * g) ^ sw), 16 * ((2 * g + 1) ^ sw)};
  // A fragments of the current substep (a[sub & 1]); a step's first substep is
  // read during the previous step's last group (the first step's here).
  i32x4v a[2][RA];
  auto readA = [&](const uint8_t* st, int sub, int i, i32x4v& dst) {
    dst = *reinterpret_cast<const i32x4v*>(st + (sub >> 1) * HALF + 2 * i * 1024 + cA[sub & 1]);
  };
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RA; ++i) readA(smem + frag, 0, i, a[0][i]);
  // The first fragment of every step is dequantised in the step before (the
  // first step's here).
  u32x4 bfirst;
  {
    DqPieces d0;
    d0.w = (uint32_t)bq[0][0][0];
    d0.s16 = sq[0][0][0][0];
    d0.z = sq[0][0][0][1];
    static_for<0, 7>([&](auto P_) { d0.template piece<decltype(P_)::value>(); });
    bfirst = d0.r;
  }
  for (int kb = kt0; kb < kend; kb += 2) {
    static_for<0, 2>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      const int kt = kb + u;
      // Stage u was written during the previous step and made visible by its
      // barrier; stage u ^ 1, read in the previous step before that barrier, is
      // written here for step kt + 1. This step's one barrier comes before its
      // last group, whose MFMAs carry the reads of step kt + 1's first substep.
      const int kta = min(kt + 2, kend - 1);  // the step whose activations and weights are loaded here
      // The step's MFMAs as 4 TJ groups g = (substep s = g / TJ, fragment j =
      // g % TJ), each RA MFMAs on one dequantised weight fragment. The wave
      // issues in order and the matrix core runs an MFMA for 16 cycles, so the
      // next group's dequantisation (the last group: the next step's first) and,
      // before a new substep, its A fragments are spread between this group's
      // MFMAs, a few VALU instructions after each, where they run under them.
      const uint8_t* st = smem + u * STAGE + frag;
      const uint8_t* stn = smem + (u ^ 1) * STAGE + frag;
      constexpr int NG = 4 * TJ;
      u32x4 bcur = bfirst;
      static_for<0, NG>([&](auto G_) {
        constexpr int gg = decltype(G_)::value, sub = gg / TJ, j = gg % TJ;
        constexpr int gn = gg + 1, subn = gn / TJ, jn = gn % TJ;
        constexpr bool in_step = gn < NG;
        DqPieces d;
        if constexpr (in_step) {
          d.w = (uint32_t)bq[u][jn][subn];
          d.s16 = sq[u][jn][subn >> 1][0];
          d.z = sq[u][jn][subn >> 1][1];
        } else {  // the next step's first fragment (its registers were loaded a step ago)
          d.w = (uint32_t)bq[u ^ 1][0][0];
          d.s16 = sq[u ^ 1][0][0][0];
          d.z = sq[u ^ 1][0][0][1];
        }
        if constexpr (!in_step) __syncthreads();  // every wave's writes of stage u ^ 1 are done
        static_for<0, RA>([&](auto I_) {
          constexpr int i = decltype(I_)::value;
          mfma_bf16_acc(acc[i][j], bcur, a[sub & 1][i]);
          if constexpr (i < 7) d.template piece<i>();
          if constexpr (in_step && jn == 0) readA(st, subn, i, a[subn & 1][i]);
          if constexpr (!in_step) readA(stn, 0, i, a[0][i]);  // substep 3 runs on a[1]
          // The step's memory work, one instruction group per MFMA slot: the
          // activation staging (each chunk written to stage u ^ 1, then its
          // register reloaded for step kt + 2) over the first groups, and each
          // weight fragment's refill for step kt + 2 once its last use (the
          // dequantisation of group 3 TJ + j, run during group 3 TJ + j - 1)
          // is behind.
          constexpr int slot = gg * RA + i;
          if constexpr (slot < NA) writeA1(u ^ 1, slot);
          if constexpr (slot >= NA && slot < 2 * NA) loadA1(kta, slot - NA);
          if constexpr (gg >= 3 * TJ && i == RA - 1) loadB1(kta, U_, gg - 3 * TJ);
          __builtin_amdgcn_sched_barrier(0);  // keep this placement: the scheduler would cluster the VALU
        });
        if constexpr (in_step) bcur = d.r;
        else bfirst = d.r;
      });
    });
  }
  W4_NOPS();
  W4_PIN();
#undef W4_PIN
#undef W4_NOPS
}

// y = bf16(acc) for one BM x 4 CW tile in the transposed accumulator layout
// (lane 16 g + r of fragment (i, j): token m0 + 16 i + r, columns n0 + wave CW +
// 16 j + 4 g .. + 3), 8-byte row pieces.
template <int BM, int CW>
__device__ __forceinline__ void w4pk_store(const f32x4 (&acc)[BM / 16][CW / 16], bf16_t* __restrict__ y,
                                           int64_t ldy, int M, int m0, int n0) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int j = 0; j < CW / 16; ++j) {
    const int col = n0 + wave * CW + 16 * j + 4 * g;
#pragma unroll
    for (int i = 0; i < BM / 16; ++i) {
      const int m = m0 + 16 * i + r16;
      if (m < M)
        *reinterpret_cast<u32x2*>(y + (int64_t)m * ldy + col) =
            pack4_bf16(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
    }
  }
}

// Plain y = bf16(x . W^T) with k split `splits` ways (pairs of k steps dealt
// evenly). With part null (then splits == 1) it stores y; otherwise each split
// stores its fp32 partial tile and a reduction adds them: ROWPART, row-major
// over the rows padded to whole tiles, part[(split Mp + row) N + col] (Mp =
// tiles_m BM; w4pk_reduce_kernel or the add_rms row kernel that takes the
// partials as its addend); else in accumulator order (f32x4 (i, j) of thread t
// at ((tile splits + split) RA TJ + i TJ + j) 256 + t; w4pk_qkv_kernel).
// SWIGLU: the weight is [gate (half rows); up (half rows)]; wave w takes gate
// channels [w CW/2, (w + 1) CW/2) of the tile's BN/2 and the matching up
// channels as fragments j = 2 t (gate) and 2 t + 1 (up), and stores
// h = bf16(bf16(silu(g)) * u) into y (M, half) with g, u = bf16(acc).
template <int BM, int CW, bool SWIGLU, bool ROWPART = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_w4a16_pk_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ wp, const float* __restrict__ sz,
    int gshift, bf16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int tiles_m, int tiles_n, int splits,
    f32x4* __restrict__ part) {
  constexpr int RA = BM / 16, TJ = CW / 16, BN = 4 * CW, CH = BN / 2, WCH = CW / 2;
  constexpr int SMEM = 2 * BM * 256;
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(!SWIGLU || TJ % 2 == 0, "gate/up fragment pairs");
  __shared__ __align__(1024) uint8_t smem[SMEM];
  __shared__ uint16_t silu_tab[SWIGLU ? kSiluEntries : 1];  // bf16(silu(g)) by g (silu_bf16)

  const int nblk = tiles_m * tiles_n * splits;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;  // one XCD walks a tile range
  const int tm = logical % tiles_m, rest = logical / tiles_m;                 // M fastest: L2 shares weights
  const int split = rest % splits, tn = rest / splits;
  const int m0 = tm * BM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int KT = K / kPkStep, kp = KT / 2;
  const int p0 = (int)((int64_t)kp * split / splits), p1 = (int)((int64_t)kp * (split + 1) / splits);
  const int half = N / 2;

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t sB[TJ], colS[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int row = SWIGLU ? (j & 1 ? half : 0) + tn * CH + wave_s * WCH + 16 * (j >> 1)
                           : tn * BN + wave_s * CW + 16 * j;
    sB[j] = (uint32_t)(row / 16) * 1024u;
    colS[j] = (uint32_t)(row + r16);
  }
  f32x4 acc[RA][TJ];
  w4pk_mainloop<BM, CW>(acc, smem, x, ldx, M, m0, wp, (uint32_t)((int64_t)N * K / 2), sB, sz,
                        (uint32_t)((int64_t)(K >> gshift) * N * 8), colS, N, gshift, 2 * p0, 2 * (p1 - p0), [&] {
                          if constexpr (SWIGLU) silu_table_fill<kThreads>(silu_tab, tid);
                        });

  if constexpr (SWIGLU) {
    // Every g of the tile and its table read first (all in flight before the
    // first result is needed), then h.
    const int c_base = tn * CH + wave * WCH + 4 * g;
    uint32_t gp[RA][TJ / 2][2], tv[RA][TJ / 2][4];
#pragma unroll
    for (int i = 0; i < RA; ++i)
#pragma unroll
      for (int t = 0; t < TJ / 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const uint32_t p = pack_bf16x2(acc[i][2 * t][r], acc[i][2 * t][r + 1]);
          gp[i][t][r / 2] = p;
          tv[i][t][r] = silu_bf16_read(p & 0xFFFFu, silu_tab);
          tv[i][t][r + 1] = silu_bf16_read(p >> 16, silu_tab);
        }
#pragma unroll
    for (int i = 0; i < RA; ++i) {
      const int m = m0 + 16 * i + r16;
#pragma unroll
      for (int t = 0; t < TJ / 2; ++t) {
        float hv[4];
        const uint32_t up[2] = {pack_bf16x2(acc[i][2 * t + 1][0], acc[i][2 * t + 1][1]),
                                pack_bf16x2(acc[i][2 * t + 1][2], acc[i][2 * t + 1][3])};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t gb = r & 1 ? gp[i][t][r / 2] >> 16 : gp[i][t][r / 2] & 0xFFFFu;
          const float uv = r & 1 ? __uint_as_float(up[r / 2] & 0xFFFF0000u) : __uint_as_float(up[r / 2] << 16);
          hv[r] = silu_bf16_finish(gb, tv[i][t][r]) * uv;  // rounded by the store's pack
        }
        if (m < M)
          *reinterpret_cast<u32x2*>(y + (int64_t)m * ldy + c_base + 16 * t) = pack4_bf16(hv[0], hv[1], hv[2], hv[3]);
      }
    }
  } else {
    if (part != nullptr && ROWPART) {
      store_tile_rows_lds<BM, CW, SMEM>(acc, smem,
                                        reinterpret_cast<float*>(part) + ((int64_t)split * tiles_m * BM + m0) * N +
                                            tn * BN,
                                        N, tid);
    } else if (part != nullptr) {
      f32x4* mine = part + ((int64_t)(tn * tiles_m + tm) * splits + split) * (RA * TJ * kThreads) + tid;
#pragma unroll
      for (int i = 0; i < RA; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) mine[(i * TJ + j) * kThreads] = acc[i][j];
    } else {
      w4pk_store<BM, CW>(acc, y, ldy, M, m0, tn * BN);
    }
  }
}

// y = bf16(sum of the splits' row-major partials) for rows < M, added in split
// order 0, 1, .. (whatever order the splits finished in); one thread per 8
// columns.
__global__ __launch_bounds__(kThreads) void w4pk_reduce_kernel(const float* __restrict__ part, int splits, int64_t mp,
                                                               bf16_t* __restrict__ y, int64_t ldy, int M, int N) {
  const int nc = N / 8;
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int m = (int)(e / nc), col = (int)(e % nc) * 8;
  if (m >= M) return;
  const float* src = part + (int64_t)m * N + col;
  f32x4 t0 = *reinterpret_cast<const f32x4*>(src), t1 = *reinterpret_cast<const f32x4*>(src + 4);
  for (int s2 = 1; s2 < splits; ++s2) {
    const float* p = src + (int64_t)s2 * mp * N;
    t0 = t0 + *reinterpret_cast<const f32x4*>(p);
    t1 = t1 + *reinterpret_cast<const f32x4*>(p + 4);
  }
  const float f[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
  *reinterpret_cast<u32x4*>(y + (int64_t)m * ldy + col) = pack8(f);
}

// Rows m <= 4 (the pick-only tail) on the packed copies: a workgroup of 4 waves
// owns 16 weight rows (one fragment row block; SWIGLU: 16 gate rows and the 16
// matching up rows) and its waves take every 4th 128-k step. Lane (g, r)
// dequantises its 32 nibbles of the fragment to the bf16 weights the tile
// kernels use (dequant8_off) and accumulates their products with the bf16 x
// pairs on v_dot2_f32_bf16 in fp32; the 4 lanes of a row, then the 4 waves in
// order, are added at the end and rounded to bf16 (SWIGLU: h = bf16(bf16(silu(
// bf16(g))) * bf16(u))). Only the fp32 order of the sum differs from the tile
// kernels.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a), __builtin_bit_cast(bf16x2v, b), c, false);
}

template <int M, bool SWIGLU>
__global__ __launch_bounds__(kThreads) void gemv_w4pk_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                             const uint8_t* __restrict__ wp,
                                                             const float* __restrict__ fs, int gshift,
                                                             bf16_t* __restrict__ y, int64_t ldy, int N, int K) {
  constexpr int NF = SWIGLU ? 2 : 1;  // fragments per k step: the rows (gate), and the up rows
  __shared__ float red[4][NF][M][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int KT = K / kPkStep;
  const int half = N / 2;
  int rowb[NF];
  rowb[0] = 16 * blockIdx.x;
  if constexpr (SWIGLU) rowb[NF - 1] = half + 16 * blockIdx.x;
  const __amdgpu_buffer_rsrc_t rX = make_rsrc(x, (uint32_t)((int64_t)M * ldx * 2));
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(wp, (uint32_t)((int64_t)N * K / 2));
  const __amdgpu_buffer_rsrc_t rS = make_rsrc(fs, (uint32_t)((int64_t)(K >> gshift) * N * 8));
  float acc[NF][M];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[f][m] = 0.f;
  for (int kt = wave; kt < KT; kt += 4) {
    i32x4v xv[M][2][2];  // row m, half h, 8 k each: k = 128 kt + 64 h + 16 g + [0, 16)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          xv[m][h][c] = bload16(rX, (uint32_t)(m * ldx + kPkStep * kt + 64 * h + 16 * g + 8 * c) * 2u, 0);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const i32x4v w = bload16(rB, 16u * (uint32_t)lane, (uint32_t)(kt * (N / 16) + rowb[f] / 16) * 1024u);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t gi = (uint32_t)(kPkStep * kt + 64 * h + 16 * g) >> gshift;
        const i32x2v sz = bload8(rS, (gi * (uint32_t)N + (uint32_t)(rowb[f] + r16)) * 8u, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const u32x4 b = dequant8_off((uint32_t)w[2 * h + t], __int_as_float(sz.x), __int_as_float(sz.y));
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const i32x4v xx = xv[m][h][t];
            acc[f][m] = dot2_bf16(b.x, (uint32_t)xx.x, acc[f][m]);
            acc[f][m] = dot2_bf16(b.y, (uint32_t)xx.y, acc[f][m]);
            acc[f][m] = dot2_bf16(b.z, (uint32_t)xx.z, acc[f][m]);
            acc[f][m] = dot2_bf16(b.w, (uint32_t)xx.w, acc[f][m]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = acc[f][m];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (g == 0) red[wave][f][m][r16] = v;
    }
  __syncthreads();
  if (tid < 16 * M) {
    const int m = tid / 16, r = tid % 16;
    float sum[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) sum[f] = ((red[0][f][m][r] + red[1][f][m][r]) + red[2][f][m][r]) + red[3][f][m][r];
    float out = sum[0];
    if constexpr (SWIGLU) out = round_bf16(round_bf16(silu(round_bf16(sum[0]))) * round_bf16(sum[NF - 1]));
    y[(int64_t)m * ldy + 16 * blockIdx.x + r] = (bf16_t)f32_to_bf16(out);
  }
}

template <bool SWIGLU>
void launch_gemv_w4pk(const void* x, int64_t ldx, const void* frag, const void* fscales, int gshift, void* y,
                      int64_t ldy, int m, int n, int k, hipStream_t s) {
  const int blocks = SWIGLU ? n / 32 : n / 16;
#define FF_GEMV_W4(MM)                                                                                          \
  case MM:                                                                                                      \
    hipLaunchKernelGGL((gemv_w4pk_kernel<MM, SWIGLU>), dim3((unsigned)blocks), dim3(kThreads), 0, s,             \
                       (const bf16_t*)x, ldx, (const uint8_t*)frag, (const float*)fscales, gshift, (bf16_t*)y, ldy, \
                       n, k);                                                                                   \
    break;
  switch (m) { FF_GEMV_W4(1) FF_GEMV_W4(2) FF_GEMV_W4(3) FF_GEMV_W4(4) }
#undef FF_GEMV_W4
}

// Shapes the packed GEMV takes: 1 <= m <= 4, n % 16 (SWIGLU: the 2 i rows,
// i % 16), k % 128, a power-of-two group >= 32 dividing k.
bool w4pk_gemv_fits(int64_t m, int64_t n, int64_t k, int64_t group) {
  return m >= 1 && m <= 4 && n > 0 && n % 16 == 0 && k % kPkStep == 0 && group >= 32 && (group & (group - 1)) == 0 &&
         k % group == 0 && n * k / 2 < (int64_t(1) << 31) && (k / group) * n * 8 < (int64_t(1) << 31) &&
         k < (1 << 24);
}

// Plans of the packed path. Plain: 144 x 384 tiles (CW 96) when they fill the
// GPU unsplit; otherwise 144 x 256 tiles (CW 64) with k split until about one
// workgroup per CU (at most 8 ways, at least one pair of k steps each). SwiGLU:
// 144 x (192 gate + 192 up) tiles when the channels divide, else 144 x (128 +
// 128). Shapes outside the packed path's limits are reported as not fitting.
constexpr int kW4BM = 144;

struct W4PkPlan {
  int cw = 0;      // 0: the packed path does not take this shape
  int splits = 1;
};

bool w4pk_common_fits(int64_t m, int64_t k, int64_t group) {
  return m > 4 && k % (2 * kPkStep) == 0 && group >= 32 && (group & (group - 1)) == 0 && k % group == 0 &&
         m < (1 << 24) && k < (1 << 24);
}

int w4_gshift(int64_t group) {
  int s = 0;
  while ((int64_t(1) << s) < group) ++s;
  return s;
}

W4PkPlan w4pk_plan(int64_t m, int64_t n, int64_t k, int64_t group) {
  W4PkPlan p;
  if (!w4pk_common_fits(m, k, group) || n % 16 || n * k / 2 >= (int64_t(1) << 31) ||
      (k / group) * n * 8 >= (int64_t(1) << 31) || m * k * 2 >= (int64_t(1) << 31))
    return p;
  const int64_t tm = (m + kW4BM - 1) / kW4BM;
  if (n % 384 == 0 && tm * (n / 384) >= 192) {
    p.cw = 96;
    return p;
  }
  if (n % 256) return p;
  const int64_t tiles = tm * (n / 256), pairs = k / (2 * kPkStep);
  int64_t s = 1;
  if (const int f = ff_tuning(FF_TUNE_W4A16_SPLITS)) s = f;
  else if (tiles < 192) s = 256 / tiles;
  p.cw = 64;
  p.splits = (int)std::max<int64_t>(1, std::min<int64_t>({s, 8, pairs}));
  return p;
}

int w4pk_swiglu_cw(int64_t m, int64_t i, int64_t k, int64_t group) {
  if (!w4pk_common_fits(m, k, group) || 2 * i * k / 2 >= (int64_t(1) << 31) ||
      (k / group) * 2 * i * 8 >= (int64_t(1) << 31) || m * k * 2 >= (int64_t(1) << 31))
    return 0;
  if (i % 192 == 0) return 96;
  if (i % 128 == 0) return 64;
  return 0;
}

int64_t w4pk_workspace(int64_t m, int64_t n, int64_t k, int64_t group) {
  const W4PkPlan p = w4pk_plan(m, n, k, group);
  if (p.cw == 0 || p.splits <= 1) return 0;
  return (m + kW4BM - 1) / kW4BM * (n / (4 * p.cw)) * p.splits * kW4BM * 4 * p.cw * 4;
}

// Row-tile height of the packed SwiGLU GEMM with 96-channel wave tiles: 160
// where it keeps the grid in one round of 256 workgroups that 144 would spill
// into a second (the 8B gate/up at 577..640 and 1153..1280 tokens), counted as
// rounds x (BM + 16) rows per CU; 144 otherwise. 160 rows is the most the
// accumulators fit (240 of 256 AGPRs), and the main loop needs at least 144.
int w4_swiglu_bm(int64_t m, int64_t tiles_n) {
  const auto cost = [&](int bm) { return ((m + bm - 1) / bm * tiles_n + 255) / 256 * (bm + 16); };
  return cost(160) < cost(kW4BM) ? 160 : kW4BM;
}

template <int CW, bool SWIGLU, int BM = kW4BM>
void launch_w4pk(const void* x, int64_t ldx, const void* frag, const void* fscales, int gshift, void* y, int64_t ldy,
                 int m, int n, int k, int splits, void* ws, hipStream_t s) {
  const int tiles_m = (m + BM - 1) / BM;
  const int tiles_n = n / (4 * CW);  // SWIGLU: n = 2 half rows, 2 CW channels of each half per tile
  hipLaunchKernelGGL((gemm_w4a16_pk_kernel<BM, CW, SWIGLU, !SWIGLU>), dim3((unsigned)(tiles_m * tiles_n * splits)),
                     dim3(kThreads), 0, s, (const bf16_t*)x, ldx, (const uint8_t*)frag, (const float*)fscales,
                     gshift, (bf16_t*)y, ldy, m, n, k, tiles_m, tiles_n, splits,
                     !SWIGLU && splits > 1 ? (f32x4*)ws : nullptr);
  if (!SWIGLU && splits > 1 && y != nullptr) {
    const int64_t chunks = (int64_t)m * (n / 8);
    hipLaunchKernelGGL(w4pk_reduce_kernel, dim3((unsigned)((chunks + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       (const float*)ws, splits, (int64_t)tiles_m * BM, (bf16_t*)y, ldy, m, n);
  }
}

}  // namespace

extern "C" int ff_pack_weight_int4(const void* packed, void* frag, int64_t n, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(packed && frag, "ff_pack_weight_int4: null pointer");
  FF_REQUIRE(n > 0 && n % 16 == 0 && k > 0 && k % kPkStep == 0 && n * k < (int64_t(1) << 40),
             "ff_pack_weight_int4: bad sizes (n %% 16, k %% 128)");
  FF_REQUIRE(ff_aligned(packed, 8) && ff_aligned(frag, 16), "ff_pack_weight_int4: alignment");
  const int64_t lanes = (n / 16) * (k / kPkStep) * 64;
  const int64_t blocks = (lanes + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(pack_int4_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)packed, (uint8_t*)frag, n, k);
  FF_LAUNCH_CHECK("ff_pack_weight_int4");
  return FF_OK;
}

namespace {

// (s, z) bf16 pairs -> (16 s, z) fp32 pairs, same [k/group, n] order.
__global__ __launch_bounds__(kThreads) void pack_scales_int4_kernel(const uint32_t* __restrict__ sz,
                                                                    float* __restrict__ out, int64_t pairs) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < pairs; i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t v = sz[i];
    out[2 * i] = 16.f * bf16_to_f32(v & 0xFFFFu);
    out[2 * i + 1] = __uint_as_float(v & 0xFFFF0000u);
  }
}

}  // namespace

extern "C" int ff_pack_scales_int4(const void* scales, void* frag_scales, int64_t n, int64_t k, int64_t group,
                                   ff_stream_t stream) {
  FF_REQUIRE(scales && frag_scales, "ff_pack_scales_int4: null pointer");
  FF_REQUIRE(n > 0 && k > 0 && group > 0 && k % group == 0 && (k / group) * n < (int64_t(1) << 40),
             "ff_pack_scales_int4: bad sizes");
  FF_REQUIRE(ff_aligned(scales, 4) && ff_aligned(frag_scales, 8), "ff_pack_scales_int4: alignment");
  const int64_t pairs = (k / group) * n, blocks = (pairs + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(pack_scales_int4_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint32_t*)scales, (float*)frag_scales, pairs);
  FF_LAUNCH_CHECK("ff_pack_scales_int4");
  return FF_OK;
}

extern "C" int ff_gemm_w4a16_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t group, int64_t* bytes) {
  FF_REQUIRE(bytes && m >= 0 && n > 0 && k > 0 && group > 0, "ff_gemm_w4a16_pk_workspace: bad arguments");
  int64_t other = 0;
  ff_gemm_w4a16_workspace(m, n, k, &other);
  *bytes = std::max(w4pk_workspace(m, n, k, group), other);
  return FF_OK;
}

namespace ff {
int gemm_w4a16_pk_partials(const void* x, int64_t ldx, const void* frag, const void* frag_scales, int64_t group,
                           int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, hipStream_t st,
                           int* splits, int64_t* mp) {
  *splits = 0;
  *mp = 0;
  if (!frag || !frag_scales || w4pk_gemv_fits(m, n, k, group)) return FF_OK;
  const W4PkPlan p = w4pk_plan(m, n, k, group);
  if (p.cw != 64 || p.splits <= 1 || ldx % 8 || ldx < k || m * ldx * 2 >= (int64_t(1) << 31) || !ff_aligned(x, 16) ||
      !ff_aligned(frag, 16) || !ff_aligned(frag_scales, 8))
    return FF_OK;
  const int64_t need = w4pk_workspace(m, n, k, group);
  FF_REQUIRE(workspace && workspace_bytes >= need && ff_aligned(workspace, 16),
             "ff_gemm_w4a16_pk: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  launch_w4pk<64, false>(x, ldx, frag, frag_scales, w4_gshift(group), nullptr, 0, (int)m, (int)n, (int)k, p.splits,
                         workspace, st);
  FF_LAUNCH_CHECK("ff_gemm_w4a16_pk");
  *splits = p.splits;
  *mp = (m + kW4BM - 1) / kW4BM * kW4BM;
  return FF_OK;
}
}  // namespace ff

extern "C" int ff_gemm_w4a16_pk(const void* x, int64_t ldx, const void* packed, const void* frag, const void* scales,
                                const void* frag_scales, int64_t group, void* y, int64_t ldy, int64_t m, int64_t n,
                                int64_t k, void* workspace, int64_t workspace_bytes, ff_stream_t stream) {
  if (frag && frag_scales && w4pk_gemv_fits(m, n, k, group) && ldx % 8 == 0 && ldx >= k && ldy >= n &&
      m * ldx * 2 < (int64_t(1) << 31) && ff_aligned(x, 16) && ff_aligned(frag, 16) && ff_aligned(frag_scales, 8) &&
      ff_aligned(y, 2)) {
    FF_REQUIRE(y, "ff_gemm_w4a16_pk: null pointer");
    launch_gemv_w4pk<false>(x, ldx, frag, frag_scales, w4_gshift(group), y, ldy, (int)m, (int)n, (int)k,
                            (hipStream_t)stream);
    FF_LAUNCH_CHECK("ff_gemm_w4a16_pk");
    return FF_OK;
  }
  const W4PkPlan p = frag && frag_scales ? w4pk_plan(m, n, k, group) : W4PkPlan{};
  if (p.cw == 0 || ldx % 8 || ldy % 8 || ldx < k || ldy < n || m * ldx * 2 >= (int64_t(1) << 31) ||
      !ff_aligned(x, 16) || !ff_aligned(frag, 16) || !ff_aligned(frag_scales, 8) || !ff_aligned(y, 8))
    return gemm_w4a16(x, ldx, packed, scales, group, y, ldy, m, n, k, workspace, workspace_bytes, stream);
  const int64_t need = w4pk_workspace(m, n, k, group);
  FF_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && ff_aligned(workspace, 16)),
             "ff_gemm_w4a16_pk: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  const hipStream_t s = (hipStream_t)stream;
  const int gs = w4_gshift(group);
  if (p.cw == 96)
    launch_w4pk<96, false>(x, ldx, frag, frag_scales, gs, y, ldy, (int)m, (int)n, (int)k, 1, nullptr, s);
  else
    launch_w4pk<64, false>(x, ldx, frag, frag_scales, gs, y, ldy, (int)m, (int)n, (int)k, p.splits, workspace, s);
  FF_LAUNCH_CHECK("ff_gemm_w4a16_pk");
  return FF_OK;
}

extern "C" int ff_gemm_w4a16_swiglu_fits(int64_t m, int64_t i, int64_t k, int64_t group, int* fits) {
  FF_REQUIRE(fits, "ff_gemm_w4a16_swiglu_fits: null pointer");
  *fits = w4pk_swiglu_cw(m, i, k, group) != 0 || (i % 16 == 0 && w4pk_gemv_fits(m, 2 * i, k, group));
  return FF_OK;
}

extern "C" int ff_gemm_w4a16_swiglu_pk(const void* x, int64_t ldx, const void* frag, const void* frag_scales,
                                       int64_t group, void* h, int64_t ldh, int64_t m, int64_t i, int64_t k,
                                       ff_stream_t stream) {
  FF_REQUIRE(x && frag && frag_scales && h, "ff_gemm_w4a16_swiglu_pk: null pointer");
  const int cw = w4pk_swiglu_cw(m, i, k, group);
  const bool gemv = cw == 0 && i % 16 == 0 && w4pk_gemv_fits(m, 2 * i, k, group);
  FF_REQUIRE(cw != 0 || gemv, "ff_gemm_w4a16_swiglu_pk: m=%lld i=%lld k=%lld group=%lld is outside the fused "
             "kernels' shapes (m > 4: i %% 128, k %% 256; m <= 4: i %% 16, k %% 128; group a power of two >= 32 "
             "dividing k)", (long long)m, (long long)i, (long long)k, (long long)group);
  FF_REQUIRE(ldx % 8 == 0 && ldx >= k && ldh % 4 == 0 && ldh >= i && m * ldx * 2 < (int64_t(1) << 31),
             "ff_gemm_w4a16_swiglu_pk: bad strides");
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(frag, 16) && ff_aligned(frag_scales, 8) && ff_aligned(h, 8),
             "ff_gemm_w4a16_swiglu_pk: alignment (x, frag 16 bytes; frag_scales, h 8)");
  const hipStream_t s = (hipStream_t)stream;
  const int gs = w4_gshift(group);
  if (gemv)
    launch_gemv_w4pk<true>(x, ldx, frag, frag_scales, gs, h, ldh, (int)m, (int)(2 * i), (int)k, s);
  else if (cw == 96 && w4_swiglu_bm(m, 2 * i / 384) == 160)
    launch_w4pk<96, true, 160>(x, ldx, frag, frag_scales, gs, h, ldh, (int)m, (int)(2 * i), (int)k, 1, nullptr, s);
  else if (cw == 96)
    launch_w4pk<96, true>(x, ldx, frag, frag_scales, gs, h, ldh, (int)m, (int)(2 * i), (int)k, 1, nullptr, s);
  else
    launch_w4pk<64, true>(x, ldx, frag, frag_scales, gs, h, ldh, (int)m, (int)(2 * i), (int)k, 1, nullptr, s);
  FF_LAUNCH_CHECK("ff_gemm_w4a16_swiglu_pk");
  return FF_OK;
}

// ------------------------------------------------------------------ fused QKV
//
// ff_gemm_w4a16_qkv: the packed GEMM of the QKV weight on 144 x 256 tiles (two
// heads of 128 per tile), its fp32 partials always going to the workspace, then
// w4pk_qkv_kernel per (tile, 16-token group): the partials added in split
// order and rounded to bf16 (the values of ff_gemm_w4a16_pk), staged in LDS,
// then q/k heads through the per-head RMSNorm + rotary of qk_pair (rope_row_pre,
// the routine of ff_qkv_post) stored head-major, v heads stored transposed
// (hk, 128, t_pad) with zeros for tokens >= m.

namespace {

struct W4Qkv {
  const bf16_t* qn;  // q_norm weight (128)
  const bf16_t* kn;  // k_norm weight (128)
  float eps_q, eps_k;
  const bf16_t* cos;  // (m, 128)
  const bf16_t* sin;
  bf16_t* yq;  // (hq, m, 128)
  bf16_t* yk;  // (hk, m, 128)
  bf16_t* vt;  // (hk, 128, t_pad)
  int hq, hk, t_pad;
};

template <int BM>
__global__ __launch_bounds__(kThreads) void w4pk_qkv_kernel(const f32x4* __restrict__ part, int splits, int M,
                                                            int tiles_m, W4Qkv qe) {
  constexpr int CW = 64, RA = BM / 16, TJ = CW / 16, BN = 4 * CW, LD = BN + 8;
  __shared__ __align__(16) bf16_t tile[16 * LD];
  const int t_idx = blockIdx.x / RA, i = blockIdx.x % RA;
  const int tm = t_idx % tiles_m, tn = t_idx / tiles_m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int m0 = tm * BM + 16 * i;
  const f32x4* tp = part + (int64_t)t_idx * splits * (RA * TJ * kThreads) + i * TJ * kThreads + tid;
  f32x4 t[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) t[j] = tp[j * kThreads];
  for (int s2 = 1; s2 < splits; ++s2)
#pragma unroll
    for (int j = 0; j < TJ; ++j) t[j] = t[j] + tp[((int64_t)s2 * RA * TJ + j) * kThreads];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
    *reinterpret_cast<u32x2*>(tile + r16 * LD + wave * CW + 16 * j + 4 * g) =
        pack4_bf16(t[j][0], t[j][1], t[j][2], t[j][3]);
  __syncthreads();
  const int head0 = tn * 2;
  // q / k rows: 16-lane group grp takes token grp of both heads (as ff_qkv_post)
  const int grp = tid >> 4, jl = tid & 15;
#pragma unroll
  for (int hl = 0; hl < 2; ++hl) {
    const int head = head0 + hl;
    if (head >= qe.hq + qe.hk) continue;
    const bool isq = head < qe.hq;
    const int m = m0 + grp;
    const bool valid = m < M;
    const int mm = valid ? m : M - 1;
    float wv[8];
    unpack8(*reinterpret_cast<const u32x4*>((isq ? qe.qn : qe.kn) + 8 * jl), wv);
    const u32x4 cs = *reinterpret_cast<const u32x4*>(qe.cos + (size_t)mm * kHeadDim + 8 * jl);
    const u32x4 sn = *reinterpret_cast<const u32x4*>(qe.sin + (size_t)mm * kHeadDim + 8 * jl);
    bf16_t* dst = (isq ? qe.yq + (size_t)head * M * kHeadDim : qe.yk + (size_t)(head - qe.hq) * M * kHeadDim) +
                  (size_t)mm * kHeadDim;
    rope_row_pre(tile + grp * LD + hl * kHeadDim, wv, isq ? qe.eps_q : qe.eps_k, cs, sn, dst, jl, valid);
  }
  // v heads: thread (d, token half) writes 8 consecutive tokens of row d
#pragma unroll
  for (int hl = 0; hl < 2; ++hl) {
    const int head = head0 + hl;
    if (head < qe.hq + qe.hk) continue;
    const int hv = head - qe.hq - qe.hk;
    const int d = tid >> 1, t0 = 8 * (tid & 1);
    const int tok = m0 + t0;
    if (tok >= qe.t_pad) continue;
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = tok + e < M ? bf16_to_f32(tile[(t0 + e) * LD + hl * kHeadDim + d]) : 0.f;
    *reinterpret_cast<u32x4*>(qe.vt + ((size_t)hv * kHeadDim + d) * qe.t_pad + tok) = pack8(f);
  }
}

// vt[:, :, t0 .. t_pad) = 0 for the tokens no tile covers (t_pad > tiles_m * BM).
__global__ __launch_bounds__(kThreads) void vt_zero_tail_kernel(bf16_t* __restrict__ vt, int rows, int t_pad,
                                                                int t0) {
  const int64_t n = (int64_t)rows * (t_pad - t0);
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    vt[(i / (t_pad - t0)) * t_pad + t0 + i % (t_pad - t0)] = 0;
}

// Splits of the QKV GEMM: the 144 x 256 tiles of w4pk_plan, k split until
// about one workgroup per CU.
int w4pk_qkv_splits(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles = (m + kW4BM - 1) / kW4BM * (n / 256), pairs = k / (2 * kPkStep);
  int64_t s = tiles >= 192 ? 1 : 256 / tiles;
  if (const int f = ff_tuning(FF_TUNE_W4A16_SPLITS)) s = f;
  return (int)std::max<int64_t>(1, std::min<int64_t>({s, 8, pairs}));
}

bool w4pk_qkv_fits(int64_t m, int64_t k, int64_t hq, int64_t hk, int64_t group) {
  const int64_t n = (hq + 2 * hk) * kHeadDim;
  return w4pk_common_fits(m, k, group) && hq > 0 && hk > 0 && n % 256 == 0 && n * k / 2 < (int64_t(1) << 31) &&
         (k / group) * n * 8 < (int64_t(1) << 31) && m * k * 2 < (int64_t(1) << 31);
}

}  // namespace

extern "C" int ff_gemm_w4a16_qkv_workspace(int64_t m, int64_t k, int64_t hq, int64_t hk, int64_t group,
                                           int64_t* bytes) {
  FF_REQUIRE(bytes && m >= 0 && k > 0 && hq > 0 && hk > 0 && group > 0, "ff_gemm_w4a16_qkv_workspace: bad arguments");
  const int64_t n = (hq + 2 * hk) * kHeadDim;
  *bytes = w4pk_qkv_fits(m, k, hq, hk, group)
               ? (m + kW4BM - 1) / kW4BM * (n / 256) * w4pk_qkv_splits(m, n, k) * kW4BM * 256 * 4
               : 0;
  return FF_OK;
}

extern "C" int ff_gemm_w4a16_qkv(const void* x, int64_t ldx, const void* frag, const void* frag_scales, int64_t group,
                                 int64_t m, int64_t k, int64_t hq, int64_t hk, const void* q_norm, const void* k_norm,
                                 float eps_q, float eps_k, const void* cos, const void* sin, void* yq, void* yk,
                                 void* vt, int64_t t_pad, void* workspace, int64_t workspace_bytes,
                                 ff_stream_t stream) {
  FF_REQUIRE(x && frag && frag_scales && q_norm && k_norm && cos && sin && yq && yk && vt,
             "ff_gemm_w4a16_qkv: null pointer");
  FF_REQUIRE(w4pk_qkv_fits(m, k, hq, hk, group),
             "ff_gemm_w4a16_qkv: m=%lld k=%lld hq=%lld hk=%lld group=%lld outside the kernel's shapes (m > 4, "
             "k %% 256, 2 (hq + 2 hk) heads per 256 columns, group a power of two >= 32 dividing k)",
             (long long)m, (long long)k, (long long)hq, (long long)hk, (long long)group);
  FF_REQUIRE(ldx % 8 == 0 && ldx >= k && m * ldx * 2 < (int64_t(1) << 31) && t_pad >= m && t_pad % 64 == 0 &&
                 t_pad < (1 << 30),
             "ff_gemm_w4a16_qkv: bad strides or t_pad");
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(frag, 16) && ff_aligned(frag_scales, 8) && ff_aligned(q_norm, 16) &&
                 ff_aligned(k_norm, 16) && ff_aligned(cos, 16) && ff_aligned(sin, 16) && ff_aligned(yq, 16) &&
                 ff_aligned(yk, 16) && ff_aligned(vt, 16),
             "ff_gemm_w4a16_qkv: operands must be 16-byte aligned");
  int64_t need = 0;
  ff_gemm_w4a16_qkv_workspace(m, k, hq, hk, group, &need);
  FF_REQUIRE(workspace && workspace_bytes >= need && ff_aligned(workspace, 16),
             "ff_gemm_w4a16_qkv: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  const int64_t n = (hq + 2 * hk) * kHeadDim;
  const int splits = w4pk_qkv_splits(m, n, k);
  const int tiles_m = (int)((m + kW4BM - 1) / kW4BM), tiles_n = (int)(n / 256);
  const hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL((gemm_w4a16_pk_kernel<kW4BM, 64, false>), dim3((unsigned)(tiles_m * tiles_n * splits)),
                     dim3(kThreads), 0, s, (const bf16_t*)x, ldx, (const uint8_t*)frag, (const float*)frag_scales,
                     w4_gshift(group), nullptr, 0, (int)m, (int)n, (int)k, tiles_m, tiles_n, splits,
                     (f32x4*)workspace);
  const W4Qkv qe{(const bf16_t*)q_norm, (const bf16_t*)k_norm, eps_q, eps_k, (const bf16_t*)cos,
                 (const bf16_t*)sin, (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)vt, (int)hq, (int)hk, (int)t_pad};
  hipLaunchKernelGGL((w4pk_qkv_kernel<kW4BM>), dim3((unsigned)(tiles_m * tiles_n * (kW4BM / 16))), dim3(kThreads),
                     0, s, (const f32x4*)workspace, splits, (int)m, tiles_m, qe);
  const int covered = tiles_m * kW4BM;
  if (t_pad > covered)
    hipLaunchKernelGGL(vt_zero_tail_kernel, dim3(64), dim3(kThreads), 0, s, (bf16_t*)vt, (int)(hk * kHeadDim),
                       (int)t_pad, covered);
  FF_LAUNCH_CHECK("ff_gemm_w4a16_qkv");
  return FF_OK;
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
  // the workspace entry point's own size, so both take the same split
  int64_t need = 0;
  const int rc = ff_gemm_w4a16_workspace(m, n, k, &need);
  if (rc != FF_OK) return rc;
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
