// Shared device helpers for the gfx950 kernels: rounding to bf16 / e4m3fn,
// 16-byte vector types, wave64 reductions and the C-ABI status plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/ff_amd.h"

namespace ff {

typedef uint16_t bf16_t;  // raw bf16 bits

struct __align__(16) u32x4 { uint32_t x, y, z, w; };
struct __align__(8) u32x2 { uint32_t x, y; };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ LDS DMA pipelines
//
// global_load_lds_dwordx4 copies 16 bytes per lane from global memory into LDS
// at M0 + 16*lane with no register round trip. It is issued from inline asm so
// that the compiler's wait-count pass does not track it: that pass otherwise
// waits for every such load before the next LDS read it cannot prove disjoint,
// and __syncthreads() (a workgroup fence) waits for all of them as well, which
// collapses a multi-stage pipeline to one stage. Kernels that use lds_dma16
// wait for their own loads with wait_vmcnt<N>() (loads complete in issue
// order) and synchronise with barrier_lds().

// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// lds (wave-uniform) receives 16 bytes from src of every lane, lane l at lds + 16*l.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds)
               : "memory", "m0");
}

// The 4-byte form: lane l's dword lands at lds + 4 l.
__device__ __forceinline__ void lds_dma4(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(src), "s"(lds)
               : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without a memory fence; this wave's LDS reads complete first.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

// ------------------------------------------------------------------ buffer loads

typedef int i32x4v __attribute__((ext_vector_type(4)));

// Raw buffer resource over `bytes` bytes (stride 0, 32-bit data format); loads
// beyond the range return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 / 8 / 4 bytes at byte offset voff + soff of the resource; ordinary
// compiler-visible loads, so the compiler's wait counts are exact.
__device__ __forceinline__ i32x4v bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}
typedef int i32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ i32x2v bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// f(integral_constant<int, I>) for I = B .. N-1, unrolled at compile time.
template <int B, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < N) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, N>(f);
  }
}

// A BM x 4 CW fp32 accumulator tile of 256 threads (lane 16 g + r of wave w,
// fragment (i, j): row 16 i + r, columns w CW + 16 j + 4 g .. + 3) stored
// row-major at dst (row stride ld floats) through the workgroup's LDS (SMEM
// bytes at smem), a group of 16-row blocks at a time, so that every store
// instruction writes whole row segments instead of 64 bytes to each of 16
// rows. Called by every thread; it opens with a barrier, so the caller's LDS
// may still be in use when it is called.
template <int BM, int CW, int SMEM>
__device__ __forceinline__ void store_tile_rows_lds(const f32x4 (&acc)[BM / 16][CW / 16], uint8_t* smem, float* dst,
                                                    int64_t ld, int tid) {
  constexpr int RA = BM / 16, TJ = CW / 16, BN = 4 * CW;
  constexpr int LDW = BN + 4;  // floats per staged row; the pad spreads the rows over the banks
  constexpr int GR = SMEM / (16 * LDW * 4);
  static_assert(GR >= 1, "one 16-row group fits the LDS");
  float* stg = reinterpret_cast<float*>(smem);
  const int lane = tid & 63, wave = tid >> 6;
  float* mine = stg + (lane & 15) * LDW + wave * CW + 4 * (lane >> 4);
  static_for<0, (RA + GR - 1) / GR>([&](auto R_) {
    constexpr int i0 = decltype(R_)::value * GR;
    constexpr int ng = RA - i0 < GR ? RA - i0 : GR;
    barrier_lds();  // the LDS (the caller's, or the previous group's) is no longer read
#pragma unroll
    for (int ii = 0; ii < ng; ++ii)
#pragma unroll
      for (int j = 0; j < TJ; ++j) *reinterpret_cast<f32x4*>(mine + ii * 16 * LDW + 16 * j) = acc[i0 + ii][j];
    barrier_lds();
#pragma unroll
    for (int e = tid; e < ng * 16 * (BN / 4); e += 256) {
      const int r = e / (BN / 4), c4 = e % (BN / 4);
      *reinterpret_cast<f32x4*>(dst + (int64_t)(16 * i0 + r) * ld + 4 * c4) =
          *reinterpret_cast<const f32x4*>(stg + r * LDW + 4 * c4);
    }
  });
}

// ------------------------------------------------------------------ bf16

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32; NaN stays a
// quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Round fp32 to the nearest bf16 value and return it as fp32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Unpack 8 bf16 (one 16-byte vector) into fp32.
__device__ __forceinline__ void unpack8(const u32x4 v, float* f) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xFFFF0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xFFFF0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xFFFF0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

// 4 bf16 (8 bytes) from 4 fp32 values, low to high.
__device__ __forceinline__ u32x2 pack4_bf16(float a, float b, float c, float d) {
  return u32x2{pack_bf16x2(a, b), pack_bf16x2(c, d)};
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
  v.x = pack_bf16x2(f[0], f[1]); v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]); v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// ------------------------------------------------------------------ e4m3fn

// fp32 -> OCP e4m3fn code, round to nearest even. |x| must already be clamped
// to <= 448 (the callers clamp, as the reference does before its cast). NaN maps
// to the NaN code with the sign kept; -0 and negative values that round to zero
// keep the sign bit. Normal range: drop 20 mantissa bits with RNE after
// re-biasing the exponent (127 -> 7); subnormal range (|x| < 2^-6): the code is
// rint(|x| * 2^9), which is exact scaling followed by RNE.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  uint32_t code;
  if (a > 0x7F800000u) {
    code = 0x7Fu;
  } else if (a >= 0x3C800000u) {
    uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
  } else {
    code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  }
  return sign | code;
}

__device__ __forceinline__ float clamp448(float v) {
  // fminf/fmaxf would drop a NaN; keep it so it encodes as NaN like torch's clamp.
  return v != v ? v : fminf(448.0f, fmaxf(-448.0f, v));
}

// x / d correctly rounded for d > 0, from r = 1/d correctly rounded: the
// product x*r is within an ulp of the quotient and one FMA residual step rounds
// it exactly (Markstein). The sign is taken from x, which keeps -0 / d = -0
// (the residual step would return +0). Quantisation divides a whole row by one
// scale, so the division is done once per row and this per element.
__device__ __forceinline__ float div_rcp(float x, float d, float r) {
  const float y = x * r;
  const float e = __builtin_fmaf(-y, d, x);
  return __builtin_copysignf(__builtin_fmaf(e, r, y), x);
}

// e4m3 codes of four values already clamped to [-448, 448], packed low to high,
// with v_cvt_pk_fp8_f32 (round to nearest even; the same codes as f32_to_e4m3
// for every fp32 value of that range).
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// SiLU as the reference writes it: g / (1 + exp(-g)), correctly rounded divide.
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// bf16(silu(g)) for a bf16 g, given as its 16 bits b, without evaluating exp
// and the divide per element: |g| in [2^-8, 128) (bits & 0x7FFF in [kSiluLo,
// kSiluHi)) reads a table of round_bf16(silu(g)) that silu_table_fill writes
// with the function above (one entry per bf16 value of that range and sign, so
// the result is the same bits by construction). Outside it:
// * |g| < 2^-8 (zero and subnormals included): exp(-g) is within 2^-8 of 1 and
//   silu(g) = g/2 (1 + g/2 + O(g^3)) is less than a quarter bf16 ulp from g/2,
//   so the result is round_bf16(g / 2);
// * |g| >= 128: for g > 0, 1 + exp(-g) rounds to 1 and the result is g; for
//   g < 0, exp(-g) overflows to inf and g / inf = -0 (NaN for g = -inf); both
//   are g * (g > 0 ? 1 : 0), and NaN stays NaN.
// Every bf16 pattern is compared with the exact form through the fused SwiGLU
// GEMM epilogues in the tests.
constexpr uint32_t kSiluLo = 0x3B80u, kSiluHi = 0x4300u, kSiluSpan = kSiluHi - kSiluLo;
constexpr int kSiluEntries = 2 * (int)kSiluSpan;  // positive g, then negative g

// NT threads (a divisor of kSiluEntries) fill the table; the entries of one
// thread are independent, so the unrolled loop overlaps their exp / divide
// latencies.
template <int NT>
__device__ __forceinline__ void silu_table_fill(uint16_t* tab, int tid) {
  static_assert(kSiluEntries % NT == 0, "whole rounds");
#pragma unroll
  for (int c = 0; c < kSiluEntries / NT; ++c) {
    const int e = tid + c * NT;
    const uint32_t neg = e >= (int)kSiluSpan;
    const uint32_t bits = (neg << 15) | (kSiluLo + (uint32_t)e - neg * kSiluSpan);
    tab[e] = (uint16_t)f32_to_bf16(silu(bf16_to_f32(bits)));
  }
}

// The table read for g (its bits b) and the result from it: split so that a
// caller can issue many reads before it needs the first.
__device__ __forceinline__ uint32_t silu_bf16_read(uint32_t b, const uint16_t* tab) {
  const uint32_t a = b & 0x7FFFu, neg = b >> 15;
  const uint32_t ia = min(max(a, kSiluLo), kSiluHi - 1u);
  return tab[ia - kSiluLo + neg * kSiluSpan];
}
__device__ __forceinline__ float silu_bf16_finish(uint32_t b, uint32_t t) {
  const uint32_t a = b & 0x7FFFu, neg = b >> 15;
  const float g = bf16_to_f32(b);
  const float small = round_bf16(g * 0.5f);
  const float big = g * (neg ? 0.0f : 1.0f);
  return a < kSiluLo ? small : (a >= kSiluHi ? big : bf16_to_f32(t));
}

// Per-token quantisation of 8 values: clamp(x / scale, +-448) -> e4m3, r = 1/scale.
__device__ __forceinline__ u32x2 quant8(const float* x, float scale, float r) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = clamp448(div_rcp(x[i], scale, r));
  u32x2 p;
  p.x = e4m3x4(v[0], v[1], v[2], v[3]);
  p.y = e4m3x4(v[4], v[5], v[6], v[7]);
  return p;
}

// Static (per-tensor) quantisation of 4 values with the calibrated multiplier
// inv: e4m3(clamp(x * inv, +-448)), the reference's runtime-scale cast.
__device__ __forceinline__ uint32_t quant4_static(float a, float b, float c, float d, float inv) {
  return e4m3x4(clamp448(a * inv), clamp448(b * inv), clamp448(c * inv), clamp448(d * inv));
}

__device__ __forceinline__ u32x2 quant8_static(const float* x, float inv) {
  u32x2 p;
  p.x = quant4_static(x[0], x[1], x[2], x[3], inv);
  p.y = quant4_static(x[4], x[5], x[6], x[7], inv);
  return p;
}


// ------------------------------------------------------------------ reductions

// Reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with the gfx950 row-swap permutes; every lane receives the result.
__device__ __forceinline__ float max_rows(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Value of the lane selected by a DPP control within each 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowMirror = 0x140;  // lane i <- 15 - i
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within each 8
constexpr int kDppRowRor8 = 0x128;    // lane i <- lane (i + 8) mod 16 of its row

// Wave-wide sum / max on DPP within rows and row swaps across them. Every step
// adds a lane's value to its partner's (a commutative pair), so all 64 lanes
// end with the same bits.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  return sum_rows(v);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  return max_rows(v);
}

// Block-wide sum / max over NW waves; every thread gets the result.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += red[i];
  return s;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) s = fmaxf(s, red[i]);
  return s;
}

// Block-wide sum / max for a runtime block of blockDim.x threads (a multiple of 64).
__device__ __forceinline__ float block_sum_rt(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}

__device__ __forceinline__ float block_max_rt(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
  for (int i = 1; i < nw; ++i) s = fmaxf(s, red[i]);
  return s;
}

// Threads per row and 16-byte chunks per thread for a row of nchunk chunks:
// up to 1024 threads (16 waves) per row, chunks spread evenly.
inline void row_shape(int64_t nchunk, int* threads, int* cpt) {
  const int c = (int)((nchunk + 1023) / 1024);
  const int64_t t = (nchunk + c - 1) / c;
  *cpt = c;
  *threads = (int)((t + 63) / 64 * 64);
}

// 1/sqrt with correctly rounded sqrt and divide (matches 1/std::sqrt on the host).
__device__ __forceinline__ float rsqrt_rn(float v) { return 1.0f / __builtin_sqrtf(v); }

}  // namespace ff

// ------------------------------------------------------------------ host side

void ff_set_error(const char* fmt, ...);
// Value of an ff_set_tuning override (FF_TUNE_*); 0 = the library's own choice.
int ff_tuning(int knob);

namespace ff {
// Row-major / GEMV form of ff_gemm_fp8_swiglu_static (defined with the row-major kernels).
int gemm_swiglu_static_rowmajor(const void* qa, const float* sa, const void* qw, const float* sw, void* hq,
                                int64_t ldh, float inv, int64_t m, int64_t i, int64_t k, hipStream_t s);
// The split-K launch of ff_gemm_fp8_pk alone (defined with the packed kernels):
// where ff_gemm_fp8_pk splits this shape, the split GEMM with its fp32 partials
// row-major in workspace ((*splits, *mp, n), *mp = m rounded up to whole
// tiles); elsewhere nothing is launched and *splits = 0.
int gemm_fp8_pk_partials(const void* qa, const float* sa, int sa_rows, const void* qw_packed, const float* sw,
                         int sw_cols, int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                         hipStream_t st, int* splits, int64_t* mp);
// The same for ff_gemm_w4a16_pk (defined with the W4A16 kernels): where it
// splits k on the packed copies, the split GEMM with its fp32 partials
// row-major in workspace ((*splits, *mp, n)); elsewhere *splits = 0.
int gemm_w4a16_pk_partials(const void* x, int64_t ldx, const void* frag, const void* frag_scales, int64_t group,
                           int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, hipStream_t st,
                           int* splits, int64_t* mp);
}  // namespace ff

#define FF_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      ff_set_error(__VA_ARGS__);       \
      return FF_EINVAL;                \
    }                                  \
  } while (0)

#define FF_LAUNCH_CHECK(what)                                               \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess) {                                                 \
      ff_set_error("%s: launch failed: %s", what, hipGetErrorString(e_));   \
      return FF_ELAUNCH;                                                    \
    }                                                                       \
  } while (0)

static inline bool ff_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
