// Bandwidth-bound kernels: SwiGLU (+ per-token e4m3 quant), activation and
// weight quantization (e4m3, int4), embedding gather, row gather/scatter and the
// M-RoPE cos/sin table. Library status functions live here too.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "ff_common.h"

using namespace ff;

// ---------------------------------------------------------------- status

static thread_local char g_err[512];

void ff_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" int ff_version(void) { return 100; }  // 0.1.0

namespace {
constexpr int kTuneKnobs = 12;
// Upper bound of each knob's values (index = FF_TUNE_*).
constexpr int kTuneMax[kTuneKnobs] = {0, 4, 3, 2, 8, 4, 3, 6, 176096, 114408, 8, 114408};
int g_tuning[kTuneKnobs] = {};
}  // namespace

int ff_tuning(int knob) { return knob > 0 && knob < kTuneKnobs ? __atomic_load_n(&g_tuning[knob], __ATOMIC_RELAXED) : 0; }

extern "C" int ff_set_tuning(int knob, int value) {
  FF_REQUIRE(knob > 0 && knob < kTuneKnobs, "ff_set_tuning: unknown knob %d", knob);
  FF_REQUIRE(value >= 0 && value <= kTuneMax[knob], "ff_set_tuning: value %d out of range for knob %d", value, knob);
  __atomic_store_n(&g_tuning[knob], value, __ATOMIC_RELAXED);
  return FF_OK;
}

extern "C" const char* ff_last_error(void) { return g_err; }

extern "C" int ff_device_check(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    ff_set_error("ff_device_check: no HIP device");
    return FF_EDEVICE;
  }
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
    ff_set_error("ff_device_check: hipGetDeviceProperties failed");
    return FF_EDEVICE;
  }
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
    ff_set_error("ff_device_check: device %d is %s, this build targets gfx950", dev, p.gcnArchName);
    return FF_EDEVICE;
  }
  return FF_OK;
}

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ uint32_t pack_e4m3x4(const float* v) {
  return f32_to_e4m3(v[0]) | (f32_to_e4m3(v[1]) << 8) | (f32_to_e4m3(v[2]) << 16) |
         (f32_to_e4m3(v[3]) << 24);
}

// ---------------------------------------------------------------- swiglu


// Elementwise over (rows, i): each thread handles one 8-wide chunk.
__global__ __launch_bounds__(kThreads) void swiglu_kernel(const bf16_t* __restrict__ g,
                                                          const bf16_t* __restrict__ u,
                                                          int64_t row_stride,
                                                          bf16_t* __restrict__ y, int64_t rows,
                                                          int i) {
  const int chunks = i >> 3;
  const int64_t total = rows * chunks;
  for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * kThreads) {
    const int64_t r = c / chunks;
    const int col = (int)(c - r * chunks) * 8;
    float gv[8], uv[8], o[8];
    unpack8(*reinterpret_cast<const u32x4*>(g + r * row_stride + col), gv);
    unpack8(*reinterpret_cast<const u32x4*>(u + r * row_stride + col), uv);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = round_bf16(silu(gv[k])) * uv[k];
    *reinterpret_cast<u32x4*>(y + r * (int64_t)i + col) = pack8(o);
  }
}

// One workgroup per row (blockDim.x threads, CPT chunks each): swiglu, then
// per-token e4m3 quant of the bf16 result.
template <int CPT>
__global__ __launch_bounds__(1024) void swiglu_quant_kernel(
    const bf16_t* __restrict__ g, const bf16_t* __restrict__ u, int64_t row_stride,
    bf16_t* __restrict__ y, uint8_t* __restrict__ q, float* __restrict__ scales, int i) {
  __shared__ float red[16];
  const int row = blockIdx.x, nt = blockDim.x;
  const int nchunk = i >> 3;
  float o[CPT][8];
  u32x4 vg[CPT], vu[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      vg[c] = *reinterpret_cast<const u32x4*>(g + row * row_stride + idx * 8);
      vu[c] = *reinterpret_cast<const u32x4*>(u + row * row_stride + idx * 8);
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      float gv[8], uv[8];
      unpack8(vg[c], gv);
      unpack8(vu[c], uv);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        o[c][k] = round_bf16(round_bf16(silu(gv[k])) * uv[k]);
        amax = fmaxf(amax, fabsf(o[c][k]));
      }
      if (y) *reinterpret_cast<u32x4*>(y + (size_t)row * i + idx * 8) = pack8(o[c]);
    }
  }
  amax = block_max_rt(amax, red);
  const float scale = fmaxf(amax, 1e-12f) / 448.0f;
  const float r = 1.0f / scale;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) *reinterpret_cast<u32x2*>(q + (size_t)row * i + idx * 8) = quant8(o[c], scale, r);
  }
  if (threadIdx.x == 0) scales[row] = scale;
}

// ---------------------------------------------------------------- activation quant

template <int CPT>
__global__ __launch_bounds__(1024) void quant_rows_kernel(const bf16_t* __restrict__ x, int64_t x_rs,
                                                         uint8_t* __restrict__ q, float* __restrict__ scales,
                                                         int k) {
  __shared__ float red[16];
  const int row = blockIdx.x, nt = blockDim.x;
  const int nchunk = k >> 3;
  float v[CPT][8];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      unpack8(*reinterpret_cast<const u32x4*>(x + row * x_rs + idx * 8), v[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[c][e]));
    }
  }
  amax = block_max_rt(amax, red);
  const float scale = fmaxf(amax, 1e-12f) / 448.0f;
  const float r = 1.0f / scale;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) *reinterpret_cast<u32x2*>(q + (size_t)row * k + idx * 8) = quant8(v[c], scale, r);
  }
  if (threadIdx.x == 0) scales[row] = scale;
}

// Per-token quantisation whose row amax comes from npart partial maxima
// (pmax[row * npart + j], written by the producer of x): the same codes and
// scales as quant_rows_kernel on x, without a reduction over the row.
template <int CPT>
__global__ __launch_bounds__(1024) void quant_rows_pmax_kernel(const bf16_t* __restrict__ x, int64_t x_rs,
                                                              const float* __restrict__ pmax, int npart,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ scales, int k) {
  __shared__ float red[16];
  const int row = blockIdx.x, nt = blockDim.x;
  const int nchunk = k >> 3;
  u32x4 v[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) v[c] = *reinterpret_cast<const u32x4*>(x + row * x_rs + idx * 8);
  }
  float amax = 0.f;
  for (int j = threadIdx.x; j < npart; j += nt) amax = fmaxf(amax, pmax[(size_t)row * npart + j]);
  amax = block_max_rt(amax, red);
  const float scale = fmaxf(amax, 1e-12f) / 448.0f;
  const float r = 1.0f / scale;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      float f[8];
      unpack8(v[c], f);
      *reinterpret_cast<u32x2*>(q + (size_t)row * k + idx * 8) = quant8(f, scale, r);
    }
  }
  if (threadIdx.x == 0) scales[row] = scale;
}

// Generic long-row fallback (k > 8*256*16): two passes over global memory.
__global__ __launch_bounds__(kThreads) void quant_rows_long_kernel(const bf16_t* __restrict__ x,
                                                                   int64_t x_rs,
                                                                   uint8_t* __restrict__ q,
                                                                   float* __restrict__ scales, int k) {
  __shared__ float red[kWaves];
  const int row = blockIdx.x;
  float amax = 0.f;
  for (int e = threadIdx.x; e < k; e += kThreads) amax = fmaxf(amax, fabsf(bf16_to_f32(x[row * x_rs + e])));
  amax = block_max<kWaves>(amax, red);
  const float scale = fmaxf(amax, 1e-12f) / 448.0f;
  for (int e = threadIdx.x; e < k; e += kThreads)
    q[(size_t)row * k + e] = (uint8_t)f32_to_e4m3(clamp448(bf16_to_f32(x[row * x_rs + e]) / scale));
  if (threadIdx.x == 0) scales[row] = scale;
}

__global__ __launch_bounds__(kThreads) void quant_static_kernel(const bf16_t* __restrict__ x,
                                                                uint8_t* __restrict__ q, int64_t n_valid,
                                                                int64_t n_total, float inv) {
  // 8 elements per thread per step; n_valid, n_total multiples of 8.
  for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c * 8 < n_total;
       c += (int64_t)gridDim.x * kThreads) {
    u32x2 p;
    if (c * 8 < n_valid) {
      float v[8];
      unpack8(*reinterpret_cast<const u32x4*>(x + c * 8), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = clamp448(v[e] * inv);
      p.x = pack_e4m3x4(v);
      p.y = pack_e4m3x4(v + 4);
    } else {
      p.x = 0;
      p.y = 0;
    }
    *reinterpret_cast<u32x2*>(q + c * 8) = p;
  }
}

// ---------------------------------------------------------------- weight quant

__global__ __launch_bounds__(kThreads) void row_amax_kernel(const bf16_t* __restrict__ w, int64_t k,
                                                            float* __restrict__ amax_out) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  float m = 0.f;
  for (int64_t e = threadIdx.x; e < k; e += kThreads) m = fmaxf(m, fabsf(bf16_to_f32(w[row * k + e])));
  m = block_max<kWaves>(m, red);
  if (threadIdx.x == 0) amax_out[row] = m;
}

// Single workgroup: per-tensor scale = max(max_n amax[n], 1e-12)/448.
__global__ __launch_bounds__(kThreads) void tensor_scale_kernel(const float* __restrict__ amax,
                                                                int64_t n, float* __restrict__ scale) {
  __shared__ float red[kWaves];
  float m = 0.f;
  for (int64_t e = threadIdx.x; e < n; e += kThreads) m = fmaxf(m, amax[e]);
  m = block_max<kWaves>(m, red);
  if (threadIdx.x == 0) scale[0] = fmaxf(m, 1e-12f) / 448.0f;
}

// Per-channel scales from the row amax (in place: amax -> scale).
__global__ void channel_scale_kernel(float* __restrict__ s, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) s[i] = fmaxf(s[i], 1e-12f) / 448.0f;
}

__global__ __launch_bounds__(kThreads) void weight_quant_kernel(const bf16_t* __restrict__ w,
                                                                uint8_t* __restrict__ q,
                                                                const float* __restrict__ scale,
                                                                int64_t k, int per_channel) {
  const int64_t row = blockIdx.x;
  const float s = scale[per_channel ? row : 0];
  for (int64_t e = threadIdx.x; e < k; e += kThreads)
    q[row * k + e] = (uint8_t)f32_to_e4m3(clamp448(bf16_to_f32(w[row * k + e]) / s));
}

// int4: one thread per (row, group). Writes packed nibbles and the (s, z) pair.
__global__ __launch_bounds__(kThreads) void int4_quant_kernel(const bf16_t* __restrict__ w,
                                                              uint8_t* __restrict__ packed,
                                                              bf16_t* __restrict__ scales, int64_t n,
                                                              int64_t k, int group, int symmetric) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t groups = k / group;
  if (gid >= n * groups) return;
  const int64_t row = gid / groups, gi = gid % groups;
  const bf16_t* src = w + row * k + gi * group;
  uint8_t* dst = packed + row * (k / 2) + gi * group / 2;
  bf16_t* sz = scales + (gi * n + row) * 2;
  if (symmetric) {
    float amax = 0.f;
    for (int e = 0; e < group; ++e) amax = fmaxf(amax, fabsf(bf16_to_f32(src[e])));
    const float s = round_bf16(fmaxf(amax, 1e-6f) / 7.0f);
    for (int e = 0; e < group; e += 2) {
      float c0 = fminf(15.f, fmaxf(0.f, __builtin_rintf(bf16_to_f32(src[e]) / s) + 8.0f));
      float c1 = fminf(15.f, fmaxf(0.f, __builtin_rintf(bf16_to_f32(src[e + 1]) / s) + 8.0f));
      dst[e / 2] = (uint8_t)(((uint32_t)c0 << 4) | (uint32_t)c1);
    }
    sz[0] = (bf16_t)f32_to_bf16(s);
    sz[1] = 0;
  } else {
    float lo = bf16_to_f32(src[0]), hi = lo;
    for (int e = 1; e < group; ++e) {
      const float v = bf16_to_f32(src[e]);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
    const float s = fmaxf((hi - lo) / 15.0f, 1e-6f);
    for (int e = 0; e < group; e += 2) {
      float c0 = fminf(15.f, fmaxf(0.f, __builtin_rintf((bf16_to_f32(src[e]) - lo) / s)));
      float c1 = fminf(15.f, fmaxf(0.f, __builtin_rintf((bf16_to_f32(src[e + 1]) - lo) / s)));
      dst[e / 2] = (uint8_t)(((uint32_t)c0 << 4) | (uint32_t)c1);
    }
    const float s8 = s * 8.0f;
    sz[0] = (bf16_t)f32_to_bf16(s);
    sz[1] = (bf16_t)f32_to_bf16(lo + s8);
  }
}

// ---------------------------------------------------------------- gathers

// One workgroup per output row; 16-byte copies.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const bf16_t* __restrict__ src,
                                                               int64_t src_rs,
                                                               const int64_t* __restrict__ idx,
                                                               bf16_t* __restrict__ out,
                                                               int64_t out_rs, int64_t width,
                                                               int64_t src_rows) {
  const int64_t r = blockIdx.x;
  int64_t s = idx ? idx[r] : r;
  if (s < 0 || s >= src_rows) s = 0;
  for (int64_t c = threadIdx.x; c * 8 < width; c += kThreads)
    *reinterpret_cast<u32x4*>(out + r * out_rs + c * 8) =
        *reinterpret_cast<const u32x4*>(src + s * src_rs + c * 8);
}

// ---------------------------------------------------------------- M-RoPE

__global__ __launch_bounds__(kThreads) void mrope_kernel(const int64_t* __restrict__ pos,
                                                         const float* __restrict__ inv_freq,
                                                         bf16_t* __restrict__ cos_out,
                                                         bf16_t* __restrict__ sin_out, int64_t t,
                                                         int d, int sec_h, int sec_w) {
  const int half = d / 2;
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= t * half) return;
  const int64_t tok = gid / half;
  const int i = (int)(gid % half);
  int src = 0;
  if (i % 3 == 1 && i < 3 * sec_h) src = 1;
  else if (i % 3 == 2 && i < 3 * sec_w) src = 2;
  const float p = (float)pos[src * t + tok];
  const float f = p * inv_freq[i];
  // cos/sin of the fp32 angle evaluated in double and rounded once to fp32
  // before the bf16 store, so the table is the correctly rounded value of the
  // fp32 argument up to the final bf16 rounding.
  const float c = (float)cos((double)f);
  const float s = (float)sin((double)f);
  const uint32_t cb = f32_to_bf16(c), sb = f32_to_bf16(s);
  cos_out[tok * d + i] = (bf16_t)cb;
  cos_out[tok * d + i + half] = (bf16_t)cb;
  sin_out[tok * d + i] = (bf16_t)sb;
  sin_out[tok * d + i + half] = (bf16_t)sb;
}

int grid_for(int64_t items, int64_t per_block, int64_t cap = 65536) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

}  // namespace

// ---------------------------------------------------------------- C ABI

extern "C" int ff_swiglu(const void* g, const void* u, int64_t row_stride, void* y, int64_t rows,
                         int64_t i, ff_stream_t stream) {
  FF_REQUIRE(g && u && y, "ff_swiglu: null pointer");
  FF_REQUIRE(i > 0 && i % 8 == 0 && row_stride >= i && row_stride % 8 == 0 && rows >= 0,
             "ff_swiglu: bad sizes i=%lld stride=%lld", (long long)i, (long long)row_stride);
  FF_REQUIRE(ff_aligned(g, 16) && ff_aligned(u, 16) && ff_aligned(y, 16), "ff_swiglu: alignment");
  if (rows == 0) return FF_OK;
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(rows * (i / 8), kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)g, (const bf16_t*)u, row_stride, (bf16_t*)y,
                     rows, (int)i);
  FF_LAUNCH_CHECK("ff_swiglu");
  return FF_OK;
}

extern "C" int ff_swiglu_quant(const void* g, const void* u, int64_t row_stride, void* y, void* q,
                               float* scales, int64_t rows, int64_t i, ff_stream_t stream) {
  FF_REQUIRE(g && u && q && scales, "ff_swiglu_quant: null pointer");
  FF_REQUIRE(i > 0 && i % 8 == 0 && row_stride >= i && row_stride % 8 == 0 && rows >= 0,
             "ff_swiglu_quant: bad sizes");
  FF_REQUIRE(ff_aligned(g, 16) && ff_aligned(u, 16) && ff_aligned(q, 8) && (!y || ff_aligned(y, 16)),
             "ff_swiglu_quant: alignment");
  if (rows == 0) return FF_OK;
  int threads, cpt;
  row_shape(i / 8, &threads, &cpt);
  hipStream_t s = (hipStream_t)stream;
#define FF_SWQ(N)                                                                                      \
  case N:                                                                                              \
    hipLaunchKernelGGL(swiglu_quant_kernel<N>, dim3((unsigned)rows), dim3((unsigned)threads), 0, s,    \
                       (const bf16_t*)g, (const bf16_t*)u, row_stride, (bf16_t*)y, (uint8_t*)q, scales, \
                       (int)i);                                                                        \
    break;
  switch (cpt) {
    FF_SWQ(1) FF_SWQ(2) FF_SWQ(3) FF_SWQ(4)
    default:
      ff_set_error("ff_swiglu_quant: i=%lld too large", (long long)i);
      return FF_EINVAL;
  }
#undef FF_SWQ
  FF_LAUNCH_CHECK("ff_swiglu_quant");
  return FF_OK;
}

extern "C" int ff_quant_rows_fp8(const void* x, int64_t x_rs, void* q, float* scales, int64_t rows,
                                 int64_t k, ff_stream_t stream) {
  FF_REQUIRE(x && q && scales, "ff_quant_rows_fp8: null pointer");
  FF_REQUIRE(k > 0 && k % 8 == 0 && x_rs >= k && x_rs % 8 == 0 && rows >= 0,
             "ff_quant_rows_fp8: bad sizes k=%lld", (long long)k);
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(q, 8), "ff_quant_rows_fp8: alignment");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  int threads, cpt;
  row_shape(k / 8, &threads, &cpt);
#define FF_QR(N)                                                                                   \
  case N:                                                                                          \
    hipLaunchKernelGGL(quant_rows_kernel<N>, dim3((unsigned)rows), dim3((unsigned)threads), 0, s,  \
                       (const bf16_t*)x, x_rs, (uint8_t*)q, scales, (int)k);                       \
    break;
  switch (cpt) {
    FF_QR(1) FF_QR(2) FF_QR(3) FF_QR(4)
    default:
      hipLaunchKernelGGL(quant_rows_long_kernel, dim3((unsigned)rows), dim3(kThreads), 0, s,
                         (const bf16_t*)x, x_rs, (uint8_t*)q, scales, (int)k);
  }
#undef FF_QR
  FF_LAUNCH_CHECK("ff_quant_rows_fp8");
  return FF_OK;
}

extern "C" int ff_quant_static_fp8(const void* x, void* q, int64_t rows, int64_t rows_pad, int64_t k,
                                   float inv, ff_stream_t stream) {
  FF_REQUIRE(x && q, "ff_quant_static_fp8: null pointer");
  FF_REQUIRE(k > 0 && k % 8 == 0 && rows >= 0 && rows_pad >= rows, "ff_quant_static_fp8: bad sizes");
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(q, 8), "ff_quant_static_fp8: alignment");
  if (rows_pad == 0) return FF_OK;
  const int64_t n_total = rows_pad * k;
  hipLaunchKernelGGL(quant_static_kernel, dim3(grid_for(n_total / 8, kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)x, (uint8_t*)q, rows * k, n_total, inv);
  FF_LAUNCH_CHECK("ff_quant_static_fp8");
  return FF_OK;
}

extern "C" int ff_quant_weight_fp8(const void* w, void* q, float* scale, float* workspace, int64_t n,
                                   int64_t k, int per_channel, ff_stream_t stream) {
  FF_REQUIRE(w && q && scale, "ff_quant_weight_fp8: null pointer");
  FF_REQUIRE(n > 0 && k > 0 && n < (1ll << 31), "ff_quant_weight_fp8: bad sizes");
  FF_REQUIRE(per_channel || workspace, "ff_quant_weight_fp8: per-tensor mode needs a workspace of n floats");
  hipStream_t s = (hipStream_t)stream;
  float* amax = per_channel ? scale : workspace;
  hipLaunchKernelGGL(row_amax_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, (const bf16_t*)w, k, amax);
  if (per_channel)
    hipLaunchKernelGGL(channel_scale_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, scale, n);
  else
    hipLaunchKernelGGL(tensor_scale_kernel, dim3(1), dim3(kThreads), 0, s, workspace, n, scale);
  hipLaunchKernelGGL(weight_quant_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, (const bf16_t*)w,
                     (uint8_t*)q, scale, k, per_channel);
  FF_LAUNCH_CHECK("ff_quant_weight_fp8");
  return FF_OK;
}

extern "C" int ff_quant_weight_int4(const void* w, void* packed, void* scales, int64_t n, int64_t k,
                                    int64_t group, int symmetric, ff_stream_t stream) {
  FF_REQUIRE(w && packed && scales, "ff_quant_weight_int4: null pointer");
  FF_REQUIRE(n > 0 && k > 0 && group > 0 && group % 2 == 0 && k % group == 0,
             "ff_quant_weight_int4: k=%lld must be a multiple of group=%lld", (long long)k,
             (long long)group);
  const int64_t items = n * (k / group);
  hipLaunchKernelGGL(int4_quant_kernel, dim3(grid_for(items, kThreads, 1ll << 30)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const bf16_t*)w, (uint8_t*)packed, (bf16_t*)scales, n, k,
                     (int)group, symmetric);
  FF_LAUNCH_CHECK("ff_quant_weight_int4");
  return FF_OK;
}

extern "C" int ff_embed(const int64_t* ids, const void* table, void* out, int64_t t, int64_t h,
                        int64_t vocab, ff_stream_t stream) {
  FF_REQUIRE(ids && table && out, "ff_embed: null pointer");
  FF_REQUIRE(h > 0 && h % 8 == 0 && t >= 0 && vocab > 0, "ff_embed: bad sizes");
  FF_REQUIRE(ff_aligned(table, 16) && ff_aligned(out, 16), "ff_embed: alignment");
  if (t == 0) return FF_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)t), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)table, h, ids, (bf16_t*)out, h, h, vocab);
  FF_LAUNCH_CHECK("ff_embed");
  return FF_OK;
}

extern "C" int ff_gather_rows(const void* src, int64_t src_rs, const int64_t* idx, void* out,
                              int64_t out_rs, int64_t n, int64_t width, int64_t src_rows,
                              ff_stream_t stream) {
  FF_REQUIRE(src && out, "ff_gather_rows: null pointer");
  FF_REQUIRE(width > 0 && width % 8 == 0 && src_rs % 8 == 0 && out_rs % 8 == 0 && n >= 0,
             "ff_gather_rows: bad sizes");
  FF_REQUIRE(ff_aligned(src, 16) && ff_aligned(out, 16), "ff_gather_rows: alignment");
  if (n == 0) return FF_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)n), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)src, src_rs, idx, (bf16_t*)out, out_rs, width, src_rows);
  FF_LAUNCH_CHECK("ff_gather_rows");
  return FF_OK;
}

extern "C" int ff_scatter_rows(const void* src, void* out, int64_t start, int64_t n, int64_t width,
                               ff_stream_t stream) {
  FF_REQUIRE(src && out && start >= 0 && width % 8 == 0, "ff_scatter_rows: bad arguments");
  FF_REQUIRE(ff_aligned(src, 16) && ff_aligned(out, 16), "ff_scatter_rows: alignment");
  if (n == 0) return FF_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)n), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)src, width, (const int64_t*)nullptr,
                     (bf16_t*)out + start * width, width, width, n);
  FF_LAUNCH_CHECK("ff_scatter_rows");
  return FF_OK;
}

extern "C" int ff_mrope_cos_sin(const int64_t* pos, const float* inv_freq, void* cos, void* sin,
                                int64_t t, int64_t d, int sec_h, int sec_w, ff_stream_t stream) {
  FF_REQUIRE(pos && inv_freq && cos && sin, "ff_mrope_cos_sin: null pointer");
  FF_REQUIRE(d > 0 && d % 2 == 0 && t >= 0 && sec_h >= 0 && sec_w >= 0, "ff_mrope_cos_sin: bad sizes");
  if (t == 0) return FF_OK;
  hipLaunchKernelGGL(mrope_kernel, dim3(grid_for(t * (d / 2), kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, pos, inv_freq, (bf16_t*)cos, (bf16_t*)sin, t, (int)d, sec_h,
                     sec_w);
  FF_LAUNCH_CHECK("ff_mrope_cos_sin");
  return FF_OK;
}

extern "C" int ff_quant_rows_pmax(const void* x, int64_t x_rs, const float* pmax, int64_t npart, void* q,
                                  float* scales, int64_t rows, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(x && pmax && q && scales, "ff_quant_rows_pmax: null pointer");
  FF_REQUIRE(k > 0 && k % 8 == 0 && x_rs >= k && x_rs % 8 == 0 && rows >= 0 && npart > 0 && npart < (1 << 20),
             "ff_quant_rows_pmax: bad sizes k=%lld npart=%lld", (long long)k, (long long)npart);
  FF_REQUIRE(ff_aligned(x, 16) && ff_aligned(q, 8), "ff_quant_rows_pmax: alignment");
  if (rows == 0) return FF_OK;
  int threads, cpt;
  row_shape(k / 8, &threads, &cpt);
  hipStream_t s = (hipStream_t)stream;
#define FF_QP(N)                                                                                      \
  case N:                                                                                             \
    hipLaunchKernelGGL(quant_rows_pmax_kernel<N>, dim3((unsigned)rows), dim3((unsigned)threads), 0, s, \
                       (const bf16_t*)x, x_rs, pmax, (int)npart, (uint8_t*)q, scales, (int)k);         \
    break;
  switch (cpt) {
    FF_QP(1) FF_QP(2) FF_QP(3) FF_QP(4)
    default:
      ff_set_error("ff_quant_rows_pmax: k=%lld too large", (long long)k);
      return FF_EINVAL;
  }
#undef FF_QP
  FF_LAUNCH_CHECK("ff_quant_rows_pmax");
  return FF_OK;
}
