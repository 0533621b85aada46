// Row-wise RMSNorm kernels: fast_norm, add_rms (+ DeepStack rows), their fused
// per-token e4m3 quant variants, and the choice readout.
//
// One workgroup of 256 threads owns one token row. Each thread loads its 16-byte
// chunks (8 bf16) up front, so a row's whole HBM traffic is in flight before the
// reduction; rows are independent, and the grid (one workgroup per row) keeps all
// rows resident at the prefill sizes (<= 2048 rows).
#include "ff_common.h"

using namespace ff;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// CPT = 16-byte chunks per thread (h <= CPT * 8 * 256).
template <int CPT, bool ADD, bool DEEP, bool WRITE_RES, bool WRITE_OUT, bool QUANT>
__global__ __launch_bounds__(kThreads) void row_norm_kernel(
    const bf16_t* __restrict__ a, const bf16_t* __restrict__ b, const bf16_t* __restrict__ deep,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ residual, bf16_t* __restrict__ out,
    uint8_t* __restrict__ q, float* __restrict__ scales, int h, float eps, int start, int nv) {
  __shared__ float red[kWaves];
  const int row = blockIdx.x;
  const int nchunk = h >> 3;
  const size_t base = (size_t)row * h;
  float x[CPT][8];
  u32x4 va[CPT], vb[CPT];
  const bool in_deep = DEEP && row >= start && row < start + nv;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * kThreads;
    if (idx < nchunk) {
      va[c] = *reinterpret_cast<const u32x4*>(a + base + (size_t)idx * 8);
      if (ADD) vb[c] = *reinterpret_cast<const u32x4*>(b + base + (size_t)idx * 8);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * kThreads;
    if (idx < nchunk) {
      unpack8(va[c], x[c]);
      if (ADD) {
        float y[8];
        unpack8(vb[c], y);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[c][i] = round_bf16(x[c][i] + y[i]);
      }
      if (DEEP && in_deep) {
        float y[8];
        unpack8(*reinterpret_cast<const u32x4*>(deep + (size_t)(row - start) * h + (size_t)idx * 8), y);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[c][i] = round_bf16(x[c][i] + y[i]);
      }
      if (WRITE_RES) *reinterpret_cast<u32x4*>(residual + base + (size_t)idx * 8) = pack8(x[c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[c][i] * x[c][i];
    }
  }
  const float var = block_sum<kWaves>(ss, red) / (float)h;
  const float inv = rsqrt_rn(var + eps);
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * kThreads;
    if (idx < nchunk) {
      float wv[8];
      unpack8(*reinterpret_cast<const u32x4*>(w + (size_t)idx * 8), wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[c][i] = round_bf16(round_bf16(x[c][i] * inv) * wv[i]);
        amax = fmaxf(amax, fabsf(x[c][i]));
      }
      if (WRITE_OUT) *reinterpret_cast<u32x4*>(out + base + (size_t)idx * 8) = pack8(x[c]);
    }
  }
  if (QUANT) {
    amax = block_max<kWaves>(amax, red);
    const float scale = fmaxf(amax, 1e-12f) / 448.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = threadIdx.x + c * kThreads;
      if (idx < nchunk) {
        u32x2 p;
        uint32_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = f32_to_e4m3(clamp448(x[c][i] / scale));
        p.x = e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24);
        p.y = e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24);
        *reinterpret_cast<u32x2*>(q + base + (size_t)idx * 8) = p;
      }
    }
    if (threadIdx.x == 0) scales[row] = scale;
  }
}

template <bool ADD, bool DEEP, bool WRITE_RES, bool WRITE_OUT, bool QUANT>
int launch_row_norm(const void* a, const void* b, const void* deep, const void* w, void* residual,
                    void* out, void* q, float* scales, int64_t rows, int64_t h, float eps,
                    int64_t start, int64_t nv, hipStream_t s, const char* name) {
  const int cpt = (int)((h / 8 + kThreads - 1) / kThreads);
  dim3 grid((unsigned)rows), block(kThreads);
#define FF_ROWNORM_CASE(N)                                                                       \
  case N:                                                                                        \
    hipLaunchKernelGGL((row_norm_kernel<N, ADD, DEEP, WRITE_RES, WRITE_OUT, QUANT>), grid, block, \
                       0, s, (const bf16_t*)a, (const bf16_t*)b, (const bf16_t*)deep,             \
                       (const bf16_t*)w, (bf16_t*)residual, (bf16_t*)out, (uint8_t*)q, scales,    \
                       (int)h, eps, (int)start, (int)nv);                                         \
    break;
  switch (cpt) {
    FF_ROWNORM_CASE(1)
    FF_ROWNORM_CASE(2)
    FF_ROWNORM_CASE(3)
    FF_ROWNORM_CASE(4)
    FF_ROWNORM_CASE(5)
    FF_ROWNORM_CASE(6)
    FF_ROWNORM_CASE(7)
    FF_ROWNORM_CASE(8)
    default:
      ff_set_error("%s: h=%lld too large", name, (long long)h);
      return FF_EINVAL;
  }
#undef FF_ROWNORM_CASE
  FF_LAUNCH_CHECK(name);
  return FF_OK;
}

int check_rows(const char* name, const void* x, int64_t rows, int64_t h) {
  FF_REQUIRE(x != nullptr, "%s: null input", name);
  FF_REQUIRE(rows >= 0 && rows < (1ll << 31), "%s: bad rows %lld", name, (long long)rows);
  FF_REQUIRE(h > 0 && h % 8 == 0 && h <= 16384, "%s: h=%lld must be a multiple of 8 <= 16384", name,
             (long long)h);
  FF_REQUIRE(ff_aligned(x, 16), "%s: input not 16-byte aligned", name);
  return FF_OK;
}

// ---------------------------------------------------------------- readout

// One workgroup: normalise the (optionally summed) row once, then each wave
// computes dot products for options w, w+4, ...
__global__ __launch_bounds__(kThreads) void readout_kernel(const bf16_t* __restrict__ x,
                                                           const bf16_t* __restrict__ x2,
                                                           const bf16_t* __restrict__ w,
                                                           const bf16_t* __restrict__ head,
                                                           float* __restrict__ y, int h, int n_opt,
                                                           float eps) {
  extern __shared__ float xs[];  // h floats (normalised row)
  __shared__ float red[kWaves];
  float ss = 0.f;
  for (int i = threadIdx.x; i < h; i += kThreads) {
    float v = bf16_to_f32(x[i]);
    if (x2) v = round_bf16(v + bf16_to_f32(x2[i]));
    xs[i] = v;
    ss += v * v;
  }
  const float inv = rsqrt_rn(block_sum<kWaves>(ss, red) / (float)h + eps);
  for (int i = threadIdx.x; i < h; i += kThreads)
    xs[i] = round_bf16(round_bf16(xs[i] * inv) * bf16_to_f32(w[i]));
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int c = wave; c < n_opt; c += kWaves) {
    float acc = 0.f;
    for (int i = lane; i < h; i += 64) acc += xs[i] * bf16_to_f32(head[(size_t)c * h + i]);
    acc = wave_sum(acc);
    if (lane == 0) y[c] = round_bf16(acc);
  }
}

}  // namespace

extern "C" int ff_fast_norm(const void* x, const void* w, void* out, int64_t rows, int64_t h,
                            float eps, ff_stream_t stream) {
  int st = check_rows("ff_fast_norm", x, rows, h);
  if (st) return st;
  FF_REQUIRE(out && w && ff_aligned(out, 16) && ff_aligned(w, 16), "ff_fast_norm: bad out/w");
  if (rows == 0) return FF_OK;
  return launch_row_norm<false, false, false, true, false>(x, nullptr, nullptr, w, nullptr, out,
                                                           nullptr, nullptr, rows, h, eps, 0, 0,
                                                           (hipStream_t)stream, "ff_fast_norm");
}

extern "C" int ff_fast_norm_quant(const void* x, const void* w, void* out, void* q, float* scales,
                                  int64_t rows, int64_t h, float eps, ff_stream_t stream) {
  int st = check_rows("ff_fast_norm_quant", x, rows, h);
  if (st) return st;
  FF_REQUIRE(q && scales && w && ff_aligned(q, 8) && ff_aligned(w, 16), "ff_fast_norm_quant: bad q/scales/w");
  FF_REQUIRE(!out || ff_aligned(out, 16), "ff_fast_norm_quant: out not aligned");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (out)
    return launch_row_norm<false, false, false, true, true>(x, nullptr, nullptr, w, nullptr, out, q,
                                                            scales, rows, h, eps, 0, 0, s,
                                                            "ff_fast_norm_quant");
  return launch_row_norm<false, false, false, false, true>(x, nullptr, nullptr, w, nullptr, nullptr,
                                                           q, scales, rows, h, eps, 0, 0, s,
                                                           "ff_fast_norm_quant");
}

extern "C" int ff_add_rms(const void* a, const void* b, const void* deep, const void* w,
                          void* residual, void* out, int64_t rows, int64_t h, float eps,
                          int64_t start, int64_t nv, ff_stream_t stream) {
  int st = check_rows("ff_add_rms", a, rows, h);
  if (st) return st;
  FF_REQUIRE(b && w && residual && out && ff_aligned(b, 16) && ff_aligned(w, 16) &&
                 ff_aligned(residual, 16) && ff_aligned(out, 16),
             "ff_add_rms: bad b/w/residual/out");
  FF_REQUIRE(!deep || (ff_aligned(deep, 16) && nv >= 0 && start >= 0), "ff_add_rms: bad deep");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (deep && nv > 0)
    return launch_row_norm<true, true, true, true, false>(a, b, deep, w, residual, out, nullptr,
                                                          nullptr, rows, h, eps, start, nv, s,
                                                          "ff_add_rms");
  return launch_row_norm<true, false, true, true, false>(a, b, nullptr, w, residual, out, nullptr,
                                                         nullptr, rows, h, eps, 0, 0, s, "ff_add_rms");
}

extern "C" int ff_add_rms_quant(const void* a, const void* b, const void* deep, const void* w,
                                void* residual, void* out, void* q, float* scales, int64_t rows,
                                int64_t h, float eps, int64_t start, int64_t nv,
                                ff_stream_t stream) {
  int st = check_rows("ff_add_rms_quant", a, rows, h);
  if (st) return st;
  FF_REQUIRE(b && w && residual && q && scales && ff_aligned(b, 16) && ff_aligned(w, 16) &&
                 ff_aligned(residual, 16) && ff_aligned(q, 8),
             "ff_add_rms_quant: bad b/w/residual/q/scales");
  FF_REQUIRE(!out || ff_aligned(out, 16), "ff_add_rms_quant: out not aligned");
  FF_REQUIRE(!deep || (ff_aligned(deep, 16) && nv >= 0 && start >= 0), "ff_add_rms_quant: bad deep");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool d = deep && nv > 0;
  if (d && out)
    return launch_row_norm<true, true, true, true, true>(a, b, deep, w, residual, out, q, scales, rows,
                                                         h, eps, start, nv, s, "ff_add_rms_quant");
  if (d)
    return launch_row_norm<true, true, true, false, true>(a, b, deep, w, residual, nullptr, q, scales,
                                                          rows, h, eps, start, nv, s,
                                                          "ff_add_rms_quant");
  if (out)
    return launch_row_norm<true, false, true, true, true>(a, b, nullptr, w, residual, out, q, scales,
                                                          rows, h, eps, 0, 0, s, "ff_add_rms_quant");
  return launch_row_norm<true, false, true, false, true>(a, b, nullptr, w, residual, nullptr, q,
                                                         scales, rows, h, eps, 0, 0, s,
                                                         "ff_add_rms_quant");
}

extern "C" int ff_lm_readout(const void* x, const void* x2, const void* norm_w, const void* head,
                             float* y, int64_t h, int64_t n_opt, float eps, ff_stream_t stream) {
  FF_REQUIRE(x && norm_w && head && y, "ff_lm_readout: null pointer");
  FF_REQUIRE(h > 0 && h <= 8192 && n_opt > 0 && n_opt <= 64, "ff_lm_readout: bad h=%lld n_opt=%lld",
             (long long)h, (long long)n_opt);
  hipLaunchKernelGGL(readout_kernel, dim3(1), dim3(kThreads), (size_t)h * sizeof(float),
                     (hipStream_t)stream, (const bf16_t*)x, (const bf16_t*)x2, (const bf16_t*)norm_w,
                     (const bf16_t*)head, y, (int)h, (int)n_opt, eps);
  FF_LAUNCH_CHECK("ff_lm_readout");
  return FF_OK;
}
