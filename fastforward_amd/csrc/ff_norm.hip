// Row-wise RMSNorm kernels: fast_norm, add_rms (+ DeepStack rows), their fused
// per-token e4m3 quant variants, and the choice readout.
//
// One workgroup owns one token row, with up to 1024 threads so that a row's
// arithmetic spreads over 16 waves. Each thread loads its 16-byte chunks (8
// bf16) up front, so a row's whole traffic is in flight before the reduction;
// rows are independent.
#include "ff_common.h"

using namespace ff;

namespace {


// e4m3 output of the normalised row: none, per-token dynamic scale (written to
// scales[row]) or a static calibrated multiplier (e4m3(clamp(x * sinv, +-448))).
constexpr int kNoQuant = 0, kDynamic = 1, kStatic = 2;

// The addend of add_rms given as the fp32 split-K partials of a GEMM
// (row-major, (splits, mp, h)) instead of bf16: b = bf16(sum_s part_s), or with
// scales (an FP8 GEMM) b = bf16((sum_s part_s * sa[row]) * sw[col]); the
// partials added in split order -- the split GEMM's own reduction, bit for bit
// -- and b stored to y (row stride h) as that GEMM's output.
struct SplitAddend {
  const float* part = nullptr;
  int64_t mp = 0;
  int splits = 0;
  const float* sa = nullptr;  // null: no scales
  int sa_rows = 0;
  const float* sw = nullptr;
  int sw_cols = 0;
  bf16_t* y = nullptr;
};

// One workgroup per row, blockDim.x threads (a multiple of 64, <= 1024) with
// CPT 16-byte chunks each (row_shape picks both from h). SPLIT > 0: the addend
// b comes from sb.splits <= SPLIT split-K partials instead of the bf16 array b.
template <int CPT, bool ADD, bool DEEP, bool WRITE_RES, bool WRITE_OUT, int QUANT, int SPLIT = 0>
__global__ __launch_bounds__(1024) void row_norm_kernel(
    const bf16_t* __restrict__ a, const bf16_t* __restrict__ b, const bf16_t* __restrict__ deep,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ residual, bf16_t* __restrict__ out,
    uint8_t* __restrict__ q, float* __restrict__ scales, int h, float eps, int start, int nv, float sinv,
    SplitAddend sb) {
  __shared__ float red[16];
  const int row = blockIdx.x;
  const int nchunk = h >> 3;
  const int nt = blockDim.x;
  const size_t base = (size_t)row * h;
  float x[CPT][8];
  u32x4 va[CPT], vb[CPT], vw[CPT];
  f32x4 vp[CPT][SPLIT > 0 ? SPLIT : 1][2], vs[CPT][2];
  float sav = 0.f;
  if constexpr (SPLIT > 0) sav = sb.sa ? sb.sa[sb.sa_rows ? row : 0] : 0.f;
  const bool in_deep = DEEP && row >= start && row < start + nv;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      va[c] = *reinterpret_cast<const u32x4*>(a + base + (size_t)idx * 8);
      if constexpr (ADD && SPLIT > 0) {
#pragma unroll
        for (int s2 = 0; s2 < SPLIT; ++s2) {
          if (s2 < sb.splits) {
            const float* src = sb.part + ((int64_t)s2 * sb.mp + row) * h + (size_t)idx * 8;
            vp[c][s2][0] = *reinterpret_cast<const f32x4*>(src);
            vp[c][s2][1] = *reinterpret_cast<const f32x4*>(src + 4);
          }
        }
        if (!sb.sa) {
        } else if (sb.sw_cols && ((uintptr_t)sb.sw & 15) == 0) {
          vs[c][0] = *reinterpret_cast<const f32x4*>(sb.sw + (size_t)idx * 8);
          vs[c][1] = *reinterpret_cast<const f32x4*>(sb.sw + (size_t)idx * 8 + 4);
        } else if (sb.sw_cols) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            vs[c][0][r] = sb.sw[(size_t)idx * 8 + r];
            vs[c][1][r] = sb.sw[(size_t)idx * 8 + 4 + r];
          }
        } else {
          const float s0 = sb.sw[0];
          vs[c][0] = vs[c][1] = f32x4{s0, s0, s0, s0};
        }
      } else if (ADD) {
        vb[c] = *reinterpret_cast<const u32x4*>(b + base + (size_t)idx * 8);
      }
      vw[c] = *reinterpret_cast<const u32x4*>(w + (size_t)idx * 8);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      unpack8(va[c], x[c]);
      if (ADD) {
        float y[8];
        if constexpr (SPLIT > 0) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            f32x4 t = vp[c][0][hh];
#pragma unroll
            for (int s2 = 1; s2 < SPLIT; ++s2)
              if (s2 < sb.splits) t = t + vp[c][s2][hh];
#pragma unroll
            for (int r = 0; r < 4; ++r) y[4 * hh + r] = sb.sa ? (t[r] * sav) * vs[c][hh][r] : t[r];
          }
          const u32x4 yb = pack8(y);
          *reinterpret_cast<u32x4*>(sb.y + base + (size_t)idx * 8) = yb;
          unpack8(yb, y);
        } else {
          unpack8(vb[c], y);
        }
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
  const float var = block_sum_rt(ss, red) / (float)h;
  const float inv = rsqrt_rn(var + eps);
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = threadIdx.x + c * nt;
    if (idx < nchunk) {
      float wv[8];
      unpack8(vw[c], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[c][i] = round_bf16(round_bf16(x[c][i] * inv) * wv[i]);
        amax = fmaxf(amax, fabsf(x[c][i]));
      }
      if (WRITE_OUT) *reinterpret_cast<u32x4*>(out + base + (size_t)idx * 8) = pack8(x[c]);
    }
  }
  if constexpr (QUANT == kStatic) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = threadIdx.x + c * nt;
      if (idx < nchunk) *reinterpret_cast<u32x2*>(q + base + (size_t)idx * 8) = quant8_static(x[c], sinv);
    }
  }
  if constexpr (QUANT == kDynamic) {
    amax = block_max_rt(amax, red);
    const float scale = fmaxf(amax, 1e-12f) / 448.0f;
    const float r = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = threadIdx.x + c * nt;
      if (idx < nchunk) *reinterpret_cast<u32x2*>(q + base + (size_t)idx * 8) = quant8(x[c], scale, r);
    }
    if (threadIdx.x == 0) scales[row] = scale;
  }
}

template <bool ADD, bool DEEP, bool WRITE_RES, bool WRITE_OUT, int QUANT, int SPLIT = 0>
int launch_row_norm(const void* a, const void* b, const void* deep, const void* w, void* residual,
                    void* out, void* q, float* scales, int64_t rows, int64_t h, float eps,
                    int64_t start, int64_t nv, hipStream_t s, const char* name, float sinv = 0.f,
                    SplitAddend sb = SplitAddend{}) {
  int threads, cpt;
  row_shape(h / 8, &threads, &cpt);
  dim3 grid((unsigned)rows), block((unsigned)threads);
#define FF_ROWNORM_CASE(N)                                                                              \
  case N:                                                                                               \
    hipLaunchKernelGGL((row_norm_kernel<N, ADD, DEEP, WRITE_RES, WRITE_OUT, QUANT, SPLIT>), grid, block, \
                       0, s, (const bf16_t*)a, (const bf16_t*)b, (const bf16_t*)deep,                    \
                       (const bf16_t*)w, (bf16_t*)residual, (bf16_t*)out, (uint8_t*)q, scales,           \
                       (int)h, eps, (int)start, (int)nv, sinv, sb);                                      \
    break;
  switch (cpt) {
    FF_ROWNORM_CASE(1)
    FF_ROWNORM_CASE(2)
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

// One workgroup per answer option c: normalise the (optionally summed) row,
// then z_c = bf16(sum_k x_hat_k * head[c, k]). Each workgroup recomputes the
// row norm (h values), so the options run in parallel with no second pass.
template <int CPT>
__global__ __launch_bounds__(1024) void readout_kernel(const bf16_t* __restrict__ x,
                                                      const bf16_t* __restrict__ x2,
                                                      const bf16_t* __restrict__ w,
                                                      const bf16_t* __restrict__ head,
                                                      float* __restrict__ y, int h, float eps) {
  __shared__ float red[16];
  const int c = blockIdx.x, nt = blockDim.x, nchunk = h >> 3;
  float v[CPT][8];
  u32x4 vx[CPT], vx2[CPT], vw[CPT], vh[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int idx = threadIdx.x + k * nt;
    if (idx < nchunk) {
      vx[k] = *reinterpret_cast<const u32x4*>(x + (size_t)idx * 8);
      if (x2) vx2[k] = *reinterpret_cast<const u32x4*>(x2 + (size_t)idx * 8);
      vw[k] = *reinterpret_cast<const u32x4*>(w + (size_t)idx * 8);
      vh[k] = *reinterpret_cast<const u32x4*>(head + (size_t)c * h + (size_t)idx * 8);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int idx = threadIdx.x + k * nt;
    if (idx < nchunk) {
      unpack8(vx[k], v[k]);
      if (x2) {
        float t[8];
        unpack8(vx2[k], t);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[k][i] = round_bf16(v[k][i] + t[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[k][i] * v[k][i];
    }
  }
  const float inv = rsqrt_rn(block_sum_rt(ss, red) / (float)h + eps);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int idx = threadIdx.x + k * nt;
    if (idx < nchunk) {
      float wv[8], hv[8];
      unpack8(vw[k], wv);
      unpack8(vh[k], hv);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += round_bf16(round_bf16(v[k][i] * inv) * wv[i]) * hv[i];
    }
  }
  acc = block_sum_rt(acc, red);
  if (threadIdx.x == 0) y[c] = round_bf16(acc);
}

}  // namespace

extern "C" int ff_fast_norm(const void* x, const void* w, void* out, int64_t rows, int64_t h,
                            float eps, ff_stream_t stream) {
  int st = check_rows("ff_fast_norm", x, rows, h);
  if (st) return st;
  FF_REQUIRE(out && w && ff_aligned(out, 16) && ff_aligned(w, 16), "ff_fast_norm: bad out/w");
  if (rows == 0) return FF_OK;
  return launch_row_norm<false, false, false, true, kNoQuant>(x, nullptr, nullptr, w, nullptr, out,
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
    return launch_row_norm<false, false, false, true, kDynamic>(x, nullptr, nullptr, w, nullptr, out, q,
                                                            scales, rows, h, eps, 0, 0, s,
                                                            "ff_fast_norm_quant");
  return launch_row_norm<false, false, false, false, kDynamic>(x, nullptr, nullptr, w, nullptr, nullptr,
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
    return launch_row_norm<true, true, true, true, kNoQuant>(a, b, deep, w, residual, out, nullptr,
                                                          nullptr, rows, h, eps, start, nv, s,
                                                          "ff_add_rms");
  return launch_row_norm<true, false, true, true, kNoQuant>(a, b, nullptr, w, residual, out, nullptr,
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
    return launch_row_norm<true, true, true, true, kDynamic>(a, b, deep, w, residual, out, q, scales, rows,
                                                         h, eps, start, nv, s, "ff_add_rms_quant");
  if (d)
    return launch_row_norm<true, true, true, false, kDynamic>(a, b, deep, w, residual, nullptr, q, scales,
                                                          rows, h, eps, start, nv, s,
                                                          "ff_add_rms_quant");
  if (out)
    return launch_row_norm<true, false, true, true, kDynamic>(a, b, nullptr, w, residual, out, q, scales,
                                                          rows, h, eps, 0, 0, s, "ff_add_rms_quant");
  return launch_row_norm<true, false, true, false, kDynamic>(a, b, nullptr, w, residual, nullptr, q,
                                                         scales, rows, h, eps, 0, 0, s,
                                                         "ff_add_rms_quant");
}

extern "C" int ff_fast_norm_quant_static(const void* x, const void* w, void* out, void* q, float inv, int64_t rows,
                                         int64_t h, float eps, ff_stream_t stream) {
  int st = check_rows("ff_fast_norm_quant_static", x, rows, h);
  if (st) return st;
  FF_REQUIRE(q && w && ff_aligned(q, 8) && ff_aligned(w, 16), "ff_fast_norm_quant_static: bad q/w");
  FF_REQUIRE(!out || ff_aligned(out, 16), "ff_fast_norm_quant_static: out not aligned");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  if (out)
    return launch_row_norm<false, false, false, true, kStatic>(x, nullptr, nullptr, w, nullptr, out, q, nullptr,
                                                               rows, h, eps, 0, 0, s, "ff_fast_norm_quant_static",
                                                               inv);
  return launch_row_norm<false, false, false, false, kStatic>(x, nullptr, nullptr, w, nullptr, nullptr, q, nullptr,
                                                              rows, h, eps, 0, 0, s, "ff_fast_norm_quant_static",
                                                              inv);
}

extern "C" int ff_add_rms_quant_static(const void* a, const void* b, const void* deep, const void* w,
                                       void* residual, void* out, void* q, float inv, int64_t rows, int64_t h,
                                       float eps, int64_t start, int64_t nv, ff_stream_t stream) {
  int st = check_rows("ff_add_rms_quant_static", a, rows, h);
  if (st) return st;
  FF_REQUIRE(b && w && residual && q && ff_aligned(b, 16) && ff_aligned(w, 16) && ff_aligned(residual, 16) &&
                 ff_aligned(q, 8),
             "ff_add_rms_quant_static: bad b/w/residual/q");
  FF_REQUIRE(!out || ff_aligned(out, 16), "ff_add_rms_quant_static: out not aligned");
  FF_REQUIRE(!deep || (ff_aligned(deep, 16) && nv >= 0 && start >= 0), "ff_add_rms_quant_static: bad deep");
  if (rows == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool d = deep && nv > 0;
  const char* nm = "ff_add_rms_quant_static";
  if (d && out)
    return launch_row_norm<true, true, true, true, kStatic>(a, b, deep, w, residual, out, q, nullptr, rows, h, eps,
                                                            start, nv, s, nm, inv);
  if (d)
    return launch_row_norm<true, true, true, false, kStatic>(a, b, deep, w, residual, nullptr, q, nullptr, rows, h,
                                                             eps, start, nv, s, nm, inv);
  if (out)
    return launch_row_norm<true, false, true, true, kStatic>(a, b, nullptr, w, residual, out, q, nullptr, rows, h,
                                                             eps, 0, 0, s, nm, inv);
  return launch_row_norm<true, false, true, false, kStatic>(a, b, nullptr, w, residual, nullptr, q, nullptr, rows,
                                                            h, eps, 0, 0, s, nm, inv);
}

extern "C" int ff_lm_readout(const void* x, const void* x2, const void* norm_w, const void* head,
                             float* y, int64_t h, int64_t n_opt, float eps, ff_stream_t stream) {
  FF_REQUIRE(x && norm_w && head && y, "ff_lm_readout: null pointer");
  FF_REQUIRE(h > 0 && h % 8 == 0 && h <= 16384 && n_opt > 0 && n_opt <= 65535,
             "ff_lm_readout: bad h=%lld n_opt=%lld", (long long)h, (long long)n_opt);
  FF_REQUIRE(ff_aligned(x, 16) && (!x2 || ff_aligned(x2, 16)) && ff_aligned(norm_w, 16) && ff_aligned(head, 16),
             "ff_lm_readout: x, x2, norm_w and head must be 16-byte aligned");
  int threads, cpt;
  row_shape(h / 8, &threads, &cpt);
  if (cpt == 1)
    hipLaunchKernelGGL(readout_kernel<1>, dim3((unsigned)n_opt), dim3((unsigned)threads), 0, (hipStream_t)stream,
                       (const bf16_t*)x, (const bf16_t*)x2, (const bf16_t*)norm_w, (const bf16_t*)head, y, (int)h,
                       eps);
  else
    hipLaunchKernelGGL(readout_kernel<2>, dim3((unsigned)n_opt), dim3((unsigned)threads), 0, (hipStream_t)stream,
                       (const bf16_t*)x, (const bf16_t*)x2, (const bf16_t*)norm_w, (const bf16_t*)head, y, (int)h,
                       eps);
  FF_LAUNCH_CHECK("ff_lm_readout");
  return FF_OK;
}

// ---------------------------------------------------------------- GEMM + add_rms

// ff_gemm_fp8_pk into y, then ff_add_rms_quant(a, y, ..) (or its static form).
// Where the GEMM splits k, the row kernel adds the split partials itself (and
// stores y) instead of a separate reduction launch; elsewhere the two entry
// points run as they are.
namespace {
template <int QUANT>
int gemm_add_rms(const char* name, const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                 const float* sw, int sw_cols, void* y, int64_t m, int64_t n, int64_t k, void* workspace,
                 int64_t workspace_bytes, const void* a, const void* deep, const void* w, void* residual, void* q,
                 float* scales, float inv, float eps, int64_t start, int64_t nv, ff_stream_t stream) {
  int st = check_rows(name, a, m, n);
  if (st) return st;
  FF_REQUIRE(qa && sa && (qw || qw_packed) && sw && y && w && residual && q && (QUANT != kDynamic || scales),
             "%s: null pointer", name);
  FF_REQUIRE(ff_aligned(y, 16) && ff_aligned(w, 16) && ff_aligned(residual, 16) && ff_aligned(q, 8),
             "%s: y, w and residual must be 16-byte aligned, q 8-byte", name);
  FF_REQUIRE(!deep || (ff_aligned(deep, 16) && nv >= 0 && start >= 0), "%s: bad deep", name);
  if (m == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  int splits = 0;
  int64_t mp = 0;
  st = ff::gemm_fp8_pk_partials(qa, sa, sa_rows, qw_packed, sw, sw_cols, m, n, k, workspace, workspace_bytes, s,
                                &splits, &mp);
  if (st) return st;
  if (splits == 0) {
    st = ff_gemm_fp8_pk(qa, sa, sa_rows, qw, qw_packed, sw, sw_cols, y, n, m, n, k, workspace, workspace_bytes,
                        stream);
    if (st) return st;
    if constexpr (QUANT == kDynamic)
      return ff_add_rms_quant(a, y, deep, w, residual, nullptr, q, scales, m, n, eps, start, nv, stream);
    else
      return ff_add_rms_quant_static(a, y, deep, w, residual, nullptr, q, inv, m, n, eps, start, nv, stream);
  }
  FF_REQUIRE(splits >= 2 && splits <= 8, "%s: unexpected split count %d", name, splits);
  SplitAddend sb;
  sb.part = (const float*)workspace;
  sb.mp = mp;
  sb.splits = splits;
  sb.sa = sa;
  sb.sa_rows = sa_rows;
  sb.sw = sw;
  sb.sw_cols = sw_cols;
  sb.y = (bf16_t*)y;
  if (deep && nv > 0)
    return splits > 4 ? launch_row_norm<true, true, true, false, QUANT, 8>(a, nullptr, deep, w, residual, nullptr, q,
                                                                          scales, m, n, eps, start, nv, s, name, inv,
                                                                          sb)
                      : launch_row_norm<true, true, true, false, QUANT, 4>(a, nullptr, deep, w, residual, nullptr, q,
                                                                          scales, m, n, eps, start, nv, s, name, inv,
                                                                          sb);
  return splits > 4 ? launch_row_norm<true, false, true, false, QUANT, 8>(a, nullptr, nullptr, w, residual, nullptr, q,
                                                                         scales, m, n, eps, 0, 0, s, name, inv, sb)
                    : launch_row_norm<true, false, true, false, QUANT, 4>(a, nullptr, nullptr, w, residual, nullptr, q,
                                                                         scales, m, n, eps, 0, 0, s, name, inv, sb);
}
}  // namespace

extern "C" int ff_gemm_fp8_pk_add_rms_quant(const void* qa, const float* sa, int sa_rows, const void* qw,
                                            const void* qw_packed, const float* sw, int sw_cols, void* y, int64_t m,
                                            int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                                            const void* a, const void* deep, const void* w, void* residual, void* q,
                                            float* scales, float eps, int64_t start, int64_t nv, ff_stream_t stream) {
  return gemm_add_rms<kDynamic>("ff_gemm_fp8_pk_add_rms_quant", qa, sa, sa_rows, qw, qw_packed, sw, sw_cols, y, m, n,
                                k, workspace, workspace_bytes, a, deep, w, residual, q, scales, 0.f, eps, start, nv,
                                stream);
}

extern "C" int ff_gemm_fp8_pk_add_rms_quant_static(const void* qa, const float* sa, int sa_rows, const void* qw,
                                                   const void* qw_packed, const float* sw, int sw_cols, void* y,
                                                   int64_t m, int64_t n, int64_t k, void* workspace,
                                                   int64_t workspace_bytes, const void* a, const void* deep,
                                                   const void* w, void* residual, void* q, float inv, float eps,
                                                   int64_t start, int64_t nv, ff_stream_t stream) {
  return gemm_add_rms<kStatic>("ff_gemm_fp8_pk_add_rms_quant_static", qa, sa, sa_rows, qw, qw_packed, sw, sw_cols, y,
                               m, n, k, workspace, workspace_bytes, a, deep, w, residual, q, nullptr, inv, eps, start,
                               nv, stream);
}

// ff_gemm_w4a16_pk into y, then ff_add_rms(a, y, ..), with the split-K
// partials (where that GEMM splits k on the packed copies) added by the
// add_rms launch in place of the reduction launch.
extern "C" int ff_gemm_w4a16_pk_add_rms(const void* x, int64_t ldx, const void* packed, const void* frag,
                                        const void* scales, const void* frag_scales, int64_t group, void* y, int64_t m,
                                        int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, const void* a,
                                        const void* deep, const void* w, void* residual, void* out, float eps,
                                        int64_t start, int64_t nv, ff_stream_t stream) {
  const char* name = "ff_gemm_w4a16_pk_add_rms";
  int st = check_rows(name, a, m, n);
  if (st) return st;
  FF_REQUIRE(x && y && w && residual && out, "%s: null pointer", name);
  FF_REQUIRE(ff_aligned(y, 16) && ff_aligned(w, 16) && ff_aligned(residual, 16) && ff_aligned(out, 16),
             "%s: y, w, residual and out must be 16-byte aligned", name);
  FF_REQUIRE(!deep || (ff_aligned(deep, 16) && nv >= 0 && start >= 0), "%s: bad deep", name);
  if (m == 0) return FF_OK;
  hipStream_t s = (hipStream_t)stream;
  int splits = 0;
  int64_t mp = 0;
  st = ff::gemm_w4a16_pk_partials(x, ldx, frag, frag_scales, group, m, n, k, workspace, workspace_bytes, s, &splits,
                                  &mp);
  if (st) return st;
  if (splits == 0) {
    st = ff_gemm_w4a16_pk(x, ldx, packed, frag, scales, frag_scales, group, y, n, m, n, k, workspace, workspace_bytes,
                          stream);
    if (st) return st;
    return ff_add_rms(a, y, deep, w, residual, out, m, n, eps, start, nv, stream);
  }
  FF_REQUIRE(splits <= 8, "%s: unexpected split count %d", name, splits);
  SplitAddend sb;
  sb.part = (const float*)workspace;
  sb.mp = mp;
  sb.splits = splits;
  sb.y = (bf16_t*)y;
  if (deep && nv > 0)
    return launch_row_norm<true, true, true, true, kNoQuant, 8>(a, nullptr, deep, w, residual, out, nullptr, nullptr,
                                                                m, n, eps, start, nv, s, name, 0.f, sb);
  return launch_row_norm<true, false, true, true, kNoQuant, 8>(a, nullptr, nullptr, w, residual, out, nullptr, nullptr,
                                                               m, n, eps, 0, 0, s, name, 0.f, sb);
}
