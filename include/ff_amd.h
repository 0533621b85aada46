/*
 * ff_amd.h — C ABI of the MI355X (gfx950) Qwen3-VL LM-step kernels.
 *
 * Every entry point takes raw device pointers, sizes, strides and scalars plus an
 * explicit HIP stream (ff_stream_t, a hipStream_t; NULL = the null stream). None
 * of them allocates device memory, synchronises the host or picks a grid size
 * from device data, so all of them may be captured into a hipGraph. Tensors are
 * bf16 (raw 16-bit), e4m3fn (raw 8-bit) or fp32 unless stated. Returns FF_OK or a
 * negative status; ff_last_error() then holds a message for the calling thread.
 *
 * Reference paths are relative to FastForward's src/fastforward_accel/.
 */
#ifndef FF_AMD_H
#define FF_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ff_stream_t;

#define FF_OK 0
#define FF_EINVAL (-1)   /* bad shape, stride, alignment or argument */
#define FF_ELAUNCH (-2)  /* kernel launch failed */
#define FF_EDEVICE (-3)  /* no usable gfx950 device */

/* Library version (major*10000 + minor*100 + patch). */
int ff_version(void);
/* Message for the last failing call on this thread ("" if none). */
const char* ff_last_error(void);
/* FF_OK if the current HIP device is a gfx950 (MI355X). */
int ff_device_check(void);

/* Tile-choice overrides for measurement sweeps and tests (no reference
 * counterpart). `value` 0 restores the library's own choice for `knob`. The
 * library never reads them from the environment: a process that does not call
 * ff_set_tuning runs the built-in choices. Set them only while no launch of an
 * affected entry point is being issued from another thread. */
#define FF_TUNE_GEMM_FP8_TILE 1   /* ff_gemm_fp8 / _qkv: 1 64x128, 2 128x128, 3 128x128 4-stage, 4 128x256 */
#define FF_TUNE_GEMM_BF16_TILE 2  /* ff_gemm_bf16: 1 64x128, 2 128x128, 3 64x128 at three per CU */
#define FF_TUNE_W4A16_TILE 3      /* ff_gemm_w4a16*: 1 64x256, 2 192x192 */
#define FF_TUNE_W4A16_SPLITS 4    /* ff_gemm_w4a16_ws: k splits of the 64x256 tile, 1..8 */
#define FF_TUNE_ATTN_QT 5         /* ff_attention_vt prefill (1, 2 or 4) / ff_attention_full (1 or 2): query tiles per wave */
#define FF_TUNE_ATTN_NS 6         /* ff_attention_vt prefill: K/V LDS stages, 2 or 3 */
#define FF_TUNE_QKV_PK_TILE 7     /* ff_gemm_fp8_qkv_pk: 1 64x256 packed, 2 64x128 packed, 3 row-major,
                                     4 96x128, 5 144x128, 6 128x128 packed */
#define FF_TUNE_SWIGLU_PK_TILE 8  /* ff_gemm_fp8_swiglu_pk / _static: 1000 BM + CW (BM x 8 CW tile) */
#define FF_TUNE_FP8_PK_SPLIT 9    /* ff_gemm_fp8_pk: 100 BM + k splits (1..6 or 8), BM 64 or 144 (256-column
                                     tiles); 100000 + 100 BM + k splits, BM 64, 80, 96, 128 or 144 (128-column
                                     tiles) */
#define FF_TUNE_BF16_PK_SPLIT 10  /* ff_gemm_bf16_pk_ws / _ln: 1 no k split, 2..8 the split count */
#define FF_TUNE_FP8_PK_SPLIT_SHORT_K 11 /* as FF_TUNE_FP8_PK_SPLIT, for k <= 4096 only (ahead of it there) */
int ff_set_tuning(int knob, int value);

/* fast_norm(x, module): out = bf16(bf16(x*rsqrt(sum(x^2)/h + eps)) * w), one row
 * per token. Replaces _legacy/sub10_runtime.py:37 (fast_norm / rms_one :31-36).
 * x, out: (rows, h) contiguous, h % 8 == 0, h <= 16384. */
int ff_fast_norm(const void* x, const void* w, void* out, int64_t rows, int64_t h, float eps,
                 ff_stream_t stream);

/* add_rms(a, b, deep, module, start, nv) -> (residual, out): x = bf16(a+b); rows
 * r in [start, start+nv) add bf16(x + deep[r-start]) when deep != NULL; residual
 * = x; out = bf16(bf16(x*rsqrt(mean(x^2)+eps))*w). Replaces
 * _legacy/lower_kernels.py:24 (kernel :7-21) and _legacy/broad_kernels.py:9. */
int ff_add_rms(const void* a, const void* b, const void* deep, const void* w, void* residual,
               void* out, int64_t rows, int64_t h, float eps, int64_t start, int64_t nv,
               ff_stream_t stream);

/* Fused producer variants (no reference counterpart as separate ops; same
 * arithmetic as ff_add_rms / ff_fast_norm followed by ff_quant_rows_fp8 on
 * `out`): additionally write the per-token e4m3 codes q (rows, h) and fp32
 * scales (rows) of the normalised output. `out` may be NULL to skip the bf16
 * normalised output. */
int ff_add_rms_quant(const void* a, const void* b, const void* deep, const void* w, void* residual,
                     void* out, void* q, float* scales, int64_t rows, int64_t h, float eps,
                     int64_t start, int64_t nv, ff_stream_t stream);
int ff_fast_norm_quant(const void* x, const void* w, void* out, void* q, float* scales,
                       int64_t rows, int64_t h, float eps, ff_stream_t stream);

/* qk_pair(q, k, qn, kn, cos, sin): per (token, head) RMSNorm over d with weight
 * wq / wk, then rotate-half M-RoPE: y = bf16(bf16(x*cos) + bf16(rot(x)*sin)).
 * q (t, hq, d) and k (t, hk, d) are strided views with token stride `row_stride`
 * elements (e.g. the packed QKV output); cos/sin (t, d) with strides
 * (cos_ts, cos_ds). Writes yq (hq, t, d), yk (hk, t, d) contiguous.
 * Replaces _legacy/broad_kernels.py:63 (kernel _legacy/lower_kernels.py:66-98).
 * d == 128. */
int ff_qk_pair(const void* q, const void* k, int64_t row_stride, const void* wq, const void* wk,
               float eps_q, float eps_k, const void* cos, const void* sin, int64_t cos_ts,
               int64_t cos_ds, int64_t sin_ts, int64_t sin_ds, void* yq, void* yk, int64_t t,
               int64_t hq, int64_t hk, int64_t d, ff_stream_t stream);

/* Fused q/k/v post-processing for the layer loop: ff_qk_pair plus a transposed
 * copy of v (hk, d, t_pad) with keys contiguous and zeros for keys in [t, t_pad),
 * the layout ff_attention_vt consumes. v is the strided view (t, hk, d) with the
 * same token stride. t_pad % 64 == 0, t_pad >= t. */
int ff_qkv_post(const void* q, const void* k, const void* v, int64_t row_stride, const void* wq,
                const void* wk, float eps_q, float eps_k, const void* cos, const void* sin,
                void* yq, void* yk, void* vt, int64_t t, int64_t t_pad, int64_t hq, int64_t hk,
                int64_t d, ff_stream_t stream);

/* Transposed copy of v (t, hk, d) [token stride v_ts, head stride v_hs] into
 * vt (hk, d, t_pad), zero-filling keys >= t. */
int ff_v_transpose(const void* v, int64_t v_ts, int64_t v_hs, void* vt, int64_t t, int64_t t_pad,
                   int64_t hk, int64_t d, ff_stream_t stream);

/* swiglu(gate, up): y = bf16(bf16(g/(1+exp(-g))) * u). g, u: (rows, i) views with
 * row stride `row_stride` elements; y (rows, i) contiguous. Replaces
 * _legacy/search_kernels.py:18 (kernel :8-15). i % 8 == 0. */
int ff_swiglu(const void* g, const void* u, int64_t row_stride, void* y, int64_t rows, int64_t i,
              ff_stream_t stream);
/* swiglu followed by per-token e4m3 quant of y (codes q (rows, i), scales (rows)).
 * y may be NULL. */
int ff_swiglu_quant(const void* g, const void* u, int64_t row_stride, void* y, void* q,
                    float* scales, int64_t rows, int64_t i, ff_stream_t stream);

/* attention_direct(q, k, v, scale, positions=None, triangular=True): causal GQA
 * attention with fp32 scores/softmax statistics, P rounded to bf16 before P.V,
 * fp32 accumulation. q (hq, s, d) contiguous, k (hk, t, d) contiguous, vt the
 * transposed v (hk, d, t_pad) from ff_qkv_post / ff_v_transpose. positions
 * (int64, s) gives each query's position (SELECTED mode) or NULL for row i at
 * position i. With gather_q != 0, q is (hq, t, d) and query i reads q row
 * positions[i] (the tail's q.index_select(2, pick) fused in). y (s, hq, d).
 * Replaces _legacy/limit_kernels.py:36 (kernel :8-33). d == 128, hq % hk == 0. */
int ff_attention_vt(const void* q, const void* k, const void* vt, const int64_t* positions,
                    int gather_q, void* y, int64_t s, int64_t t, int64_t t_pad, int64_t hq,
                    int64_t hk, int64_t d, float scale, ff_stream_t stream);

/* lm_readout(x, norm, weight): x_hat = bf16(bf16(x*rsqrt(mean(x^2)+eps))*w);
 * y[c] = bf16(sum_k x_hat_k * head[c,k]) stored as fp32. If x2 != NULL the
 * input row is bf16(x + x2) (the tail's `residual + mlp` add). x (h), head
 * (n_opt, h) contiguous, h % 8 == 0, h <= 16384, x / x2 / norm_w / head
 * 16-byte aligned; y (n_opt) fp32. Replaces _legacy/limit_kernels.py:60
 * (kernel :48-57). */
int ff_lm_readout(const void* x, const void* x2, const void* norm_w, const void* head, float* y,
                  int64_t h, int64_t n_opt, float eps, ff_stream_t stream);

/* Per-token dynamic activation quant: scale[m] = max(amax_k|x[m,k]|, 1e-12)/448,
 * q = e4m3(clamp(x/scale, +-448)). x (rows, k) with row stride x_rs elements.
 * Replaces quantize_rows, _legacy/fp8_private.py:11-18. */
int ff_quant_rows_fp8(const void* x, int64_t x_rs, void* q, float* scales, int64_t rows, int64_t k,
                      ff_stream_t stream);

/* Static per-tensor activation quant: q = e4m3(clamp(x*inv, +-448)) for the first
 * `rows` rows; rows in [rows, rows_pad) are written as zero codes. Replaces
 * _runtime_scale / quantize_runtime, _family/depth_fp8.py:8-19. */
int ff_quant_static_fp8(const void* x, void* q, int64_t rows, int64_t rows_pad, int64_t k,
                        float inv, ff_stream_t stream);

/* Setup-time weight quant. per_channel != 0: scale[n] = max(amax_k|W[n,k]|,
 * 1e-12)/448 (FP8Linear.__init__, _legacy/fp8_private.py:22-27); else one scale
 * for the tensor (StaticFP8Linear.__init__, _legacy/limit_kernels.py:122-127),
 * which needs a caller-provided fp32 workspace of n floats (row amax).
 * q = e4m3(clamp(W/scale, +-448)). w (n, k) bf16 contiguous. */
int ff_quant_weight_fp8(const void* w, void* q, float* scale, float* workspace, int64_t n,
                        int64_t k, int per_channel, ff_stream_t stream);

/* FP8 GEMM: y (m, n) bf16 = bf16(sum_k qa[m,k]*qw[n,k] * sa * sw) with fp32
 * accumulation (torch._scaled_mm as called at _legacy/fp8_private.py:36 and
 * _family/depth_fp8.py:25). qa (m, k) and qw (n, k) e4m3 row-major; sa is per-row
 * (m floats) if sa_rows else one float; sw is per-column (n floats) if sw_cols
 * else one float. y row stride ldy elements. k % 128 == 0. */
int ff_gemm_fp8(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw,
                int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                ff_stream_t stream);

/* Fused gate/up GEMM + SwiGLU (no reference counterpart as one op; the same
 * arithmetic as ff_gemm_fp8 on the packed gate/up weight followed by ff_swiglu):
 * qw (2i, k) e4m3 = [gate rows; up rows] with per-row scales sw (2i); qa (m, k)
 * with per-token scales sa (m). Writes h (m, i) bf16 (row stride ldh) =
 * bf16(bf16(silu(g)) * u) for g, u the bf16 GEMM outputs, and pmax (m, i/64)
 * fp32, the max |h| of each row over each 64-channel block, for
 * ff_quant_rows_pmax. i % 64 == 0, k % 128 == 0. */
int ff_gemm_fp8_swiglu(const void* qa, const float* sa, const void* qw, const float* sw, void* h,
                       int64_t ldh, float* pmax, int64_t m, int64_t i, int64_t k, ff_stream_t stream);

/* Setup-time repack of e4m3 weights w (n, k) row-major into the MFMA fragment
 * layout read by ff_gemm_fp8_swiglu_pk, ff_gemm_fp8_pk and ff_gemm_fp8_qkv_pk
 * (no reference counterpart: a storage layout of this library): fragment (f,
 * kt), rows [16 f, 16 f + 16) x k bytes [128 kt, 128 kt + 128), is the 2048
 * bytes at (kt * n/16 + f) * 2048 (k-step major); lane
 * l = 16 g + r holds row 16 f + r, k bytes [128 kt + 32 g, +16) at 16 l and
 * [128 kt + 32 g + 16, +16) at 1024 + 16 l (two 1 KB planes, one load
 * instruction each). packed holds n * k bytes. n % 16 == 0, k % 128 == 0. */
int ff_pack_weight_fp8(const void* w, void* packed, int64_t n, int64_t k, ff_stream_t stream);
/* The inverse (no reference counterpart): the row-major (n, k) codes w from the
 * packed copy, for callers that keep only the packed copy and read the codes
 * themselves. n % 16 == 0, k % 128 == 0. */
int ff_unpack_weight_fp8(const void* packed, void* w, int64_t n, int64_t k, ff_stream_t stream);

/* ff_gemm_fp8_swiglu with an optional packed copy of the same weight
 * (ff_pack_weight_fp8 of qw): identical results (same products and summation
 * order); when qw_packed is given and the shape suits it (k % 512 == 0, m > 4,
 * i % 192 == 0 for BM x 384 tiles or i % 128 == 0 for BM x 256 tiles with
 * enough tiles to fill the GPU, or up to 176 tokens with i / 64 >= 192 for one
 * row tile of 64 channels per workgroup) the weights are read from the packed
 * copy straight into the matrix-core operands, otherwise this is
 * ff_gemm_fp8_swiglu on qw. qw may be NULL when the caller keeps only the
 * packed copy (i % 64 == 0, k % 512 == 0): every m then runs on it, m <= 4 on a
 * single-row kernel whose fp32 sums differ in order from the row-major one. */
int ff_gemm_fp8_swiglu_pk(const void* qa, const float* sa, const void* qw, const void* qw_packed,
                          const float* sw, void* h, int64_t ldh, float* pmax, int64_t m, int64_t i, int64_t k,
                          ff_stream_t stream);

/* ff_gemm_fp8 with an optional packed copy of the weight (ff_pack_weight_fp8 of
 * qw) and a workspace (no reference counterpart: the down projection of the
 * step, Linear.apply of scaled_qwen_runtime.py:35-39). When qw_packed is given
 * and the shape suits it the weights are read from the packed copy: 144 x 256
 * tiles when 192 or more fill the GPU; with fewer tiles and k >= 8192 k split
 * 2, 3, 4 or 8 ways; up to 256 tokens 64 x 256 tiles with k split 2, 4 or 8
 * ways; else smaller unsplit tiles (n % 128 == 0, k % 512 == 0). Each split
 * writes its fp32 partial tile to the workspace and a second launch adds the
 * partials in split order (same math as ff_gemm_fp8 up to the fp32 order of
 * adding the partials; repeatable bit for bit). Otherwise this is ff_gemm_fp8
 * on qw. qw may be NULL when the caller keeps only the packed copy (n % 128 ==
 * 0, k % 512 == 0): every m then runs on it, m <= 4 on a single-row kernel
 * whose fp32 sums differ in order from the row-major one. workspace:
 * ff_gemm_fp8_pk_workspace bytes (0 when no split is used), 16-byte aligned;
 * calls that overlap must not share it. */
int ff_gemm_fp8_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes);
int ff_gemm_fp8_pk(const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                   const float* sw, int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                   void* workspace, int64_t workspace_bytes, ff_stream_t stream);

/* Down projection + the next add_rms (no reference counterpart as one op: the
 * down Linear of scaled_qwen_runtime.py:35-39 followed by the add_rms of
 * _legacy/lower_kernels.py:7-32 with the per-token quant of
 * _legacy/fp8_private.py:11-18, or, _static, the runtime-scale cast of
 * _family/depth_fp8.py:8-19 with multiplier inv): ff_gemm_fp8_pk into y (m, n)
 * bf16 (row stride n), then ff_add_rms_quant(a, y, deep, w, residual, NULL, q,
 * scales, m, n, eps, start, nv) (_static: ff_add_rms_quant_static with inv),
 * bit for bit. Where the GEMM splits k the add_rms launch adds the fp32
 * partials itself, taking the place of the reduction launch; the workspace is
 * ff_gemm_fp8_pk_workspace bytes as for ff_gemm_fp8_pk. */
int ff_gemm_fp8_pk_add_rms_quant(const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                                 const float* sw, int sw_cols, void* y, int64_t m, int64_t n, int64_t k,
                                 void* workspace, int64_t workspace_bytes, const void* a, const void* deep,
                                 const void* w, void* residual, void* q, float* scales, float eps, int64_t start,
                                 int64_t nv, ff_stream_t stream);
int ff_gemm_fp8_pk_add_rms_quant_static(const void* qa, const float* sa, int sa_rows, const void* qw,
                                        const void* qw_packed, const float* sw, int sw_cols, void* y, int64_t m,
                                        int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                                        const void* a, const void* deep, const void* w, void* residual, void* q,
                                        float inv, float eps, int64_t start, int64_t nv, ff_stream_t stream);

/* Fused QKV GEMM + q/k norm + rotary + V transpose (no reference counterpart as
 * one op; the same arithmetic as ff_gemm_fp8 on the packed QKV weight followed
 * by ff_qkv_post): qw ((hq + 2 hk) * 128, k) e4m3 with scales sw (per row if
 * sw_cols, else sw[0]), qa (m, k) with scales sa (per token if sa_rows, else
 * sa[0]: the static-scale linears). Writes yq (hq, m, 128), yk (hk, m, 128)
 * (per-head RMSNorm with q_norm / k_norm, then rotary with cos / sin (m, 128))
 * and vt (hk, 128, t_pad) with zeros for tokens in [m, t_pad). Head dim 128.
 * Replaces the qkv linear + qk_pair of scaled_qwen_runtime.py:150-155. */
int ff_gemm_fp8_qkv(const void* qa, const float* sa, int sa_rows, const void* qw, const float* sw, int sw_cols,
                    int64_t m, int64_t k, int64_t hq, int64_t hk, const void* q_norm, const void* k_norm,
                    float eps_q, float eps_k, const void* cos, const void* sin, void* yq, void* yk, void* vt,
                    int64_t t_pad, ff_stream_t stream);
/* ff_gemm_fp8_qkv on the MFMA-fragment copy of qw (ff_pack_weight_fp8):
 * 64-token x 128-channel tiles (one head) while their grid has at most 512
 * tiles (the 8B step at 576 tokens), else 64-token x 256-channel tiles (two
 * heads) when the grid has 192..512 tiles, for m > 4, k % 512 == 0 and t_pad
 * <= the tiles' token range; the same bits as ff_gemm_fp8_qkv, which it calls
 * for every other shape (qw_packed may then be NULL). qw may be NULL when the
 * caller keeps only the packed copy: every m then runs on the packed tiles.
 * Same reference replacement as ff_gemm_fp8_qkv. */
int ff_gemm_fp8_qkv_pk(const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                       const float* sw, int sw_cols, int64_t m, int64_t k, int64_t hq, int64_t hk,
                       const void* q_norm, const void* k_norm, float eps_q, float eps_k, const void* cos,
                       const void* sin, void* yq, void* yk, void* vt, int64_t t_pad, ff_stream_t stream);

/* Static-scale (calibrated) FP8 producers of the step, no reference counterpart
 * as separate ops: each is the op it extends followed by the runtime-scale cast
 * q = e4m3(clamp(x * inv, +-448)) of _family/depth_fp8.py:8-19 (quantize_runtime)
 * on its bf16 output, with inv the consuming linear's inverse_scale, so the
 * next GEMM reads e4m3 codes directly.
 * ff_fast_norm_quant_static / ff_add_rms_quant_static: ff_fast_norm_quant /
 * ff_add_rms_quant with that cast in place of the per-token scale (out may be
 * NULL). ff_attention_vt_q: the causal prefill of ff_attention_vt (no
 * positions, s == t) writing the codes of its (s, hq, 128) output. */
int ff_fast_norm_quant_static(const void* x, const void* w, void* out, void* q, float inv, int64_t rows, int64_t h,
                              float eps, ff_stream_t stream);
int ff_add_rms_quant_static(const void* a, const void* b, const void* deep, const void* w, void* residual, void* out,
                            void* q, float inv, int64_t rows, int64_t h, float eps, int64_t start, int64_t nv,
                            ff_stream_t stream);
int ff_attention_vt_q(const void* q, const void* k, const void* vt, void* yq, float inv, int64_t s, int64_t t,
                      int64_t t_pad, int64_t hq, int64_t hk, int64_t d, float scale, ff_stream_t stream);
/* Gate/up GEMM with the SwiGLU epilogue for static-scale linears: per-tensor
 * scales sa[0], sw[0]; h = bf16(bf16(silu(g)) * u) written as the codes
 * e4m3(clamp(h * inv, +-448)) (m, i) with row pitch ldh bytes (inv: the down
 * projection's inverse_scale). The packed tile when qw_packed is given and
 * the shape suits it (as ff_gemm_fp8_swiglu_pk), else the row-major tile or,
 * for m <= 4, the GEMV kernel; with qw NULL (only the packed copy kept) every
 * m runs on the packed copy, as in ff_gemm_fp8_swiglu_pk. */
int ff_gemm_fp8_swiglu_static(const void* qa, const float* sa, const void* qw, const void* qw_packed, const float* sw,
                              void* hq, int64_t ldh, float inv, int64_t m, int64_t i, int64_t k, ff_stream_t stream);

/* ff_quant_rows_fp8 with the row amax given as npart partial maxima per row
 * (pmax (rows, npart), as ff_gemm_fp8_swiglu writes them): identical codes and
 * scales, no reduction over x. */
int ff_quant_rows_pmax(const void* x, int64_t x_rs, const float* pmax, int64_t npart, void* q,
                       float* scales, int64_t rows, int64_t k, ff_stream_t stream);

/* Setup-time int4 quant of w (n, k) bf16 into packed nibbles (n, k/2) (even k in
 * the high nibble) and scales [k/group, n, 2] bf16 (scale, zero).
 * symmetric != 0: s = bf16(max(amax|w|,1e-6)/7), q = clamp(rint(w/s)+8, 0, 15),
 * zero = 0. symmetric == 0: the reference's asymmetric min/max form
 * (Int4.__init__, _family/night_runtime.py:16-26). */
int ff_quant_weight_int4(const void* w, void* packed, void* scales, int64_t n, int64_t k,
                         int64_t group, int symmetric, ff_stream_t stream);

/* W4A16 GEMM: y (m, n) bf16 = x (m, k) bf16 @ dequant(W)^T with dequant
 * w = (q-8)*s + z fused into the B-operand load, fp32 accumulation (Int4.__call__,
 * _family/night_runtime.py:31-42). x row stride ldx; k % 128 == 0, group 32 or
 * a multiple of 64 dividing k; n, ldx, ldy multiples of 8; x, packed, scales and
 * y 16-byte aligned. */
int ff_gemm_w4a16(const void* x, int64_t ldx, const void* packed, const void* scales,
                  int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                  ff_stream_t stream);

/* The same product with a caller-provided device workspace (the reference's
 * _weight_int4pack_mm call at _family/night_runtime.py:33 allocates inside its
 * library; here the caller allocates, so the call stays graph-capturable). Shapes
 * whose tile grid would leave CUs idle split K; the fp32 partial sums go to the
 * workspace and a second launch adds them in split order (deterministic) and
 * rounds to bf16. ff_gemm_w4a16_workspace stores the bytes the split wants (0:
 * none); a smaller workspace lowers the split, and 0 bytes is ff_gemm_w4a16.
 * workspace must be 16-byte aligned. */
int ff_gemm_w4a16_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes);
int ff_gemm_w4a16_ws(const void* x, int64_t ldx, const void* packed, const void* scales,
                     int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                     void* workspace, int64_t workspace_bytes, ff_stream_t stream);

/* ff_gemm_w4a16_ws without a workspace argument and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The split-K partials go to a static device scratch of
 * 32 MiB per GPU, held until the process ends. The split the library picks by
 * itself always fits (it keeps splits * m * n <= 2^23); a split forced with
 * ff_set_tuning that wants more is rejected with FF_EINVAL. Results equal
 * ff_gemm_w4a16_ws given ff_gemm_w4a16_workspace bytes, bit for bit. All calls
 * on one GPU share its scratch: calls that overlap in time on one GPU race. */
int ff_gemm_w4a16_noalloc(const void* x, int64_t ldx, const void* packed, const void* scales,
                          int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                          ff_stream_t stream);

/* Setup-time copy of an int4 weight in MFMA fragment order for the packed
 * kernels below (no reference counterpart: the reference repacks its Int4
 * weights once for its library kernel, _family/night_runtime.py:27). packed
 * (n, k/2) in the ff_quant_weight_int4 layout; frag receives n * k / 2 bytes:
 * the 16 rows x 128 k of fragment (f, kt) at (kt n/16 + f) * 1024, lane
 * l = 16 g + r holding row 16 f + r, the bytes of k = 128 kt + 64 h + 16 g +
 * [0, 16) for h = 0, 1 at 16 l, each nibble q stored as q ^ 8. n % 16 == 0,
 * k % 128 == 0. */
int ff_pack_weight_int4(const void* packed, void* frag, int64_t n, int64_t k, ff_stream_t stream);

/* Setup-time copy of the (scale, zero) pairs for the packed kernels: scales
 * [k/group, n, 2] bf16 -> frag_scales [k/group, n, 2] fp32 holding (16 s, z)
 * (16 s is exact for |s| < 2^124; larger scales must stay on ff_gemm_w4a16). */
int ff_pack_scales_int4(const void* scales, void* frag_scales, int64_t n, int64_t k, int64_t group,
                        ff_stream_t stream);

/* ff_gemm_w4a16_ws with the fragment copies (ff_pack_weight_int4 of packed and
 * ff_pack_scales_int4 of scales): the weights are read from frag straight into
 * registers (Int4.__call__,
 * _family/night_runtime.py:31-42). The same dequantised values and, unsplit,
 * the same bits as ff_gemm_w4a16; where it splits K (grids that would leave
 * CUs idle) the fp32 partials go to the workspace and a second launch adds them
 * in split order. Rows m <= 4 (n % 16, k % 128) run a GEMV on the same
 * copies: the same bf16 weights, summed in another fp32 order. Shapes neither
 * takes (k % 256 for m > 4, group not a power of two >= 32, n % 256 unless the
 * 144 x 384 tiles fill the GPU) and a null frag run ff_gemm_w4a16_ws on
 * packed / scales. ff_gemm_w4a16_pk_workspace stores
 * the bytes either path wants; workspace 16-byte aligned; calls that overlap
 * must not share it. */
int ff_gemm_w4a16_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t group, int64_t* bytes);
int ff_gemm_w4a16_pk(const void* x, int64_t ldx, const void* packed, const void* frag, const void* scales,
                     const void* frag_scales, int64_t group, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                     void* workspace, int64_t workspace_bytes, ff_stream_t stream);

/* An Int4 linear + the add_rms it feeds (no reference counterpart as one op:
 * Linear.apply of an Int4, _family/night_runtime.py:31-42, followed by the
 * add_rms of _legacy/lower_kernels.py:7-32): ff_gemm_w4a16_pk into y (m, n)
 * bf16 (row stride n), then ff_add_rms(a, y, deep, w, residual, out, m, n,
 * eps, start, nv), bit for bit. Where the GEMM splits k on the packed copies
 * the add_rms launch adds the fp32 partials itself, taking the place of the
 * reduction launch; workspace as for ff_gemm_w4a16_pk. */
int ff_gemm_w4a16_pk_add_rms(const void* x, int64_t ldx, const void* packed, const void* frag, const void* scales,
                             const void* frag_scales, int64_t group, void* y, int64_t m, int64_t n, int64_t k,
                             void* workspace, int64_t workspace_bytes, const void* a, const void* deep, const void* w,
                             void* residual, void* out, float eps, int64_t start, int64_t nv, ff_stream_t stream);

/* Gate/up W4A16 GEMM with SwiGLU in its epilogue: h (m, i) = bf16(bf16(silu(g))
 * * u) with g, u = bf16 of x @ dequant(W)^T for W = [gate (i rows); up (i rows)]
 * (frag / frag_scales: ff_pack_weight_int4 / ff_pack_scales_int4 of the
 * (2 i, k) weight and its [k/group, 2 i, 2] scales).
 * No reference counterpart as one op: Int4.__call__ (_family/night_runtime.py:
 * 31-42) then swiglu (_legacy/search_kernels.py:8-23), the same bits.
 * ff_gemm_w4a16_swiglu_fits (no GPU needed) reports whether a kernel takes the
 * shape (m > 4: the tile kernel, i % 128, k % 256; 1 <= m <= 4: the GEMV,
 * i % 16, k % 128; group a power of two >= 32 dividing k); other shapes are
 * rejected with FF_EINVAL. h row stride ldh (multiple of 4). */
int ff_gemm_w4a16_swiglu_fits(int64_t m, int64_t i, int64_t k, int64_t group, int* fits);
int ff_gemm_w4a16_swiglu_pk(const void* x, int64_t ldx, const void* frag, const void* frag_scales, int64_t group,
                            void* h, int64_t ldh, int64_t m, int64_t i, int64_t k, ff_stream_t stream);

/* W4A16 QKV GEMM + q/k norm + rotary + V transpose (no reference counterpart as
 * one op: the QKV Int4.__call__ (_family/night_runtime.py:31-42) followed by
 * qk_pair and the V transpose of attention_direct, scaled_qwen_runtime.py:
 * 165-171; the same bits). frag / frag_scales / group: the fragment copies of
 * the (hq + 2 hk) * 128 x k Int4 weight. Writes yq (hq, m, 128), yk (hk, m, 128)
 * (per-head RMSNorm with q_norm / k_norm, then rotary with cos / sin (m, 128))
 * and vt (hk, 128, t_pad) with zeros for tokens in [m, t_pad); head dim 128.
 * workspace: ff_gemm_w4a16_qkv_workspace bytes (0 there: shape not taken --
 * m > 4, k % 256, group a power of two >= 32 dividing k), 16-byte aligned. */
int ff_gemm_w4a16_qkv_workspace(int64_t m, int64_t k, int64_t hq, int64_t hk, int64_t group, int64_t* bytes);
int ff_gemm_w4a16_qkv(const void* x, int64_t ldx, const void* frag, const void* frag_scales, int64_t group, int64_t m,
                      int64_t k, int64_t hq, int64_t hk, const void* q_norm, const void* k_norm, float eps_q,
                      float eps_k, const void* cos, const void* sin, void* yq, void* yk, void* vt, int64_t t_pad,
                      void* workspace, int64_t workspace_bytes, ff_stream_t stream);

/* Embedding gather h[t] = table[ids[t]] (scaled_qwen_runtime.py:145
 * embed_tokens). Ids outside [0, vocab) read row 0 (the host validates ids). */
int ff_embed(const int64_t* ids, const void* table, void* out, int64_t t, int64_t h,
             int64_t vocab, ff_stream_t stream);

/* Copy rows: out[i] = src[idx[i]] for i < n (index_copy / index_select of the
 * layer loop, scaled_qwen_runtime.py:145, _family/night_runtime.py:100,103).
 * Row width `width` elements of 2 bytes; src/out row strides in elements. */
int ff_gather_rows(const void* src, int64_t src_rs, const int64_t* idx, void* out, int64_t out_rs,
                   int64_t n, int64_t width, int64_t src_rows, ff_stream_t stream);
/* out[start + i] = src[i] for i < n (visual rows into the embedding). */
int ff_scatter_rows(const void* src, void* out, int64_t start, int64_t n, int64_t width,
                    ff_stream_t stream);

/* M-RoPE cos/sin (lm.rotary_emb, scaled_qwen_runtime.py:145): pos (3, t) int64,
 * inv_freq (d/2) fp32; slot i of the half uses the H position if i%3==1 and
 * i < 3*sec_h, W if i%3==2 and i < 3*sec_w, else T; emb = cat(f, f);
 * cos/sin (t, d) bf16. */
int ff_mrope_cos_sin(const int64_t* pos, const float* inv_freq, void* cos, void* sin, int64_t t,
                     int64_t d, int sec_h, int sec_w, ff_stream_t stream);

#ifdef __cplusplus
/* ---------------------------------------------------------------- vision tower
 * The reference runs the vision tower as bf16 torch modules inside
 * NativeNormVision.core (scaled_qwen_runtime.py:42-55) with only the rotary
 * fused (vision_rope); the entry points below replace those modules. */

/* pack_rectangle / pack_rgb (_family/depth_runtime.py:18-25,
 * _legacy/sub10_runtime.py:22-29): rgb (height, width, 3) uint8 -> patches
 * (height/16 * width/16, 1536) bf16 in the processor's 2 x 2 merge-block order,
 * both temporal frames the same image, value bf16((u8 - 127.5) / 127.5).
 * height % 32 == 0, width % 32 == 0. */
int ff_pack_pixels(const void* rgb, void* out, int64_t height, int64_t width, ff_stream_t stream);

/* The vision tower's interpolated position embedding
 * (fast_pos_embed_interpolate, transformers modeling_qwen3_vl.py:664-679, which
 * the reference computes once per image geometry in VisionGraph.geo,
 * _legacy/vision_graph_runtime.py:11-15): out[p] = bf16(sum_t table[idx[p, t]] *
 * wt[p, t]) in fp32, taps in order; table (rows, hidden) bf16, idx (n, taps)
 * int64 (clamped to [0, rows)), wt (n, taps) fp32. hidden % 8 == 0. */
int ff_pos_interp(const void* table, const int64_t* idx, const float* wt, void* out, int64_t n,
                  int64_t taps, int64_t hidden, int64_t rows, ff_stream_t stream);

/* torch.nn.LayerNorm (the vision blocks' norm1/norm2 and the patch mergers'
 * norm, transformers modeling_qwen3_vl.py:122-137,279-306): y = bf16((x - mean)
 * * rstd * w + b) per row of h elements, statistics in fp32. Row strides x_rs,
 * y_rs. h % 8 == 0, h <= 6144. */
int ff_layer_norm(const void* x, int64_t x_rs, const void* w, const void* b, void* y, int64_t y_rs,
                  int64_t rows, int64_t h, float eps, ff_stream_t stream);

/* A bf16 torch.nn.Linear with its neighbours fused (the vision tower's qkv,
 * proj, linear_fc1/fc2 and patch-embedding projection, modeling_qwen3_vl.py:77-107,
 * 196-306): v = bf16(a . w^T + bias) for a (m, k) row stride lda and w (n, k);
 * act 1: v = bf16(gelu_tanh(v)), act 2: v = bf16(gelu(v)) (erf); with resid
 * (row stride ldr, may be y): y = bf16(resid + v). y row stride ldy.
 * k % 64 == 0 (pad k with zero columns of a and w), n % 4 == 0. */
int ff_gemm_bf16(const void* a, int64_t lda, const void* w, const void* bias, void* y, int64_t ldy,
                 const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, int act, ff_stream_t stream);

/* Setup-time repack of bf16 weights w (n, k) row-major into the operand order
 * of ff_gemm_bf16_pk (no reference counterpart: a storage layout of this
 * library): fragment (f, kt), rows [16 f, 16 f + 16) x k [128 kt, 128 kt +
 * 128), is the 4 KB at (kt * n/16 + f) * 4096; its sub-block s (1 KB at s *
 * 1024) holds for lane l = 16 g + r the 16 bytes of row 16 f + r at k 128 kt +
 * 64 (s / 2) + 16 g + 8 (s % 2). packed holds 2 n k bytes. n % 16 == 0,
 * k % 128 == 0. */
int ff_pack_weight_bf16(const void* w, void* packed, int64_t n, int64_t k, ff_stream_t stream);
/* ff_gemm_bf16 with the weight read from its packed copy (ff_pack_weight_bf16
 * of w) straight into the matrix-core operands: the same products in the same
 * order, so the same bits. Taken when w_packed is given, k % 128 == 0 and a
 * tile of 128 x 192, 64 x 256, 64 x 192 or 64 x 128 divides n and gives a grid
 * of 192..256 workgroups; otherwise this is ff_gemm_bf16 on w (w_packed may be
 * NULL). Same reference replacement as ff_gemm_bf16. */
int ff_gemm_bf16_pk(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias, void* y,
                    int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, int act,
                    ff_stream_t stream);

/* Bytes of workspace ff_gemm_bf16_pk_ws / ff_gemm_bf16_pk_ln need for an
 * m x n x k product (0: it runs unsplit). Host-only. */
int ff_gemm_bf16_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes);
/* ff_gemm_bf16_pk with a k split where the packed kernel has no tile whose
 * grid fills the GPU in one round (short m: the tower at 400 patches, the
 * patch mergers): the split launches store fp32 partials in workspace
 * (ff_gemm_bf16_pk_workspace bytes, 16-byte aligned) and a second launch adds
 * them in split order and applies the epilogue (bias, act, resid). The same
 * products summed in another order: within an fp32 rounding of the unsplit
 * sums before the bf16 rounding. Splits need 16-byte aligned a, bias, y,
 * resid and ldy, ldr % 8; otherwise, or with no split planned, this is
 * ff_gemm_bf16_pk. Same reference replacement as ff_gemm_bf16. */
int ff_gemm_bf16_pk_ws(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias, void* y,
                       int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, int act,
                       void* workspace, int64_t workspace_bytes, ff_stream_t stream);
/* A vision block's residual linear and the LayerNorm that reads its output
 * (attn.proj + residual + norm2, mlp.linear_fc2 + residual + the next block's
 * norm1: transformers modeling_qwen3_vl.py:196-306, NativeNormVision.core,
 * scaled_qwen_runtime.py:42-55): y = bf16(resid + bf16(a . w^T + bias)) as
 * ff_gemm_bf16_pk_ws (resid required, may be y), then ln_out = LayerNorm(y)
 * with ln_w, ln_b, eps as ff_layer_norm (row stride ln_ld; ln_w NULL: no
 * LayerNorm). With a k split the LayerNorm launch adds the partials, stores y
 * and normalises it: two launches either way. */
int ff_gemm_bf16_pk_ln(const void* a, int64_t lda, const void* w, const void* w_packed, const void* bias, void* y,
                       int64_t ldy, const void* resid, int64_t ldr, int64_t m, int64_t n, int64_t k, void* workspace,
                       int64_t workspace_bytes, const void* ln_w, const void* ln_b, float eps, void* ln_out,
                       int64_t ln_ld, ff_stream_t stream);

/* vision_rope (_legacy/search_kernels.py:111-134): yq/yk = bf16(x * cos +
 * rotate_half(x) * sin) in fp32, cos/sin (n, hd) fp32. q, k with token stride
 * x_ts and head stride x_hs (views of the packed qkv output); outputs with
 * y_ts / y_hs and columns [hd, dpad) of each head set to 0 (dpad = hd for the
 * reference's (n, heads, hd) layout, 128 for the zero-padded head-major layout
 * ff_attention_full reads). hd % 8 == 0. */
int ff_vision_rope(const void* q, const void* k, int64_t x_ts, int64_t x_hs, const float* cos,
                   const float* sin, void* yq, void* yk, int64_t y_ts, int64_t y_hs, int64_t n,
                   int64_t heads, int64_t hd, int64_t dpad, ff_stream_t stream);

/* The transposed, zero-padded V of the vision attention (no reference
 * counterpart: the layout ff_attention_full reads): v (token stride v_ts, head
 * stride v_hs, hd columns) -> vt (heads, 128, t_pad), zeros for d >= hd and
 * tokens >= n. hd <= 128, t_pad % 64 == 0. */
int ff_vision_vt(const void* v, int64_t v_ts, int64_t v_hs, void* vt, int64_t n, int64_t t_pad,
                 int64_t heads, int64_t hd, ff_stream_t stream);

/* ff_vision_rope + ff_vision_vt on the packed qkv output of a vision block in
 * one launch (no reference counterpart as one op): qkv (n, 3, heads, hd)
 * contiguous -> yq, yk (heads, n, 128) rotated and zero-padded, vt (heads,
 * 128, t_pad) zero-padded. hd % 8 == 0, hd <= 128, t_pad % 64 == 0; every
 * pointer 16-byte aligned. */
int ff_vision_qkv(const void* qkv, const float* cos, const float* sin, void* yq, void* yk, void* vt,
                  int64_t n, int64_t t_pad, int64_t heads, int64_t hd, ff_stream_t stream);

/* Bidirectional multi-head attention of the vision blocks (the sdpa call with
 * is_causal=False of scaled_qwen_runtime.py:51): q, k (heads, t, 128) with head
 * dims past the model's zero, vt (heads, 128, t_pad) from ff_vision_vt; fp32
 * scores and softmax statistics, P rounded to bf16 before P.V, fp32
 * accumulation. y (t, heads, d_out) bf16. d_out in {64, 72, 128}. */
int ff_attention_full(const void* q, const void* k, const void* vt, void* y, int64_t t, int64_t t_pad,
                      int64_t heads, int64_t d_out, float scale, ff_stream_t stream);

}
#endif
#endif /* FF_AMD_H */
