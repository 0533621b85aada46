"""Per-op CPU restatement of the reference's LM-step arithmetic (test infrastructure).

Paths are relative to the reference's ``src/fastforward_accel/``. Each function
reproduces the rounding points of the cited kernel: values are carried in fp32
and rounded to bf16 (round-to-nearest-even) exactly where the reference stores
or casts to bf16, and to e4m3fn where it casts to FP8.

Not the product: only tests/, smoke() and bench.py's cpu_baseline use it.
"""
import math

import torch

BF16 = torch.bfloat16
F32 = torch.float32
E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0


def bf16(x):
    """Round fp32 -> bf16 (RNE) and return it widened back to fp32."""
    return x.to(BF16).to(F32)


def _rsqrt(v):
    return torch.rsqrt(v)


# ---------------------------------------------------------------- norms

def fast_norm(x, weight, eps):
    """``fast_norm`` / ``rms_one`` (_legacy/sub10_runtime.py:31-41).

    out = bf16(bf16(x * rsqrt(sum(x^2)/H + eps)) * w), one row per token.
    """
    xf = x.to(F32)
    h = xf.shape[-1]
    var = (xf * xf).sum(-1, keepdim=True) / h
    n = bf16(xf * _rsqrt(var + eps))
    return (n * weight.to(F32)).to(BF16)


def add_rms(a, b, deep, weight, eps, start=0, nv=0):
    """``add_rms`` / ``_add_rms`` (_legacy/lower_kernels.py:7-32).

    x = bf16(a+b); rows in [start, start+nv) get x = bf16(x + deep[row-start]);
    returns (residual = x, out = bf16(bf16(x*rsqrt(mean(x^2)+eps))*w)).
    """
    assert a.shape == b.shape
    h = a.shape[-1]
    x = bf16(a.to(F32) + b.to(F32)).reshape(-1, h)
    if deep is not None:
        assert deep.shape == (nv, h)
        x = x.clone()
        rows = torch.arange(x.shape[0])
        sel = (rows >= start) & (rows < start + nv)
        idx = rows[sel]
        x[idx] = bf16(x[idx] + deep.to(F32)[idx - start])
    var = (x * x).sum(-1, keepdim=True) / h
    n = bf16(x * _rsqrt(var + eps))
    out = (n * weight.to(F32)).to(BF16)
    return x.to(BF16).reshape(a.shape), out.reshape(a.shape)


# ---------------------------------------------------------------- rotary

def _rope_rows(x, weight, eps, cos, sin):
    """``_rope_rows`` (_legacy/lower_kernels.py:66-86) for x (1,T,H,D) -> (1,H,T,D)."""
    xf = x.to(F32)
    d = xf.shape[-1]
    inv = _rsqrt((xf * xf).sum(-1, keepdim=True) / d + eps)
    xn = bf16(bf16(xf * inv) * weight.to(F32))
    r = torch.cat((-xn[..., d // 2:], xn[..., : d // 2]), -1)
    c = cos.to(F32).reshape(1, -1, 1, d)
    s = sin.to(F32).reshape(1, -1, 1, d)
    y = bf16(bf16(xn * c) + bf16(r * s))
    return y.permute(0, 2, 1, 3).contiguous().to(BF16)


def qk_pair(q, k, q_weight, k_weight, q_eps, k_eps, cos, sin):
    """``qk_pair`` -> ``_pair_rows`` (_legacy/broad_kernels.py:63-74,
    _legacy/lower_kernels.py:89-98): per-head q/k RMSNorm then M-RoPE rotate-half.

    q (1,T,HQ,D), k (1,T,HK,D) (strided views allowed), cos/sin (1,T,D) bf16.
    Returns yq (1,HQ,T,D), yk (1,HK,T,D) bf16 contiguous.
    """
    return (_rope_rows(q, q_weight, q_eps, cos, sin),
            _rope_rows(k, k_weight, k_eps, cos, sin))


def mrope_positions(prefix_tokens, grid_h, grid_w, total):
    """M-RoPE position ids (3, total) for one image, as the reference obtains them
    from transformers' ``get_rope_index`` at setup (_family/depth_runtime.py:45-49):
    text tokens t < s0 get (t,t,t); the image token at merged-grid (r,c) gets
    (s0, s0+r, s0+c); text after the image resumes at s0+max(gh,gw).
    """
    s0 = prefix_tokens
    nv = grid_h * grid_w
    assert s0 + nv <= total
    pos = torch.zeros(3, total, dtype=torch.int64)
    t = torch.arange(s0)
    pos[:, :s0] = t
    r = torch.arange(grid_h).repeat_interleave(grid_w)
    c = torch.arange(grid_w).repeat(grid_h)
    pos[0, s0:s0 + nv] = s0
    pos[1, s0:s0 + nv] = s0 + r
    pos[2, s0:s0 + nv] = s0 + c
    rest = total - s0 - nv
    pos[:, s0 + nv:] = s0 + max(grid_h, grid_w) + torch.arange(rest)
    return pos


def mrope_inv_freq(theta, head_dim):
    """``inv_freq = 1/(theta ** (arange(0,D,2)/D))`` in fp32 (transformers
    Qwen3VLTextRotaryEmbedding default rope parameters)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def mrope_cos_sin(pos, theta, head_dim, sections=(24, 20, 20)):
    """``lm.rotary_emb(h, pos)`` (scaled_qwen_runtime.py:145) ->
    Qwen3VLTextRotaryEmbedding.forward + apply_interleaved_mrope (transformers).

    pos (3,T) int64 -> cos, sin (1,T,D) bf16. Frequency slot i takes the H
    position if i%3==1 and i<3*sections[1], W if i%3==2 and i<3*sections[2],
    else T; emb = cat(f, f).
    """
    inv = mrope_inv_freq(theta, head_dim)
    freqs = pos.to(F32)[:, :, None] * inv[None, None, :]          # (3,T,D/2)
    f = freqs[0].clone()
    for dim, offset in ((1, 1), (2, 2)):
        idx = slice(offset, sections[dim] * 3, 3)
        f[:, idx] = freqs[dim][:, idx]
    emb = torch.cat((f, f), -1)
    return emb.cos().to(BF16)[None], emb.sin().to(BF16)[None]


# ---------------------------------------------------------------- MLP

def swiglu(g, u):
    """``swiglu`` / ``_swiglu`` (_legacy/search_kernels.py:8-23):
    y = bf16(bf16(g / (1 + exp(-g))) * u)."""
    gf = g.to(F32)
    act = bf16(gf / (1.0 + torch.exp(-gf)))
    return (act * u.to(F32)).to(BF16)


# ---------------------------------------------------------------- attention

def attention_direct(q, k, v, scale, positions=None, block_n=64):
    """``attention_direct`` / ``_attention_direct`` (_legacy/limit_kernels.py:8-45).

    q (1,HQ,S,D), k (1,HK,T,D), v (1,HK,T,D) bf16 -> y (1,S,HQ,D) bf16.
    Per key block of ``block_n``: s = (q.k) * scale in fp32, causal mask
    key <= position, online max / denominator with exp, P rounded to bf16
    before P.V, fp32 accumulation, out = acc/den rounded to bf16.
    ``positions`` (S,) selects the query positions (SELECTED mode); otherwise
    query row i sits at position i.
    """
    _, hq, s_len, d = q.shape
    hk, t = k.shape[1], k.shape[2]
    group = hq // hk
    pos = torch.arange(s_len) if positions is None else positions.to(torch.int64).reshape(-1)
    qf = q[0].to(F32)                                     # (HQ,S,D)
    kf = k[0].to(F32).repeat_interleave(group, 0)         # (HQ,T,D)
    vf = v[0].to(F32).repeat_interleave(group, 0)
    mx = torch.full((hq, s_len, 1), -math.inf)
    den = torch.zeros(hq, s_len, 1)
    acc = torch.zeros(hq, s_len, d)
    for start in range(0, t, block_n):
        n = torch.arange(start, min(start + block_n, t))
        score = torch.matmul(qf, kf[:, n].transpose(1, 2)) * scale
        allowed = pos[:, None] >= n[None, :]
        score = torch.where(allowed[None], score, torch.tensor(-math.inf))
        new = torch.maximum(mx, score.amax(-1, keepdim=True))
        alpha = torch.exp(mx - new)
        alpha = torch.where(torch.isnan(alpha), torch.zeros(()), alpha)
        p = torch.exp(score - new)
        p = torch.where(torch.isnan(p), torch.zeros(()), p)
        den = den * alpha + p.sum(-1, keepdim=True)
        acc = acc * alpha + torch.matmul(bf16(p), vf[:, n])
        mx = new
    y = (acc / den).to(BF16)                              # (HQ,S,D)
    return y.permute(1, 0, 2).unsqueeze(0).contiguous()


def attention_exact(q, k, v, scale, positions=None):
    """Plain softmax attention in fp64 (no block structure), for tolerance checks."""
    _, hq, s_len, d = q.shape
    hk, t = k.shape[1], k.shape[2]
    group = hq // hk
    pos = torch.arange(s_len) if positions is None else positions.to(torch.int64).reshape(-1)
    qf = q[0].double()
    kf = k[0].double().repeat_interleave(group, 0)
    vf = v[0].double().repeat_interleave(group, 0)
    score = torch.matmul(qf, kf.transpose(1, 2)) * scale
    allowed = pos[:, None] >= torch.arange(t)[None, :]
    score = score.masked_fill(~allowed[None], -math.inf)
    p = torch.softmax(score, -1)
    y = torch.matmul(p, vf)
    return y.permute(1, 0, 2).unsqueeze(0)


# ---------------------------------------------------------------- readout

def lm_readout(x, norm_weight, eps, head):
    """``lm_readout`` / ``_lm_readout`` (_legacy/limit_kernels.py:48-66):
    x_hat = bf16(bf16(x*rsqrt(mean(x^2)+eps))*w); z_c = bf16(sum_k x_hat_k*head[c,k])
    stored fp32. Returns (1, n_options) fp32."""
    xf = x.to(F32).reshape(-1)
    h = xf.shape[0]
    inv = _rsqrt((xf * xf).sum() / h + eps)
    xn = bf16(bf16(xf * inv) * norm_weight.to(F32))
    z = bf16((head.to(F32) * xn[None, :]).sum(-1))
    return z[None]


def choose(logits):
    """Answer index: max logit, ties -> lowest index (_family/family_api.py:41)."""
    return max(range(len(logits)), key=lambda i: (logits[i], -i))


def response(logits, candidates, item_id):
    """Response dict with softmax probabilities (api.py:28-34)."""
    if len(logits) != len(candidates) or not all(math.isfinite(x) for x in logits):
        raise RuntimeError('Invalid model output')
    pred = max(range(len(logits)), key=lambda i: logits[i])
    exps = [math.exp(x - max(logits)) for x in logits]
    return dict(id=item_id, answer=dict(letter=chr(65 + pred), text=candidates[pred]),
                logits=logits, probabilities=[e / sum(exps) for e in exps])


# ---------------------------------------------------------------- FP8 linear

def fp8_weight_quant(w, per_channel=True):
    """Setup-time weight quantization.

    per_channel: ``FP8Linear.__init__`` (_legacy/fp8_private.py:22-27),
    scale[n] = max(amax_k |W[n,k]|, 1e-12)/448, returns scale (N,) fp32.
    per-tensor: ``StaticFP8Linear.__init__`` (_legacy/limit_kernels.py:122-127),
    scale = max(amax |W|, 1e-12)/448, returns scale (1,) fp32.
    q = e4m3(clamp(W/scale, -448, 448)).
    """
    wf = w.detach().to(F32)
    if per_channel:
        scale = wf.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / E4M3_MAX
        q = (wf / scale).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3).contiguous()
        return q, scale.reshape(-1)
    scale = wf.abs().amax().clamp_min(1e-12) / E4M3_MAX
    q = (wf / scale).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3).contiguous()
    return q, scale.reshape(1)


def quant_rows_dynamic(x):
    """Per-token dynamic activation quant ``quantize_rows`` (_legacy/fp8_private.py:11-18):
    scale[m] = max(amax_k |x[m,k]|, 1e-12)/448; q = e4m3(clamp(x/scale, +-448)).
    Returns (q (M,K) e4m3, scale (M,) fp32)."""
    xf = x.reshape(-1, x.shape[-1]).to(F32)
    scale = xf.abs().amax(-1, keepdim=True).clamp_min(1e-12) / E4M3_MAX
    q = (xf / scale).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3)
    return q, scale.reshape(-1)


def quant_static(x, inverse_scale):
    """Static per-tensor activation quant ``_runtime_scale`` (_family/depth_fp8.py:8-12):
    q = e4m3(clamp(x * INV, +-448)), INV an fp32 kernel argument."""
    xf = x.reshape(-1, x.shape[-1]).to(F32)
    inv = torch.tensor(inverse_scale, dtype=F32)
    return (xf * inv).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3)


def fp8_gemm(qa, sa, qw, sw):
    """``torch._scaled_mm(qA, qW.T, scale_a, scale_b, out_dtype=bf16)``
    (_legacy/fp8_private.py:36-37, _family/depth_fp8.py:25-26):
    y = bf16(acc * sA * sW) with acc = sum_k f32(qA)*f32(qW) in fp32; sA is (M,)
    or (1,), sW is (N,) or (1,)."""
    acc = qa.to(F32) @ qw.to(F32).T
    return (acc * sa.reshape(-1, 1) * sw.reshape(1, -1)).to(BF16)


def fp8_gemm_exact(qa, sa, qw, sw):
    """``fp8_gemm`` with exact accumulation: the sum of e4m3 products is formed
    in fp64, where every such sum of up to 2^22 terms is exact, then scaled and
    rounded like ``fp8_gemm``. The formulation's value without any summation
    error (a sensitivity check, not a reference kernel)."""
    acc = qa.double() @ qw.double().T
    return (acc * sa.double().reshape(-1, 1) * sw.double().reshape(1, -1)).to(BF16)


def round_sig_(x, bits):
    """Round the fp64 tensor x in place to ``bits`` significant bits, nearest
    even (normal values and zero; the fp64 bit pattern's low 53 - bits bits are
    rounded away)."""
    u = x.view(torch.int64)
    drop = 53 - bits
    u.add_(((u >> drop) & 1) + ((1 << (drop - 1)) - 1))
    u.bitwise_and_(~((1 << drop) - 1))
    return x


def fp8_gemm_blocks(qa, sa, qw, sw, bits=14, block=32, chunk=2048):
    """``fp8_gemm`` on a model of a matrix unit with reduced-precision block sums:
    k is cut into blocks of ``block`` products, each block's sum (exact) is rounded
    to ``bits`` significant bits, and the blocks are added into an fp32
    accumulator in k order; then the scaling and bf16 rounding of ``fp8_gemm``.

    Not a restatement of the reference: its ``_scaled_mm`` runs on FP8 tensor
    cores whose block accumulation is of this class (about 14 significant bits
    retained per block), and so does gfx950's v_mfma_f32_16x16x128_f8f6f4. The
    oracle with this GEMM in place of the fp32 one measures how far a
    correctly computed step moves when only the GEMMs' accumulation has the
    precision of such a unit."""
    m, k = qa.shape
    n = qw.shape[0]
    assert k % block == 0 and 2 <= bits <= 52
    a = qa.double().reshape(m, k // block, block).permute(1, 0, 2).contiguous()
    wd = qw.double()
    out = torch.empty(m, n, dtype=BF16)
    sa_, sw_ = sa.to(F32).reshape(-1, 1), sw.to(F32).reshape(1, -1).expand(1, n)
    for c0 in range(0, n, chunk):
        w = wd[c0:c0 + chunk].reshape(-1, k // block, block).permute(1, 2, 0).contiguous()
        blk = round_sig_(torch.bmm(a, w), bits).to(F32)      # exact block sums -> bits -> fp32 (exact)
        acc = blk[0].clone()
        for b in range(1, blk.shape[0]):
            acc.add_(blk[b])
        out[:, c0:c0 + chunk] = ((acc * sa_) * sw_[:, c0:c0 + chunk]).to(BF16)
    return out


def fp8_linear_dynamic(x, qw, sw):
    """``FP8Linear.__call__`` (_legacy/fp8_private.py:29-38)."""
    qa, sa = quant_rows_dynamic(x)
    y = fp8_gemm(qa, sa, qw, sw)
    return y.reshape(*x.shape[:-1], qw.shape[0])


def fp8_linear_static(x, qw, sw, inverse_scale, input_scale):
    """``RuntimeScaleLinear.__call__`` (_family/depth_fp8.py:22-26): static activation
    scale ``input_scale`` (fp32 (1,)) with quant multiplier ``inverse_scale``."""
    qa = quant_static(x, inverse_scale)
    y = fp8_gemm(qa, input_scale.reshape(1), qw, sw)
    return y.reshape(*x.shape[:-1], qw.shape[0])


# ---------------------------------------------------------------- W4A16 linear

def int4_quantize_asym(w, group=32):
    """``Int4.__init__`` (_family/night_runtime.py:16-26): asymmetric min/max per
    group along K; s = max((hi-lo)/15, 1e-6); q = clamp(round((w-lo)/s), 0, 15);
    z = lo + 8s; scales [K/g, N, 2] bf16 (s, z); nibbles packed (N, K/2) with
    even k in the high nibble. Returns (q (N,K) uint8, packed, scales)."""
    n, k = w.shape
    x = w.to(F32).reshape(n, -1, group)
    low = x.amin(-1, keepdim=True)
    high = x.amax(-1, keepdim=True)
    scale = ((high - low) / 15).clamp_min(1e-6)
    q = ((x - low) / scale).round().clamp(0, 15).to(torch.uint8).reshape(n, k)
    zeros = low + scale * 8
    scales = torch.stack((scale.squeeze(-1), zeros.squeeze(-1)), dim=-1).transpose(0, 1).contiguous().to(BF16)
    packed = (q[:, 0::2] << 4) | q[:, 1::2]
    return q, packed.contiguous(), scales


def int4_quantize_sym(w, group=128):
    """Symmetric int4 (the measured W4A16 configuration): the reference's dequant
    form ``(q-8)*s + z`` (_family/night_runtime.py:28-30) with z = 0 and
    s = bf16(max(amax_group |w|, 1e-6)/7); q = clamp(round(w/s) + 8, 0, 15) using
    the stored (bf16) scale. Same packing and [K/g, N, 2] layout as the reference."""
    n, k = w.shape
    x = w.to(F32).reshape(n, -1, group)
    s = bf16(x.abs().amax(-1, keepdim=True).clamp_min(1e-6) / 7)
    q = ((x / s).round() + 8).clamp(0, 15).to(torch.uint8).reshape(n, k)
    scales = torch.stack((s.squeeze(-1), torch.zeros_like(s.squeeze(-1))), dim=-1)
    scales = scales.transpose(0, 1).contiguous().to(BF16)
    packed = (q[:, 0::2] << 4) | q[:, 1::2]
    return q, packed.contiguous(), scales


def int4_unpack(packed):
    """(N, K/2) uint8 -> (N, K) nibble codes; even k from the high nibble."""
    n, kh = packed.shape
    q = torch.empty(n, kh * 2, dtype=torch.uint8)
    q[:, 0::2] = packed >> 4
    q[:, 1::2] = packed & 15
    return q


def int4_dequant(packed, scales, group):
    """Dequantized fp32 weight (N,K): (q-8)*s + z with s,z = scales[k//g, n]
    (_family/night_runtime.py:28-30)."""
    q = int4_unpack(packed).to(F32)
    n, k = q.shape
    s, z = scales.to(F32).transpose(0, 1).unbind(-1)        # (N, K/g)
    return ((q.reshape(n, -1, group) - 8) * s[..., None] + z[..., None]).reshape(n, k)


def w4a16_linear(x, packed, scales, group, weight_bf16=False):
    """``Int4.__call__`` (_family/night_runtime.py:31-42): y = x @ Wdq^T, bf16 out.

    ``weight_bf16=False``: against the fp32 dequantized weight, as the reference's
    own operator check does (:28-30, :36-40).
    ``weight_bf16=True``: the dequantized weight rounded to bf16 first, the form
    the reference's runtime GEMM ``_weight_int4pack_mm`` (:33) multiplies on bf16
    tensor cores: a bf16 matrix unit takes bf16 operands, so each dequantized
    weight bf16((q-8)*s + z) enters the products rounded once."""
    flat = x.reshape(-1, x.shape[-1]).to(F32)
    w = int4_dequant(packed, scales, group)
    if weight_bf16:
        w = bf16(w)
    y = (flat @ w.T).to(BF16)
    return y.reshape(*x.shape[:-1], w.shape[0])
