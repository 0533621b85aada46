"""Drop-in LM-step ops with the reference's Python signatures, on gfx950 kernels.

Each function keeps the reference op's name, argument meaning, output layout and
assertion behaviour (shape/dtype/contiguity violations raise AssertionError
before any launch) and launches the HIP kernel on the current stream through
the C ABI. Triton tuning knobs (``rows``, ``warps``, ``bm``, ``bn``, ``block``,
``half``, ``pad``, ``fusion``) are accepted and ignored: the kernels pick their
own gfx950 tiles. Outputs are fresh ``torch.empty`` tensors (graph-pool memory
under capture); inputs are never written.

Reference paths are relative to FastForward's src/fastforward_accel/.
"""
import torch

from . import _lib
from ._lib import call, ptr, stream

BF16 = torch.bfloat16


def fast_norm(x, module):
    """``fast_norm`` (_legacy/sub10_runtime.py:37-41)."""
    assert x.is_contiguous() and x.dtype == module.weight.dtype == BF16
    out = torch.empty_like(x)
    d = x.shape[-1]
    call("ff_fast_norm", ptr(x), ptr(module.weight), ptr(out), x.numel() // d, d,
         float(module.variance_epsilon), stream())
    return out


def add_rms(a, b, deep, module, start=0, nv=0, warps=4, fusion=False):
    """``add_rms`` (_legacy/lower_kernels.py:24-32; knob variant _legacy/broad_kernels.py:9-17)."""
    assert a.shape == b.shape and a.is_contiguous() and b.is_contiguous()
    assert a.dtype == b.dtype == module.weight.dtype == BF16
    if deep is not None:
        assert deep.shape == (nv, a.shape[-1]) and deep.is_contiguous()
    residual = torch.empty_like(a)
    out = torch.empty_like(a)
    d = a.shape[-1]
    call("ff_add_rms", ptr(a), ptr(b), ptr(deep), ptr(module.weight), ptr(residual), ptr(out),
         a.numel() // d, d, float(module.variance_epsilon), int(start), int(nv), stream())
    return residual, out


def qk_pair(q, k, qn, kn, cos, sin, rows=4, warps=4, half=False, pad=1, fusion=False):
    """``qk_pair`` (_legacy/broad_kernels.py:63-74): per-head q/k RMSNorm + M-RoPE.

    q (1,T,HQ,D), k (1,T,HK,D) strided views with equal token strides; returns
    yq (1,HQ,T,D), yk (1,HK,T,D)."""
    assert q.shape[0] == k.shape[0] == 1 and q.shape[1] == k.shape[1]
    assert q.stride(1) == k.stride(1) and q.stride(-1) == k.stride(-1) == 1
    _, t, hq, d = q.shape
    hk = k.shape[2]
    assert q.stride(2) == d and k.stride(2) == d, "heads must be packed along the row"
    yq = torch.empty((1, hq, t, d), device=q.device, dtype=q.dtype)
    yk = torch.empty((1, hk, t, d), device=k.device, dtype=k.dtype)
    cos2 = cos.reshape(-1, cos.shape[-1])
    sin2 = sin.reshape(-1, sin.shape[-1])
    if cos2.stride(-1) != 1:
        cos2 = cos2.contiguous()
    if sin2.stride(-1) != 1:
        sin2 = sin2.contiguous()
    call("ff_qk_pair", ptr(q), ptr(k), q.stride(1), ptr(qn.weight), ptr(kn.weight),
         float(qn.variance_epsilon), float(kn.variance_epsilon), ptr(cos2), ptr(sin2),
         cos2.stride(0), cos2.stride(1), sin2.stride(0), sin2.stride(1), ptr(yq), ptr(yk),
         t, hq, hk, d, stream())
    return yq, yk


def swiglu(gate, up, block=1024, warps=4):
    """``swiglu`` (_legacy/search_kernels.py:18-23): gate/up may be strided halves."""
    assert gate.shape == up.shape and gate.stride() == up.stride()
    assert gate.stride(-1) == 1 and gate.dtype == up.dtype == BF16
    y = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    i = gate.shape[-1]
    rows = gate.numel() // i
    rs = gate.stride(-2) if gate.dim() > 1 else i
    call("ff_swiglu", ptr(gate), ptr(up), rs, ptr(y), rows, i, stream())
    return y


def _t_pad(t):
    return (t + 63) // 64 * 64


def attention_direct(q, k, v, scale, bm=16, bn=64, warps=4, positions=None, triangular=True):
    """``attention_direct`` (_legacy/limit_kernels.py:36-45): causal GQA attention.

    q (1,HQ,S,D) and k (1,HK,T,D) contiguous, v (1,HK,T,D) with stride(-1)==1
    (a strided view of the packed QKV is fine); returns y (1,S,HQ,D). With
    ``positions`` (S,) int64 each query attends to keys <= its position."""
    assert q.is_contiguous() and k.is_contiguous() and q.shape[0] == k.shape[0] == v.shape[0] == 1
    _, hq, s, d = q.shape
    _, hk, t, kd = k.shape
    assert kd == d and v.shape == (1, hk, t, d) and v.stride(-1) == 1 and hq % hk == 0
    if positions is not None:
        assert positions.shape == (s,) and positions.is_contiguous()
    tp = _t_pad(t)
    vt = torch.empty((hk, d, tp), device=v.device, dtype=v.dtype)
    call("ff_v_transpose", ptr(v), v.stride(2), v.stride(1), ptr(vt), t, tp, hk, d, stream())
    y = torch.empty((1, s, hq, d), device=q.device, dtype=q.dtype)
    call("ff_attention_vt", ptr(q), ptr(k), ptr(vt), ptr(positions), 0, ptr(y), s, t, tp, hq, hk, d,
         float(scale), stream())
    return y


def lm_readout(x, norm, weight):
    """``lm_readout`` (_legacy/limit_kernels.py:60-66): returns (1, n_options) fp32."""
    assert x.numel() == x.shape[-1] == weight.shape[1] and x.is_contiguous() and weight.is_contiguous()
    assert x.dtype == weight.dtype == norm.weight.dtype == BF16
    y = torch.empty((1, weight.shape[0]), device=x.device, dtype=torch.float32)
    call("ff_lm_readout", ptr(x), None, ptr(norm.weight), ptr(weight), ptr(y), x.shape[-1],
         weight.shape[0], float(norm.variance_epsilon), stream())
    return y


class RMSNorm:
    """Parameter holder with the attributes the ops read from HF's RMSNorm
    modules: ``weight`` (bf16) and ``variance_epsilon``."""

    def __init__(self, weight, eps=1e-6):
        self.weight = weight
        self.variance_epsilon = eps


__all__ = ["fast_norm", "add_rms", "qk_pair", "swiglu", "attention_direct", "lm_readout", "RMSNorm"]
_ = _lib
