"""Linear-op protocol of the reference on gfx950 GEMMs.

An op is a callable ``op(x) -> y2d`` with ``op.weight`` (N,K) (its ``.shape`` is
read by ``Linear.apply``), used through ``Linear.apply(x, op)``
(scaled_qwen_runtime.py:35-39). Three families, each keeping the reference's
attributes:

* ``FP8Linear``: per-token dynamic activation scale, per-output-channel weight
  scale (_legacy/fp8_private.py:21-38) -- the measured configuration.
* ``StaticFP8Linear`` / ``RuntimeScaleLinear``: per-tensor weight scale and a
  static activation scale ``input_scale`` = 1/``inverse_scale`` from a
  calibration profile (_legacy/limit_kernels.py:110-135, _family/depth_fp8.py:22-26).
* ``Int4``: W4A16 with nibble codes and [K/g, N, 2] (scale, zero) pairs
  (_family/night_runtime.py:15-42); symmetric group-128 or the reference's
  asymmetric group-32 quantizer.

Weight quantization runs once on the GPU at construction. All calls allocate
their outputs with torch.empty and launch on the current stream.
"""
import ctypes
import types

import torch

from ._lib import call, ptr, stream

E4M3 = torch.float8_e4m3fn
BF16 = torch.bfloat16


def gemm_pk_workspace(m, n, k):
    """Bytes of workspace ff_gemm_fp8_pk needs for an m x n x k GEMM (0: none)."""
    need = ctypes.c_int64(0)
    call("ff_gemm_fp8_pk_workspace", m, n, k, ctypes.byref(need))
    return need.value


# Execution modes that mix the FP8 and int4 banks per layer and role.
MIXED_MODES = ("int4_half", "int4_ffn")


def bank_of(mode, layer, layers, role):
    """Bank ("fp8" or "int4") of linear ``role`` ("qkv", "o", "gateup", "down")
    of layer ``layer`` of ``layers`` under the reference's execution ``mode``
    (``set_mode``, _family/night_runtime.py:56-65): with final = layers - 1 the
    interior layers are 3 <= layer < final - 3; "int4_half" takes every role of
    the even interior layers from the int4 bank, "int4_ffn" the gate/up and
    down projections of every interior layer; "int4" every linear; any other
    mode the FP8 bank."""
    if mode == "int4":
        return "int4"
    interior = 3 <= layer < layers - 1 - 3
    if mode == "int4_half" and interior and layer % 2 == 0:
        return "int4"
    if mode == "int4_ffn" and interior and role in ("gateup", "down"):
        return "int4"
    return "fp8"


def _rows(x):
    return x.reshape(-1, x.shape[-1])


class Linear:
    @staticmethod
    def apply(x, op):
        """``Linear.apply`` (scaled_qwen_runtime.py:35-39), forward only."""
        return op(x).reshape(*x.shape[:-1], op.weight.shape[0])


class PackedCodes:
    """The ``weight`` of a linear that keeps only the MFMA-fragment copy of its
    e4m3 codes: ``shape``, ``dtype`` and ``device`` of the row-major (N, K)
    tensor it replaces, and a NULL data pointer, so the entry points that take
    both copies run on the packed one. A caller that reads the codes gets them
    unpacked on the device (``rowmajor()``, ``cpu()``, ``view()``), each time."""

    def __init__(self, packed, shape):
        self._packed = packed
        self.shape = torch.Size(shape)
        self.dtype, self.device = E4M3, packed.device

    def data_ptr(self):
        return 0

    def numel(self):
        return self.shape[0] * self.shape[1]

    def rowmajor(self):
        n, k = self.shape
        w = torch.empty((n, k), device=self.device, dtype=E4M3)
        call("ff_unpack_weight_fp8", ptr(self._packed), ptr(w), n, k, stream())
        return w

    def cpu(self):
        return self.rowmajor().cpu()

    def view(self, dtype):
        return self.rowmajor().view(dtype)


def _single_copy(op, keep_rowmajor):
    """Pack ``op``'s codes and, unless ``keep_rowmajor``, keep the packed copy
    alone where the packed kernels take every row count of its shape (n % 128,
    k % 512): one copy of the weights in HBM."""
    op.pack()
    n, k = op.weight.shape
    if not keep_rowmajor and op.packed is not None and n % 128 == 0 and k % 512 == 0:
        op.weight = PackedCodes(op.packed, (n, k))


def _packed_gemm(op, q, s, s_rows, sw, sw_cols, y):
    """y = bf16((q . W^T * s) * sw) through ff_gemm_fp8_pk on ``op``'s packed
    copy, with a k-split workspace the op keeps (calls ordered on one stream)."""
    m, k = q.shape
    n = op.weight.shape[0]
    need = gemm_pk_workspace(m, n, k)
    ws = getattr(op, "_ws", None)
    if need and (ws is None or ws.numel() < need):
        op._ws = ws = torch.empty(need, device=q.device, dtype=torch.uint8)
    call("ff_gemm_fp8_pk", ptr(q), ptr(s), s_rows, ptr(op.weight), ptr(op.packed), ptr(sw), sw_cols, ptr(y),
         y.stride(0), m, n, k, ptr(ws) if need else None, need, stream())
    return y


class FP8Linear:
    """Per-channel e4m3 weights + per-token dynamic activation quant
    (_legacy/fp8_private.py:21-38). ``scale`` is (1, N) fp32 as in the reference.

    The codes are packed into MFMA-fragment order at construction
    (ff_pack_weight_fp8), the layout every GEMM of this op reads; where the
    packed kernels take every row count of the shape (n % 128 == 0, k % 512 ==
    0) that copy is the only one kept and ``weight`` is a ``PackedCodes``
    (``keep_rowmajor`` keeps the row-major tensor too, for callers of the
    row-major entry points)."""

    def __init__(self, weight, keep_rowmajor=False):
        assert weight.is_cuda and weight.ndim == 2 and weight.shape[0] % 16 == weight.shape[1] % 16 == 0
        w = weight.detach().to(BF16).contiguous()
        n, k = w.shape
        self.weight = torch.empty((n, k), device=w.device, dtype=E4M3)
        scale = torch.empty((n,), device=w.device, dtype=torch.float32)
        call("ff_quant_weight_fp8", ptr(w), ptr(self.weight), ptr(scale), None, n, k, 1, stream())
        self.scale = scale.reshape(1, n)
        self.packed = None
        _single_copy(self, keep_rowmajor)

    def pack(self):
        """Add the MFMA-fragment copy of the weight (ff_pack_weight_fp8) that the
        packed tile kernels read (once; construction already does it)."""
        n, k = self.weight.shape
        if self.packed is None and n % 16 == 0 and k % 128 == 0:
            self.packed = torch.empty((n, k), device=self.weight.device, dtype=E4M3)
            call("ff_pack_weight_fp8", ptr(self.weight), ptr(self.packed), n, k, stream())
        return self

    def quantize(self, x):
        """Per-token e4m3 codes and scales of x (2-D view, bf16)."""
        flat = _rows(x)
        if flat.stride(-1) != 1:
            flat = flat.contiguous()
        m, k = flat.shape
        q = torch.empty((m, k), device=x.device, dtype=E4M3)
        s = torch.empty((m,), device=x.device, dtype=torch.float32)
        call("ff_quant_rows_fp8", ptr(flat), flat.stride(0), ptr(q), ptr(s), m, k, stream())
        return q, s

    def gemm(self, q, s, out=None, workspace=None):
        """y = bf16(q_a . W^T * s_a * s_w) from pre-quantized activations. With the
        packed copy this is ff_gemm_fp8_pk, whose k split needs a workspace:
        ``workspace`` if given (a caller's, reused across calls that are ordered
        on one stream), else one this op keeps."""
        m, k = q.shape
        n = self.weight.shape[0]
        y = torch.empty((m, n), device=q.device, dtype=BF16) if out is None else out
        if self.packed is None:
            call("ff_gemm_fp8", ptr(q), ptr(s), 1, ptr(self.weight), ptr(self.scale), 1, ptr(y), y.stride(0),
                 m, n, k, stream())
            return y
        if workspace is None:
            return _packed_gemm(self, q, s, 1, self.scale, 1, y)
        call("ff_gemm_fp8_pk", ptr(q), ptr(s), 1, ptr(self.weight), ptr(self.packed), ptr(self.scale), 1, ptr(y),
             y.stride(0), m, n, k, ptr(workspace), workspace.numel(), stream())
        return y

    def __call__(self, x):
        assert x.is_cuda and x.dtype == BF16
        q, s = self.quantize(x)
        return self.gemm(q, s).reshape(*x.shape[:-1], self.weight.shape[0])


class StaticFP8Linear:
    """Per-tensor e4m3 weight scale and a static activation scale
    (_legacy/limit_kernels.py:110-135). ``input_scale`` is an fp32 (1,) device
    tensor that callers may update in place (``select``,
    _family/night_runtime.py:48-54); ``inverse_scale`` is the quant multiplier."""

    def __init__(self, weight, inverse_scale=16., keep_rowmajor=False):
        w = weight.detach().to(BF16).contiguous()
        n, k = w.shape
        self.weight = torch.empty((n, k), device=w.device, dtype=E4M3)
        self.weight_scale = torch.empty((1,), device=w.device, dtype=torch.float32)
        work = torch.empty((n,), device=w.device, dtype=torch.float32)
        call("ff_quant_weight_fp8", ptr(w), ptr(self.weight), ptr(self.weight_scale), ptr(work), n, k, 0,
             stream())
        self.inverse_scale = inverse_scale
        self.input_scale = torch.tensor([1. / inverse_scale], device=w.device, dtype=torch.float32)
        self.fast_accum = True
        self.packed = None
        _single_copy(self, keep_rowmajor)     # as FP8Linear: the packed copy alone where it serves every shape

    pack = FP8Linear.pack

    def set_bound(self, bound):
        """Calibrate to activation bound ``bound`` as the reference's ``select``
        does per op (_family/night_runtime.py:52-54): ``inverse_scale = 448/bound``
        and ``input_scale`` refilled in place with ``bound/448``. A graph captured
        before this call keeps the old multiplier; the graph runners re-capture."""
        self.inverse_scale = 448. / bound
        self.input_scale.fill_(bound / 448.)

    def __call__(self, x):
        flat = _rows(x)
        if not flat.is_contiguous():
            flat = flat.contiguous()
        m, k = flat.shape
        n = self.weight.shape[0]
        q = torch.empty((m, k), device=x.device, dtype=E4M3)
        call("ff_quant_static_fp8", ptr(flat), ptr(q), m, m, k, float(self.inverse_scale), stream())
        y = torch.empty((m, n), device=x.device, dtype=BF16)
        if self.packed is not None:
            return _packed_gemm(self, q, self.input_scale, 0, self.weight_scale, 0, y)
        call("ff_gemm_fp8", ptr(q), ptr(self.input_scale), 0, ptr(self.weight), ptr(self.weight_scale), 0,
             ptr(y), n, m, n, k, stream())
        return y


def parity(op, x):
    """``parity`` (_family/depth_fp8.py:29-37) for a static-scale linear and an
    activation x: the e4m3 codes of the runtime-scale cast (ff_quant_static_fp8,
    the cast the fused producers share) against an independent cast of the
    same formula (torch: e4m3(clamp(x * inverse_scale, +-448)), round to nearest
    even), byte for byte, and the op's output against the GEMM on those codes.
    Returns {shape, inverse_scale, quant_bytes_exact, output_exact}; asserts both."""
    flat = _rows(x).contiguous()
    m, k = flat.shape
    n = op.weight.shape[0]
    q = torch.empty((m, k), device=flat.device, dtype=E4M3)
    call("ff_quant_static_fp8", ptr(flat), ptr(q), m, m, k, float(op.inverse_scale), stream())
    ref = (flat.float() * float(op.inverse_scale)).clamp(-448., 448.).to(E4M3)
    exact = torch.equal(q.view(torch.uint8), ref.view(torch.uint8))
    new = op(flat)
    prev = torch.empty((m, n), device=flat.device, dtype=BF16)
    if op.packed is not None:
        _packed_gemm(op, ref, op.input_scale, 0, op.weight_scale, 0, prev)
    else:
        call("ff_gemm_fp8", ptr(ref), ptr(op.input_scale), 0, ptr(op.weight), ptr(op.weight_scale), 0, ptr(prev), n,
             m, n, k, stream())
    result = dict(shape=[m, k], inverse_scale=op.inverse_scale, quant_bytes_exact=exact,
                  output_exact=torch.equal(new.reshape(m, n), prev))
    assert exact and result["output_exact"], result
    return result


class RuntimeScaleLinear(StaticFP8Linear):
    """``RuntimeScaleLinear`` (_family/depth_fp8.py:22-26): the activation multiplier is
    read at call time, so ``select`` can change it without re-building the op.

    ``fast_accum`` (set by the reference's ``set_mode``, _family/night_runtime.py:59)
    is accepted and does not change the arithmetic. The reference's ``precise``
    mode (``use_fast_accum=False``) promotes tensor-core partial sums to fp32
    registers at intervals, its ``fp8`` mode keeps them in the tensor core. The
    gfx950 matrix instruction here sums each block of 32 products with ~13
    significant bits and adds the blocks in fp32, i.e. a promotion every 32
    products, which is at least as exact as either mode."""


class Int4:
    """W4A16 linear (_family/night_runtime.py:15-42). ``symmetric=True`` (default,
    group 128) stores s = bf16(amax/7) and z = 0; ``symmetric=False`` is the
    reference's asymmetric min/max quantizer (group 32 there).

    ``oracle=True`` keeps the fp32 dequantised weight ((q - 8) s + z) until the
    first call, which checks its first output row against that weight in fp32:
    ``operator_check`` = {passed: relative RMS <= 0.01, relative_rms, max_abs,
    shape}, asserted (the reference's setup-time check, :28-41). The first call
    must be eager (the check reads the result on the host)."""

    def __init__(self, w, group=128, symmetric=True, oracle=False):
        n, k = w.shape
        assert n % 8 == 0 and k % 128 == 0 and k % group == 0
        w = w.detach().to(BF16).contiguous()
        self.weight = types.SimpleNamespace(shape=(n, k))
        self.group = group
        self.symmetric = symmetric
        self.packed = torch.empty((n, k // 2), device=w.device, dtype=torch.uint8)
        self.scales = torch.empty((k // group, n, 2), device=w.device, dtype=BF16)
        call("ff_quant_weight_int4", ptr(w), ptr(self.packed), ptr(self.scales), n, k, group,
             1 if symmetric else 0, stream())
        self.frag = self.frag_scales = None
        self.oracle = self.operator_check = None
        if oracle:
            q = torch.stack((self.packed >> 4, self.packed & 15), -1).reshape(n, k).float()
            s, z = self.scales.float().permute(2, 1, 0)                      # (n, k / group) each
            self.oracle = ((q.reshape(n, -1, group) - 8) * s[..., None] + z[..., None]).reshape(n, k)

    def _check(self, flat, y):
        """The first-call operator check against the fp32 dequantised weight."""
        reference = torch.nn.functional.linear(flat[:1].float(), self.oracle)
        delta = y[:1].float() - reference
        rms = float(delta.square().mean().sqrt() / (reference.square().mean().sqrt() + 1e-12))
        self.operator_check = dict(passed=rms <= .01, relative_rms=rms, max_abs=float(delta.abs().max()),
                                   shape=list(flat.shape))
        self.oracle = None
        assert self.operator_check["passed"], self.operator_check

    def pack(self):
        """Add the copies the packed kernels read: the nibbles in MFMA-fragment
        order (ff_pack_weight_int4) and the (s, z) pairs as fp32 (16 s, z)
        (ff_pack_scales_int4). ``packed`` / ``scales`` stay for the shapes the
        packed kernels do not take. Weights with a scale of 2^120 or more stay
        unpacked (16 s must be exact)."""
        n, k = self.weight.shape
        if self.frag is None and n % 16 == 0 and k % 128 == 0:
            if float(self.scales[..., 0].abs().max()) >= 2.0 ** 120:
                return self
            self.frag = torch.empty_like(self.packed)
            call("ff_pack_weight_int4", ptr(self.packed), ptr(self.frag), n, k, stream())
            self.frag_scales = torch.empty(self.scales.shape, device=self.scales.device, dtype=torch.float32)
            call("ff_pack_scales_int4", ptr(self.scales), ptr(self.frag_scales), n, k, self.group, stream())
        return self

    def __call__(self, x, out=None):
        flat = _rows(x)
        if flat.stride(-1) != 1 or flat.stride(0) % 8:
            flat = flat.contiguous()
        m, k = flat.shape
        n = self.weight.shape[0]
        y = torch.empty((m, n), device=x.device, dtype=BF16) if out is None else out
        need = ctypes.c_int64(0)
        if self.frag is not None:
            call("ff_gemm_w4a16_pk_workspace", m, n, k, self.group, ctypes.byref(need))
            ws = torch.empty(need.value, device=x.device, dtype=torch.uint8) if need.value else None
            call("ff_gemm_w4a16_pk", ptr(flat), flat.stride(0), ptr(self.packed), ptr(self.frag), ptr(self.scales),
                 ptr(self.frag_scales), self.group, ptr(y), y.stride(0), m, n, k, ptr(ws), need.value, stream())
        else:
            call("ff_gemm_w4a16_workspace", m, n, k, ctypes.byref(need))
            ws = torch.empty(need.value, device=x.device, dtype=torch.uint8) if need.value else None
            call("ff_gemm_w4a16_ws", ptr(flat), flat.stride(0), ptr(self.packed), ptr(self.scales), self.group,
                 ptr(y), y.stride(0), m, n, k, ptr(ws), need.value, stream())
        if self.oracle is not None:
            self._check(flat, y)
        return y

    def add_rms(self, x, a, deep, module, start=0, nv=0):
        """``ops.add_rms(a, self(x), deep, module, start, nv)`` in one op
        (ff_gemm_w4a16_pk_add_rms: where the packed GEMM splits k, the add_rms
        launch adds its fp32 partials; the same bits). Returns (residual, out)
        like ``ops.add_rms``."""
        from . import ops
        if self.frag is None:
            return ops.add_rms(a, self(x), deep, module, start, nv)
        flat = _rows(x)
        if flat.stride(-1) != 1 or flat.stride(0) % 8:
            flat = flat.contiguous()
        if self.oracle is not None:
            # the first-call operator check on row 0 of the full-m product: ff_gemm_w4a16_pk
            # runs the packed tile kernel the fused op runs (a one-row call would take the GEMV)
            self(flat)
        m, k = flat.shape
        n = self.weight.shape[0]
        assert a.is_contiguous() and a.dtype == BF16 and a.shape[-1] == n and a.numel() == m * n
        if deep is not None:
            assert deep.shape == (nv, n) and deep.is_contiguous()
        need = ctypes.c_int64(0)
        call("ff_gemm_w4a16_pk_workspace", m, n, k, self.group, ctypes.byref(need))
        ws = torch.empty(need.value, device=x.device, dtype=torch.uint8) if need.value else None
        y = torch.empty((m, n), device=x.device, dtype=BF16)
        residual, out = torch.empty_like(a), torch.empty_like(a)
        call("ff_gemm_w4a16_pk_add_rms", ptr(flat), flat.stride(0), ptr(self.packed), ptr(self.frag), ptr(self.scales),
             ptr(self.frag_scales), self.group, ptr(y), m, n, k, ptr(ws), need.value, ptr(a), ptr(deep),
             ptr(module.weight), ptr(residual), ptr(out), float(module.variance_epsilon), int(start), int(nv),
             stream())
        return residual, out

    def qkv(self, x, hq, hk, q_norm, k_norm, cos, sin):
        """The QKV linear with qk_pair and the V transpose in one op
        (ff_gemm_w4a16_qkv): x (1, T, H) -> yq (1, hq, T, 128), yk (1, hk, T, 128),
        vt (hk, 128, t_pad), t_pad; None where the packed kernel does not take
        the shape (the caller then runs the separate ops)."""
        if self.frag is None:
            return None
        flat = _rows(x)
        if flat.stride(-1) != 1 or flat.stride(0) % 8:
            flat = flat.contiguous()
        if self.oracle is not None:
            # the first-call operator check on row 0 of the full-m product: ff_gemm_w4a16_pk
            # runs the packed tile kernel the fused op runs (a one-row call would take the GEMV)
            self(flat)
        m, k = flat.shape
        need = ctypes.c_int64(0)
        call("ff_gemm_w4a16_qkv_workspace", m, k, hq, hk, self.group, ctypes.byref(need))
        if need.value == 0:
            return None
        d, tp = 128, (m + 63) // 64 * 64
        yq = torch.empty((1, hq, m, d), device=x.device, dtype=BF16)
        yk = torch.empty((1, hk, m, d), device=x.device, dtype=BF16)
        vt = torch.empty((hk, d, tp), device=x.device, dtype=BF16)
        ws = torch.empty(need.value, device=x.device, dtype=torch.uint8)
        cos2, sin2 = cos.reshape(-1, d).contiguous(), sin.reshape(-1, d).contiguous()
        call("ff_gemm_w4a16_qkv", ptr(flat), flat.stride(0), ptr(self.frag), ptr(self.frag_scales), self.group, m, k,
             hq, hk, ptr(q_norm.weight), ptr(k_norm.weight), float(q_norm.variance_epsilon),
             float(k_norm.variance_epsilon), ptr(cos2), ptr(sin2), ptr(yq), ptr(yk), ptr(vt), tp, ptr(ws),
             need.value, stream())
        return yq, yk, vt, tp

    def swiglu_fits(self, m):
        """Whether ``swiglu`` runs the fused kernel for ``m`` rows."""
        if self.frag is None:
            return False
        n, k = self.weight.shape
        ok = ctypes.c_int(0)
        call("ff_gemm_w4a16_swiglu_fits", m, n // 2, k, self.group, ctypes.byref(ok))
        return bool(ok.value)

    def swiglu(self, x):
        """swiglu(g, u) for [g, u] = self(x).chunk(2, -1) (gate rows first): one
        fused launch where the packed kernel takes the shape (ff_gemm_w4a16_swiglu_pk,
        the same bits), else the GEMM and ``ops.swiglu``."""
        flat = _rows(x)
        if flat.stride(-1) != 1 or flat.stride(0) % 8:
            flat = flat.contiguous()
        if self.oracle is not None:
            # the first-call operator check on row 0 of the full-m product: ff_gemm_w4a16_pk
            # runs the packed tile kernel the fused op runs (a one-row call would take the GEMV)
            self(flat)
        m, k = flat.shape
        i = self.weight.shape[0] // 2
        if not self.swiglu_fits(m):
            from . import ops
            g, u = self(x).chunk(2, -1)
            return ops.swiglu(g, u)
        h = torch.empty((m, i), device=x.device, dtype=BF16)
        call("ff_gemm_w4a16_swiglu_pk", ptr(flat), flat.stride(0), ptr(self.frag), ptr(self.frag_scales), self.group,
             ptr(h), i, m, i, k, stream())
        return h.reshape(*x.shape[:-1], i)
