"""The W4A16 kernels on fragment-packed int4 weights (ff_pack_weight_int4,
ff_gemm_w4a16_pk, ff_gemm_w4a16_swiglu_pk) against the LDS-staged kernel and
the oracle's exact dequantisation (Int4, _family/night_runtime.py:15-42).

Bars: where neither kernel splits k, the packed kernel runs the same MFMAs on
the same dequantised values in the same k order, so the bits are equal; with a
k split, or on the single-row GEMV (m <= 4: the same bf16 weights, summed on
v_dot2_f32_bf16 in another fp32 order), only the order of the fp32 sum
differs (|difference| <= 1 bf16 ulp + 2^-21 sum |x w|, under 1% of outputs
differing). Every shape is also held to the fp64 product
with the exactly dequantised weight (relative RMS <= 5e-3, worst element <=
0.05 of the output RMS), as the LDS-staged kernel's tests are."""
import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import bf16_ulps

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda"

FF_TUNE_W4A16_SPLITS = 4


def _g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.fixture
def tuning(gpu):
    from fastforward_amd._lib import call
    used = []

    def set_(knob, value):
        used.append(knob)
        call("ff_set_tuning", knob, value)
    yield set_
    for knob in used:
        call("ff_set_tuning", knob, 0)


def _unsplit_lds(op, x, tuning):
    """The LDS-staged kernel (ff_gemm_w4a16_ws) with k unsplit."""
    frag, op.frag = op.frag, None
    tuning(FF_TUNE_W4A16_SPLITS, 1)
    try:
        return op(x)
    finally:
        op.frag = frag
        tuning(FF_TUNE_W4A16_SPLITS, 0)


def _pk_splits(m, n, k):
    """Splits the packed plan takes (mirrors w4pk_plan for the tested shapes)."""
    tm = (m + 143) // 144
    if n % 384 == 0 and tm * (n // 384) >= 192:
        return 1
    tiles = tm * (n // 256)
    s = 1 if tiles >= 192 else 256 // tiles
    return max(1, min(s, 8, k // 256))


def test_pack_weight_int4_layout(gpu):
    """ff_pack_weight_int4 stores fragment (f, kt) at (kt * n/16 + f) * 1024 with
    lane l = 16 g + r holding row 16 f + r, the packed bytes of k = 128 kt +
    64 h + 16 g + [0, 16) for h = 0, 1 (8 bytes each), every nibble q as q ^ 8."""
    from fastforward_amd._lib import call, ptr, stream
    n, k = 48, 384
    src = torch.randint(0, 256, (n, k // 2), generator=_g(69), dtype=torch.uint8)
    frag = torch.empty(n * k // 2, device=DEV, dtype=torch.uint8)
    src_d = src.to(DEV)
    call("ff_pack_weight_int4", ptr(src_d), ptr(frag), n, k, stream())
    got = frag.cpu().numpy().reshape(k // 128, n // 16, 64, 16)
    s = src.numpy() ^ 0x88
    for f in range(n // 16):
        for kt in range(k // 128):
            for lane in range(64):
                r, g = lane % 16, lane // 16
                row = s[16 * f + r]
                want = np.concatenate([row[64 * kt + 8 * g: 64 * kt + 8 * g + 8],
                                       row[64 * kt + 32 + 8 * g: 64 * kt + 32 + 8 * g + 8]])
                assert np.array_equal(got[kt, f, lane], want), (f, kt, lane)


SHAPES = [(576, 4096, 24576), (576, 4096, 6144), (576, 12288, 4096), (576, 4096, 4096), (320, 2048, 6144),
          (100, 1024, 512), (1, 12288, 4096), (1, 4096, 4096), (3, 4096, 1040), (4, 1024, 16)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("sym,group", [(True, 128), (False, 32)])
def test_w4a16_packed_vs_lds_kernel_and_exact(gpu, tuning, m, k, n, sym, group):
    from fastforward_amd.linear import Int4
    x = torch.randn(m, k, generator=_g(70)).to(BF16)
    w = (torch.randn(n, k, generator=_g(71)) * 0.02).to(BF16)
    op = Int4(w.to(DEV), group=group, symmetric=sym).pack()
    xd = x.to(DEV)
    outs = [op(xd) for _ in range(3)]
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    dq = O.int4_dequant(op.packed.cpu(), op.scales.cpu(), group).double()
    ref = _unsplit_lds(op, xd, tuning)
    if m > 4 and _pk_splits(m, n, k) == 1:
        assert torch.equal(outs[0], ref), (m, k, n)
    else:
        # adding the splits' partials reassociates the fp32 sum: an absolute
        # error of a few fp32 ulps of sum |x w|, plus each side's bf16 rounding
        got, want = outs[0].cpu().double(), ref.cpu().double()
        mag = torch.maximum(got.abs(), want.abs()).clamp_min(2.0 ** -126)
        ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
        scale = x.double().abs() @ dq.abs().T
        assert bool(((got - want).abs() <= ulp + 2.0 ** -21 * scale).all())
        assert float((bf16_ulps(outs[0], ref) > 0).float().mean()) < 0.01
    y = outs[0].cpu().double()
    exact = x.double() @ dq.T
    rms = exact.pow(2).mean().sqrt()
    assert float((y - exact).pow(2).mean().sqrt() / rms) <= 5e-3
    assert float((y - exact).abs().max() / rms) <= 0.05


@pytest.mark.parametrize("n,k", [(256, 256), (256, 512)])
def test_w4a16_packed_dequant_bit_exact_via_one_hot(gpu, n, k):
    """x = rows of the identity, so y[r, c] = bf16((q-8)*s + z) for k = r exactly,
    unsplit (k 256) and split in two (k 512; each output has one nonzero
    product, so adding the partials is exact). Columns 0-39 hold 64.0 in their
    first 32 k: the asymmetric quantizer stores s = bf16(1e-6), z = 64 there,
    where z - 8s is not exact in fp32 (the case the LDS-staged kernel routes to
    its exact form; the packed kernel's v_cvt_off form is exact throughout)."""
    from fastforward_amd.linear import Int4
    w = (torch.randn(n, k, generator=_g(72)) * 0.02).to(BF16)
    w[:40, :32] = 64.0
    for sym, group in ((True, 128), (False, 32)):
        op = Int4(w.to(DEV), group=group, symmetric=sym).pack()
        y = op(torch.eye(k, dtype=BF16, device=DEV)).cpu()
        dq = O.int4_dequant(op.packed.cpu(), op.scales.cpu(), group).to(BF16)
        assert torch.equal(y, dq.T.contiguous()), (sym, group)


@pytest.mark.parametrize("m,k,i", [(1, 4096, 12288), (3, 1024, 656)])
@pytest.mark.parametrize("sym,group", [(True, 128), (False, 32)])
def test_w4a16_swiglu_gemv_vs_exact(gpu, m, k, i, sym, group):
    """The tail's fused gate/up + SwiGLU (single-row GEMV on the packed copies)
    against the fp64 product with the dequantised weights rounded to bf16 (the
    MFMA operand; the oracle's bf16-weight form), SwiGLU in fp64: relative RMS
    <= 5e-3, and per element |h - want| <= 2^-6 |want| + 1e-3 RMS (h rounds g,
    u, silu(g) and the product to bf16, about 4 ulps of its own size); the
    unfused ops (tile kernel + swiglu) meet the same bar."""
    from fastforward_amd import ops
    from fastforward_amd.linear import Int4
    x = torch.randn(m, k, generator=_g(80)).to(BF16)
    w = (torch.randn(2 * i, k, generator=_g(81)) * 0.02).to(BF16)
    op = Int4(w.to(DEV), group=group, symmetric=sym).pack()
    assert op.swiglu_fits(m)
    h = op.swiglu(x.to(DEV)).cpu().double()
    dq = O.int4_dequant(op.packed.cpu(), op.scales.cpu(), group).to(BF16).double()
    gu = x.double() @ dq.T
    g, u = gu[:, :i], gu[:, i:]
    want = g / (1 + torch.exp(-g)) * u
    rms = want.pow(2).mean().sqrt()
    bound = 2.0 ** -6 * want.abs() + 1e-3 * rms
    assert float((h - want).pow(2).mean().sqrt() / rms) <= 5e-3
    assert bool(((h - want).abs() <= bound).all())
    gg, uu = op(x.to(DEV)).chunk(2, -1)
    unf = ops.swiglu(gg, uu).cpu().double()
    assert bool(((unf - want).abs() <= bound).all())


# 576 tokens: 144-row tiles; 640: 160-row tiles (one round of 256 workgroups)
@pytest.mark.parametrize("m,k,i", [(576, 4096, 12288), (640, 4096, 12288), (320, 2048, 6144), (100, 1024, 640)])
@pytest.mark.parametrize("sym,group", [(True, 128), (False, 32)])
def test_w4a16_swiglu_packed_equals_unfused(gpu, tuning, m, k, i, sym, group):
    """ff_gemm_w4a16_swiglu_pk == ops.swiglu of the unsplit gate/up product, bit
    for bit (144 x 384 and 144 x 256 tiles; ragged m)."""
    from fastforward_amd import ops
    from fastforward_amd.linear import Int4
    x = torch.randn(m, k, generator=_g(73)).to(BF16).to(DEV)
    w = (torch.randn(2 * i, k, generator=_g(74)) * 0.02).to(BF16)
    op = Int4(w.to(DEV), group=group, symmetric=sym).pack()
    assert op.swiglu_fits(m)
    h = op.swiglu(x)
    g, u = _unsplit_lds(op, x, tuning).chunk(2, -1)
    assert torch.equal(h, ops.swiglu(g, u))
    assert torch.equal(h, op.swiglu(x))


@pytest.mark.parametrize("m,k,hq,hk", [(576, 4096, 32, 8), (320, 2048, 16, 8), (144, 1024, 8, 4), (100, 1024, 8, 2)])
@pytest.mark.parametrize("sym,group", [(True, 128), (False, 32)])
def test_w4a16_qkv_fused_equals_unfused(gpu, m, k, hq, hk, sym, group):
    """Int4.qkv (ff_gemm_w4a16_qkv) == the packed QKV GEMM, qk_pair and the V
    transpose of attention_direct (ff_v_transpose), bit for bit, with zeros in
    V^T for the padded tokens (m = 144: t_pad 192 lies beyond the last tile)."""
    from fastforward_amd import ops
    from fastforward_amd._lib import call, ptr, stream
    from fastforward_amd.linear import Int4
    d = 128
    n = (hq + 2 * hk) * d
    x = torch.randn(1, m, k, generator=_g(75)).to(BF16).to(DEV)
    w = (torch.randn(n, k, generator=_g(76)) * 0.02).to(BF16)
    op = Int4(w.to(DEV), group=group, symmetric=sym).pack()
    qn = ops.RMSNorm((1 + 0.2 * torch.randn(d, generator=_g(77))).to(BF16).to(DEV), 1e-6)
    kn = ops.RMSNorm((1 + 0.2 * torch.randn(d, generator=_g(78))).to(BF16).to(DEV), 1e-6)
    ang = torch.randn(m, d, generator=_g(79)) * 3
    cos, sin = ang.cos().to(BF16).to(DEV)[None], ang.sin().to(BF16).to(DEV)[None]
    yq, yk, vt, tp = op.qkv(x, hq, hk, qn, kn, cos, sin)
    q, kk, v = op(x).reshape(1, m, n).split([hq * d, hk * d, hk * d], -1)
    rq, rk = ops.qk_pair(q.view(1, m, hq, d), kk.view(1, m, hk, d), qn, kn, cos, sin)
    assert torch.equal(yq, rq) and torch.equal(yk, rk)
    vv = v.view(1, m, hk, d).transpose(1, 2)
    rvt = torch.full((hk, d, tp), float("nan"), device=DEV, dtype=BF16)
    call("ff_v_transpose", ptr(vv), vv.stride(2), vv.stride(1), ptr(rvt), m, tp, hk, d, stream())
    assert torch.equal(vt, rvt)
    assert int(vt[:, :, m:].abs().sum()) == 0


@pytest.mark.parametrize("m,k,n,deep", [(576, 12288, 4096, True), (576, 4096, 4096, False), (500, 12288, 4096, False),
                                        (320, 6144, 2048, True), (576, 4096, 12288, False), (1, 12288, 4096, False)])
def test_w4a16_add_rms_equals_unfused(gpu, m, k, n, deep):
    """Int4.add_rms (ff_gemm_w4a16_pk_add_rms) == ops.add_rms of the packed GEMM's
    output, bit for bit, residual and normalised rows: where the GEMM splits k
    (o and down of the 8B step, 500 rows with a ragged last tile, DeepStack
    rows) the add_rms launch adds the partials; elsewhere (144 x 384 tiles
    unsplit, the one-row GEMV) the two ops run."""
    from fastforward_amd import ops
    from fastforward_amd.linear import Int4
    x = torch.randn(m, k, generator=_g(80)).to(BF16).to(DEV)
    w = (torch.randn(n, k, generator=_g(81)) * 0.02).to(BF16)
    op = Int4(w.to(DEV), group=128, symmetric=True).pack()
    a = (torch.randn(1, m, n, generator=_g(82)) * 3).to(BF16).to(DEV)
    norm = ops.RMSNorm((1 + 0.2 * torch.randn(n, generator=_g(83))).to(BF16).to(DEV), 1e-6)
    start, nv = (min(5, m - 1), min(40, m - min(5, m - 1))) if deep else (0, 0)
    dp = torch.randn(nv, n, generator=_g(84)).to(BF16).to(DEV) if deep else None
    r0, o0 = ops.add_rms(a, op(x).reshape(1, m, n), dp, norm, start, nv)
    r1, o1 = op.add_rms(x, a, dp, norm, start, nv)
    assert torch.equal(r0, r1) and torch.equal(o0, o1)
    assert not torch.isnan(o1.float()).any()
