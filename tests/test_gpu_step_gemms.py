"""Every FP8 GEMM launch of the LM step, at the 2B / 8B / 32B shapes, against the oracle.

Each case goes through the entry point and weight layout the step itself uses
(``Runtime._attention_fused`` / ``_gemm`` / ``_mlp_fused``), so every tile that
the dispatch picks at these shapes -- the row-major 128 x 128 four-stage QKV
tile with its norm / rotary / V^T epilogue, the 64 x 128 and 128 x 128 tiles,
the packed gate/up tile with SwiGLU, the packed k-split tile with its
reduction, the row-major fallbacks and the single-row GEMV of the pick-only
tail -- is compared with the oracle on seeded inputs. Reference formulation:
``FP8Linear.__call__`` / ``torch._scaled_mm`` (_legacy/fp8_private.py:29-38),
``qk_pair`` (_legacy/lower_kernels.py:66-98), ``swiglu``
(_legacy/search_kernels.py:8-23).

Bars:
* Plain GEMM outputs (o, down, the V columns of QKV, the tail's rows): within
  the accumulation bound of the exact fp64 product of the codes (one bf16 ulp
  plus 2^-16 * sum |a w| * sa * sw) and equal to the oracle's bf16 result for
  >= 98 % of elements (97 % beyond K = 16384): the matrix unit sums each
  32-product block with ~13 bits, so ~1 % of outputs round to the neighbouring
  bf16 of the fp32 result.
* Fused epilogues (QKV's norm + rotary + V^T, gate/up's SwiGLU): every
  unsplit FP8 tile adds the same 128-deep MFMA steps in the same k order, so
  the raw product of the same codes from ff_gemm_fp8 is what the fused kernel
  sums; that raw product meets the plain-GEMM bar, V^T holds exactly its V
  columns, SwiGLU output equals the oracle's swiglu of it within the swiglu bar
  (<= 1 bf16 ulp, all but 0.1 % exact), and q / k equal the oracle's qk_pair of
  it for all but 0.2 % of values, the rest within two bf16 ulps of the larger
  of the rotary's two terms bf16(xn cos) and bf16(r sin) (the per-head norm may
  round xn one ulp apart; where the two terms cancel, that ulp is many ulps of
  their sum).
* Row maxima of the SwiGLU output per 64 channels: exactly max |h| of the
  GPU's own h (the quantizer reads them instead of the row).
"""
import pytest
import torch

from oracle import ops as O
from tests.helpers import assert_bf16_close
from tests.numerics import ulp_bf16

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda"

# preset -> (tokens, hidden, q heads, kv heads, mlp)
SHAPES = {"2b": (320, 2048, 16, 8, 6144), "4b": (576, 2560, 32, 8, 9728), "8b": (576, 4096, 32, 8, 12288),
          "32b": (1024, 5120, 64, 8, 25600)}
D = 128


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _act(m, k, seed):
    """N(0,1) activations with 0.1 % outliers at x20, bf16."""
    x = torch.randn(m, k, generator=_g(seed))
    x[torch.rand(m, k, generator=_g(seed + 1)) < 0.001] *= 20
    return x.to(BF16)


def _op(n, k, seed):
    from fastforward_amd.linear import FP8Linear
    w = (torch.randn(n, k, generator=_g(seed)) * 0.02).to(BF16)
    return FP8Linear(w.to(DEV), keep_rowmajor=True)   # the tests call the row-major entry points too


def _rows(m):
    """Rows checked against the fp64 exact product: every row of small GEMMs,
    else a spread that includes both ends of every 144- and 128-row tile."""
    if m <= 128:
        return torch.arange(m)
    r = set(range(0, m, 7)) | {m - 1}
    for t in (128, 144):
        r |= {min(i, m - 1) for b in range(0, m, t) for i in (b, b + t - 1)}
    return torch.tensor(sorted(r))


def _assert_plain(y, qa, sa, qw, sw, what):
    """y (m, n) bf16 against the exact product and the oracle's fp32 GEMM on the
    sampled rows."""
    rows = _rows(qa.shape[0])
    a, w = qa[rows].double(), qw.double()
    sa_, sw_ = sa[rows].double().reshape(-1, 1), sw.double().reshape(1, -1)
    exact = (a @ w.T) * sa_ * sw_
    abs_sum = (a.abs() @ w.abs().T) * sa_.abs() * sw_.abs()
    got = y[rows].double()
    bound = torch.from_numpy(ulp_bf16(exact.numpy())) + abs_sum * 2.0 ** -16
    excess = float(((got - exact).abs() - bound).max())
    assert excess <= 0, f"{what}: exceeds the accumulation bound by {excess}"
    want = O.fp8_gemm(qa[rows], sa[rows], qw, sw)
    frac = float((y[rows] != want).float().mean())
    assert frac <= (0.02 if qa.shape[1] <= 16384 else 0.03), f"{what}: {frac:.4f} differ from the oracle"
    print(f"{what}: {frac:.4f} of outputs differ from the oracle's fp32 GEMM", flush=True)


@pytest.mark.parametrize("preset", list(SHAPES))
@pytest.mark.parametrize("role", ["o", "down"])
@pytest.mark.parametrize("rows", ["full", "tail"])
def test_step_plain_gemm_vs_oracle(gpu, preset, role, rows):
    """o and down projections through ff_gemm_fp8_pk with the step's packed
    weights and a runtime-sized workspace (the k-split reduction where it is
    taken); ``tail``: the pick-only final layer's single row (GEMV)."""
    from fastforward_amd._lib import call, ptr, stream
    from fastforward_amd.linear import gemm_pk_workspace
    t, h, hq, _, inter = SHAPES[preset]
    m = t if rows == "full" else 1
    n, k = (h, hq * D) if role == "o" else (h, inter)
    op = _op(n, k, 300 + len(role))
    x = _act(m, k, 310)
    qa, sa = O.quant_rows_dynamic(x)
    qa_d, sa_d = qa.to(DEV), sa.to(DEV)
    ws = torch.full((max(gemm_pk_workspace(m, n, k), 256),), 0xFF, device=DEV, dtype=torch.uint8)
    y = torch.full((m, n), float("nan"), device=DEV, dtype=BF16)
    call("ff_gemm_fp8_pk", ptr(qa_d), ptr(sa_d), 1, ptr(op.weight), ptr(op.packed), ptr(op.scale), 1, ptr(y), n,
         m, n, k, ptr(ws), ws.numel(), stream())
    _assert_plain(y.cpu(), qa, sa, op.weight.cpu(), op.scale.reshape(-1).cpu(), f"{preset} {role} {m}x{k}x{n}")


@pytest.mark.parametrize("preset", list(SHAPES))
@pytest.mark.parametrize("rows", ["full", "tail"])
def test_step_gateup_swiglu_vs_oracle(gpu, preset, rows):
    """gate/up through ff_gemm_fp8_swiglu_pk (packed tile where the shape takes
    it, else the row-major SwiGLU tile; GEMV for the tail's row). The GEMM part:
    the raw gate/up product of the same codes (ff_gemm_fp8; every unsplit FP8
    tile adds the same 128-deep MFMA steps in the same k order, so the fused
    kernel sums identical values) meets the plain-GEMM bar against the exact
    product. The epilogue: h equals the oracle's swiglu of those g and u within
    the swiglu bar (<= 1 bf16 ulp, all but 0.1 % exact); the row maxima it
    writes equal max |h| per 64 channels."""
    from fastforward_amd._lib import call, ptr, stream
    t, h, _, _, inter = SHAPES[preset]
    m = t if rows == "full" else 1
    op = _op(2 * inter, h, 320)
    x = _act(m, h, 330)
    qa, sa = O.quant_rows_dynamic(x)
    qa_d, sa_d = qa.to(DEV), sa.to(DEV)
    hh = torch.full((m, inter), float("nan"), device=DEV, dtype=BF16)
    pmax = torch.full((m, inter // 64), float("nan"), device=DEV)
    call("ff_gemm_fp8_swiglu_pk", ptr(qa_d), ptr(sa_d), ptr(op.weight), ptr(op.packed), ptr(op.scale), ptr(hh),
         inter, ptr(pmax), m, inter, h, stream())
    raw = torch.empty(m, 2 * inter, device=DEV, dtype=BF16)
    call("ff_gemm_fp8", ptr(qa_d), ptr(sa_d), 1, ptr(op.weight), ptr(op.scale), 1, ptr(raw), 2 * inter, m,
         2 * inter, h, stream())
    raw, got = raw.cpu(), hh.cpu()
    _assert_plain(raw, qa, sa, op.weight.cpu(), op.scale.reshape(-1).cpu(), f"{preset} gate/up {m}x{h}x{2 * inter}")
    want = O.swiglu(raw[:, :inter], raw[:, inter:])
    assert_bf16_close(got, want, 1, 1e-3, f"{preset} gate/up swiglu(raw)")
    assert torch.equal(pmax.cpu(), got.float().abs().view(m, inter // 64, 64).amax(-1))


@pytest.mark.parametrize("preset", list(SHAPES))
def test_step_qkv_epilogue_vs_oracle(gpu, preset):
    """The QKV GEMM with the per-head q/k RMSNorm, the M-RoPE rotary and the V
    transpose in its epilogue: ff_gemm_fp8_qkv_pk (the step's launch, packed
    weights) gives the same bits as ff_gemm_fp8_qkv (row-major weights), which
    is checked here. The GEMM part: the raw product of the same codes
    (ff_gemm_fp8, the same tile) meets the plain-GEMM bar against the exact
    product, and V^T is exactly its V columns (the fused kernel sums the same
    values); V^T padding is zero. The epilogue: q and k equal the oracle's
    qk_pair of that raw product within the rotary-term bar of the module
    docstring."""
    from fastforward_amd._lib import call, ptr, stream
    from fastforward_amd.ops import RMSNorm
    t, h, hq, hk, _ = SHAPES[preset]
    tp = (t + 63) // 64 * 64
    n = (hq + 2 * hk) * D
    op = _op(n, h, 340)
    x = _act(t, h, 350)
    qa, sa = O.quant_rows_dynamic(x)
    qa_d, sa_d = qa.to(DEV), sa.to(DEV)
    qn = (1 + 0.3 * torch.randn(D, generator=_g(360))).to(BF16)
    kn = (1 + 0.3 * torch.randn(D, generator=_g(361))).to(BF16)
    qn_d, kn_d = RMSNorm(qn.to(DEV)), RMSNorm(kn.to(DEV))
    grid = {"2b": (16, 16), "4b": (16, 32), "8b": (16, 32), "32b": (30, 32)}[preset]
    cos, sin = O.mrope_cos_sin(O.mrope_positions(4, *grid, t), 5e6, D)
    cos_d, sin_d = cos[0].to(DEV), sin[0].to(DEV)
    yq = torch.full((hq, t, D), float("nan"), device=DEV, dtype=BF16)
    yk = torch.full((hk, t, D), float("nan"), device=DEV, dtype=BF16)
    vt = torch.full((hk, D, tp), float("nan"), device=DEV, dtype=BF16)
    call("ff_gemm_fp8_qkv", ptr(qa_d), ptr(sa_d), 1, ptr(op.weight), ptr(op.scale), 1, t, h, hq, hk, ptr(qn_d.weight),
         ptr(kn_d.weight), 1e-6, 1e-6, ptr(cos_d), ptr(sin_d), ptr(yq), ptr(yk), ptr(vt), tp, stream())
    # the step's launch on the packed copy: the same bits
    pq, pk_, pv = (torch.full_like(b, float("nan")) for b in (yq, yk, vt))
    call("ff_gemm_fp8_qkv_pk", ptr(qa_d), ptr(sa_d), 1, ptr(op.weight), ptr(op.packed), ptr(op.scale), 1, t, h,
         hq, hk, ptr(qn_d.weight), ptr(kn_d.weight), 1e-6, 1e-6, ptr(cos_d), ptr(sin_d), ptr(pq), ptr(pk_), ptr(pv),
         tp, stream())
    assert torch.equal(pq, yq) and torch.equal(pk_, yk) and torch.equal(pv, vt), f"{preset}: packed != row-major"
    raw = torch.empty(t, n, device=DEV, dtype=BF16)
    call("ff_gemm_fp8", ptr(qa_d), ptr(sa_d), 1, ptr(op.weight), ptr(op.scale), 1, ptr(raw), n, t, n, h, stream())
    raw = raw.cpu()
    _assert_plain(raw, qa, sa, op.weight.cpu(), op.scale.reshape(-1).cpu(), f"{preset} qkv {t}x{h}x{n}")
    vt = vt.cpu()
    assert torch.equal(vt[:, :, t:], torch.zeros_like(vt[:, :, t:])), "V^T padding must be zero"
    assert torch.equal(vt[:, :, :t].permute(2, 0, 1).reshape(t, hk * D), raw[:, (hq + hk) * D:])
    xq, xk = raw[:, : hq * D].reshape(1, t, hq, D), raw[:, hq * D:(hq + hk) * D].reshape(1, t, hk, D)
    wq, wk = O.qk_pair(xq, xk, qn, kn, 1e-6, 1e-6, cos, sin)
    for got, want, x_, w_, name in ((yq.cpu(), wq[0], xq, qn, "q"), (yk.cpu(), wk[0], xk, kn, "k")):
        # the rotary's two bf16 terms: y = bf16(bf16(xn c) + bf16(r s)) with r = rotate_half(xn)
        xn = O.qk_pair(x_, x_, w_, w_, 1e-6, 1e-6, torch.ones_like(cos), torch.zeros_like(sin))[0][0].float()
        r = torch.cat((-xn[..., D // 2:], xn[..., : D // 2]), -1)
        terms = torch.maximum((xn * cos[0].float()).abs(), (r * sin[0].float()).abs())
        bound = 2 * torch.from_numpy(ulp_bf16(terms.numpy())).float()
        dif = (got.float() - want.float()).abs()
        frac = float((dif > 0).float().mean())
        print(f"{preset} qkv {name}: {frac:.4f} differ from qk_pair(raw); worst |d| / bound "
              f"{float((dif / bound).max()):.3f}", flush=True)
        assert bool((dif <= bound).all()), f"{preset} qkv {name}: beyond two ulps of the larger rotary term"
        assert frac <= 2e-3, (name, frac)
