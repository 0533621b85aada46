"""Setup-time self-checks on the weights as loaded, as the reference runs them:
the Int4 operator check (_family/night_runtime.py:28-41) and the static-FP8
cast parity (_family/depth_fp8.py:29-62)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("sym,group", [(True, 128), (False, 32)])
@pytest.mark.parametrize("how", ["plain", "packed", "packed_qkv", "packed_swiglu"])
def test_int4_operator_check(gpu, sym, group, how):
    """Int4(oracle=True): the first call (plain GEMM, packed GEMM, or the fused
    QKV / gate-up forms, which check through the GEMM on the first row) records
    operator_check with relative RMS <= 0.01 against the fp32 dequantised
    weight and drops that weight; later calls do not check again."""
    from fastforward_amd import ops
    from fastforward_amd.linear import Int4
    hq, hk, d, k, m = 8, 4, 128, 1024, 96
    n = (hq + 2 * hk) * d
    w = (torch.randn(n, k, generator=_g(90)) * 0.02).to(BF16).to(DEV)
    op = Int4(w, group=group, symmetric=sym, oracle=True)
    assert op.oracle is not None and op.operator_check is None
    if how != "plain":
        op.pack()
    x = torch.randn(1, m, k, generator=_g(91)).to(BF16).to(DEV)
    if how == "packed_qkv":
        qn = ops.RMSNorm(torch.ones(d, dtype=BF16, device=DEV), 1e-6)
        ang = torch.randn(m, d, generator=_g(92))
        assert op.qkv(x, hq, hk, qn, qn, ang.cos().to(BF16).to(DEV), ang.sin().to(BF16).to(DEV)) is not None
    elif how == "packed_swiglu":
        op.swiglu(x)
    else:
        op(x)
    chk = op.operator_check
    assert chk["passed"] and chk["relative_rms"] <= 0.01 and op.oracle is None, chk
    op(x)
    assert op.operator_check is chk


def test_int4_operator_check_trips(gpu):
    """The check fails loudly when the weights disagree with its fp32 reference
    (the mistake is planted in that reference, scaled by 1.05)."""
    from fastforward_amd.linear import Int4
    w = (torch.randn(256, 512, generator=_g(93)) * 0.02).to(BF16).to(DEV)
    op = Int4(w, oracle=True)
    op.oracle *= 1.05
    with pytest.raises(AssertionError):
        op(torch.randn(8, 512, generator=_g(94)).to(BF16).to(DEV))
    assert op.operator_check["passed"] is False and op.operator_check["relative_rms"] > 0.01


def test_fp8_static_parity(gpu):
    """linear.parity: the runtime-scale e4m3 cast equals an independent cast of
    the same formula byte for byte (outliers beyond the clamp included), and
    the op's output equals the GEMM on those codes."""
    from fastforward_amd.linear import RuntimeScaleLinear, parity
    w = (torch.randn(512, 1024, generator=_g(95)) * 0.02).to(BF16).to(DEV)
    op = RuntimeScaleLinear(w, 448.0 / 6.0)
    x = torch.randn(77, 1024, generator=_g(96)) * 2
    x[3, :5] = 40.0                       # beyond the bound: clamped to +-448 codes
    res = parity(op, x.to(BF16).to(DEV))
    assert res["quant_bytes_exact"] and res["output_exact"] and res["shape"] == [77, 1024]


def test_model_parity_restores_scales(gpu):
    """profiles.model_parity on a small static-FP8 model: every observed linear
    (all roles of the middle layer, gate/up and down of the final one) passes
    under each calibration variant, and each op's scales are restored."""
    from fastforward_amd.profiles import model_parity
    from fastforward_amd.runtime import LMConfig
    from fastforward_amd.synthetic import make_model, make_request
    cfg = LMConfig("tiny", 4, 512, 4, 2, 128, 1024, 1000)
    w = make_model(cfg, mode="fp8_static", seed=5, norm_jitter=0.2)
    ids, pos, pick = make_request(cfg, 128, 4, 4, seed=6)
    before = [(L.qkv.inverse_scale, float(L.qkv.input_scale)) for L in w.layers]
    prof = {"a": {f"{j}:{r}": 6.0 for j in range(4) for r in ("qkv", "output", "gateup", "down")},
            "b": {f"{j}:{r}": 3.0 + j for j in range(4) for r in ("qkv", "output", "gateup", "down")}}
    checks = model_parity(cfg, w, ids, pos, pick, profiles=prof)
    roles = sorted({c["role"] for c in checks})
    assert roles == ["2:down", "2:gateup", "2:output", "2:qkv", "3:down", "3:gateup"], roles
    assert len(checks) == 2 * len(roles)
    assert all(c["quant_bytes_exact"] and c["output_exact"] for c in checks)
    assert [(L.qkv.inverse_scale, float(L.qkv.input_scale)) for L in w.layers] == before
