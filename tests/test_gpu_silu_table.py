"""The fused SwiGLU GEMM epilogues look bf16(silu(g)) up in a table for
|g| in [2^-8, 128) and use closed forms outside it (silu_bf16). These tests put
every bf16 gate value through them and require the same bits as the exact
form (ff_swiglu: g / (1 + exp(-g)) with a correctly rounded divide,
_legacy/search_kernels.py:8-15).

One-hot GEMMs make g a chosen value per channel: a single nonzero product
per output, 1 x 1 (FP8 codes 0x38) scaled by sw = g, or 1 x z (W4A16 with
every nibble 8 and s = 0, so each dequantised weight is z), with no rounding
before the epilogue's own bf16 rounding."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda"


def _every_bf16():
    return torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16)).view(BF16)


def _same(a, b):
    """Bit equality, NaN at the same places (NaN payloads may differ)."""
    na, nb = torch.isnan(a.float()), torch.isnan(b.float())
    return torch.equal(na, nb) and torch.equal(a.view(torch.int16)[~na], b.view(torch.int16)[~nb])


def test_fp8_gate_up_epilogue_every_bf16_gate(gpu):
    """ff_gemm_fp8_swiglu_pk (packed tile) against ff_gemm_fp8 + ff_swiglu and the
    row-major fused kernel: h for all 65536 gate patterns (NaN, inf, zeros and
    subnormals included) and the per-64-channel row maxima."""
    from fastforward_amd import ops
    from fastforward_amd._lib import call, ptr, stream
    m, i, k = 144, 65664, 512
    qa = torch.zeros(m, k, dtype=torch.uint8, device=DEV)
    qa[:, 0] = 0x38
    qw = torch.zeros(2 * i, k, dtype=torch.uint8, device=DEV)
    qw[:, 0] = 0x38
    packed = torch.empty_like(qw)
    call("ff_pack_weight_fp8", ptr(qw), ptr(packed), 2 * i, k, stream())
    sa = torch.ones(m, device=DEV)
    sw = torch.zeros(2 * i)
    sw[:65536] = _every_bf16().float()
    sw[i:] = torch.randn(i, generator=torch.Generator().manual_seed(3)).to(BF16).float()
    sw = sw.to(DEV)
    gu = torch.empty(m, 2 * i, device=DEV, dtype=BF16)
    call("ff_gemm_fp8", ptr(qa), ptr(sa), 1, ptr(qw), ptr(sw), 1, ptr(gu), 2 * i, m, 2 * i, k, stream())
    assert _same(gu[0, :65536], _every_bf16().to(DEV))
    want = ops.swiglu(*gu.chunk(2, -1))
    wmax = torch.nan_to_num(want.float().abs(), nan=0.0, posinf=float("inf")).reshape(m, i // 64, 64).amax(-1)
    for entry in ("ff_gemm_fp8_swiglu_pk", "ff_gemm_fp8_swiglu"):
        h = torch.full((m, i), 7.0, device=DEV, dtype=BF16)
        pmax = torch.full((m, i // 64), -1.0, device=DEV)
        args = [ptr(qa), ptr(sa), ptr(qw)] + ([ptr(packed)] if entry.endswith("pk") else [])
        call(entry, *args, ptr(sw), ptr(h), i, ptr(pmax), m, i, k, stream())
        assert _same(h, want), entry
        assert torch.equal(pmax, wmax), entry


@pytest.mark.parametrize("i", [65664, 65536])  # 144 x 384 and 144 x 256 tiles
def test_w4a16_gate_up_epilogue_every_finite_bf16_gate(gpu, i):
    """ff_gemm_w4a16_swiglu_pk against the packed GEMM + ff_swiglu for every
    finite gate pattern (an inf or NaN z would reach the other products of its
    group as 0 x inf)."""
    from fastforward_amd import ops
    from fastforward_amd.linear import Int4
    m, k = 144, 256
    op = Int4(torch.zeros(2 * i, k, dtype=BF16, device=DEV), group=128)
    op.packed.fill_(0x88)
    z = _every_bf16()
    z[torch.isinf(z.float()) | torch.isnan(z.float())] = 0
    sc = torch.zeros(op.scales.shape, dtype=BF16)
    sc[0, :65536, 1] = z
    sc[0, i:, 1] = torch.randn(i, generator=torch.Generator().manual_seed(4)).to(BF16)
    op.scales.copy_(sc)
    op.pack()
    assert op.frag is not None and op.swiglu_fits(m)
    x = torch.zeros(m, k, dtype=BF16, device=DEV)
    x[:, 0] = 1
    gu = op(x)
    normal = (z.float().abs() >= 2.0 ** -126).to(DEV)  # the bf16 MFMA may flush subnormal operands
    assert _same(gu[0, :65536][normal], z.to(DEV)[normal])
    assert _same(op.swiglu(x), ops.swiglu(*gu.chunk(2, -1)))
