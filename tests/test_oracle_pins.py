"""Pins the CPU oracle against checks that do not restate its own formulas:
bit-level numpy rounding, exhaustive e4m3 search, fp64 closed forms and brute
force, and the installed transformers Qwen3-VL modules (third-party code that
the reference calls for embeddings, RMSNorm, rotary and position ids).

The reference ships no golden vectors for this path (its only tests pin request
validation and the response contract, mirrored at the bottom of this file).
"""
import math
import types

import numpy as np
import pytest
import torch

from oracle import ops
from oracle import model as omodel
from tests.numerics import bf16_round_np, e4m3_encode_np, e4m3_decode_np, ulp_bf16

torch.manual_seed(0)


def _gen(seed):
    g = torch.Generator().manual_seed(seed)
    return g


# ------------------------------------------------------------------ rounding

def test_bf16_rounding_matches_bit_rne():
    g = _gen(1)
    x = torch.randn(200000, generator=g) * torch.exp2(torch.randint(-30, 30, (200000,), generator=g).float())
    # exact ties: low 16 bits = 0x8000 with odd and even upper halves
    u = torch.randint(0, 2 ** 31 - 1, (20000,), generator=g, dtype=torch.int64)
    ties = ((u & ~0xFFFF) | 0x8000).to(torch.int32).view(torch.float32)
    ties = ties[torch.isfinite(ties)]
    x = torch.cat([x, ties])
    got = ops.bf16(x).numpy()
    want = bf16_round_np(x.numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_e4m3_cast_exhaustive():
    g = _gen(2)
    vals = e4m3_decode_np(np.arange(0, 0x7F))
    mids = (vals[1:] + vals[:-1]) / 2                     # exact midpoints -> ties
    x = np.concatenate([
        np.random.default_rng(3).uniform(-448, 448, 50000),
        np.random.default_rng(4).standard_normal(50000) * 0.01,
        mids, -mids, vals, -vals, [0.0, -0.0, 448.0, -448.0, 2.0 ** -10, 3 * 2.0 ** -11]])
    x32 = x.astype(np.float32)
    x32 = x32[np.abs(x32) <= 448]
    got = torch.from_numpy(x32).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    want = e4m3_encode_np(x32.astype(np.float64))
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ norms

def _np_rms(x, w, eps):
    x = x.astype(np.float64)
    var = (x.astype(np.float32).astype(np.float64) ** 2).mean(-1, keepdims=True)
    n = bf16_round_np((x / np.sqrt(var + eps)).astype(np.float32)).astype(np.float64)
    return bf16_round_np((n * w.astype(np.float64)).astype(np.float32))


def _close_bf16(got, want, frac=0.002):
    """At most one bf16 ulp apart everywhere, and exact for all but ``frac``."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    diff = np.abs(got - want)
    assert np.all(diff <= ulp_bf16(want) * 1.0001), diff.max()
    assert (diff > 0).mean() <= frac, (diff > 0).mean()


def test_rms_fast_norm_matches_fp64():
    g = _gen(5)
    x = (torch.randn(64, 2048, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    got = ops.fast_norm(x, w, 1e-6).float().numpy()
    want = _np_rms(x.float().numpy(), w.float().numpy(), 1e-6)
    _close_bf16(got, want)


def test_rms_matches_hf_rmsnorm_module():
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRMSNorm
    g = _gen(6)
    m = Qwen3VLTextRMSNorm(1024, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_((1 + 0.2 * torch.randn(1024, generator=g)).to(torch.bfloat16))
    x = (torch.randn(3, 17, 1024, generator=g) * 2).to(torch.bfloat16)
    with torch.no_grad():
        want = m(x)
    got = ops.fast_norm(x, m.weight.detach(), m.variance_epsilon)
    assert torch.equal(got, want)


def test_add_rms_matches_fp64_with_deepstack():
    g = _gen(7)
    t, h = 40, 512
    a = torch.randn(1, t, h, generator=g).to(torch.bfloat16)
    b = torch.randn(1, t, h, generator=g).to(torch.bfloat16)
    deep = torch.randn(10, h, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    res, out = ops.add_rms(a, b, deep, w, 1e-6, start=5, nv=10)
    x = bf16_round_np(a.float().numpy()[0] + b.float().numpy()[0])
    x[5:15] = bf16_round_np(x[5:15] + deep.float().numpy())
    assert np.array_equal(res.float().numpy()[0], x)
    _close_bf16(out.float().numpy()[0], _np_rms(x, w.float().numpy(), 1e-6))
    # rows outside [start, start+nv) see no injection
    res0, _ = ops.add_rms(a, b, None, w, 1e-6)
    assert torch.equal(res0[0, :5], res[0, :5]) and torch.equal(res0[0, 15:], res[0, 15:])
    assert not torch.equal(res0[0, 5:15], res[0, 5:15])


# ------------------------------------------------------------------ rotary

def _hf_cfg(head_dim=128, sections=(24, 20, 20), theta=5e6, hidden=256, heads=4, kv=2, layers=2,
            inter=512, vocab=512):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    cfg = Qwen3VLTextConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                            num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv,
                            head_dim=head_dim, rms_norm_eps=1e-6,
                            rope_parameters=dict(rope_type='default', rope_theta=theta,
                                                 mrope_section=list(sections), mrope_interleaved=True))
    cfg._attn_implementation = 'eager'
    return cfg


def _hf_positions(s0, gh, gw, total):
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLModel
    fake = types.SimpleNamespace(config=types.SimpleNamespace(
        vision_config=types.SimpleNamespace(spatial_merge_size=2)))
    fake.get_vision_position_ids = lambda *a, **k: Qwen3VLModel.get_vision_position_ids(fake, *a, **k)
    ids = torch.zeros(1, total, dtype=torch.long)
    tt = torch.zeros(1, total, dtype=torch.int)
    tt[0, s0:s0 + gh * gw] = 1
    p, _ = Qwen3VLModel.get_rope_index(fake, ids, tt, image_grid_thw=torch.tensor([[1, 2 * gh, 2 * gw]]))
    return p[:, 0]


@pytest.mark.parametrize("s0,gh,gw,total", [(4, 16, 16, 320), (4, 16, 32, 576), (4, 30, 32, 1024),
                                            (3, 5, 7, 50), (0, 4, 2, 8)])
def test_mrope_positions_match_hf(s0, gh, gw, total):
    got = ops.mrope_positions(s0, gh, gw, total)
    want = _hf_positions(s0, gh, gw, total)
    assert torch.equal(got, want)


def test_mrope_positions_brute_force():
    s0, gh, gw, total = 2, 3, 5, 24
    pos = ops.mrope_positions(s0, gh, gw, total)
    t = 0
    for i in range(s0):
        assert pos[:, t].tolist() == [i, i, i]; t += 1
    for r in range(gh):
        for c in range(gw):
            assert pos[:, t].tolist() == [s0, s0 + r, s0 + c]; t += 1
    nxt = s0 + max(gh, gw)
    while t < total:
        assert pos[:, t].tolist() == [nxt] * 3; t += 1; nxt += 1


@pytest.mark.parametrize("head_dim,sections", [(128, (24, 20, 20)), (64, (12, 10, 10))])
def test_mrope_cos_sin_match_hf(head_dim, sections):
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRotaryEmbedding
    rot = Qwen3VLTextRotaryEmbedding(_hf_cfg(head_dim=head_dim, sections=sections))
    pos = ops.mrope_positions(4, 16, 32, 576)
    x = torch.zeros(1, 576, 8, dtype=torch.bfloat16)
    cos_w, sin_w = rot(x, pos[:, None, :])
    cos, sin = ops.mrope_cos_sin(pos, 5e6, head_dim, sections)
    assert torch.equal(cos, cos_w) and torch.equal(sin, sin_w)


def test_mrope_section_assignment_closed_form():
    # frequency slot i must use H iff i%3==1 and i<60, W iff i%3==2 and i<60, else T
    pos = torch.tensor([[1], [1000], [1000000]], dtype=torch.int64).expand(3, 1).clone()
    inv = ops.mrope_inv_freq(5e6, 128)
    cos, _ = ops.mrope_cos_sin(pos, 5e6, 128)
    for i in range(64):
        src = 1 if (i % 3 == 1 and i < 60) else 2 if (i % 3 == 2 and i < 60) else 0
        ang = float(pos[src, 0]) * float(inv[i])
        want = math.cos(np.float32(ang))
        assert abs(float(cos[0, 0, i]) - want) <= 2 ** -8, i
        assert torch.equal(cos[0, 0, i], cos[0, 0, i + 64])


def test_qk_pair_matches_hf_norm_and_rotary():
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLTextRMSNorm, apply_rotary_pos_emb)
    g = _gen(8)
    t, hq, hk, d = 48, 4, 2, 128
    packed = torch.randn(1, t, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16) * 2
    q = packed[..., : hq * d].view(1, t, hq, d)          # strided views as in the reference
    k = packed[..., hq * d:(hq + hk) * d].view(1, t, hk, d)
    qn = Qwen3VLTextRMSNorm(d).to(torch.bfloat16)
    kn = Qwen3VLTextRMSNorm(d).to(torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_((1 + 0.3 * torch.randn(d, generator=g)).to(torch.bfloat16))
        kn.weight.copy_((1 + 0.3 * torch.randn(d, generator=g)).to(torch.bfloat16))
    pos = ops.mrope_positions(2, 4, 6, t)
    cos, sin = ops.mrope_cos_sin(pos, 5e6, d)
    yq, yk = ops.qk_pair(q, k, qn.weight.detach(), kn.weight.detach(), 1e-6, 1e-6, cos, sin)
    with torch.no_grad():
        wq, wk = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    assert torch.equal(yq, wq) and torch.equal(yk, wk)
    # rotate-half is an isometry on each (i, i+D/2) pair: norms agree up to bf16 rounding
    xn = qn(q).transpose(1, 2).float()
    assert torch.allclose(yq.float().norm(dim=-1), xn.norm(dim=-1), rtol=2e-2)


# ------------------------------------------------------------------ MLP / readout

def test_swiglu_matches_fp64():
    g = _gen(9)
    gate = (torch.randn(64, 300, generator=g) * 4).to(torch.bfloat16)
    up = torch.randn(64, 300, generator=g).to(torch.bfloat16)
    got = ops.swiglu(gate, up).float().numpy()
    gf = gate.double().numpy()
    act = bf16_round_np((gf / (1 + np.exp(-gf))).astype(np.float32)).astype(np.float64)
    want = bf16_round_np((act * up.double().numpy()).astype(np.float32))
    _close_bf16(got, want, frac=0.01)


def test_lm_readout_matches_fp64():
    g = _gen(10)
    h = 2048
    x = (torch.randn(h, generator=g) * 5).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    head = (torch.randn(8, h, generator=g) * 0.02).to(torch.bfloat16)
    got = ops.lm_readout(x, w, 1e-6, head)
    assert got.shape == (1, 8) and got.dtype == torch.float32
    xn = _np_rms(x.float().numpy()[None], w.float().numpy(), 1e-6)[0].astype(np.float64)
    want = bf16_round_np((head.double().numpy() @ xn).astype(np.float32))
    _close_bf16(got.numpy()[0], want, frac=0.25)
    # stored values are bf16-representable
    assert torch.equal(got, got.to(torch.bfloat16).float())


# ------------------------------------------------------------------ attention

def _attention_loops(q, k, v, scale, positions):
    """Brute-force fp64 softmax attention, one (head, query) at a time."""
    _, hq, s, d = q.shape
    hk, t = k.shape[1], k.shape[2]
    out = np.zeros((s, hq, d))
    qn, kn, vn = q.double().numpy()[0], k.double().numpy()[0], v.double().numpy()[0]
    for hh in range(hq):
        kv = hh // (hq // hk)
        for i in range(s):
            p = positions[i]
            sc = np.array([qn[hh, i] @ kn[kv, n] * scale for n in range(p + 1)])
            e = np.exp(sc - sc.max())
            out[i, hh] = (e[:, None] * vn[kv, : p + 1]).sum(0) / e.sum()
    return out


def test_attention_matches_bruteforce_gqa_causal():
    g = _gen(11)
    hq, hk, t, d = 4, 2, 150, 32
    q = torch.randn(1, hq, t, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, hk, t, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, hk, t, d, generator=g).to(torch.bfloat16)
    # make the two kv heads very different so a wrong GQA mapping fails
    v[:, 1] += 3
    got = ops.attention_direct(q, k, v, d ** -0.5).float().numpy()[0]
    want = _attention_loops(q, k, v, d ** -0.5, list(range(t)))
    assert np.abs(got - want).max() < 3e-2
    assert np.abs(got - want).mean() < 3e-3
    exact = ops.attention_exact(q, k, v, d ** -0.5).numpy()[0]
    assert np.abs(exact - want).max() < 1e-9


def test_attention_selected_rows_equal_full_rows():
    g = _gen(12)
    hq, hk, t, d = 8, 2, 130, 64
    q = torch.randn(1, hq, t, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, hk, t, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, hk, t, d, generator=g).to(torch.bfloat16)
    full = ops.attention_direct(q, k, v, d ** -0.5)
    pick = torch.tensor([0, 63, 64, 129])
    sel = ops.attention_direct(q.index_select(2, pick), k, v, d ** -0.5, positions=pick)
    assert torch.equal(sel[0], full[0, pick])


# ------------------------------------------------------------------ FP8

def test_fp8_dynamic_rows_match_numpy():
    g = _gen(13)
    x = torch.randn(33, 512, generator=g)
    x[torch.rand(33, 512, generator=g) < 0.001] *= 20
    x[5] = 0                                                 # zero row -> scale clamp 1e-12
    x = x.to(torch.bfloat16)
    q, s = ops.quant_rows_dynamic(x)
    xf = x.float().numpy()
    amax = np.maximum(np.abs(xf).max(-1), np.float32(1e-12)).astype(np.float32)
    scale = (amax / np.float32(448)).astype(np.float32)
    assert np.array_equal(s.numpy(), scale)
    qq = np.clip((xf / scale[:, None]).astype(np.float32), -448, 448)
    assert np.array_equal(q.view(torch.uint8).numpy(), e4m3_encode_np(qq.astype(np.float64)))
    assert float(s[5]) == np.float32(np.float32(1e-12) / np.float32(448))


def test_fp8_static_matches_numpy():
    g = _gen(14)
    x = (torch.randn(20, 256, generator=g) * 30).to(torch.bfloat16)
    inv = 448 / 37.5
    q = ops.quant_static(x, inv)
    qq = np.clip(x.float().numpy() * np.float32(inv), -448, 448)
    assert np.array_equal(q.view(torch.uint8).numpy(), e4m3_encode_np(qq.astype(np.float64)))


def test_fp8_weight_quant_matches_numpy():
    g = _gen(15)
    w = (torch.randn(48, 256, generator=g) * 0.02).to(torch.bfloat16)
    q, s = ops.fp8_weight_quant(w, per_channel=True)
    wf = w.float().numpy()
    sc = (np.maximum(np.abs(wf).max(1), np.float32(1e-12)) / np.float32(448)).astype(np.float32)
    assert np.array_equal(s.numpy(), sc)
    qq = np.clip((wf / sc[:, None]).astype(np.float32), -448, 448)
    assert np.array_equal(q.view(torch.uint8).numpy(), e4m3_encode_np(qq.astype(np.float64)))
    q1, s1 = ops.fp8_weight_quant(w, per_channel=False)
    sc1 = np.float32(np.abs(wf).max()) / np.float32(448)
    assert s1.shape == (1,) and float(s1) == sc1
    qq1 = np.clip((wf / sc1).astype(np.float32), -448, 448)
    assert np.array_equal(q1.view(torch.uint8).numpy(), e4m3_encode_np(qq1.astype(np.float64)))


def test_fp8_linear_matches_fp64():
    g = _gen(16)
    m, k, n = 40, 256, 96
    x = torch.randn(m, k, generator=g)
    x[torch.rand(m, k, generator=g) < 0.001] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    qw, sw = ops.fp8_weight_quant(w)
    y = ops.fp8_linear_dynamic(x, qw, sw).float().numpy()
    qa, sa = ops.quant_rows_dynamic(x)
    a = e4m3_decode_np(qa.view(torch.uint8).numpy())
    b = e4m3_decode_np(qw.view(torch.uint8).numpy())
    acc = a @ b.T
    want = bf16_round_np((acc * sa.double().numpy()[:, None] * sw.double().numpy()[None, :]).astype(np.float32))
    _close_bf16(y, want, frac=0.01)
    # and the quantized product tracks the unquantized one
    ref = x.double().numpy() @ w.double().numpy().T
    assert np.abs(y - ref).max() < 0.05 * np.abs(ref).max()


def _rne_sig(v, bits):
    """v (a Python float) rounded to ``bits`` significant bits, nearest even, by
    math.frexp and Python's round (ties to even on an exact double)."""
    if v == 0.0:
        return v
    m, e = math.frexp(v)
    return math.ldexp(round(m * 2.0 ** bits), e - bits)


@pytest.mark.parametrize("bits", [8, 13, 14, 24])
def test_round_sig_matches_frexp_rounding(bits):
    g = _gen(40)
    x = torch.randn(2000, generator=g, dtype=torch.float64) * torch.exp2(torch.randint(-60, 60, (2000,),
                                                                                    generator=g).double())
    # exact ties (half an ulp of the kept width, both parities) and carries into the next binade
    base = torch.tensor([1.0, 1.5, -1.25, 3.0, -0.75], dtype=torch.float64)
    ulp = torch.exp2(torch.floor(torch.log2(base.abs())) - (bits - 1))
    ties = torch.cat([base + ulp / 2, base + 3 * ulp / 2, -(base.abs() + ulp / 2),
                      torch.tensor([2.0 - 2.0 ** -(bits + 1), -(2.0 - 2.0 ** -(bits + 1)), 0.0])])
    for v in (x, ties):
        got = ops.round_sig_(v.clone(), bits).tolist()
        want = [_rne_sig(a, bits) for a in v.tolist()]
        assert got == want


def test_fp8_gemm_exact_and_blocks_brute_force():
    """The exact-accumulation GEMM and the reduced-precision block model against
    pure-Python sums of the decoded codes (Fractions): the exact block sums,
    their rounding to the kept bits, fp32 accumulation in k order (numpy
    float32), then the scaling and bf16 rounding."""
    from fractions import Fraction
    g = _gen(41)
    m, k, n, block = 3, 128, 5, 32
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    qa, sa = ops.quant_rows_dynamic(x)
    qw, sw = ops.fp8_weight_quant(w)
    a = e4m3_decode_np(qa.view(torch.uint8).numpy())
    b = e4m3_decode_np(qw.view(torch.uint8).numpy())
    exact = ops.fp8_gemm_exact(qa, sa, qw, sw).float().numpy()
    for bits in (10, 14):
        blocks = ops.fp8_gemm_blocks(qa, sa, qw, sw, bits=bits, block=block, chunk=2).float().numpy()
        for i in range(m):
            for j in range(n):
                prods = [Fraction(float(a[i, t])) * Fraction(float(b[j, t])) for t in range(k)]
                tot = float(sum(prods, Fraction(0)))                   # exact in fp64
                want_exact = bf16_round_np(np.float32(tot * float(sa[i]) * float(sw[j])))
                assert exact[i, j] == want_exact
                acc = np.float32(0.0)
                for c in range(k // block):
                    part = float(sum(prods[c * block:(c + 1) * block], Fraction(0)))
                    acc = np.float32(acc + np.float32(_rne_sig(part, bits)))
                want = bf16_round_np(np.float32(np.float32(acc * np.float32(sa[i])) * np.float32(sw[j])))
                assert blocks[i, j] == want, (bits, i, j)


# ------------------------------------------------------------------ int4

def test_int4_asym_pack_and_scale_indexing_by_loops():
    g = _gen(17)
    n, k, grp = 4, 64, 32
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    q, packed, scales = ops.int4_quantize_asym(w, grp)
    wf = w.float().numpy()
    assert packed.shape == (n, k // 2) and scales.shape == (k // grp, n, 2)
    for r in range(n):
        for gi in range(k // grp):
            blk = wf[r, gi * grp:(gi + 1) * grp]
            lo, hi = np.float32(blk.min()), np.float32(blk.max())
            s = max(np.float32((hi - lo) / np.float32(15)), np.float32(1e-6))
            z = np.float32(lo + np.float32(s * np.float32(8)))
            assert float(scales[gi, r, 0]) == float(torch.tensor(s).to(torch.bfloat16))
            assert float(scales[gi, r, 1]) == float(torch.tensor(z).to(torch.bfloat16))
            for j in range(grp):
                code = int(np.clip(np.round(np.float32((blk[j] - lo) / s)), 0, 15))
                assert int(q[r, gi * grp + j]) == code
        for c in range(k // 2):
            assert int(packed[r, c]) == (int(q[r, 2 * c]) << 4) | int(q[r, 2 * c + 1])
    assert torch.equal(ops.int4_unpack(packed), q)


def test_int4_sym_codes_and_dequant():
    g = _gen(18)
    n, k, grp = 6, 256, 128
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    q, packed, scales = ops.int4_quantize_sym(w, grp)
    assert torch.all(scales[..., 1] == 0)
    wf = w.float().numpy()
    for r in range(n):
        for gi in range(k // grp):
            blk = wf[r, gi * grp:(gi + 1) * grp]
            s = float(torch.tensor(max(np.abs(blk).max(), 1e-6) / np.float32(7), dtype=torch.float32).to(torch.bfloat16))
            assert float(scales[gi, r, 0]) == s
            codes = np.clip(np.round(blk / np.float32(s)) + 8, 0, 15)
            assert np.array_equal(q[r, gi * grp:(gi + 1) * grp].numpy(), codes.astype(np.uint8))
    dq = ops.int4_dequant(packed, scales, grp).numpy()
    s_full = np.repeat(scales[..., 0].float().numpy().T, grp, axis=1)
    assert np.array_equal(dq, ((q.numpy().astype(np.float32) - 8) * s_full).astype(np.float32))
    assert np.abs(dq - wf).max() <= s_full.max() / 2 + 1e-9


def test_w4a16_linear_matches_fp64():
    g = _gen(19)
    m, k, n = 24, 256, 40
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    for quant, grp in ((ops.int4_quantize_asym, 32), (ops.int4_quantize_sym, 128)):
        q, packed, scales = quant(w, grp)
        y = ops.w4a16_linear(x, packed, scales, grp).float().numpy()
        s = scales.double().numpy()                       # [K/g, N, 2]
        wd = np.zeros((n, k))
        for r in range(n):
            for c in range(k):
                wd[r, c] = (int(q[r, c]) - 8) * s[c // grp, r, 0] + s[c // grp, r, 1]
        want = x.double().numpy() @ wd.T
        _close_bf16(y, bf16_round_np(want.astype(np.float32)), frac=0.05)
        # the reference's own operator bar: relative RMS <= 1% against the fp32 dequant
        ref = x.double().numpy() @ w.double().numpy().T
        assert np.sqrt(((y - ref) ** 2).mean()) / np.sqrt((ref ** 2).mean()) < 0.2
        # the bf16-operand form: each dequantized weight rounded once to bf16 (numpy bit RNE)
        yb = ops.w4a16_linear(x, packed, scales, grp, weight_bf16=True).float().numpy()
        wb = bf16_round_np(wd.astype(np.float32)).astype(np.float64)
        _close_bf16(yb, bf16_round_np((x.double().numpy() @ wb.T).astype(np.float32)), frac=0.05)
        assert not np.array_equal(wb, wd), "the test weights must have dequantized values that bf16 rounds"


def test_w4a16_linear_matches_torch_int4pack_cpu():
    """The fp32-dequant form equals torch's own CPU int4 GEMM
    (aten._weight_int4pack_mm_for_cpu, the CPU sibling of the reference's
    _weight_int4pack_mm, _family/night_runtime.py:33) given the same nibble codes
    and [K/g, N, 2] (scale, zero) table, bit for bit on the symmetric group-128
    form and for >= 99% of outputs on the asymmetric group-32 form (the library
    folds the zero point in a different order)."""
    g = _gen(20)
    m, k, n = 8, 1024, 256
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g) * 0.02
    for quant, grp, need in ((ops.int4_quantize_sym, 128, 1.0), (ops.int4_quantize_asym, 32, 0.99)):
        q, packed, scales = quant(w, grp)
        wp = torch.ops.aten._convert_weight_to_int4pack_for_cpu(q.to(torch.int32), 1)
        lib = torch.ops.aten._weight_int4pack_mm_for_cpu(x, wp, grp, scales)
        ours = ops.w4a16_linear(x, packed, scales, grp)
        assert float((lib == ours).float().mean()) >= need, (grp, float((lib == ours).float().mean()))


# ------------------------------------------------------------------ composition vs HF

def _oracle_weights_from_hf(hf, head_rows):
    layers = []
    for L in hf.layers:
        a, m = L.self_attn, L.mlp
        layers.append(omodel.Layer(
            input_norm=L.input_layernorm.weight.detach(), post_norm=L.post_attention_layernorm.weight.detach(),
            q_norm=a.q_norm.weight.detach(), k_norm=a.k_norm.weight.detach(),
            qkv=dict(kind='bf16', w=torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).detach()),
            o=dict(kind='bf16', w=a.o_proj.weight.detach()),
            gateup=dict(kind='bf16', w=torch.cat([m.gate_proj.weight, m.up_proj.weight]).detach()),
            down=dict(kind='bf16', w=m.down_proj.weight.detach())))
    return omodel.Weights(embed=hf.embed_tokens.weight.detach(), layers=layers,
                          norm=hf.norm.weight.detach(), head=head_rows)


@pytest.mark.parametrize("use_deep", [False, True])
def test_model_matches_hf_text_model(use_deep):
    """Layer wiring (residuals, norms, q/k-norm, GQA, M-RoPE, DeepStack, pick-only
    tail, readout) against transformers' Qwen3VLTextModel with the same weights."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel
    torch.manual_seed(20)
    cfg = _hf_cfg(head_dim=64, sections=(12, 10, 10), hidden=256, heads=4, kv=2, layers=3, inter=512, vocab=512)
    hf = Qwen3VLTextModel(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():
        for p in hf.parameters():
            if p.ndim == 1:
                p.copy_(1 + 0.1 * torch.randn_like(p.float()))
            else:
                p.copy_(torch.randn_like(p.float()) * 0.05)
    g = _gen(21)
    t, s0, gh, gw = 70, 3, 4, 6
    nv = gh * gw
    ids = torch.randint(0, 512, (t,), generator=g)
    pos = ops.mrope_positions(s0, gh, gw, t)
    head = (torch.randn(4, 256, generator=g) * 0.05).to(torch.bfloat16)
    visual = (torch.randn(nv, 256, generator=g)).to(torch.bfloat16)
    deep = [(torch.randn(nv, 256, generator=g) * 0.5).to(torch.bfloat16) for _ in range(2)] if use_deep else None
    pick = t - 5
    shape = omodel.Shape(layers=3, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=512,
                         sections=(12, 10, 10))
    w = _oracle_weights_from_hf(hf, head)
    trace = []
    z = omodel.step(shape, w, ids, pos, pick, visual=visual, image_start=s0, deep=deep, trace=trace)
    emb = hf.embed_tokens(ids)[None].detach().clone()
    emb[0, s0:s0 + nv] = visual
    mask = torch.zeros(1, t, dtype=torch.bool)
    mask[0, s0:s0 + nv] = True
    # HF in fp32 is the unrounded composition; the oracle differs from it only by
    # its bf16 / rounding points (about 1% relative per layer).
    hf32 = Qwen3VLTextModel(cfg).eval()
    hf32.load_state_dict({k: v.float() for k, v in hf.state_dict().items()})
    with torch.no_grad():
        out = hf32(inputs_embeds=emb.float(), position_ids=pos[:, None, :],
                   visual_pos_masks=mask if use_deep else None,
                   deepstack_visual_embeds=[d.float() for d in deep] if use_deep else None,
                   output_hidden_states=True)
    for j, h in enumerate(trace):
        a, b = h[0].float(), out.hidden_states[j + 1][0].clone()
        if use_deep and j < len(deep):        # HF records the layer output before its DeepStack add
            b[s0:s0 + nv] += deep[j].float()
        assert float((a - b).norm() / b.norm()) < 0.02, j
    want = out.last_hidden_state[0, pick] @ head.float().T
    assert torch.allclose(z, want, rtol=0, atol=0.02 * float(want.abs().max())), (z, want)
    assert ops.choose(z.tolist()) == ops.choose(want.tolist())


# ------------------------------------------------------------------ choice contract

def test_choice_ties_lowest_index_and_probabilities():
    """Mirrors the reference's tests/test_contract.py:13-17 for the oracle."""
    r = ops.response([1., 1.], ["a", "b"], "x")
    assert r["answer"]["letter"] == "A"
    assert abs(sum(r["probabilities"]) - 1) < 1e-12
    with pytest.raises(RuntimeError):
        ops.response([float("nan"), 0.], ["a", "b"], "x")
    assert ops.choose([0.5, 2.0, 2.0, 1.0]) == 1
