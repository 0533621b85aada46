"""Test helpers: hand the product's quantized device weights to the CPU oracle,
and compare bf16 tensors in units in the last place."""
import numpy as np
import torch

from oracle import model as omodel


def bf16_ulps(a, b):
    """Elementwise distance in bf16 ulps between two bf16 tensors (same device)."""
    ia = a.to(torch.bfloat16).view(torch.int16).to(torch.int32).cpu()
    ib = b.to(torch.bfloat16).view(torch.int16).to(torch.int32).cpu()
    # map sign-magnitude to a monotonic integer line
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return (ia - ib).abs()


def assert_bf16_close(got, want, max_ulps=1, max_frac=1e-3, what=""):
    """At most ``max_ulps`` bf16 ulps apart everywhere and exact for all but ``max_frac``."""
    d = bf16_ulps(got, want)
    frac = float((d > 0).float().mean())
    assert int(d.max()) <= max_ulps, f"{what}: max ulp distance {int(d.max())} > {max_ulps}"
    assert frac <= max_frac, f"{what}: {frac:.2e} of elements differ (> {max_frac})"


def linear_to_oracle(op, int4_bf16=False):
    from fastforward_amd.linear import FP8Linear, Int4, StaticFP8Linear
    if isinstance(op, FP8Linear):
        return dict(kind="fp8_dynamic", q=op.weight.cpu(), scale=op.scale.reshape(-1).cpu())
    if isinstance(op, StaticFP8Linear):
        return dict(kind="fp8_static", q=op.weight.cpu(), scale=op.weight_scale.cpu(),
                    inverse_scale=op.inverse_scale, input_scale=op.input_scale.cpu())
    if isinstance(op, Int4):
        return dict(kind="w4a16", packed=op.packed.cpu(), scales=op.scales.cpu(), group=op.group,
                    weight_bf16=int4_bf16)
    raise TypeError(type(op))


def to_oracle(cfg, w, layers=None, only=None, int4_bf16=False):
    """(oracle Shape, oracle Weights) holding CPU copies of the product's weights.
    ``only``: indices of the layers whose linears are copied (the others keep
    their norms and None linears), for shapes too large to copy whole.
    ``int4_bf16``: W4A16 linears use the oracle's bf16-operand form (each
    dequantized weight rounded to bf16, as a bf16 matrix unit consumes it)."""
    shape = omodel.Shape(layers=cfg.layers, hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads,
                         head_dim=cfg.head_dim, inter=cfg.inter, vocab=cfg.vocab, eps=cfg.eps,
                         theta=cfg.theta, sections=tuple(cfg.sections))
    out = []
    for j, lw in enumerate(w.layers[: layers or len(w.layers)]):
        lin = only is None or j in only
        out.append(omodel.Layer(
            input_norm=lw.input_norm.weight.cpu(), post_norm=lw.post_norm.weight.cpu(),
            q_norm=lw.q_norm.weight.cpu(), k_norm=lw.k_norm.weight.cpu(),
            qkv=linear_to_oracle(lw.qkv, int4_bf16) if lin else None,
            o=linear_to_oracle(lw.o, int4_bf16) if lin else None,
            gateup=linear_to_oracle(lw.gateup, int4_bf16) if lin else None,
            down=linear_to_oracle(lw.down, int4_bf16) if lin else None))
    return shape, omodel.Weights(embed=w.embed.cpu(), layers=out, norm=w.norm.weight.cpu(), head=w.head.cpu())


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))
