"""CPU restatement of the whole LM prefill + choice-score step (test infrastructure).

Follows ``Runtime.prefix`` / ``attention`` / ``mlp`` (scaled_qwen_runtime.py:143-176)
and the pick-only tail of the fp8/precise execution modes
(_family/night_runtime.py:92-105). Weights are passed in explicitly so the same
quantized tensors can be handed to the product on the GPU.

Not the product: only tests/, smoke() and bench.py's cpu_baseline use it.
"""
from dataclasses import dataclass, field

import torch

from . import ops
from .ops import BF16, F32


@dataclass
class Shape:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    eps: float = 1e-6
    theta: float = 5e6
    sections: tuple = (24, 20, 20)

    @property
    def scaling(self):
        return self.head_dim ** -0.5


@dataclass
class Layer:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    qkv: dict        # linear spec, see ``linear``
    o: dict
    gateup: dict
    down: dict


@dataclass
class Weights:
    embed: torch.Tensor               # (vocab, H) bf16
    layers: list
    norm: torch.Tensor                # final RMSNorm weight (H,)
    head: torch.Tensor                # option rows of lm_head (n_opt, H) bf16
    extra: dict = field(default_factory=dict)


def linear(x, spec):
    """``Linear.apply(x, op)`` (scaled_qwen_runtime.py:35-39) for the linear-op kinds:

    fp8_dynamic: {q (N,K) e4m3, scale (N,)}           -> ops.fp8_linear_dynamic
    fp8_static:  {q, scale (1,), inverse_scale, input_scale} -> ops.fp8_linear_static
    w4a16:       {packed (N,K/2) u8, scales [K/g,N,2], group, weight_bf16 (optional)}
                                                       -> ops.w4a16_linear
    bf16:        {w (N,K) bf16}                        -> bf16(x @ w^T) in fp32
    """
    kind = spec['kind']
    if kind == 'fp8_dynamic':
        return ops.fp8_linear_dynamic(x, spec['q'], spec['scale'])
    if kind == 'fp8_static':
        return ops.fp8_linear_static(x, spec['q'], spec['scale'], spec['inverse_scale'], spec['input_scale'])
    if kind == 'w4a16':
        return ops.w4a16_linear(x, spec['packed'], spec['scales'], spec['group'], spec.get('weight_bf16', False))
    if kind == 'bf16':
        flat = x.reshape(-1, x.shape[-1]).to(F32)
        return (flat @ spec['w'].to(F32).T).to(BF16).reshape(*x.shape[:-1], spec['w'].shape[0])
    raise ValueError(kind)


def attention_block(shape, layer, x, cos, sin):
    """``Runtime.attention`` (scaled_qwen_runtime.py:165-172)."""
    hq, hk, d = shape.heads, shape.kv_heads, shape.head_dim
    z = linear(x, layer.qkv)
    q, k, v = z.split([hq * d, hk * d, hk * d], -1)
    q, k = ops.qk_pair(q.reshape(1, -1, hq, d), k.reshape(1, -1, hk, d), layer.q_norm, layer.k_norm,
                       shape.eps, shape.eps, cos, sin)
    v = v.reshape(1, -1, hk, d).transpose(1, 2)
    out = ops.attention_direct(q, k, v, shape.scaling)
    return linear(out.reshape(*x.shape[:-1], -1), layer.o)


def mlp(layer, x):
    """``Runtime.mlp`` (scaled_qwen_runtime.py:174-176)."""
    g, u = linear(x, layer.gateup).chunk(2, -1)
    return linear(ops.swiglu(g, u), layer.down)


def tail(shape, layer, weights, h, cos, sin, pick):
    """Pick-only final layer + readout (_family/night_runtime.py:92-105)."""
    hq, hk, d = shape.heads, shape.kv_heads, shape.head_dim
    x = ops.fast_norm(h, layer.input_norm, shape.eps)
    z = linear(x, layer.qkv)
    q, k, v = z.split([hq * d, hk * d, hk * d], -1)
    q, k = ops.qk_pair(q.reshape(1, -1, hq, d), k.reshape(1, -1, hk, d), layer.q_norm, layer.k_norm,
                       shape.eps, shape.eps, cos, sin)
    v = v.reshape(1, -1, hk, d).transpose(1, 2)
    pick_t = torch.tensor([pick])
    query = q.index_select(2, pick_t)
    out = ops.attention_direct(query, k, v, shape.scaling, positions=pick_t)
    value = linear(out.reshape(1, 1, -1), layer.o)
    residual, post = ops.add_rms(h.index_select(1, pick_t), value, None, layer.post_norm, shape.eps)
    chosen = (residual[0].to(F32) + mlp(layer, post[0]).to(F32)).to(BF16)
    return ops.lm_readout(chosen, weights.norm, shape.eps, weights.head)[0].float()


def step(shape, weights, ids, pos, pick, visual=None, image_start=0, deep=None, n_choices=None,
         trace=None):
    """``Runtime.prefix`` (scaled_qwen_runtime.py:143-163) with the fp8/precise tail.

    ids (T,) int64, pos (3,T) int64, pick int. ``visual`` (nv,H) replaces the image
    rows of the embedding (``index_copy``, :145); ``deep`` is the list of DeepStack
    features injected by the carry ``add_rms`` of layers 0..len(deep)-1 (:161-162).
    Returns the choice logits (n_choices,) fp32. ``trace`` (a list) receives the
    residual stream after every full layer when given.
    """
    h = weights.embed[ids][None].clone()
    nv = 0
    if visual is not None:
        nv = visual.shape[0]
        h[0, image_start:image_start + nv] = visual.to(BF16)
    cos, sin = ops.mrope_cos_sin(pos, shape.theta, shape.head_dim, shape.sections)
    deep = deep or []
    if deep and visual is None:
        nv = deep[0].shape[0]
    layers = weights.layers
    normalized = ops.fast_norm(h, layers[0].input_norm, shape.eps)
    for j in range(shape.layers - 1):
        layer = layers[j]
        attn = attention_block(shape, layer, normalized, cos, sin)
        residual, post = ops.add_rms(h, attn, None, layer.post_norm, shape.eps)
        value = mlp(layer, post)
        injection = deep[j] if j < len(deep) else None
        h, normalized = ops.add_rms(residual, value, injection, layers[j + 1].input_norm, shape.eps,
                                    image_start, nv)
        if trace is not None:
            trace.append(h)
    z = tail(shape, layers[-1], weights, h, cos, sin, pick)
    return z if n_choices is None else z[:n_choices]
