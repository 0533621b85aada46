"""CPU restatement of the reference's vision tower (test infrastructure).

The reference runs the Qwen3-VL vision tower as bf16 torch modules inside
``NativeNormVision.core`` (scaled_qwen_runtime.py:42-55, paths relative to the
reference's ``src/fastforward_accel/``): patch embedding + interpolated
position embedding, then per block h += proj(sdpa(rope(qkv(LN1(h))))) and
h += fc2(gelu_tanh(fc1(LN2(h)))), DeepStack mergers after the listed blocks
and the final patch merger. The modules are transformers' Qwen3-VL vision
classes (modeling_qwen3_vl.py:77-137,196-306,606-744 in the installed
transformers). Here every module is restated in fp32 (fp64 for the matrix
products and the attention) and rounded to bf16 where the module returns a
bf16 tensor.

Not the product: only tests/, smoke() and bench.py's cpu_baseline use it.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from .ops import BF16, F32, bf16


@dataclass(frozen=True)
class VisionShape:
    depth: int
    hidden: int
    heads: int
    inter: int
    out_hidden: int
    deepstack: tuple
    pos_side: int = 48        # the learned position grid is pos_side x pos_side
    patch: int = 16
    merge: int = 2
    temporal: int = 2
    eps: float = 1e-6
    theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden // self.heads


@dataclass
class VisionBlock:
    norm1_w: torch.Tensor
    norm1_b: torch.Tensor
    qkv_w: torch.Tensor       # (3 hidden, hidden)
    qkv_b: torch.Tensor
    proj_w: torch.Tensor
    proj_b: torch.Tensor
    norm2_w: torch.Tensor
    norm2_b: torch.Tensor
    fc1_w: torch.Tensor       # (inter, hidden)
    fc1_b: torch.Tensor
    fc2_w: torch.Tensor       # (hidden, inter)
    fc2_b: torch.Tensor


@dataclass
class Merger:
    norm_w: torch.Tensor      # (hidden,) or (4 hidden,) with the post-shuffle norm
    norm_b: torch.Tensor
    fc1_w: torch.Tensor       # (4 hidden, 4 hidden)
    fc1_b: torch.Tensor
    fc2_w: torch.Tensor       # (out_hidden, 4 hidden)
    fc2_b: torch.Tensor
    postshuffle: bool


@dataclass
class VisionWeights:
    patch_w: torch.Tensor     # (hidden, 1536): the Conv3d kernel flattened (c, t, y, x)
    patch_b: torch.Tensor
    pos_embed: torch.Tensor   # (pos_side^2, hidden)
    blocks: list
    merger: Merger
    deep: list = field(default_factory=list)


# ---------------------------------------------------------------- pixels

def pack_pixels(rgb):
    """``pack_rectangle`` (_family/depth_runtime.py:18-25; square form pack_rgb,
    _legacy/sub10_runtime.py:22-29): rgb (H, W, 3) uint8 -> (H/16 * W/16, 1536)
    bf16 patches, 2 x 2 merge blocks row-major, the 4 patches of a block
    row-major, element (c, frame, y, x) with both frames the same image,
    value (u8 - 127.5) / 127.5 in fp32."""
    rgb = np.asarray(rgb)
    h, w, _ = rgb.shape
    x = (torch.from_numpy(rgb.astype(np.float32)) - 127.5) / 127.5          # (H, W, 3)
    x = x.reshape(h // 32, 2, 16, w // 32, 2, 16, 3)                         # gy my y0 gx mx x0 c
    x = x.permute(0, 3, 1, 4, 6, 2, 5)                                       # gy gx my mx c y0 x0
    x = x.unsqueeze(5).expand(-1, -1, -1, -1, -1, 2, -1, -1)                 # frame axis
    return x.reshape(-1, 1536).to(BF16)


# ---------------------------------------------------------------- geometry

def rot_pos_freqs(shape, gh, gw):
    """Per-patch rotary angles (n, head_dim/2) fp32 of the vision rotary
    (Qwen3VLVisionModel.rot_pos_emb): patch (row, col) in merge-block order
    gets [row * inv_freq, col * inv_freq], inv_freq = theta^(-2i/(head_dim/2))."""
    dim = shape.head_dim // 2
    inv = 1.0 / (shape.theta ** (torch.arange(0, dim, 2, dtype=F32) / dim))
    m = shape.merge
    rows = torch.arange(gh).reshape(gh // m, m, 1, 1).expand(gh // m, m, gw // m, m)
    cols = torch.arange(gw).reshape(1, 1, gw // m, m).expand(gh // m, m, gw // m, m)
    rows = rows.permute(0, 2, 1, 3).reshape(-1)
    cols = cols.permute(0, 2, 1, 3).reshape(-1)
    return torch.cat([rows[:, None].to(F32) * inv, cols[:, None].to(F32) * inv], dim=1)


def rope_cos_sin(shape, gh, gw):
    """cos, sin (n, head_dim) fp32: emb = cat(freqs, freqs) (modeling_qwen3_vl.py:704-707)."""
    f = rot_pos_freqs(shape, gh, gw)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def pos_interp(shape, gh, gw):
    """Bilinear align-corners resampling of the pos_side^2 learned grid to the
    (gh, gw) patch grid in merge-block order: (indices (n, 4), weights (n, 4)
    fp32) (fast_pos_embed_interpolate, modeling_qwen3_vl.py:664-679). Source
    coordinate of patch row r: r (side - 1) / (gh - 1) in fp32; taps floor and
    floor + 1 (clamped to the grid), hat weights 1 - |src - tap|."""
    s = shape.pos_side
    def axis(size):
        i = torch.arange(size, dtype=F32)
        src = i * (s - 1) / max(size - 1, 1)
        fl = torch.floor(src)
        off = torch.arange(2)
        taps = (fl.long()[:, None] + off).clamp(0, s - 1)
        wts = (1 - (src[:, None] - fl[:, None] - off).abs()).clamp(min=0)
        return taps, wts
    ht, hw = axis(gh)
    wt_, ww = axis(gw)
    idx = (ht[:, None, :, None] * s + wt_[None, :, None, :]).reshape(gh, gw, 4)
    wt = (hw[:, None, :, None] * ww[None, :, None, :]).reshape(gh, gw, 4)
    m = shape.merge
    def order(x):
        x = x.reshape(gh // m, m, gw // m, m, 4).permute(0, 2, 1, 3, 4)
        return x.reshape(-1, 4)
    return order(idx), order(wt)


def pos_embeds(shape, pos_embed, gh, gw):
    """(n, hidden) bf16: the 4 corner embeddings times their fp32 weights,
    summed in tap order in fp32."""
    idx, wt = pos_interp(shape, gh, gw)
    e = pos_embed.to(F32)[idx]                            # (n, 4, hidden)
    acc = e[:, 0] * wt[:, 0, None]
    for t in range(1, 4):
        acc = acc + e[:, t] * wt[:, t, None]
    return acc.to(BF16)


# ---------------------------------------------------------------- modules

def linear(x, w, b):
    """bf16 nn.Linear: bf16(x . w^T + b), the product in fp64."""
    y = x.to(torch.float64) @ w.to(torch.float64).T + b.to(torch.float64)
    return y.to(F32).to(BF16)


def layer_norm(x, w, b, eps):
    """nn.LayerNorm on bf16: statistics and affine map in fp32, one rounding."""
    xf = x.to(F32)
    mean = xf.mean(-1, keepdim=True)
    var = ((xf - mean) ** 2).mean(-1, keepdim=True)
    return ((xf - mean) * torch.rsqrt(var + eps) * w.to(F32) + b.to(F32)).to(BF16)


def gelu_tanh(x):
    """ACT2FN['gelu_pytorch_tanh'] on bf16 (fp32 inside, one rounding)."""
    return torch.nn.functional.gelu(x.to(F32), approximate="tanh").to(BF16)


def gelu_erf(x):
    """nn.GELU() on bf16 (fp32 inside, one rounding)."""
    return torch.nn.functional.gelu(x.to(F32)).to(BF16)


def vision_rope(q, k, cos, sin):
    """``vision_rope`` (_legacy/search_kernels.py:111-134) = apply_rotary_pos_emb_vision:
    bf16(x * cos + rotate_half(x) * sin) in fp32; q, k (n, heads, hd), cos/sin (n, hd)."""
    def rot(x):
        xf = x.to(F32)
        h = xf.shape[-1] // 2
        r = torch.cat([-xf[..., h:], xf[..., :h]], dim=-1)
        return (xf * cos[:, None, :] + r * sin[:, None, :]).to(BF16)
    return rot(q), rot(k)


def attention(q, k, v, scale):
    """Bidirectional sdpa (is_causal=False) per head, exact in fp64: q, k, v
    (n, heads, hd) bf16 -> (n, heads * hd) bf16."""
    qf, kf, vf = (t.to(torch.float64).transpose(0, 1) for t in (q, k, v))
    p = torch.softmax(qf @ kf.transpose(1, 2) * scale, dim=-1)
    o = (p @ vf).transpose(0, 1)
    return o.reshape(o.shape[0], -1).to(F32).to(BF16)


def block(shape, blk, h, cos, sin, trace=None):
    """One vision block (Qwen3VLVisionBlock.forward, modeling_qwen3_vl.py:288-306,
    as NativeNormVision.core runs it)."""
    n, hd = h.shape[0], shape.head_dim
    x = layer_norm(h, blk.norm1_w, blk.norm1_b, shape.eps)
    qkv = linear(x, blk.qkv_w, blk.qkv_b).reshape(n, 3, shape.heads, hd)
    q, k = vision_rope(qkv[:, 0], qkv[:, 1], cos, sin)
    z = attention(q, k, qkv[:, 2], hd ** -0.5)
    h = bf16(h.to(F32) + linear(z, blk.proj_w, blk.proj_b).to(F32)).to(BF16)
    x = layer_norm(h, blk.norm2_w, blk.norm2_b, shape.eps)
    y = linear(gelu_tanh(linear(x, blk.fc1_w, blk.fc1_b)), blk.fc2_w, blk.fc2_b)
    h = bf16(h.to(F32) + y.to(F32)).to(BF16)
    if trace is not None:
        trace.append(h)
    return h


def merge(shape, mg, h):
    """Qwen3VLVisionPatchMerger.forward (modeling_qwen3_vl.py:122-137)."""
    width = shape.hidden * shape.merge ** 2
    x = layer_norm(h.reshape(-1, width), mg.norm_w, mg.norm_b, shape.eps) if mg.postshuffle else \
        layer_norm(h, mg.norm_w, mg.norm_b, shape.eps).reshape(-1, width)
    return linear(gelu_erf(linear(x, mg.fc1_w, mg.fc1_b)), mg.fc2_w, mg.fc2_b)


def tower(shape, w, pixels, gh, gw, trace=None):
    """The whole vision step: (merged (n/4, out_hidden), [deepstack features])."""
    cos, sin = rope_cos_sin(shape, gh, gw)
    h = linear(pixels, w.patch_w, w.patch_b)
    h = bf16(h.to(F32) + pos_embeds(shape, w.pos_embed, gh, gw).to(F32)).to(BF16)
    deep = []
    for j, blk in enumerate(w.blocks):
        h = block(shape, blk, h, cos, sin, trace)
        if j in shape.deepstack:
            deep.append(merge(shape, w.deep[shape.deepstack.index(j)], h))
    return merge(shape, w.merger, h), deep


def from_hf(model):
    """VisionWeights from a transformers Qwen3VLVisionModel (any dtype)."""
    g = lambda t: t.detach().to(BF16).clone()  # noqa: E731
    def mg(m, post):
        return Merger(g(m.norm.weight), g(m.norm.bias), g(m.linear_fc1.weight), g(m.linear_fc1.bias),
                      g(m.linear_fc2.weight), g(m.linear_fc2.bias), post)
    blocks = [VisionBlock(g(b.norm1.weight), g(b.norm1.bias), g(b.attn.qkv.weight), g(b.attn.qkv.bias),
                          g(b.attn.proj.weight), g(b.attn.proj.bias), g(b.norm2.weight), g(b.norm2.bias),
                          g(b.mlp.linear_fc1.weight), g(b.mlp.linear_fc1.bias), g(b.mlp.linear_fc2.weight),
                          g(b.mlp.linear_fc2.bias)) for b in model.blocks]
    return VisionWeights(g(model.patch_embed.proj.weight.reshape(model.patch_embed.proj.weight.shape[0], -1)),
                         g(model.patch_embed.proj.bias), g(model.pos_embed.weight), blocks,
                         mg(model.merger, False), [mg(m, True) for m in model.deepstack_merger_list])
