"""Qwen3-VL vision tower on gfx950 kernels, hipGraph-captured.

Restates the reference's vision step: pixel packing (``pack_rectangle``,
_family/depth_runtime.py:18-25) and ``NativeNormVision.core``
(scaled_qwen_runtime.py:42-55): patch embedding + interpolated position
embedding, per block h += proj(sdpa(vision_rope(qkv(LN1(h))))) and
h += fc2(gelu_tanh(fc1(LN2(h)))), the DeepStack mergers after the listed
blocks and the final patch merger, with the per-geometry constants cached as
``VisionGraph.geo`` does (_legacy/vision_graph_runtime.py:11-15) and the step
captured in one graph as ``VisionGraph.build`` does (:28-36).

Every op runs on the library's HIP kernels (``ff_pack_pixels``,
``ff_layer_norm``, ``ff_gemm_bf16``, ``ff_vision_qkv`` (rotary + padded
layouts in one launch), ``ff_attention_full``, ``ff_pos_interp``). Layout choices of this build: the
attention reads q and k head-major with each head zero-padded to 128 dims and
V transposed (heads, 128, n_pad); the MLP intermediate is zero-padded to a
multiple of 64 (fc1 rows and fc2 columns), which leaves every sum exact.

The outputs feed the LM step: ``merged`` (n/4, out_hidden) are the image-token
embeddings that ``Runtime`` scatters into the hidden states, and ``deep`` the
DeepStack features its first layers add (``add_rms`` with ``deep``).
"""
import ctypes
import types
from dataclasses import dataclass

import torch

from ._lib import call, ptr, stream
from .runtime import _Carver

BF16 = torch.bfloat16
F32 = torch.float32
ACT_NONE, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2


@dataclass(frozen=True)
class VisionConfig:
    """Vision tower dimensions (Qwen3VLVisionConfig)."""
    name: str
    depth: int
    hidden: int
    heads: int
    inter: int
    out_hidden: int
    deepstack: tuple
    pos_side: int = 48           # num_position_embeddings = pos_side ** 2
    merge: int = 2
    eps: float = 1e-6
    theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden // self.heads

    @property
    def inter_pad(self):
        return (self.inter + 63) // 64 * 64


VISION_PRESETS = {
    "qwen3vl-2b": VisionConfig("qwen3vl-2b", 24, 1024, 16, 4096, 2048, (5, 11, 17)),
    "qwen3vl-4b": VisionConfig("qwen3vl-4b", 24, 1024, 16, 4096, 2560, (5, 11, 17)),
    "qwen3vl-8b": VisionConfig("qwen3vl-8b", 27, 1152, 16, 4304, 4096, (8, 16, 24)),
    "qwen3vl-32b": VisionConfig("qwen3vl-32b", 27, 1152, 16, 4304, 5120, (8, 16, 24)),
}


@dataclass
class Lin:
    """A bf16 linear: weight (n, k) and bias (n,) on the device, and once
    ``pack`` has run the weight's copy in the packed GEMM's operand order
    (ff_pack_weight_bf16; ``linear`` then reads it, the same bits)."""
    w: torch.Tensor
    b: torch.Tensor
    p: torch.Tensor = None

    def pack(self):
        n, k = self.w.shape
        if self.p is None and n % 16 == 0 and k % 128 == 0:
            self.p = torch.empty_like(self.w)
            call("ff_pack_weight_bf16", ptr(self.w), ptr(self.p), n, k, stream())
        return self


def pack_linears(obj):
    """``Lin.pack`` on every linear reachable from a weights object (dataclass
    fields, lists and tuples)."""
    if isinstance(obj, Lin):
        obj.pack()
    elif isinstance(obj, (list, tuple)):
        for o in obj:
            pack_linears(o)
    elif hasattr(obj, "__dataclass_fields__"):
        for f in obj.__dataclass_fields__:
            pack_linears(getattr(obj, f))


@dataclass
class Norm:
    w: torch.Tensor
    b: torch.Tensor


@dataclass
class VBlock:
    norm1: Norm
    qkv: Lin
    proj: Lin
    norm2: Norm
    fc1: Lin          # rows padded to inter_pad (zero rows, zero bias)
    fc2: Lin          # columns padded to inter_pad (zero columns)


@dataclass
class VMerger:
    norm: Norm
    fc1: Lin
    fc2: Lin
    postshuffle: bool


@dataclass
class VisionWeights:
    patch: Lin        # (hidden, 1536): the Conv3d kernel flattened (c, frame, y, x)
    pos_embed: torch.Tensor
    blocks: list
    merger: VMerger
    deep: list


def pad_mlp(cfg, fc1_w, fc1_b, fc2_w):
    """Zero-pad the MLP intermediate to a multiple of 64: fc1 gains zero rows
    (zero bias, so those channels are gelu(0) = 0) and fc2 zero columns."""
    ip = cfg.inter_pad
    if ip == fc1_w.shape[0]:
        return fc1_w.contiguous(), fc1_b.contiguous(), fc2_w.contiguous()
    w1 = torch.zeros((ip, fc1_w.shape[1]), device=fc1_w.device, dtype=BF16)
    w1[:fc1_w.shape[0]] = fc1_w
    b1 = torch.zeros((ip,), device=fc1_b.device, dtype=BF16)
    b1[:fc1_b.shape[0]] = fc1_b
    w2 = torch.zeros((fc2_w.shape[0], ip), device=fc2_w.device, dtype=BF16)
    w2[:, :fc2_w.shape[1]] = fc2_w
    return w1, b1, w2


def weights_from_hf(cfg, model, device="cuda"):
    """VisionWeights from a transformers Qwen3VLVisionModel."""
    d = lambda t: t.detach().to(device=device, dtype=BF16).contiguous()  # noqa: E731
    blocks = []
    for b in model.blocks:
        w1, b1, w2 = pad_mlp(cfg, d(b.mlp.linear_fc1.weight), d(b.mlp.linear_fc1.bias), d(b.mlp.linear_fc2.weight))
        blocks.append(VBlock(Norm(d(b.norm1.weight), d(b.norm1.bias)), Lin(d(b.attn.qkv.weight), d(b.attn.qkv.bias)),
                             Lin(d(b.attn.proj.weight), d(b.attn.proj.bias)),
                             Norm(d(b.norm2.weight), d(b.norm2.bias)), Lin(w1, b1),
                             Lin(w2, d(b.mlp.linear_fc2.bias))))
    def mg(m, post):
        return VMerger(Norm(d(m.norm.weight), d(m.norm.bias)), Lin(d(m.linear_fc1.weight), d(m.linear_fc1.bias)),
                       Lin(d(m.linear_fc2.weight), d(m.linear_fc2.bias)), post)
    pw = model.patch_embed.proj.weight
    return VisionWeights(Lin(d(pw.reshape(pw.shape[0], -1)), d(model.patch_embed.proj.bias)),
                         d(model.pos_embed.weight), blocks, mg(model.merger, False),
                         [mg(m, True) for m in model.deepstack_merger_list])


def make_vision(cfg, seed=0, device="cuda", std=0.02):
    """Seeded random-init tower (no checkpoint here): linear weights and biases
    N(0, std), position embeddings N(0, std), LayerNorm weights 1 + N(0, 0.1)
    and biases N(0, 0.1) (varied so the affine map is exercised)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed * 7919 + 11)
    def rnd(*s, scale=std):
        return (torch.randn(s, generator=g, device=device) * scale).to(BF16)
    def lin(n, k):
        return Lin(rnd(n, k), rnd(n))
    def norm(n):
        return Norm((1 + torch.randn(n, generator=g, device=device) * 0.1).to(BF16), rnd(n, scale=0.1))
    H, W4 = cfg.hidden, cfg.hidden * cfg.merge ** 2
    blocks = []
    for _ in range(cfg.depth):
        n1, qkv, proj, n2 = norm(H), lin(3 * H, H), lin(H, H), norm(H)
        fc1, fc2 = lin(cfg.inter, H), lin(H, cfg.inter)
        w1, b1, w2 = pad_mlp(cfg, fc1.w, fc1.b, fc2.w)
        blocks.append(VBlock(n1, qkv, proj, n2, Lin(w1, b1), Lin(w2, fc2.b)))
    def merger(post):
        return VMerger(norm(W4 if post else H), lin(W4, W4), lin(cfg.out_hidden, W4), post)
    return VisionWeights(lin(H, 1536), rnd(cfg.pos_side ** 2, H), blocks, merger(False),
                         [merger(True) for _ in cfg.deepstack])


# ---------------------------------------------------------------- geometry

def merge_order(x, gh, gw, m=2):
    """Rows of an (gh, gw, ...) grid in the 2 x 2 merge-block walk."""
    rest = x.shape[2:]
    return x.reshape(gh // m, m, gw // m, m, *rest).transpose(1, 2).reshape(gh * gw, *rest)


def rope_tables(cfg, gh, gw):
    """cos, sin (n, head_dim) fp32 of the vision rotary for a (gh, gw) patch
    grid: patch (row, col) rotates its first head_dim/4 frequency pairs by row
    and the next by col, inv_freq = theta^(-2i/(head_dim/2)), emb = cat(f, f)
    (Qwen3VLVisionModel.rot_pos_emb; modeling_qwen3_vl.py:654-662,704-707).
    A per-geometry constant computed once on the host at setup."""
    dim = cfg.head_dim // 2
    inv = 1.0 / (cfg.theta ** (torch.arange(0, dim, 2, dtype=F32) / dim))
    rows = torch.arange(gh)[:, None].expand(gh, gw)
    cols = torch.arange(gw)[None, :].expand(gh, gw)
    r = merge_order(rows, gh, gw, cfg.merge).to(F32)
    c = merge_order(cols, gh, gw, cfg.merge).to(F32)
    f = torch.cat([r[:, None] * inv, c[:, None] * inv], dim=1)
    emb = torch.cat([f, f], dim=1)
    return emb.cos(), emb.sin()


def interp_taps(cfg, gh, gw):
    """Bilinear align-corners taps of the pos_side^2 position grid for a
    (gh, gw) patch grid in merge-block order: idx (n, 4) int64, wt (n, 4) fp32
    (fast_pos_embed_interpolate; transformers vision_utils.py:191-289). Source
    coordinate r (side - 1) / (size - 1) in fp32, taps floor and floor + 1
    clamped to the grid, hat weights 1 - |src - tap|."""
    s = cfg.pos_side
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
    return merge_order(idx, gh, gw, cfg.merge).contiguous(), merge_order(wt, gh, gw, cfg.merge).contiguous()


# ---------------------------------------------------------------- drop-in ops

def vision_rope(q, k, cos, sin, block=512):
    """``vision_rope(q, k, cos, sin)`` (_legacy/search_kernels.py:127-134): q, k
    (n, heads, hd) bf16 views with equal strides and stride(-1) == 1, cos/sin
    (n, hd) fp32 contiguous -> new (n, heads, hd) tensors. ``block`` (a Triton
    knob) is accepted and ignored."""
    assert q.shape == k.shape and q.stride() == k.stride()
    assert q.ndim == 3 and q.stride(-1) == 1 and cos.is_contiguous() and sin.is_contiguous()
    n, h, d = q.shape
    yq = torch.empty((n, h, d), device=q.device, dtype=q.dtype)
    yk = torch.empty_like(yq)
    call("ff_vision_rope", ptr(q), ptr(k), q.stride(0), q.stride(1), ptr(cos), ptr(sin), ptr(yq), ptr(yk),
         h * d, d, n, h, d, d, stream())
    return yq, yk


def pack_rgb(rgb):
    """``pack_rectangle`` / ``pack_rgb``: rgb (H, W, 3) uint8 on the device ->
    (H/16 * W/16, 1536) bf16 patches."""
    assert rgb.dtype == torch.uint8 and rgb.ndim == 3 and rgb.shape[2] == 3 and rgb.is_contiguous()
    hgt, wid = rgb.shape[:2]
    out = torch.empty(((hgt // 16) * (wid // 16), 1536), device=rgb.device, dtype=BF16)
    call("ff_pack_pixels", ptr(rgb), ptr(out), hgt, wid, stream())
    return out


def linear(x, lin, act=ACT_NONE, resid=None, out=None, ws=None):
    """bf16 linear with its fused neighbours (bias, GELU, residual add). With a
    workspace ``ws`` (at least ``split_workspace`` bytes) short grids split k."""
    m, k = x.shape
    n = lin.w.shape[0]
    y = torch.empty((m, n), device=x.device, dtype=BF16) if out is None else out
    args = [ptr(x), x.stride(0), ptr(lin.w), ptr(lin.p), ptr(lin.b), ptr(y), y.stride(0), ptr(resid),
            0 if resid is None else resid.stride(0), m, n, k, act]
    if ws is None:
        call("ff_gemm_bf16_pk", *args, stream())
    else:
        call("ff_gemm_bf16_pk_ws", *args, ptr(ws), ws.numel() * ws.element_size(), stream())
    return y


def linear_ln(x, lin, resid, out, ws, norm=None, eps=0.0, ln_out=None):
    """A block's residual linear, out = bf16(resid + bf16(x . w^T + b)), and the
    LayerNorm ``norm`` of its output into ``ln_out`` (None: no LayerNorm), as
    two launches: with a k split the LayerNorm launch adds the partials."""
    m, k = x.shape
    n = lin.w.shape[0]
    call("ff_gemm_bf16_pk_ln", ptr(x), x.stride(0), ptr(lin.w), ptr(lin.p), ptr(lin.b), ptr(out), out.stride(0),
         ptr(resid), resid.stride(0), m, n, k, ptr(ws), ws.numel() * ws.element_size(),
         None if norm is None else ptr(norm.w), None if norm is None else ptr(norm.b), float(eps),
         None if ln_out is None else ptr(ln_out), 0 if ln_out is None else ln_out.stride(0), stream())
    return out


def split_workspace(m, n, k):
    """Bytes of fp32 partials the k-split bf16 GEMM needs for an m x n x k product."""
    b = ctypes.c_int64(0)
    call("ff_gemm_bf16_pk_workspace", m, n, k, ctypes.byref(b))
    return b.value


def layer_norm(x, norm, eps, out=None):
    rows, h = x.shape
    y = torch.empty((rows, h), device=x.device, dtype=BF16) if out is None else out
    call("ff_layer_norm", ptr(x), x.stride(0), ptr(norm.w), ptr(norm.b), ptr(y), y.stride(0), rows, h, float(eps),
         stream())
    return y


# ---------------------------------------------------------------- runtime

def _lay_out_vision(rt, cfg, n, n_pad, nm, a):
    """Give ``rt`` the tower's activation buffers, each from ``a(*shape, dt=dtype)``
    (an arena carve, a plain allocation, or a byte counter), in a fixed order.
    The activations grow with the patch count; the k-split partials ``part``
    exist only for grids too short to fill the GPU, so a variant's arena is
    sized by the largest layout over its canvases."""
    H, NH = cfg.hidden, cfg.heads
    W4 = H * cfg.merge ** 2
    rt.pixels = a(n, 1536)
    rt.h = a(n, H)
    rt.x = a(n, H)
    rt.qkv = a(n, 3 * H)
    rt.q, rt.k = a(NH, n, 128), a(NH, n, 128)
    rt.vt = a(NH, 128, n_pad)
    rt.z = a(n, H)
    rt.u = a(n, cfg.inter_pad)
    rt.x4 = a(nm, W4)
    rt.u4 = a(nm, W4)
    ip = cfg.inter_pad
    need = max(split_workspace(n, H, 1536), split_workspace(n, 3 * H, H), split_workspace(n, H, H),
               split_workspace(n, ip, H), split_workspace(n, H, ip), split_workspace(nm, W4, W4),
               split_workspace(nm, cfg.out_hidden, W4))
    rt.part = a(max(need // 4, 64), dt=torch.float32)


class VisionRuntime:
    """The vision step for one image geometry (a (gh, gw) patch grid, i.e. an
    image of 16 gh x 16 gw pixels) with static device buffers.

    ``merged`` / ``deep`` may be given (the LM runtime's ``visual`` and ``deep``
    buffers) so the step writes the image tokens straight where the LM step
    reads them. ``arena``: a ``runtime.Arena`` that the activations alias,
    shared with the towers of the model's other image geometries (their steps
    must not overlap in time); the per-geometry tables stay private.
    """

    @staticmethod
    def arena_bytes(cfg, gh, gw):
        """Arena bytes a tower of a (gh, gw) patch grid lays its activations out in."""
        counter = _Carver(None)
        n = gh * gw
        _lay_out_vision(types.SimpleNamespace(), cfg, n, (n + 63) // 64 * 64, n // cfg.merge ** 2,
                        lambda *s, dt=BF16: counter(s, dt, None))
        return counter.cursor

    def __init__(self, cfg, weights, gh, gw, merged=None, deep=None, arena=None):
        if gh % cfg.merge or gw % cfg.merge:
            raise ValueError("the patch grid must be a whole number of merge blocks")
        self.cfg, self.w = cfg, weights
        pack_linears(weights)  # packed weight copies for the packed GEMM (once per weights object)
        self.gh, self.gw = gh, gw
        n = gh * gw
        self.n, self.nm = n, n // cfg.merge ** 2
        self.n_pad = (n + 63) // 64 * 64
        dev = weights.pos_embed.device
        H = cfg.hidden
        e = lambda *s, dt=BF16: torch.empty(s, device=dev, dtype=dt)  # noqa: E731
        # activations (written in full by every step): aliased into a shared arena when one is given
        if arena is not None:
            carve = _Carver(arena)
            a = lambda *s, dt=BF16: carve(s, dt, dev)  # noqa: E731
        else:
            a = e
        self.rgb = torch.zeros((16 * gh, 16 * gw, 3), device=dev, dtype=torch.uint8)
        # per-geometry constants (VisionGraph.geo)
        cos, sin = rope_tables(cfg, gh, gw)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        idx, wt = interp_taps(cfg, gh, gw)
        rows = weights.pos_embed.shape[0]
        if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= rows):
            raise ValueError(f"position-embedding taps outside the {rows}-row table")
        # the tap tables stay referenced until the kernel has read them: a
        # temporary freed inside the argument list could hand its memory to
        # the next one before the launch
        self._taps = (idx.to(dev), wt.to(dev))
        self.pos = e(n, H)
        call("ff_pos_interp", ptr(weights.pos_embed), ptr(self._taps[0]), ptr(self._taps[1]), ptr(self.pos), n, 4,
             H, weights.pos_embed.shape[0], stream())
        _lay_out_vision(self, cfg, n, self.n_pad, self.nm, a)
        self.merged = e(self.nm, cfg.out_hidden) if merged is None else merged
        self.deep = [e(self.nm, cfg.out_hidden) for _ in cfg.deepstack] if deep is None else deep
        if len(self.deep) != len(cfg.deepstack):
            raise ValueError("one DeepStack buffer per DeepStack merger")
        self.graph = None

    def set_image(self, rgb):
        """Refill the static rgb input ((16 gh, 16 gw, 3) uint8, host or device)."""
        rgb = torch.as_tensor(rgb)
        if tuple(rgb.shape) != tuple(self.rgb.shape) or rgb.dtype != torch.uint8:
            raise ValueError(f"image must be uint8 {tuple(self.rgb.shape)}")
        self.rgb.copy_(rgb, non_blocking=True)

    def _merge(self, mg, h, out):
        cfg, s = self.cfg, stream()
        W4 = cfg.hidden * cfg.merge ** 2
        if mg.postshuffle:   # LayerNorm over the 4 merged patches
            layer_norm(h.view(self.nm, W4), mg.norm, cfg.eps, out=self.x4)
        else:                # LayerNorm per patch, then the 4 patches side by side
            layer_norm(h, mg.norm, cfg.eps, out=self.x4.view(self.n, cfg.hidden))
        linear(self.x4, mg.fc1, ACT_GELU_ERF, out=self.u4, ws=self.part)
        linear(self.u4, mg.fc2, out=out, ws=self.part)
        return s

    def step(self, trace=None):
        """Run the tower eagerly on the current stream; returns (merged, deep).
        ``trace`` (a list) receives a copy of h after every block."""
        cfg, w, s = self.cfg, self.w, stream()
        n, H, HD, NH = self.n, cfg.hidden, cfg.head_dim, cfg.heads
        call("ff_pack_pixels", ptr(self.rgb), ptr(self.pixels), 16 * self.gh, 16 * self.gw, s)
        # each residual linear carries the LayerNorm that reads its output: the
        # patch embedding block 0's norm1, proj norm2, fc2 the next block's norm1
        linear_ln(self.pixels, w.patch, self.pos, self.h, self.part, w.blocks[0].norm1, cfg.eps, self.x)
        for j, blk in enumerate(w.blocks):
            linear(self.x, blk.qkv, out=self.qkv, ws=self.part)
            call("ff_vision_qkv", ptr(self.qkv), ptr(self.cos), ptr(self.sin), ptr(self.q), ptr(self.k),
                 ptr(self.vt), n, self.n_pad, NH, HD, s)
            call("ff_attention_full", ptr(self.q), ptr(self.k), ptr(self.vt), ptr(self.z), n, self.n_pad, NH, HD,
                 float(HD ** -0.5), s)
            linear_ln(self.z, blk.proj, self.h, self.h, self.part, blk.norm2, cfg.eps, self.x)
            linear(self.x, blk.fc1, ACT_GELU_TANH, out=self.u, ws=self.part)
            nxt = w.blocks[j + 1].norm1 if j + 1 < len(w.blocks) else None
            linear_ln(self.u, blk.fc2, self.h, self.h, self.part, nxt, cfg.eps, self.x)
            if j in cfg.deepstack:
                self._merge(w.deep[cfg.deepstack.index(j)], self.h, self.deep[cfg.deepstack.index(j)])
            if trace is not None:
                trace.append(self.h.clone())
        self._merge(w.merger, self.h, self.merged)
        return self.merged, self.deep

    def capture(self, warmup=2):
        """Capture the whole tower into one hipGraph (VisionGraph.build)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g
        return g

    def replay(self):
        if self.graph is None:
            self.capture()
        self.graph.replay()
        return self.merged, self.deep
