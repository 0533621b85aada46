"""Qwen3-VL LM prefill + choice-score step on gfx950 kernels, hipGraph-captured.

Restates ``Runtime.prefix`` / ``attention`` / ``mlp`` (scaled_qwen_runtime.py:143-176)
and the pick-only tail of the fp8/precise execution modes
(_family/night_runtime.py:92-105), with graph capture and input refill as in
``graph`` (_family/night_runtime.py:106-125).

Two step bodies produce identical numbers:

* ``fused`` (FP8Linear weights): every activation buffer is allocated once per
  token bucket (or laid out in an ``Arena`` that the buckets share); the per-token e4m3 quantization of each GEMM input is fused into
  the kernel that produces it (add_rms, fast_norm, swiglu), and V is written
  transposed by the QKV GEMM's epilogue; the down projection's split-K partials
  are added by the next add_rms launch. 9 launches per layer.
* ``generic`` (any linear op): the reference's own op sequence through the
  drop-in ops of ``fastforward_amd.ops`` and ``Linear.apply``.

Inputs are a bucket-sized token id buffer (zero padded), M-RoPE positions
(3, T) and the picked row; the step writes the choice logits (n_options,) fp32.
"""
import types
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from ._lib import call, ptr, stream
from .linear import FP8Linear, Int4, Linear, StaticFP8Linear, gemm_pk_workspace

BF16 = torch.bfloat16
E4M3 = torch.float8_e4m3fn


@dataclass(frozen=True)
class LMConfig:
    """Language-model dimensions (Qwen3-VL text config)."""
    name: str
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
    tie_embed: bool = False

    @property
    def scaling(self):
        return self.head_dim ** -0.5

    @property
    def qkv_out(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim


PRESETS = {
    "qwen3vl-2b": LMConfig("qwen3vl-2b", 28, 2048, 16, 8, 128, 6144, 151936, tie_embed=True),
    "qwen3vl-4b": LMConfig("qwen3vl-4b", 36, 2560, 32, 8, 128, 9728, 151936, tie_embed=True),
    "qwen3vl-8b": LMConfig("qwen3vl-8b", 36, 4096, 32, 8, 128, 12288, 151936),
    "qwen3vl-32b": LMConfig("qwen3vl-32b", 64, 5120, 64, 8, 128, 25600, 151936),
}


def mrope_positions(prefix_tokens, grid_h, grid_w, total):
    """M-RoPE position ids (3, total) int64 for a prompt with one image of merged
    grid (grid_h, grid_w) after ``prefix_tokens`` text tokens, the layout the
    reference precomputes per bucket with transformers' get_rope_index
    (_family/depth_runtime.py:45-49): text t -> (t,t,t); image (r,c) ->
    (s0, s0+r, s0+c); later text continues at s0 + max(gh, gw)."""
    s0, nv = prefix_tokens, grid_h * grid_w
    if s0 + nv > total:
        raise ValueError("image does not fit in the bucket")
    pos = np.empty((3, total), dtype=np.int64)
    pos[:, :s0] = np.arange(s0)
    rows = np.repeat(np.arange(grid_h), grid_w)
    cols = np.tile(np.arange(grid_w), grid_h)
    pos[0, s0:s0 + nv] = s0
    pos[1, s0:s0 + nv] = s0 + rows
    pos[2, s0:s0 + nv] = s0 + cols
    pos[:, s0 + nv:] = s0 + max(grid_h, grid_w) + np.arange(total - s0 - nv)
    return pos


def rope_inv_freq(theta, head_dim):
    """The rotary module's constant ``inv_freq`` buffer, computed once at setup
    on the host exactly as transformers does at module init (fp32)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


@dataclass
class LayerWeights:
    input_norm: ops.RMSNorm
    post_norm: ops.RMSNorm
    q_norm: ops.RMSNorm
    k_norm: ops.RMSNorm
    qkv: object
    o: object
    gateup: object
    down: object


@dataclass
class ModelWeights:
    embed: torch.Tensor       # (vocab, H) bf16
    layers: list
    norm: ops.RMSNorm
    head: torch.Tensor        # (n_options, H) bf16, option rows of lm_head
    extra: dict = field(default_factory=dict)


class Arena:
    """Device bytes that the activation buffers of several step runtimes share.

    Requests run one at a time, and a step writes each activation buffer before
    it reads it, so nothing lives in them between steps: the runtimes of all
    token buckets (and image canvases) of one model can alias a single region
    instead of holding one set each (about 100 MB per 576-token bucket at the
    8B shape). Static inputs (ids, positions, pick), the image-token buffers and
    the logits stay per runtime. Steps of runtimes that share an arena must not
    overlap in time.

    The region must hold the largest layout over every bucket, which is not
    always the largest bucket's: the k-split workspace of the packed GEMMs
    depends on whether a shape's tiles fill the GPU unsplit, so a smaller
    bucket can need more bytes (``size_for_buckets``).
    """

    ALIGN = 256

    def __init__(self, nbytes, device):
        self.nbytes = int(nbytes)
        self.buf = torch.empty(max(self.nbytes, self.ALIGN), dtype=torch.uint8, device=device)

    @staticmethod
    def size_for(cfg, tokens, path="fused"):
        """Bytes of arena a Runtime of ``tokens`` tokens on ``path`` takes
        (counted by laying its activation buffers out without allocating them)."""
        counter = _Carver(None)
        _lay_out_activations(types.SimpleNamespace(), cfg, tokens, path, lambda *s, dt=BF16: counter(s, dt, None))
        return counter.cursor

    @staticmethod
    def size_for_buckets(cfg, buckets, path="fused"):
        """Bytes of arena that every bucket of ``buckets`` fits in."""
        return max(Arena.size_for(cfg, int(b), path) for b in buckets)


class _Carver:
    """Lays one runtime's activation buffers out from offset 0 of an arena
    (``arena`` None: only counts the bytes)."""

    def __init__(self, arena):
        self.arena, self.cursor = arena, 0

    def __call__(self, shape, dtype, device):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype, device="meta").element_size()
        off = (self.cursor + Arena.ALIGN - 1) // Arena.ALIGN * Arena.ALIGN
        self.cursor = off + n
        if self.arena is None:
            return torch.empty(shape, dtype=dtype, device="meta")
        if self.cursor > self.arena.nbytes:
            raise ValueError(f"arena of {self.arena.nbytes} bytes is too small for this runtime")
        return self.arena.buf[off:off + n].view(dtype).view(shape)


def _lay_out_activations(rt, cfg, tokens, path, a):
    """Give ``rt`` the step's activation buffers, each from ``a(*shape, dt=dtype)``
    (an arena carve, a plain allocation, or a byte counter), in a fixed order."""
    T, Tp, H, D = tokens, (tokens + 63) // 64 * 64, cfg.hidden, cfg.head_dim
    HQ, HK, I = cfg.heads, cfg.kv_heads, cfg.inter
    rt.cos, rt.sin = a(T, D), a(T, D)
    rt.h = [a(T, H), a(T, H)]
    rt.res = a(T, H)
    if path == "fused_static":
        # static-scale linears: every GEMM input is e4m3 written by its producer
        rt.xq = a(T, H, dt=E4M3)
        rt.yq, rt.yk, rt.vt = a(HQ, T, D), a(HK, T, D), a(HK, D, Tp)
        rt.aq = a(T, HQ * D, dt=E4M3)
        rt.attn = a(1, HQ * D)                             # the tail's attention row (bf16)
        rt.o = a(T, H)
        rt.pq = a(T, H, dt=E4M3)
        rt.mq = a(T, I, dt=E4M3)
        rt.dn = a(T, H)
        rt.hp = a(1, H)
        need = max(gemm_pk_workspace(T, H, HQ * D), gemm_pk_workspace(T, H, I), 256)
        rt.gws = a(need, dt=torch.uint8)
        return
    if path != "fused":
        return
    rt.xq, rt.xs = a(T, H, dt=E4M3), a(T, dt=torch.float32)
    rt.yq, rt.yk, rt.vt = a(HQ, T, D), a(HK, T, D), a(HK, D, Tp)
    rt.attn = a(T, HQ * D)
    rt.aq, rt.as_ = a(T, HQ * D, dt=E4M3), a(T, dt=torch.float32)
    rt.o = a(T, H)
    rt.pq, rt.ps = a(T, H, dt=E4M3), a(T, dt=torch.float32)
    rt.hm = a(T, I)                                    # swiglu output (bf16)
    rt.pmax = a(T, I // 64, dt=torch.float32)          # its row maxima per 64 channels
    rt.mq, rt.ms = a(T, I, dt=E4M3), a(T, dt=torch.float32)
    rt.dn = a(T, H)
    rt.hp = a(1, H)
    # k-split partials of ff_gemm_fp8_pk (o and down share it: their calls are ordered)
    need = max(gemm_pk_workspace(T, H, HQ * D), gemm_pk_workspace(T, H, I), 256)
    rt.gws = a(need, dt=torch.uint8)


class Runtime:
    """One bucket (T tokens) of the LM step with static device buffers.

    ``arena``: an ``Arena`` whose bytes the activation buffers alias (shared
    with the other runtimes of the same model; see ``Arena``); None allocates
    them for this runtime alone."""

    def __init__(self, cfg, weights, tokens, path=None, visual_rows=0, image_start=0, deep_layers=0, arena=None):
        self.cfg, self.w = cfg, weights
        self.T = tokens
        self.Tp = (tokens + 63) // 64 * 64
        dev = weights.embed.device
        self.dev = dev
        natural = self.path_for(weights)
        self.path = path or natural
        if self.path in ("fused", "fused_static") and self.path != natural:
            raise ValueError(f"the {self.path} path needs "
                             + ("FP8Linear (per-token / per-channel)" if self.path == "fused"
                                else "StaticFP8Linear / RuntimeScaleLinear (calibrated per-tensor)") + " weights")
        if self.path in ("fused", "fused_static"):
            for L in weights.layers:  # MFMA-fragment copies for the packed tile kernels (once per weight)
                L.qkv.pack()
                L.o.pack()
                L.gateup.pack()
                L.down.pack()
        else:
            for L in weights.layers:  # fragment copies of the int4 weights for the packed W4A16 kernels
                for op in (L.qkv, L.o, L.gateup, L.down):
                    if isinstance(op, Int4):
                        op.pack()
        T, H, D = tokens, cfg.hidden, cfg.head_dim
        e = lambda *s, dt=BF16: torch.empty(s, device=dev, dtype=dt)  # noqa: E731
        # activations: aliased into the shared arena when one is given
        if arena is not None:
            carve = _Carver(arena)
            a = lambda *s, dt=BF16: carve(s, dt, dev)  # noqa: E731
        else:
            a = e
        # static inputs
        self.ids = torch.zeros(T, device=dev, dtype=torch.int64)
        self.pos = torch.zeros(3, T, device=dev, dtype=torch.int64)
        self.pick = torch.zeros(1, device=dev, dtype=torch.int64)
        if visual_rows and not 0 <= image_start <= tokens - visual_rows:
            raise ValueError("visual rows do not fit in the bucket")
        self.nv, self.image_start = visual_rows, image_start
        self.visual = e(visual_rows, H) if visual_rows else None
        self.deep = [e(visual_rows, H) for _ in range(deep_layers)] if visual_rows else []
        self.inv_freq = rope_inv_freq(cfg.theta, D).to(dev)
        self.logits = torch.zeros(weights.head.shape[0], device=dev, dtype=torch.float32)
        _lay_out_activations(self, cfg, tokens, self.path, a)
        self.graph = None
        self.graph_out = None

    @staticmethod
    def path_for(weights):
        """"fused" when every linear is an FP8Linear (per-token / per-channel),
        "fused_static" when every linear is a StaticFP8Linear /
        RuntimeScaleLinear (calibrated per-tensor scales), else "generic" (the
        reference's op sequence through the drop-in ops)."""
        ops_ = [op for L in weights.layers for op in (L.qkv, L.o, L.gateup, L.down)]
        if all(isinstance(op, FP8Linear) for op in ops_):
            return "fused"
        if all(isinstance(op, StaticFP8Linear) for op in ops_):
            return "fused_static"
        return "generic"

    # ------------------------------------------------------------ inputs

    def set_inputs(self, ids, pos, pick, visual=None, deep=None):
        """Refill the static inputs (graph replay reads them in place)."""
        ids = torch.as_tensor(ids, dtype=torch.int64)
        n = ids.numel()
        if not 0 < n <= self.T:
            raise ValueError(f"{n} tokens do not fit the {self.T}-token bucket")
        if not 0 <= int(pick) < n:
            raise ValueError("pick must index a real token")
        if int(ids.min()) < 0 or int(ids.max()) >= self.cfg.vocab:
            raise ValueError("token id outside the vocabulary")
        pos = torch.as_tensor(pos, dtype=torch.int64)
        if pos.shape != (3, self.T):
            raise ValueError(f"positions must be (3, {self.T})")
        self.ids.zero_()
        self.ids[:n].copy_(ids, non_blocking=True)
        self.pos.copy_(pos, non_blocking=True)
        self.pick.fill_(int(pick))
        if visual is not None:
            self.visual.copy_(visual)
        for d, src in zip(self.deep, deep or []):
            d.copy_(src)

    # ------------------------------------------------------------ step bodies

    def _prologue(self):
        cfg, s = self.cfg, stream()
        T, H, D = self.T, cfg.hidden, cfg.head_dim
        h = self.h[0]
        call("ff_embed", ptr(self.ids), ptr(self.w.embed), ptr(h), T, H, cfg.vocab, s)
        if self.visual is not None:
            call("ff_scatter_rows", ptr(self.visual), ptr(h), self.image_start, self.nv, H, s)
        call("ff_mrope_cos_sin", ptr(self.pos), ptr(self.inv_freq), ptr(self.cos), ptr(self.sin), T, D,
             cfg.sections[1], cfg.sections[2], s)
        return h

    def _step_fused(self, trace=None):
        cfg, w, s = self.cfg, self.w, stream()
        T, Tp, H, D = self.T, self.Tp, cfg.hidden, cfg.head_dim
        HQ, HK, I, eps = cfg.heads, cfg.kv_heads, cfg.inter, cfg.eps
        h = self._prologue()
        L = w.layers
        call("ff_fast_norm_quant", ptr(h), ptr(L[0].input_norm.weight), None, ptr(self.xq), ptr(self.xs), T, H,
             float(L[0].input_norm.variance_epsilon), s)
        cur = 0
        for j in range(cfg.layers - 1):
            lw = L[j]
            h = self.h[cur]
            self._attention_fused(lw, s)
            # o projection + the post-attention add_rms: where o splits k (the 32B shape) the add_rms
            # launch adds its partials; elsewhere the two launches as they are
            ow = lw.o
            call("ff_gemm_fp8_pk_add_rms_quant", ptr(self.aq), ptr(self.as_), 1, ptr(ow.weight), ptr(ow.packed),
                 ptr(ow.scale), 1, ptr(self.o), T, H, HQ * D, ptr(self.gws), self.gws.numel(), ptr(h), None,
                 ptr(lw.post_norm.weight), ptr(self.res), ptr(self.pq), ptr(self.ps),
                 float(lw.post_norm.variance_epsilon), 0, 0, s)
            self._gateup_fused(lw, self.pq, self.ps, T, s)
            nxt = self.h[cur ^ 1]
            deep = self.deep[j] if j < len(self.deep) else None
            nn = L[j + 1].input_norm
            # down projection + the next layer's add_rms (the split-K partials added by the add_rms launch)
            dw = lw.down
            call("ff_gemm_fp8_pk_add_rms_quant", ptr(self.mq), ptr(self.ms), 1, ptr(dw.weight), ptr(dw.packed),
                 ptr(dw.scale), 1, ptr(self.dn), T, H, I, ptr(self.gws), self.gws.numel(), ptr(self.res), ptr(deep),
                 ptr(nn.weight), ptr(nxt), ptr(self.xq), ptr(self.xs), float(nn.variance_epsilon), self.image_start,
                 self.nv if deep is not None else 0, s)
            cur ^= 1
            if trace is not None:
                trace.append(nxt.clone())
        # pick-only tail (_family/night_runtime.py:92-105)
        lw = L[-1]
        h = self.h[cur]
        self._attention_fused(lw, s, tail=True)
        self._gemm(self.aq, self.as_, lw.o, self.o, 1, s)
        call("ff_gather_rows", ptr(h), H, ptr(self.pick), ptr(self.hp), H, 1, H, T, s)
        call("ff_add_rms_quant", ptr(self.hp), ptr(self.o), None, ptr(lw.post_norm.weight), ptr(self.res), None,
             ptr(self.pq), ptr(self.ps), 1, H, float(lw.post_norm.variance_epsilon), 0, 0, s)
        self._mlp_fused(lw, self.pq, self.ps, 1, self.dn, s)
        call("ff_lm_readout", ptr(self.res), ptr(self.dn), ptr(w.norm.weight), ptr(w.head), ptr(self.logits), H,
             w.head.shape[0], float(w.norm.variance_epsilon), s)
        return self.logits

    def _attention_fused(self, lw, s, tail=False):
        cfg = self.cfg
        T, Tp, H, D = self.T, self.Tp, cfg.hidden, cfg.head_dim
        HQ, HK = cfg.heads, cfg.kv_heads
        # QKV GEMM with q/k norm + rotary and the V transpose in its epilogue
        call("ff_gemm_fp8_qkv_pk", ptr(self.xq), ptr(self.xs), 1, ptr(lw.qkv.weight), ptr(lw.qkv.packed),
             ptr(lw.qkv.scale), 1, T, H, HQ, HK, ptr(lw.q_norm.weight), ptr(lw.k_norm.weight),
             float(lw.q_norm.variance_epsilon), float(lw.k_norm.variance_epsilon), ptr(self.cos), ptr(self.sin),
             ptr(self.yq), ptr(self.yk), ptr(self.vt), Tp, s)
        if tail:
            call("ff_attention_vt", ptr(self.yq), ptr(self.yk), ptr(self.vt), ptr(self.pick), 1, ptr(self.attn),
                 1, T, Tp, HQ, HK, D, float(cfg.scaling), s)
            call("ff_quant_rows_fp8", ptr(self.attn), HQ * D, ptr(self.aq), ptr(self.as_), 1, HQ * D, s)
        else:
            call("ff_attention_vt", ptr(self.yq), ptr(self.yk), ptr(self.vt), None, 0, ptr(self.attn), T, T, Tp,
                 HQ, HK, D, float(cfg.scaling), s)
            call("ff_quant_rows_fp8", ptr(self.attn), HQ * D, ptr(self.aq), ptr(self.as_), T, HQ * D, s)

    def _gemm(self, q, sc, op, out, m, s):
        """out[:m] = bf16(q . W^T * sc * s_w) for an FP8Linear op: ff_gemm_fp8_pk (packed
        weights, k split over the Runtime's workspace where it pays; otherwise the
        row-major kernels, GEMV for m <= 4)."""
        n, k = op.weight.shape
        call("ff_gemm_fp8_pk", ptr(q), ptr(sc), 1, ptr(op.weight), ptr(op.packed), ptr(op.scale), 1, ptr(out), n,
             m, n, k, ptr(self.gws), self.gws.numel(), s)

    def _gateup_fused(self, lw, q, sc, m, s):
        I, H = self.cfg.inter, self.cfg.hidden
        # gate/up GEMM with SwiGLU in its epilogue, then per-token quant from its row maxima
        call("ff_gemm_fp8_swiglu_pk", ptr(q), ptr(sc), ptr(lw.gateup.weight), ptr(lw.gateup.packed),
             ptr(lw.gateup.scale), ptr(self.hm), I, ptr(self.pmax), m, I, H, s)
        call("ff_quant_rows_pmax", ptr(self.hm), I, ptr(self.pmax), I // 64, ptr(self.mq), ptr(self.ms), m, I, s)

    def _mlp_fused(self, lw, q, sc, m, out, s):
        self._gateup_fused(lw, q, sc, m, s)
        self._gemm(self.mq, self.ms, lw.down, out, m, s)

    def _step_static(self, trace=None):
        """The fused step for static-scale linears (the reference's calibrated
        mode: RuntimeScaleLinear, _family/depth_fp8.py:8-26, with select()'s
        bounds): every GEMM input is cast to e4m3 with the consuming linear's
        inverse_scale inside the kernel that produces it (norms, attention, the
        gate/up SwiGLU epilogue), and the GEMMs take the per-tensor
        input_scale / weight_scale. 7 launches per full layer; where the down
        projection splits k its partials are added by the add_rms launch."""
        cfg, w, s = self.cfg, self.w, stream()
        T, Tp, H, D = self.T, self.Tp, cfg.hidden, cfg.head_dim
        HQ, HK, I = cfg.heads, cfg.kv_heads, cfg.inter
        h = self._prologue()
        L = w.layers
        call("ff_fast_norm_quant_static", ptr(h), ptr(L[0].input_norm.weight), None, ptr(self.xq),
             float(L[0].qkv.inverse_scale), T, H, float(L[0].input_norm.variance_epsilon), s)
        cur = 0
        for j in range(cfg.layers - 1):
            lw = L[j]
            h = self.h[cur]
            self._qkv_static(lw, T, s)
            call("ff_attention_vt_q", ptr(self.yq), ptr(self.yk), ptr(self.vt), ptr(self.aq),
                 float(lw.o.inverse_scale), T, T, Tp, HQ, HK, D, float(cfg.scaling), s)
            ow = lw.o
            call("ff_gemm_fp8_pk_add_rms_quant_static", ptr(self.aq), ptr(ow.input_scale), 0, ptr(ow.weight),
                 ptr(ow.packed), ptr(ow.weight_scale), 0, ptr(self.o), T, H, HQ * D, ptr(self.gws),
                 self.gws.numel(), ptr(h), None, ptr(lw.post_norm.weight), ptr(self.res), ptr(self.pq),
                 float(lw.gateup.inverse_scale), float(lw.post_norm.variance_epsilon), 0, 0, s)
            self._gateup_static(lw, T, s)
            nxt = self.h[cur ^ 1]
            deep = self.deep[j] if j < len(self.deep) else None
            nn = L[j + 1].input_norm
            dw = lw.down
            call("ff_gemm_fp8_pk_add_rms_quant_static", ptr(self.mq), ptr(dw.input_scale), 0, ptr(dw.weight),
                 ptr(dw.packed), ptr(dw.weight_scale), 0, ptr(self.dn), T, H, I, ptr(self.gws), self.gws.numel(),
                 ptr(self.res), ptr(deep), ptr(nn.weight), ptr(nxt), ptr(self.xq), float(L[j + 1].qkv.inverse_scale),
                 float(nn.variance_epsilon), self.image_start, self.nv if deep is not None else 0, s)
            cur ^= 1
            if trace is not None:
                trace.append(nxt.clone())
        # pick-only tail (_family/night_runtime.py:92-105)
        lw = L[-1]
        h = self.h[cur]
        self._qkv_static(lw, T, s)
        call("ff_attention_vt", ptr(self.yq), ptr(self.yk), ptr(self.vt), ptr(self.pick), 1, ptr(self.attn), 1, T,
             Tp, HQ, HK, D, float(cfg.scaling), s)
        call("ff_quant_static_fp8", ptr(self.attn), ptr(self.aq), 1, 1, HQ * D, float(lw.o.inverse_scale), s)
        self._gemm_static(self.aq, lw.o, self.o, 1, s)
        call("ff_gather_rows", ptr(h), H, ptr(self.pick), ptr(self.hp), H, 1, H, T, s)
        call("ff_add_rms_quant_static", ptr(self.hp), ptr(self.o), None, ptr(lw.post_norm.weight), ptr(self.res), None,
             ptr(self.pq), float(lw.gateup.inverse_scale), 1, H, float(lw.post_norm.variance_epsilon), 0, 0, s)
        self._mlp_static(lw, 1, s)
        call("ff_lm_readout", ptr(self.res), ptr(self.dn), ptr(w.norm.weight), ptr(w.head), ptr(self.logits), H,
             w.head.shape[0], float(w.norm.variance_epsilon), s)
        return self.logits

    def _qkv_static(self, lw, m, s):
        cfg = self.cfg
        op = lw.qkv
        call("ff_gemm_fp8_qkv_pk", ptr(self.xq), ptr(op.input_scale), 0, ptr(op.weight), ptr(op.packed),
             ptr(op.weight_scale), 0, m, cfg.hidden, cfg.heads, cfg.kv_heads, ptr(lw.q_norm.weight), ptr(lw.k_norm.weight),
             float(lw.q_norm.variance_epsilon), float(lw.k_norm.variance_epsilon), ptr(self.cos), ptr(self.sin),
             ptr(self.yq), ptr(self.yk), ptr(self.vt), self.Tp, s)

    def _gemm_static(self, q, op, out, m, s):
        n, k = op.weight.shape
        call("ff_gemm_fp8_pk", ptr(q), ptr(op.input_scale), 0, ptr(op.weight), ptr(op.packed), ptr(op.weight_scale),
             0, ptr(out), n, m, n, k, ptr(self.gws), self.gws.numel(), s)

    def _gateup_static(self, lw, m, s):
        I, H = self.cfg.inter, self.cfg.hidden
        op = lw.gateup
        call("ff_gemm_fp8_swiglu_static", ptr(self.pq), ptr(op.input_scale), ptr(op.weight), ptr(op.packed),
             ptr(op.weight_scale), ptr(self.mq), I, float(lw.down.inverse_scale), m, I, H, s)

    def _mlp_static(self, lw, m, s):
        self._gateup_static(lw, m, s)
        self._gemm_static(self.mq, lw.down, self.dn, m, s)

    def _step_generic(self, trace=None):
        """The reference's op sequence (scaled_qwen_runtime.py:143-176,
        _family/night_runtime.py:92-105) through the drop-in ops."""
        cfg, w = self.cfg, self.w
        HQ, HK, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        h = self._prologue()[None]
        cos, sin = self.cos[None], self.sin[None]
        L = w.layers
        normalized = ops.fast_norm(h, L[0].input_norm)
        for j in range(cfg.layers - 1):
            lw = L[j]
            attn = self._attention_generic(lw, normalized, cos, sin)
            residual, post = self._linear_add_rms(attn, lw.o, h, None, lw.post_norm)
            deep = self.deep[j] if j < len(self.deep) else None
            h, normalized = self._linear_add_rms(self._swiglu(post, lw.gateup), lw.down, residual, deep,
                                                 L[j + 1].input_norm, self.image_start,
                                                 self.nv if deep is not None else 0)
            if trace is not None:
                trace.append(h[0].clone())
        lw = L[-1]
        x = ops.fast_norm(h, lw.input_norm)
        fused = lw.qkv.qkv(x, HQ, HK, lw.q_norm, lw.k_norm, cos, sin) if isinstance(lw.qkv, Int4) else None
        if fused is not None:
            # the picked query row read in place (gather_q), K/V for every token
            q, k, vt, tp = fused
            t = x.shape[-2]
            out = torch.empty((1, 1, HQ, D), device=x.device, dtype=x.dtype)
            call("ff_attention_vt", ptr(q), ptr(k), ptr(vt), ptr(self.pick), 1, ptr(out), 1, t, tp, HQ, HK, D,
                 float(cfg.scaling), stream())
        else:
            q, k, v = Linear.apply(x, lw.qkv).split([HQ * D, HK * D, HK * D], -1)
            shape = (*x.shape[:-1], -1, D)
            q, k = ops.qk_pair(q.view(shape), k.view(shape), lw.q_norm, lw.k_norm, cos, sin)
            v = v.view(shape).transpose(1, 2)
            query = self._index_rows(q[0], self.pick)[None]        # q.index_select(2, pick)
            out = ops.attention_direct(query, k, v, cfg.scaling, positions=self.pick)
        value = Linear.apply(out.reshape(1, 1, -1), lw.o)
        hp = self._index_rows(h[0], self.pick, dim1=True)           # h.index_select(1, pick)
        residual, post = ops.add_rms(hp, value, None, lw.post_norm)
        mlp = Linear.apply(self._swiglu(post[0], lw.gateup), lw.down)
        y = torch.empty((1, w.head.shape[0]), device=self.dev, dtype=torch.float32)
        call("ff_lm_readout", ptr(residual), ptr(mlp), ptr(w.norm.weight), ptr(w.head), ptr(y), cfg.hidden,
             w.head.shape[0], float(w.norm.variance_epsilon), stream())
        self.logits.copy_(y[0])
        return self.logits

    @staticmethod
    def _linear_add_rms(x, op, a, deep, module, start=0, nv=0):
        """add_rms(a, Linear.apply(x, op), deep, module, start, nv)
        (scaled_qwen_runtime.py:158-162): one fused op for a packed Int4 (the
        add_rms launch adds the GEMM's split-K partials; the same bits), else
        the two ops."""
        if isinstance(op, Int4) and op.frag is not None:
            return op.add_rms(x, a, deep, module, start, nv)
        return ops.add_rms(a, Linear.apply(x, op), deep, module, start, nv)

    @staticmethod
    def _swiglu(x, op):
        """swiglu(g, u) for [g, u] = Linear.apply(x, op).chunk(2, -1)
        (scaled_qwen_runtime.py:174-176): one fused launch for a packed Int4
        gate/up whose shape the kernel takes (the same bits), else the two ops."""
        if isinstance(op, Int4) and op.swiglu_fits(x.numel() // x.shape[-1]):
            return op.swiglu(x)
        g, u = Linear.apply(x, op).chunk(2, -1)
        return ops.swiglu(g, u)

    def _attention_generic(self, lw, x, cos, sin):
        cfg = self.cfg
        HQ, HK, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        fused = lw.qkv.qkv(x, HQ, HK, lw.q_norm, lw.k_norm, cos, sin) if isinstance(lw.qkv, Int4) else None
        if fused is not None:
            # packed Int4 QKV: GEMM + qk_pair + V transpose in one op (the same bits),
            # then the attention kernel attention_direct runs on that layout
            yq, yk, vt, tp = fused
            t = x.shape[-2]
            out = torch.empty((1, t, HQ, D), device=x.device, dtype=x.dtype)
            call("ff_attention_vt", ptr(yq), ptr(yk), ptr(vt), None, 0, ptr(out), t, t, tp, HQ, HK, D,
                 float(cfg.scaling), stream())
            return out.reshape(*x.shape[:-1], -1)
        q, k, v = Linear.apply(x, lw.qkv).split([HQ * D, HK * D, HK * D], -1)
        shape = (*x.shape[:-1], -1, D)
        q, k = ops.qk_pair(q.view(shape), k.view(shape), lw.q_norm, lw.k_norm, cos, sin)
        v = v.view(shape).transpose(1, 2)
        out = ops.attention_direct(q, k, v, cfg.scaling)
        return out.reshape(*x.shape[:-1], -1)

    def _index_rows(self, x, idx, dim1=False):
        """Rows ``idx`` of x along its token axis on the device (index_select);
        x is (heads, T, D) or, with dim1, (1, T, H) -> (1, n, H)."""
        if dim1:
            x2 = x.reshape(-1, x.shape[-1])
            out = torch.empty((1, idx.numel(), x2.shape[-1]), device=x.device, dtype=x.dtype)
            call("ff_gather_rows", ptr(x2), x2.stride(0), ptr(idx), ptr(out), x2.shape[-1], idx.numel(),
                 x2.shape[-1], x2.shape[0], stream())
            return out
        heads, t, d = x.shape
        out = torch.empty((heads, idx.numel(), d), device=x.device, dtype=x.dtype)
        for hh in range(heads):
            call("ff_gather_rows", x[hh].data_ptr(), d, ptr(idx), out[hh].data_ptr(), d, idx.numel(), d, t,
                 stream())
        return out

    def step(self, trace=None):
        """Run the step eagerly on the current stream; returns the logits buffer.
        ``trace`` (a list) receives a copy of the residual stream after every
        full layer (eager runs only)."""
        if self.path == "fused":
            return self._step_fused(trace)
        if self.path == "fused_static":
            return self._step_static(trace)
        return self._step_generic(trace)

    # ------------------------------------------------------------ hipGraph

    def capture(self, warmup=2):
        """Capture the whole step into one hipGraph (torch.cuda.CUDAGraph is a
        hipGraph on ROCm). The inputs of the last ``set_inputs`` are used for the
        warmup runs; replays read the static input buffers in place."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self.step()
        self.graph, self.graph_out = g, out
        return g

    def replay(self):
        if self.graph is None:
            self.capture()
        self.graph.replay()
        return self.graph_out
