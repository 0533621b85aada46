"""Image requests over a local Qwen3-VL checkpoint: decode, canvas, prompt,
tokens, one captured image + prompt step per (canvas, token bucket).

Restates the request half of the reference's family runtime:

* ``setup_side`` (_family/depth_runtime.py:35-52): per canvas, the prompt
  prefix with its single image placeholder expanded to one token per merged
  32 x 32 block, and the M-RoPE position template of every bucket;
* ``prepare`` (_family/depth_runtime.py:54-76): decode, canvas + fit +
  letterbox for the selected variant, the question's suffix tokens appended
  to the prefix, no truncation (the prompt must fit the largest bucket), the
  scored row is the last real token;
* ``graph`` (scaled_qwen_runtime.py:218-234, _family/night_runtime.py:106-125):
  the smallest bucket that holds the prompt; its first request captures the
  step, later ones refill the static rgb / ids / pick through pinned staging;
  the first k option logits are the answer scores;
* ``select`` (_family/night_runtime.py:48-54): a calibration variant's
  activation bounds for static FP8 linears; captured steps are dropped.

The image branch runs the vision tower and the LM step in one hipGraph
(``pipeline.ImageStep``); weights come from ``checkpoint.load_pretrained``.
"""
import os
import threading

import numpy as np
import torch

from .checkpoint import load_pretrained
from .pipeline import ImageStep
from .prepare import canvas, canvases, decode_image, prepare_image, text_parts
from .runtime import Arena, Runtime, mrope_positions
from .vision import VisionRuntime

# The reference's execution modes (_family/night_runtime.py:56-65) -> the
# linear format loaded here (None: FP8, static with a calibration profile).
# "int4_half" / "int4_ffn" mix the int4 bank into the interior layers
# (linear.bank_of). The FP8 modes share one accumulation (the matrix
# instruction promotes every 32 products to fp32; fast_accum changes nothing).
EXECUTION_MODES = {"precise": None, "fp8": None, "anchor": None, "int4": "int4", "int4_half": "int4_half",
                   "int4_ffn": "int4_ffn"}


class FamilyRuntime:
    """One checkpoint on one GPU, serving image + question requests.

    ``config`` is the bundle dict: ``model`` (checkpoint directory with
    config.json, safetensors and tokenizer.json), ``buckets`` (token counts),
    and optionally ``variant`` (canvas policy, default 'square256'),
    ``prompt_style`` ('short' / 'minimal' / 'standard'), ``linear`` ('fp8',
    'fp8_static', 'w4a16', 'int4'), ``execution_mode``, ``expected_dimensions``
    ([LM layers, LM width, vision blocks]).
    """

    def __init__(self, config, profiles=None, warmup=3):
        c = dict(config)
        self.c = c
        path = c["model"]
        mode = c.get("execution_mode", "precise")
        if mode not in EXECUTION_MODES:
            raise ValueError(f"execution mode {mode!r} is not supported by this build")
        linear = c.get("linear") or EXECUTION_MODES[mode] or ("fp8_static" if "profile_path" in c else "fp8")
        self.linear = linear
        fp8_bank = "fp8_static" if "profile_path" in c else "fp8"
        self.lm_cfg, self.lm_w, self.vis_cfg, self.vis_w, self.meta = load_pretrained(path, mode=linear,
                                                                                      fp8_bank=fp8_bank)
        dims = (self.lm_cfg.layers, self.lm_cfg.hidden, self.vis_cfg.depth)
        if "expected_dimensions" in c and tuple(c["expected_dimensions"]) != dims:
            raise ValueError(f"checkpoint dimensions {dims} differ from the bundle's {tuple(c['expected_dimensions'])}")
        from tokenizers import Tokenizer
        self.tokenizer = Tokenizer.from_file(os.path.join(path, "tokenizer.json"))
        self.image_token = self.meta["image_token_id"]
        self.buckets = sorted({int(b) for b in c["buckets"]})
        self.max_tokens = self.buckets[-1]
        self.style = c.get("prompt_style", "short")
        self.variant = c.get("variant", "square256")
        self.profiles = profiles or {}
        self.warmup = warmup
        # the LM activations of every (canvas, bucket) step alias one region, the vision tower's
        # another (requests run one at a time); the tower's is sized per variant
        self.arena = Arena(Arena.size_for_buckets(self.lm_cfg, self.buckets, Runtime.path_for(self.lm_w)),
                           self.lm_w.embed.device)
        self.vision_arena = None
        self.geometry = {}   # canvas (h, w) -> prefix ids, image start, merged grid
        self.cache = {}      # (canvas, bucket) -> (ImageStep, pinned rgb, pinned ids, pinned pick, event)
        # every step shares the two arenas, so requests (refill, replay, read-back) are serialised
        self.lock = threading.RLock()
        if self.profiles:
            self.select(self.variant)

    # ------------------------------------------------------------ geometry

    def setup_side(self, side):
        """Prefix token ids (image placeholder expanded) and image placement of
        one canvas (height, width) in pixels; computed once per canvas."""
        side = (int(side[0]), int(side[1]))
        if side in self.geometry:
            return self.geometry[side]
        height, width = side
        if height % 32 or width % 32:
            raise ValueError("canvas sides must be multiples of 32")
        prefix, _ = text_parts(dict(instruction="fixture", candidates=["a", "b"]), self.style)
        tokens = self.tokenizer.encode(prefix, add_special_tokens=False).ids
        if tokens.count(self.image_token) != 1:
            raise ValueError("the prompt prefix must hold exactly one image placeholder token")
        at = tokens.index(self.image_token)
        mh, mw = height // 32, width // 32
        expanded = tokens[:at] + [self.image_token] * (mh * mw) + tokens[at + 1:]
        g = dict(prefix=np.asarray(expanded, dtype=np.int64), image_start=at, grid=(mh, mw))
        self.geometry[side] = g
        return g

    def positions(self, side, bucket):
        g = self.setup_side(side)
        return torch.from_numpy(mrope_positions(g["image_start"], *g["grid"], bucket))

    # ------------------------------------------------------------ requests

    def prepare(self, row):
        """Request row {'image_path', 'instruction', 'candidates'} -> graph
        inputs {'rgb', 'ids', 'pick', 'k', 'side', 'prompt'}."""
        rgb = row["rgb"] if "rgb" in row else decode_image(row["image_path"])
        image = prepare_image(rgb, self.variant)
        side = image.shape[:2]
        g = self.setup_side(side)
        prefix, suffix = text_parts(row, self.style)
        ids = self.tokenizer.encode(suffix, add_special_tokens=False).ids
        full = np.concatenate((g["prefix"], np.asarray(ids, dtype=np.int64)))
        if len(full) > self.max_tokens:
            raise ValueError(f"prompt of {len(full)} tokens exceeds the largest bucket ({self.max_tokens}); "
                             "text is never truncated")
        return dict(rgb=image, ids=full, pick=len(full) - 1, k=len(row["candidates"]), side=tuple(side),
                    prompt=prefix + suffix)

    def bucket_for(self, n):
        b = next((b for b in self.buckets if b >= n), None)
        if b is None:
            raise ValueError(f"{n} tokens exceed the largest bucket ({self.max_tokens})")
        return b

    def graph(self, g):
        """Option logits (first k, fp32 device tensor, a view of the step's
        static output: valid until the next request, so a caller on another
        thread reads it under ``lock``) of prepared inputs and whether this call
        captured the (canvas, bucket) step."""
        with self.lock:
            return self._graph(g)

    def _graph(self, g):
        n = len(g["ids"])
        bucket = self.bucket_for(n)
        key = (g["side"], bucket)
        captured = key not in self.cache
        if captured:
            geo = self.setup_side(g["side"])
            gh, gw = g["side"][0] // 16, g["side"][1] // 16
            if self.vision_arena is None:    # sized so that every canvas of the variant fits
                need = max(VisionRuntime.arena_bytes(self.vis_cfg, c[0] // 16, c[1] // 16)
                           for c in canvases(self.variant))
                self.vision_arena = Arena(need, self.lm_w.embed.device)
            st = ImageStep(self.lm_cfg, self.lm_w, self.vis_cfg, self.vis_w, gh, gw, bucket, geo["image_start"],
                           arena=self.arena, vision_arena=self.vision_arena)
            st.set_inputs(torch.from_numpy(g["rgb"]), torch.from_numpy(g["ids"]), self.positions(g["side"], bucket),
                          g["pick"])
            st.capture(warmup=self.warmup)
            ev = torch.cuda.Event()
            ev.record()
            self.cache[key] = (st, torch.zeros(tuple(g["rgb"].shape), dtype=torch.uint8, pin_memory=True),
                               torch.zeros(bucket, dtype=torch.int64, pin_memory=True),
                               torch.zeros(1, dtype=torch.int64, pin_memory=True), ev)
        st, srgb, sid, spick, ev = self.cache[key]
        ids = torch.from_numpy(np.asarray(g["ids"], dtype=np.int64))
        if int(ids.min()) < 0 or int(ids.max()) >= self.lm_cfg.vocab:
            raise ValueError("token id outside the vocabulary")
        if not 0 <= int(g["pick"]) < n:
            raise ValueError("pick must index a real token")
        ev.synchronize()     # the previous request's copies out of the pinned buffers are done
        srgb.copy_(torch.from_numpy(np.ascontiguousarray(g["rgb"])))
        sid.zero_()
        sid[:n].copy_(ids)
        spick[0] = int(g["pick"])
        st.vision.rgb.copy_(srgb, non_blocking=True)
        st.lm.ids.copy_(sid, non_blocking=True)
        st.lm.pick.copy_(spick, non_blocking=True)
        ev.record()
        z = st.replay()
        return z[:g["k"]], captured

    def predict(self, row):
        """Option logits (python floats) of one request row."""
        g = self.prepare(row)
        with self.lock:
            z, _ = self._graph(g)
            return z.float().cpu().tolist()

    # ------------------------------------------------------------ calibration

    def select(self, variant):
        """Canvas variant and, for static FP8 linears, its calibration bounds;
        captured steps are dropped (the activation multiplier is recorded at
        capture)."""
        with self.lock:
            from .prepare import VARIANTS
            if variant not in VARIANTS and variant not in self.profiles:
                raise ValueError(f"Unknown variant {variant!r}")
            torch.cuda.synchronize()
            if self.profiles:
                if variant not in self.profiles:
                    raise ValueError(f"Unknown calibration variant {variant!r}")
                from .profiles import apply_profile
                apply_profile(self.lm_w, self.profiles[variant])
            if variant in VARIANTS:
                self.variant = variant
            self.cache.clear()
            self.vision_arena = None      # re-sized for the new variant's canvases at the next capture

    def canvas_of(self, height, width):
        """The canvas (height, width) a height x width image gets under the
        current variant."""
        return canvas(height, width, self.variant)

