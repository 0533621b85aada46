"""Host-side request preparation: canvas geometry, letterboxing and prompt text.

Restates the host steps in front of the graph (pure Python / numpy, no GPU
work):

* ``canvas`` / ``fit`` -- the canvas each image variant uses and the
  aspect-preserving fit inside it (_family/depth_geometry.py:7-22);
* ``letterbox`` -- the image placed in a gray (128) canvas at the fitted
  offset, as ``prepare`` does for the aspect variants
  (_family/depth_runtime.py:66-70); the resize itself (cv2.resize with
  INTER_AREA in the reference) is the caller's, since OpenCV is not part of
  this build;
* ``text_parts`` -- the prompt prefix (up to and including the image
  placeholder) and the per-question suffix ending at the readout position
  (_legacy/sub10_runtime.py:43-49 and, for the 'standard' style,
  _legacy/vdm/models/prompts.py:31-62).

Token ids come from the model's tokenizer, which needs the model's assets;
``graphs.StepGraphs`` takes the resulting ids.
"""
import math

import numpy as np

VARIANTS = ("square256", "aspect256", "square320", "aspect320")

# Candidate (rows, cols) of 32-pixel merge blocks per canvas side; both
# orientations are allowed (_family/depth_geometry.py:13-14).
_PAIRS = {256: ((8, 8), (6, 10), (4, 16), (2, 32)),
          320: ((10, 10), (8, 12), (6, 16), (4, 24), (2, 50))}


def canvas(height, width, variant):
    """(canvas height, canvas width) in pixels for an image of height x width.
    'square*' variants use side x side; 'aspect*' variants pick the block grid
    whose aspect ratio is closest in log space to the image's, ties to the
    larger area, then to the smaller (rows, cols)."""
    if not (height > 0 and width > 0 and variant in VARIANTS):
        raise ValueError(f"bad canvas request {height}x{width} {variant!r}")
    side = 256 if variant.endswith("256") else 320
    if variant.startswith("square"):
        return side, side
    base = _PAIRS[side]
    pairs = sorted(set(base + tuple((w, h) for h, w in base)))
    target = height / width
    h, w = min(pairs, key=lambda p: (abs(math.log((p[0] / p[1]) / target)), -p[0] * p[1], p))
    return h * 32, w * 32


def fit(height, width, target):
    """(new height, new width, top, left) of an image scaled to fit inside
    ``target`` = (rows, cols) keeping its aspect ratio, centred."""
    h, w = target
    ratio = min(h / height, w / width)
    nh = min(h, max(1, round(height * ratio)))
    nw = min(w, max(1, round(width * ratio)))
    return nh, nw, (h - nh) // 2, (w - nw) // 2


def letterbox(resized, shape, top, left, fill=128):
    """``resized`` (nh, nw, 3) uint8 placed at (top, left) of a ``shape`` canvas
    filled with ``fill``."""
    resized = np.asarray(resized)
    if resized.dtype != np.uint8 or resized.ndim != 3 or resized.shape[2] != 3:
        raise ValueError("expected an (h, w, 3) uint8 image")
    nh, nw = resized.shape[:2]
    if top < 0 or left < 0 or top + nh > shape[0] or left + nw > shape[1]:
        raise ValueError("the image does not fit the canvas at that offset")
    out = np.full((shape[0], shape[1], 3), fill, dtype=np.uint8)
    out[top:top + nh, left:left + nw] = resized
    return out


def prepare_image(rgb, variant, resize):
    """The canvas image of ``rgb`` for ``variant``: square variants resize to
    the canvas, aspect variants resize to the fitted size and letterbox.
    ``resize(image, (height, width)) -> uint8 image`` is the caller's resampler."""
    rgb = np.asarray(rgb)
    height, width = rgb.shape[:2]
    shape = canvas(height, width, variant)
    if variant.startswith("aspect"):
        nh, nw, top, left = fit(height, width, shape)
        return letterbox(resize(rgb, (nh, nw)), shape, top, left)
    return np.asarray(resize(rgb, shape), dtype=np.uint8)


SYSTEM = ("You are a visual decision model. You inspect the image and answer each "
          "question by choosing exactly one of the given options. You never explain.")
IMAGE = "<|vision_start|><|image_pad|><|vision_end|>"


def _letters(n):
    if n > 26:
        raise ValueError("at most 26 options")
    return [chr(ord("A") + i) for i in range(n)]


def prefix_text(shared_context=""):
    """System turn, user turn opener, the image and any shared context."""
    ctx = f"\n{shared_context.strip()}" if shared_context.strip() else ""
    return f"<|im_start|>system\n{SYSTEM}<|im_end|>\n<|im_start|>user\n{IMAGE}{ctx}"


def suffix_text(instruction, options, qtype="choice"):
    """Per-question continuation ending at 'Answer:' (the readout position)."""
    lines = [f"\n\nQuestion: {instruction.strip()}"]
    if qtype == "claim":
        lines.append("Decide whether the statement above is:")
    lines.append("Options:")
    lines += [f"{c}. {o}" for c, o in zip(_letters(len(options)), options)]
    lines.append("Reply with the single letter of the correct option.")
    return "\n".join(lines) + "<|im_end|>\n<|im_start|>assistant\nAnswer:"


def text_parts(row, style="short"):
    """(prefix, suffix) of a request row {'instruction', 'candidates'} in the
    'short' (default), 'minimal' or 'standard' prompt style."""
    if style == "standard":
        return prefix_text(""), suffix_text(row["instruction"], row["candidates"], "choice")
    if style not in ("short", "minimal"):
        raise ValueError(f"unknown prompt style {style!r}")
    prefix = f"<|im_start|>user\n{IMAGE}"
    options = "\n".join(f"{c}. {x}" for c, x in zip(_letters(len(row["candidates"])), row["candidates"]))
    suffix = ("\n" + row["instruction"].strip() + "\nOptions:\n" + options +
              "\nReply with one letter.<|im_end|>\n<|im_start|>assistant\nAnswer:")
    if style == "minimal":
        suffix = suffix.replace("\nReply with one letter.", "")
    return prefix, suffix


def option_strings(n):
    """The strings whose first token scores each option (' A', ' B', ...)."""
    return [f" {c}" for c in _letters(n)]
