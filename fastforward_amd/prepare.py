"""Host-side request preparation: canvas geometry, letterboxing and prompt text.

Restates the host steps in front of the graph (pure Python / numpy, no GPU
work):

* ``canvas`` / ``fit`` -- the canvas each image variant uses and the
  aspect-preserving fit inside it (_family/depth_geometry.py:7-22);
  ``canvases`` lists every canvas a variant can produce;
* ``decode_image`` / ``area_resize`` -- decode to RGB and the INTER_AREA
  resampling the reference does with cv2 (_family/depth_runtime.py:54-71);
* ``letterbox`` -- the image placed in a gray (128) canvas at the fitted
  offset, as ``prepare`` does for the aspect variants
  (_family/depth_runtime.py:66-70);
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


def canvases(variant):
    """Every (canvas height, canvas width) ``canvas`` can return for ``variant``."""
    if variant not in VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    side = 256 if variant.endswith("256") else 320
    if variant.startswith("square"):
        return [(side, side)]
    return sorted({(32 * h, 32 * w) for a, b in _PAIRS[side] for h, w in ((a, b), (b, a))})


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


def decode_image(path):
    """(h, w, 3) uint8 RGB of an image file. The reference decodes JPEG with
    imagecodecs, PNG with pyspng and anything else with PIL
    (_family/depth_runtime.py:55-65); PIL (libjpeg-turbo / zlib) decodes all
    three here."""
    from PIL import Image
    with Image.open(path) as im:
        rgb = np.array(im.convert("RGB"))
    if rgb.dtype != np.uint8 or rgb.ndim != 3 or rgb.shape[2] != 3 or 0 in rgb.shape:
        raise ValueError(f"could not decode {path} as an RGB image")
    return rgb


def _area_weights(n_in, n_out):
    """(n_out, n_in) coverage matrix of area resampling for n_out <= n_in: output
    pixel d covers source [d s, (d+1) s), s = n_in/n_out; each row sums to 1."""
    s = n_in / n_out
    w = np.zeros((n_out, n_in))
    for d in range(n_out):
        lo, hi = d * s, (d + 1) * s
        for i in range(int(np.floor(lo)), min(n_in, int(np.ceil(hi)))):
            w[d, i] = min(hi, i + 1) - max(lo, i)
    return w / s


def _area_linear_weights(n_in, n_out):
    """(n_out, n_in) interpolation matrix of area mode when the image grows on
    some axis: output d reads source s = floor(d n_in/n_out) and s + 1 with
    weight f = frac((d+1) - (s+1) n_out/n_in), f = 0 where that is <= 0 (pixel
    replication with a linear blend across source pixel edges)."""
    scale = n_in / n_out
    w = np.zeros((n_out, n_in))
    for d in range(n_out):
        s = int(np.floor(d * scale))
        f = (d + 1) - (s + 1) / scale
        f = 0.0 if f <= 0 else f - np.floor(f)
        if s >= n_in - 1:
            s, f = n_in - 1, 0.0
        w[d, s] += 1 - f
        if f:
            w[d, s + 1] += f
    return w


def area_resize(img, size):
    """``img`` (h, w, 3) uint8 resampled to ``size`` = (height, width) the way
    OpenCV's INTER_AREA is specified: when neither side grows, every output
    pixel is the coverage-weighted mean of the source pixels under it; when a
    side grows, area-mode linear weights (``_area_linear_weights``) on both
    axes. Separable, float64, rounded half to even. The reference calls
    cv2.resize(..., INTER_AREA) (_family/depth_runtime.py:70-71); cv2 is not
    part of this build and its fixed-point paths can differ by one level."""
    img = np.asarray(img)
    h, w = img.shape[:2]
    nh, nw = int(size[0]), int(size[1])
    if nh <= 0 or nw <= 0:
        raise ValueError("resize target must be positive")
    if (nh, nw) == (h, w):
        return img.astype(np.uint8, copy=True)
    weights = _area_weights if nh <= h and nw <= w else _area_linear_weights
    wy, wx = weights(h, nh), weights(w, nw)
    out = np.einsum("yh,hwc,xw->yxc", wy, img.astype(np.float64), wx, optimize=True)
    return np.clip(np.rint(out), 0, 255).astype(np.uint8)


def prepare_image(rgb, variant, resize=area_resize):
    """The canvas image of ``rgb`` for ``variant``: square variants resize to
    the canvas, aspect variants resize to the fitted size and letterbox.
    ``resize(image, (height, width)) -> uint8 image`` is the resampler
    (default ``area_resize``)."""
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
