"""Request API over the gfx950 step: the reference's public surface
(api.py:9-99 -- ``sha256``, ``validate_request``, ``response``,
``Accelerator``) with the same argument meaning and error types.

What differs: this build has no vision encoder, tokenizer or checkpoint
loader, so a bundle names a Qwen3-VL LM shape and a linear format, the weights
are the seeded synthetic ones, and requests enter as token ids plus the image
block's place in the prompt (``predict_tokens``). ``predict`` keeps the
reference's validation and then raises, because turning an image and a
question into tokens is outside this build.

Bundle (JSON): ``{"schema_version": 1, "task": "visual_choice",
"architecture": "qwen3_vl_lm", "preset": "qwen3vl-8b", "linear": "fp8" |
"fp8_static" | "w4a16", "seed": 0, "tokens": 576, "image_grid": [16, 32],
"prefix_tokens": 4, "buckets": [576]}``; ``buckets`` (token buckets, each a
captured graph, as the reference's ``buckets`` config) defaults to
``[tokens]``. With ``linear: "fp8_static"`` a bundle may name a calibration
profile (``profile_path``, ``profile_sha256``, ``variant``), selected at
construction.
"""
import hashlib
import json
import math
import threading
from pathlib import Path

BACKENDS = ("fast", "native", "established")
LINEAR_MODES = ("fp8", "fp8_static", "w4a16")


def sha256(path):
    """Hex SHA-256 of a file, read in 1 MiB blocks (api.py:9-14)."""
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1024 * 1024), b""):
            h.update(block)
    return h.hexdigest()


def validate_request(image, question, candidates):
    """Request checks of api.py:17-25: the image file exists, the question is a
    nonempty string, two to eight nonempty string choices."""
    if not Path(image).is_file():
        raise FileNotFoundError(image)
    if not isinstance(question, str) or not question.strip():
        raise ValueError("A nonempty question is required")
    validate_candidates(candidates)


def validate_candidates(candidates):
    if not isinstance(candidates, (list, tuple)) or not 2 <= len(candidates) <= 8:
        raise ValueError("Provide two to eight choices")
    if any(not isinstance(x, str) or not x.strip() for x in candidates):
        raise ValueError("Choices must be nonempty strings")


def response(logits, candidates, item_id):
    """Response dict of api.py:28-34: argmax (first index on ties), softmax
    probabilities; non-finite or mismatched logits raise RuntimeError."""
    if len(logits) != len(candidates) or not all(math.isfinite(x) for x in logits):
        raise RuntimeError("Invalid model output")
    top = max(logits)
    prediction = max(range(len(logits)), key=lambda i: (logits[i], -i))
    exps = [math.exp(x - top) for x in logits]
    total = sum(exps)
    return dict(id=item_id, answer=dict(letter=chr(65 + prediction), text=candidates[prediction]),
                logits=list(logits), probabilities=[x / total for x in exps])


def read_bundle(bundle):
    """Parse and check a bundle file; ValueError for an unsupported schema,
    task, architecture, preset or linear format."""
    from .runtime import PRESETS
    c = json.loads(Path(bundle).read_text())
    if c.get("schema_version") != 1 or c.get("task") != "visual_choice":
        raise ValueError("Unsupported adaptation bundle schema or task")
    if c.get("architecture") != "qwen3_vl_lm":
        raise ValueError("No adapter registered for this architecture")
    if c.get("preset") not in PRESETS:
        raise ValueError(f"Unknown model preset {c.get('preset')!r}")
    if c.get("linear", "fp8") not in LINEAR_MODES:
        raise ValueError(f"Unknown linear format {c.get('linear')!r}")
    tokens = int(c.get("tokens", 576))
    gh, gw = c.get("image_grid", (16, 32))
    prefix = int(c.get("prefix_tokens", 4))
    if tokens <= 0 or gh < 0 or gw < 0 or prefix < 0 or prefix + gh * gw > tokens:
        raise ValueError("tokens must hold the prefix and the image grid")
    buckets = c.get("buckets", [tokens])
    if (not isinstance(buckets, list) or not buckets or any(not isinstance(b, int) for b in buckets)
            or min(buckets) < prefix + gh * gw):
        raise ValueError("buckets must be token counts that hold the prefix and the image grid")
    if "profile_path" in c:
        from .profiles import read_profiles
        if c.get("linear") != "fp8_static":
            raise ValueError("a calibration profile needs static FP8 linears (linear: fp8_static)")
        profiles = read_profiles(c["profile_path"], c.get("profile_sha256"))
        if c.get("variant") not in profiles:
            raise ValueError(f"Unknown calibration variant {c.get('variant')!r}")
    if "checkpoint" in c:
        if not Path(c["checkpoint"]).exists():
            raise FileNotFoundError(c["checkpoint"])
        if sha256(c["checkpoint"]) != c.get("checkpoint_sha256"):
            raise ValueError("Recovery checkpoint SHA256 mismatch")
    return c


class Accelerator:
    """One model on one MI355X, its step captured as a hipGraph.

    Instances serialise calls (one request at a time, as the reference's
    RLock does); graph buffers are never shared across instances. The first
    call captures the graph.
    """

    def __init__(self, bundle, *, backend="fast"):
        self.bundle = Path(bundle).resolve()
        c = read_bundle(self.bundle)
        if backend not in BACKENDS:
            raise ValueError("Unknown backend")
        if backend != "fast":
            raise RuntimeError(f"The {backend!r} backend is not part of this build; use 'fast'")
        from . import _lib
        _lib.check_device()      # exactly the gfx950 path; there is no CPU fallback
        from .graphs import StepGraphs
        from .runtime import PRESETS
        from .synthetic import OPTION_IDS, make_model
        self.config = c
        self.backend = backend
        self.lock = threading.RLock()
        self.cfg = PRESETS[c["preset"]]
        self.tokens = int(c.get("tokens", 576))
        self.grid = tuple(c.get("image_grid", (16, 32)))
        self.prefix_tokens = int(c.get("prefix_tokens", 4))
        self.weights = make_model(self.cfg, mode=c.get("linear", "fp8"), seed=int(c.get("seed", 0)),
                                  n_options=len(OPTION_IDS))
        self.buckets = sorted(set(c.get("buckets", [self.tokens])))
        self.graphs = StepGraphs(self.cfg, self.weights, self.buckets, self.grid, self.prefix_tokens)
        self.variant = None
        if "profile_path" in c:
            from .profiles import read_profiles
            self.profiles = read_profiles(c["profile_path"], c.get("profile_sha256"))
            self.select(c["variant"])

    def select(self, variant):
        """Switch the static FP8 activation bounds to calibration ``variant``
        (the reference's ``select``); graphs re-capture on their next request."""
        if variant not in getattr(self, "profiles", {}):
            raise ValueError(f"Unknown calibration variant {variant!r}")
        with self.lock:
            self.graphs.select(self.profiles[variant])
            self.variant = variant

    def predict(self, image, question, candidates, item_id="request", *, backend=None):
        """The reference's entry point: validated as there, then refused --
        image decoding, the prompt template and the vision encoder are not
        part of this build (use predict_tokens)."""
        validate_request(image, question, candidates)
        mode = self.backend if backend is None else backend
        if mode not in BACKENDS:
            raise ValueError("Unknown backend")
        raise RuntimeError("Image requests need the vision encoder and tokenizer, which this build "
                           "does not include; call predict_tokens with token ids")

    def predict_tokens(self, ids, candidates, item_id="request", *, pick=None):
        """Score ``candidates`` (2..8 strings, answer letters A.. in order) for a
        prompt of token ids (1-D int, at most the largest bucket long) whose
        image block sits after ``prefix_tokens`` tokens on the bundle's grid.
        ``pick`` is the scored row (default: the last token). The request runs
        in the smallest bucket that holds it; the bucket's first request
        captures its graph. Returns the response dict."""
        import torch
        validate_candidates(candidates)
        ids = torch.as_tensor(ids, dtype=torch.int64).reshape(-1)
        n = ids.numel()
        if n > self.buckets[-1]:
            raise ValueError(f"expected at most {self.buckets[-1]} token ids, got {n}")
        pick = n - 1 if pick is None else int(pick)
        with self.lock, torch.no_grad():
            z, _ = self.graphs.run(ids, pick, len(candidates))
            logits = z.cpu().tolist()
        return response(logits, list(candidates), item_id)

    def warmup(self, requests):
        for r in requests:
            self.predict_tokens(r["ids"], r["candidates"], r.get("item_id", "warmup"))
