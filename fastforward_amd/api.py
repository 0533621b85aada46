"""Request API over the gfx950 step: the reference's public surface
(api.py:9-99 -- ``sha256``, ``validate_request``, ``response``,
``Accelerator``) with the same argument meaning and error types.

Two bundle architectures:

* ``"qwen3_vl_family"`` -- the reference's: a local Qwen3-VL checkpoint
  directory (``model``: config.json, safetensors, tokenizer.json) served by
  ``family.FamilyRuntime``: ``predict(image, question, candidates)`` decodes the
  image, fits it to the variant's canvas, builds the prompt, runs the vision
  tower + LM step as one hipGraph per (canvas, token bucket) and answers.
  Keys as the reference's bundles: ``buckets``, ``variant``, ``prompt_style``,
  ``execution_mode``, ``expected_dimensions``, ``checkpoint`` +
  ``checkpoint_sha256`` (the repair adapter; only the identity -- all-zero --
  adapter the reference's family runtime accepts), ``profile_path`` +
  ``profile_sha256`` (static FP8 calibration), plus ``linear`` to pick the
  linear format ('fp8' per-token dynamic, 'fp8_static', 'w4a16', 'int4').
* ``"qwen3_vl_lm"`` -- synthetic weights of a named LM preset, requests as
  token ids (``predict_tokens``): ``{"schema_version": 1, "task":
  "visual_choice", "architecture": "qwen3_vl_lm", "preset": "qwen3vl-8b",
  "linear": "fp8" | "fp8_static" | "w4a16", "seed": 0, "tokens": 576,
  "image_grid": [16, 32], "prefix_tokens": 4, "buckets": [576]}``;
  ``buckets`` defaults to ``[tokens]``. With ``linear: "fp8_static"`` a bundle
  may name a calibration profile (``profile_path``, ``profile_sha256``,
  ``variant``), selected at construction.
"""
import hashlib
import json
import math
import threading
from pathlib import Path

BACKENDS = ("fast", "native", "established")
LINEAR_MODES = ("fp8", "fp8_static", "w4a16", "int4")
ARCHITECTURES = ("qwen3_vl_lm", "qwen3_vl_family")


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
    task, architecture, preset or linear format, FileNotFoundError for a
    missing model, checkpoint or profile."""
    c = json.loads(Path(bundle).read_text())
    if c.get("schema_version") != 1 or c.get("task") != "visual_choice":
        raise ValueError("Unsupported adaptation bundle schema or task")
    if c.get("architecture") not in ARCHITECTURES:
        raise ValueError("No adapter registered for this architecture")
    if c.get("linear", "fp8") not in LINEAR_MODES:
        raise ValueError(f"Unknown linear format {c.get('linear')!r}")
    if c["architecture"] == "qwen3_vl_family":
        if "model" not in c or not Path(c["model"]).exists():
            raise FileNotFoundError(c.get("model"))
        buckets = c.get("buckets")
        if (not isinstance(buckets, list) or not buckets
                or any(not isinstance(b, int) or b <= 0 for b in buckets)):
            raise ValueError("buckets must be a list of positive token counts")
    else:
        from .runtime import PRESETS
        if c.get("preset") not in PRESETS:
            raise ValueError(f"Unknown model preset {c.get('preset')!r}")
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
        if c.get("linear", "fp8_static" if c["architecture"] == "qwen3_vl_family" else "fp8") != "fp8_static":
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


def check_identity_repair(path):
    """The family runtime's repair adapter must be the identity: its 'up' and
    'bias' tensors all zero (_family/family_api.py:21-23). Loaded with
    weights_only=True (no code from the file runs)."""
    import torch
    state = torch.load(path, map_location="cpu", weights_only=True)
    state = state.get("state_dict", state) if isinstance(state, dict) else None
    if not isinstance(state, dict) or "up" not in state or "bias" not in state:
        raise ValueError("repair checkpoint has no state_dict with 'up' and 'bias'")
    if bool(torch.count_nonzero(state["up"])) or bool(torch.count_nonzero(state["bias"])):
        raise ValueError("only the identity (all-zero) repair adapter is supported")


class Accelerator:
    """One model on one MI355X, its step captured as a hipGraph.

    Instances serialise calls (one request at a time, as the reference's
    RLock does); graph buffers are never shared across instances. The first
    request of each (canvas, bucket) captures its graph.
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
        self.config = c
        self.backend = backend
        self.lock = threading.RLock()
        self.variant = None
        self.profiles = {}
        if "profile_path" in c:
            from .profiles import read_profiles
            self.profiles = read_profiles(c["profile_path"], c.get("profile_sha256"))
        if c["architecture"] == "qwen3_vl_family":
            if "checkpoint" in c:
                check_identity_repair(c["checkpoint"])
            from .family import FamilyRuntime
            self.runtime = FamilyRuntime(c, profiles=self.profiles)
            self.variant = self.runtime.variant
            return
        self.runtime = None
        from .graphs import StepGraphs
        from .runtime import PRESETS
        from .synthetic import OPTION_IDS, make_model
        self.cfg = PRESETS[c["preset"]]
        self.tokens = int(c.get("tokens", 576))
        self.grid = tuple(c.get("image_grid", (16, 32)))
        self.prefix_tokens = int(c.get("prefix_tokens", 4))
        self.weights = make_model(self.cfg, mode=c.get("linear", "fp8"), seed=int(c.get("seed", 0)),
                                  n_options=len(OPTION_IDS))
        self.buckets = sorted(set(c.get("buckets", [self.tokens])))
        self.graphs = StepGraphs(self.cfg, self.weights, self.buckets, self.grid, self.prefix_tokens)
        if self.profiles:
            self.select(c["variant"])

    def select(self, variant):
        """Switch to calibration ``variant`` (the reference's ``select``): its
        static FP8 activation bounds and, for image bundles, its canvas policy;
        graphs re-capture on their next request."""
        with self.lock:
            if self.runtime is not None:
                self.runtime.select(variant)
            else:
                if variant not in self.profiles:
                    raise ValueError(f"Unknown calibration variant {variant!r}")
                self.graphs.select(self.profiles[variant])
            self.variant = variant

    def predict(self, image, question, candidates, item_id="request", *, backend=None):
        """The reference's entry point (api.py:71-80): validate, answer, respond.
        Image bundles run the whole request; token-level bundles have no
        tokenizer or vision weights and refuse (use predict_tokens)."""
        validate_request(image, question, candidates)
        mode = self.backend if backend is None else backend
        if mode not in BACKENDS:
            raise ValueError("Unknown backend")
        if mode != "fast":
            raise RuntimeError(f"The {mode!r} backend is not part of this build; use 'fast'")
        if self.runtime is None:
            raise RuntimeError("This bundle serves token ids only (architecture qwen3_vl_lm); "
                               "call predict_tokens, or use a qwen3_vl_family bundle for image requests")
        import torch
        row = dict(image_path=str(image), instruction=question, candidates=list(candidates), item_id=item_id)
        with self.lock, torch.no_grad():
            logits = self.runtime.predict(row)
        return response(logits, list(candidates), item_id)

    def predict_tokens(self, ids, candidates, item_id="request", *, pick=None):
        """Score ``candidates`` (2..8 strings, answer letters A.. in order) for a
        prompt of token ids (1-D int, at most the largest bucket long) whose
        image block sits after ``prefix_tokens`` tokens on the bundle's grid.
        ``pick`` is the scored row (default: the last token). The request runs
        in the smallest bucket that holds it; the bucket's first request
        captures its graph. Returns the response dict."""
        import torch
        if self.runtime is not None:
            raise RuntimeError("image bundles take image requests (predict)")
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
        """Run requests to capture their graphs ahead of time: image rows
        ({'image_path', 'instruction', 'candidates'}) for image bundles, token
        rows ({'ids', 'candidates'}) otherwise."""
        for r in requests:
            if self.runtime is not None:
                self.predict(r["image_path"], r["instruction"], r["candidates"], r.get("item_id", "warmup"))
            else:
                self.predict_tokens(r["ids"], r["candidates"], r.get("item_id", "warmup"))

    def activate_fast(self):
        """The reference converts a bf16 instance to FP8 here; this build
        quantises at load, so this only reports the resident linear format."""
        with self.lock:
            self.backend = "fast"
            linear = self.runtime.linear if self.runtime is not None else self.config.get("linear", "fp8")
            return dict(linear=linear, runtime_activation_scale=linear == "fp8_static")
