"""Static-FP8 calibration profiles: the activation bounds of every static FP8
linear, per variant, and ``select`` of one of them.

Reference: the profile file read by ``activate_fast`` (_family/family_api.py:
28-30: ``read(profile_path)['profiles']``, checked against ``profile_sha256``)
and ``select(variant)`` (_family/depth_runtime.py:84-91,
_family/night_runtime.py:48-54), which gives each op of layer j and role r
``inverse_scale = 448/bound`` and ``input_scale <- bound/448`` for
``bound = profiles[variant]['j:r']``. Roles are the reference's pack roles:
``qkv``, ``output`` (o_proj), ``gateup``, ``down``.
"""
import json
from pathlib import Path

from .linear import StaticFP8Linear

# LayerWeights attribute -> the reference's profile role
ROLE_KEYS = {"qkv": "qkv", "o": "output", "gateup": "gateup", "down": "down"}


def read_profiles(path, sha256_hex=None):
    """{variant: {"j:role": bound}} from a profile file; with ``sha256_hex`` the
    file's digest must match (ValueError otherwise)."""
    from .api import sha256
    path = Path(path)
    if not path.exists():
        raise FileNotFoundError(path)
    if sha256_hex is not None and sha256(path) != sha256_hex:
        raise ValueError("Calibration profile SHA256 mismatch")
    data = json.loads(path.read_text())
    profiles = data.get("profiles") if isinstance(data, dict) else None
    if not isinstance(profiles, dict) or not profiles:
        raise ValueError("profile file has no 'profiles' mapping")
    for variant, bounds in profiles.items():
        if not isinstance(bounds, dict):
            raise ValueError(f"profile {variant!r} is not a mapping")
        for key, b in bounds.items():
            if not isinstance(b, (int, float)) or not b > 0:
                raise ValueError(f"profile {variant!r}: bound of {key!r} must be a positive number")
    return profiles


def apply_profile(weights, bounds):
    """Set every static FP8 linear of ``weights`` from ``bounds`` ({"j:role":
    bound}). ValueError if the model has no static FP8 linear, KeyError naming
    the first missing entry."""
    n = 0
    for j, layer in enumerate(weights.layers):
        for attr, role in ROLE_KEYS.items():
            op = getattr(layer, attr)
            if not isinstance(op, StaticFP8Linear):
                continue
            key = f"{j}:{role}"
            if key not in bounds:
                raise KeyError(f"calibration profile has no bound for {key}")
            op.set_bound(float(bounds[key]))
            n += 1
    if n == 0:
        raise ValueError("the model has no static FP8 linears to calibrate")
    return n


def model_parity(cfg, weights, ids, pos, pick, profiles=None):
    """``model_parity`` (_family/depth_fp8.py:40-62): one step of the
    reference's op sequence (the generic path) with the static FP8 linears of
    the middle layer (every role) and of the final layer (gate/up, down)
    observed, then ``linear.parity`` for each observed (op, activation) under
    every calibration variant of ``profiles`` ({variant: {"j:role": bound}};
    None: the ops' current scales). The ops' scales are restored afterwards.
    Returns the checks {role, variant, shape, inverse_scale, quant_bytes_exact,
    output_exact}; ``parity`` asserts each."""
    import torch
    from .linear import parity
    from .runtime import Runtime
    captured = {}

    class Observe:
        def __init__(self, op, key):
            self.op, self.key = op, key

        def __getattr__(self, name):
            return getattr(self.op, name)

        def __call__(self, x):
            captured[self.key] = (self.op, x.detach().clone())
            return self.op(x)

    layers = weights.layers
    mid, final = len(layers) // 2, len(layers) - 1
    originals = []
    for j in sorted({mid, final}):
        for attr, role in ROLE_KEYS.items():
            op = getattr(layers[j], attr)
            if isinstance(op, StaticFP8Linear) and (j == mid or role in ("gateup", "down")):
                originals.append((layers[j], attr, op))
                setattr(layers[j], attr, Observe(op, f"{j}:{role}"))
    try:
        rt = Runtime(cfg, weights, len(ids), path="generic")
        rt.set_inputs(ids, pos, pick)
        rt.step()
        torch.cuda.synchronize()
    finally:
        for layer, attr, op in originals:
            setattr(layer, attr, op)
    checks = []
    for key, (op, x) in captured.items():
        inverse, scale = op.inverse_scale, op.input_scale.clone()
        try:
            for name, bounds in (profiles or {"anchor": None}).items():
                if bounds is not None:
                    op.set_bound(float(bounds[key]))
                checks.append(dict(role=key, variant=name, **parity(op, x)))
        finally:
            op.inverse_scale = inverse
            op.input_scale.copy_(scale)
    return checks
