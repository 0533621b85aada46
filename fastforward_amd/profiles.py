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
