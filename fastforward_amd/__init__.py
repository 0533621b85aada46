"""MI355X (gfx950) Qwen3-VL LM prefill + choice-score step.

Drop-in for FastForward's per-op API (``ops``: fast_norm, add_rms, qk_pair,
swiglu, attention_direct, lm_readout; ``linear``: FP8Linear, StaticFP8Linear,
RuntimeScaleLinear, Int4, Linear) and its ``Accelerator``/``predict`` request
API, on hand-written HIP kernels reached through the C ABI in include/ff_amd.h.
"""
__version__ = "0.1.0"


def __getattr__(name):
    if name == "Accelerator":
        from .api import Accelerator
        return Accelerator
    raise AttributeError(name)


__all__ = ["Accelerator"]
