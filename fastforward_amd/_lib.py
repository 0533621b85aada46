"""ctypes binding of the gfx950 C-ABI library ``libffamd.so`` (declared in include/ff_amd.h).

The library is loaded from this package directory; there is no fallback. A
missing library, a missing symbol or a non-gfx950 device raises.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libffamd.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
PI64 = ctypes.POINTER(ctypes.c_int64)
PI32 = ctypes.POINTER(ctypes.c_int)

# name -> argtypes (restype int unless noted); mirrors include/ff_amd.h
SIGNATURES = {
    "ff_version": [],
    "ff_last_error": [],
    "ff_device_check": [],
    "ff_set_tuning": [I32, I32],
    "ff_fast_norm": [P, P, P, I64, I64, F32, P],
    "ff_add_rms": [P, P, P, P, P, P, I64, I64, F32, I64, I64, P],
    "ff_add_rms_quant": [P, P, P, P, P, P, P, P, I64, I64, F32, I64, I64, P],
    "ff_fast_norm_quant": [P, P, P, P, P, I64, I64, F32, P],
    "ff_qk_pair": [P, P, I64, P, P, F32, F32, P, P, I64, I64, I64, I64, P, P, I64, I64, I64, I64, P],
    "ff_qkv_post": [P, P, P, I64, P, P, F32, F32, P, P, P, P, P, I64, I64, I64, I64, I64, P],
    "ff_v_transpose": [P, I64, I64, P, I64, I64, I64, I64, P],
    "ff_swiglu": [P, P, I64, P, I64, I64, P],
    "ff_swiglu_quant": [P, P, I64, P, P, P, I64, I64, P],
    "ff_attention_vt": [P, P, P, P, I32, P, I64, I64, I64, I64, I64, I64, F32, P],
    "ff_lm_readout": [P, P, P, P, P, I64, I64, F32, P],
    "ff_quant_rows_fp8": [P, I64, P, P, I64, I64, P],
    "ff_quant_static_fp8": [P, P, I64, I64, I64, F32, P],
    "ff_quant_weight_fp8": [P, P, P, P, I64, I64, I32, P],
    "ff_gemm_fp8": [P, P, I32, P, P, I32, P, I64, I64, I64, I64, P],
    "ff_gemm_fp8_swiglu": [P, P, P, P, P, I64, P, I64, I64, I64, P],
    "ff_pack_weight_fp8": [P, P, I64, I64, P],
    "ff_unpack_weight_fp8": [P, P, I64, I64, P],
    "ff_gemm_fp8_swiglu_pk": [P, P, P, P, P, P, I64, P, I64, I64, I64, P],
    "ff_gemm_fp8_pk_workspace": [I64, I64, I64, PI64],
    "ff_gemm_fp8_pk": [P, P, I32, P, P, P, I32, P, I64, I64, I64, I64, P, I64, P],
    "ff_gemm_fp8_pk_add_rms_quant": [P, P, I32, P, P, P, I32, P, I64, I64, I64, P, I64, P, P, P, P, P, P, F32, I64,
                                     I64, P],
    "ff_gemm_fp8_pk_add_rms_quant_static": [P, P, I32, P, P, P, I32, P, I64, I64, I64, P, I64, P, P, P, P, P, F32,
                                            F32, I64, I64, P],
    "ff_quant_rows_pmax": [P, I64, P, I64, P, P, I64, I64, P],
    "ff_gemm_fp8_qkv": [P, P, I32, P, P, I32, I64, I64, I64, I64, P, P, F32, F32, P, P, P, P, P, I64, P],
    "ff_gemm_fp8_qkv_pk": [P, P, I32, P, P, P, I32, I64, I64, I64, I64, P, P, F32, F32, P, P, P, P, P, I64, P],
    "ff_fast_norm_quant_static": [P, P, P, P, F32, I64, I64, F32, P],
    "ff_add_rms_quant_static": [P, P, P, P, P, P, P, F32, I64, I64, F32, I64, I64, P],
    "ff_attention_vt_q": [P, P, P, P, F32, I64, I64, I64, I64, I64, I64, F32, P],
    "ff_gemm_fp8_swiglu_static": [P, P, P, P, P, P, I64, F32, I64, I64, I64, P],
    "ff_quant_weight_int4": [P, P, P, I64, I64, I64, I32, P],
    "ff_gemm_w4a16": [P, I64, P, P, I64, P, I64, I64, I64, I64, P],
    "ff_gemm_w4a16_workspace": [I64, I64, I64, PI64],
    "ff_gemm_w4a16_ws": [P, I64, P, P, I64, P, I64, I64, I64, I64, P, I64, P],
    "ff_gemm_w4a16_noalloc": [P, I64, P, P, I64, P, I64, I64, I64, I64, P],
    "ff_pack_weight_int4": [P, P, I64, I64, P],
    "ff_pack_scales_int4": [P, P, I64, I64, I64, P],
    "ff_gemm_w4a16_pk_workspace": [I64, I64, I64, I64, PI64],
    "ff_gemm_w4a16_pk": [P, I64, P, P, P, P, I64, P, I64, I64, I64, I64, P, I64, P],
    "ff_gemm_w4a16_pk_add_rms": [P, I64, P, P, P, P, I64, P, I64, I64, I64, P, I64, P, P, P, P, P, F32, I64, I64, P],
    "ff_gemm_w4a16_swiglu_fits": [I64, I64, I64, I64, PI32],
    "ff_gemm_w4a16_swiglu_pk": [P, I64, P, P, I64, P, I64, I64, I64, I64, P],
    "ff_gemm_w4a16_qkv_workspace": [I64, I64, I64, I64, I64, PI64],
    "ff_gemm_w4a16_qkv": [P, I64, P, P, I64, I64, I64, I64, I64, P, P, F32, F32, P, P, P, P, P, I64, P, I64, P],
    "ff_embed": [P, P, P, I64, I64, I64, P],
    "ff_gather_rows": [P, I64, P, P, I64, I64, I64, I64, P],
    "ff_scatter_rows": [P, P, I64, I64, I64, P],
    "ff_mrope_cos_sin": [P, P, P, P, I64, I64, I32, I32, P],
    "ff_pack_pixels": [P, P, I64, I64, P],
    "ff_layer_norm": [P, I64, P, P, P, I64, I64, I64, F32, P],
    "ff_gemm_bf16": [P, I64, P, P, P, I64, P, I64, I64, I64, I64, I32, P],
    "ff_pack_weight_bf16": [P, P, I64, I64, P],
    "ff_gemm_bf16_pk": [P, I64, P, P, P, P, I64, P, I64, I64, I64, I64, I32, P],
    "ff_gemm_bf16_pk_workspace": [I64, I64, I64, PI64],
    "ff_gemm_bf16_pk_ws": [P, I64, P, P, P, P, I64, P, I64, I64, I64, I64, I32, P, I64, P],
    "ff_gemm_bf16_pk_ln": [P, I64, P, P, P, P, I64, P, I64, I64, I64, I64, P, I64, P, P, F32, P, I64, P],
    "ff_vision_rope": [P, P, I64, I64, P, P, P, P, I64, I64, I64, I64, I64, I64, P],
    "ff_vision_vt": [P, I64, I64, P, I64, I64, I64, I64, P],
    "ff_attention_full": [P, P, P, P, I64, I64, I64, I64, F32, P],
    "ff_pos_interp": [P, P, P, P, I64, I64, I64, I64, P],
    "ff_vision_qkv": [P, P, P, P, P, P, I64, I64, I64, I64, P],
}

_lib = None


def load():
    """Load the library (once) and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m fastforward_amd.build` "
                           "(there is no CPU or PyTorch fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "ff_last_error" else ctypes.c_int
    _lib = lib
    return lib


def check_device():
    """Raise unless the current torch device is a gfx950 GPU."""
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU visible; the gfx950 kernels have no CPU fallback")
    lib = load()
    torch.cuda.current_device()
    st = lib.ff_device_check()
    if st != 0:
        raise RuntimeError(lib.ff_last_error().decode())


def call(name, *args):
    """Call a C-ABI entry point; a nonzero status raises RuntimeError with the message."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        raise RuntimeError(f"{name} failed ({st}): {lib.ff_last_error().decode()}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    """The current torch stream as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
