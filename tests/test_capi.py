"""CPU checks of the C ABI: the library loads without a GPU, exports every
function include/ff_amd.h declares, and the ctypes binding agrees with the
header on names and parameter counts. No compute call is made."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ff_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"(?:int64_t|int|const char\*)\s+(ff_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        n = 0 if params in ("", "void") else len(params.split(","))
        decls[m.group(1)] = n
    return decls


@pytest.fixture(scope="module")
def lib_path():
    from fastforward_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from fastforward_amd import build
        build.build(verbose=False)
    return _lib.LIB_PATH


def test_header_declares_entry_points():
    d = _declared()
    assert len(d) >= 24
    for name in ("ff_gemm_fp8", "ff_gemm_w4a16", "ff_attention_vt", "ff_add_rms", "ff_qk_pair",
                 "ff_swiglu", "ff_fast_norm", "ff_lm_readout"):
        assert name in d


def test_library_exports_every_declared_symbol(lib_path):
    lib = ctypes.CDLL(lib_path)
    for name in _declared():
        assert hasattr(lib, name), name


def test_binding_matches_header(lib_path):
    from fastforward_amd import _lib
    d = _declared()
    assert set(d) == set(_lib.SIGNATURES)
    for name, n in d.items():
        assert len(_lib.SIGNATURES[name]) == n, name
    lib = _lib.load()
    assert lib.ff_version() >= 100
    assert lib.ff_last_error() == b""


def test_tuning_knobs_validate_without_a_gpu(lib_path):
    """ff_set_tuning checks knob and value ranges on the host and never reads the
    environment; 0 restores the built-in choice."""
    from fastforward_amd import _lib
    _lib.load()
    _lib.call("ff_set_tuning", 3, 2)
    _lib.call("ff_set_tuning", 3, 0)
    with pytest.raises(RuntimeError, match="unknown knob"):
        _lib.call("ff_set_tuning", 99, 1)
    with pytest.raises(RuntimeError, match="out of range"):
        _lib.call("ff_set_tuning", 4, 9)
    text = "".join(open(os.path.join(ROOT, "fastforward_amd", "csrc", f)).read()
                   for f in os.listdir(os.path.join(ROOT, "fastforward_amd", "csrc")))
    assert "getenv" not in text


def test_w4a16_swiglu_shape_query_without_a_gpu(lib_path):
    """ff_gemm_w4a16_swiglu_fits answers on the host: m > 4 with i % 128 and k % 256,
    or m <= 4 with i % 16 and k % 128; a power-of-two group >= 32 dividing k."""
    import ctypes
    from fastforward_amd import _lib
    _lib.load()

    def fits(m, i, k, group):
        ok = ctypes.c_int(-1)
        _lib.call("ff_gemm_w4a16_swiglu_fits", m, i, k, group, ctypes.byref(ok))
        return ok.value

    assert fits(576, 12288, 4096, 128) == 1 and fits(320, 6144, 2048, 32) == 1 and fits(100, 640, 1024, 64) == 1
    assert fits(4, 12288, 4096, 128) == 1 and fits(1, 16, 128, 32) == 1  # the tail's rows: the packed GEMV
    assert fits(1, 8, 128, 32) == 0                # the GEMV takes 16-row blocks
    assert fits(576, 12288 + 64, 4096, 128) == 0   # i % 128
    assert fits(576, 12288, 4096 + 128, 128) == 0  # k % 256
    assert fits(576, 12288, 4096, 96) == 0         # group not a power of two


# (m, n, k, row tile, splits) the packed FP8 plain GEMM takes: the 8B down
# projection at the bucket sizes that pick 5 (64-row tiles, short m), 4, 3 and 2
# splits (k = 12288), the 176-token o projection on 64-row tiles split 5 ways
# (short m: 6 or 5 splits with uneven k ranges where 8, 4 or 2 do not fit: the
# 2B down at 250 tokens 6, the 4B o at 176 tokens 5; the 2B o at 176 tokens, 16
# k steps, keeps 4),
# splits of unequal length where k is not a multiple of 4 x splits x 128 (the
# 4B and 32B down projections, k = 9728 and 25600),
# unsplit grids and shapes left to the small tiles or the row-major kernels (0):
# at k = 8192 a split only where no small tile fills the GPU (the 32B o
# projection at 1024 and 576 tokens runs unsplit on small tiles).
# The plan is host code, so the workspace query pins it without a GPU.
PLAN_SHAPES = [(176, 4096, 12288, 64, 5), (576, 4096, 12288, 144, 4), (640, 4096, 12288, 144, 3),
               (1152, 4096, 12288, 144, 2), (300, 2048, 8192, 144, 8), (1000, 6144, 8192, 0, 0),
               (1024, 5120, 8192, 0, 0), (576, 5120, 8192, 0, 0),
               (576, 12288, 4096, 144, 1), (576, 4096, 4096, 0, 0), (176, 4096, 4096, 64, 5), (64, 2048, 2048, 64, 4),
               (250, 2048, 6144, 64, 6), (176, 2560, 2560, 64, 5), (176, 2048, 2048, 64, 4),
               (300, 4096, 2048, 0, 0), (3, 4096, 4096, 0, 0), (1024, 5120, 25600, 144, 3),
               (576, 2560, 9728, 144, 4), (576, 5120, 25600, 144, 3)]


@pytest.mark.parametrize("m,n,k,bm,splits", PLAN_SHAPES)
def test_fp8_pk_split_plan(lib_path, m, n, k, bm, splits):
    from fastforward_amd.linear import gemm_pk_workspace
    need = gemm_pk_workspace(m, n, k)
    assert need == ((m + bm - 1) // bm * (n // 256) * splits * bm * 256 * 4 if splits > 1 else 0)
