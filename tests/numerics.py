"""Independent numeric helpers for tests: bit-level bf16 / e4m3 in numpy.

These do not use torch's casts, so they can pin the oracle's use of them.
"""
import numpy as np


def bf16_round_np(x):
    """fp32 -> bf16 round-to-nearest-even by integer arithmetic; returns fp32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(x)
    out = np.where(nan, x, out)
    return out


def e4m3_table():
    """Values of all 256 OCP e4m3fn codes from the format definition
    (bias 7, 3 mantissa bits, subnormals at exponent 0, S.1111.111 = NaN)."""
    vals = np.zeros(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 7
        if e == 0xF and m == 7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[code] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return vals


_TABLE = e4m3_table()
_POS_CODES = np.arange(0, 0x7F)            # 0 .. 0x7E, finite non-negative
_POS_VALS = _TABLE[_POS_CODES]


def e4m3_encode_np(x):
    """Nearest e4m3fn code by exhaustive search over the finite codes, ties to the
    even code (even mantissa). Inputs must already be clamped to [-448, 448]."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    assert np.all(a <= 448.0)
    d = np.abs(a[..., None] - _POS_VALS[None, :])
    best = d.min(-1, keepdims=True)
    cand = d == best
    # among tied candidates prefer the even code
    even = (_POS_CODES % 2 == 0)[None, :]
    pick_even = cand & even
    has_even = pick_even.any(-1)
    code = np.where(has_even, pick_even.argmax(-1), cand.argmax(-1)).astype(np.uint8)
    # the sign bit is kept even when the magnitude rounds to zero (-0 code 0x80)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    return code | sign


def e4m3_decode_np(codes):
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def ulp_bf16(x):
    """bf16 unit in the last place at |x| (fp64)."""
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)
