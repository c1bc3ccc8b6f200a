"""Low-precision codecs from the format definitions (numpy only).

TEST INFRASTRUCTURE: see ``oracle/__init__.py``.

* OCP FP8 E4M3FN ("e4m3fn"): 1 sign, 4 exponent (bias 7), 3 mantissa bits, no
  infinities, S.1111.111 is NaN, largest finite 448. Subnormals are m/8 * 2^-6.
* OCP FP4 E2M1: 1 sign, 2 exponent (bias 1), 1 mantissa bit; magnitudes
  {0, .5, 1, 1.5, 2, 3, 4, 6}.
* UE8M0: an unsigned 8-bit biased exponent, value 2^(e-127).

Encoding is round-to-nearest, ties to the even code, which for a monotone
positive code table is "ties to the code whose mantissa LSB is 0". Magnitudes
in (448, 464] saturate to 448 and larger ones become NaN: that is what a
float32 -> float8_e4m3fn cast does (measured with torch 2.10 CPU; the tests pin
this module against that cast on every representable value and on midpoints).

Pinned by: ``tests/test_oracle.py::test_e4m3_table_*`` (closed-form values of
all 256 codes vs torch's float8_e4m3fn view), ``test_e4m3_encode_matches_torch``
(random + all midpoints), ``test_e2m1_*``, ``test_ue8m0_*``.
"""
import numpy as np

E4M3_MAX = 448.0


def _e4m3_code_value(code: int) -> float:
    """Value of one e4m3fn code from the field definition."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float('nan')
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


E4M3_TABLE = np.array([_e4m3_code_value(c) for c in range(256)], dtype=np.float64)
# Positive finite codes 0..126 are strictly increasing in value.
_E4M3_POS = E4M3_TABLE[:127].copy()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (exact: every e4m3 value is an fp32)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 values -> uint8 e4m3fn codes, RNE, overflow past 464 -> NaN code.

    Arithmetic form: the quantum of |x| is 2^(e-3) for the binade 2^e >= 2^-6 and
    2^-9 below it; |x| / quantum is exact, np.rint rounds it half-to-even, and
    the rounded multiple of the quantum is re-encoded from its own binade.
    ``e4m3_encode_table`` is an independent nearest-value search used to pin it.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x)
    neg = np.signbit(x)
    bits = a.view(np.int32)
    e = ((bits >> 23) & 0xFF).astype(np.int32) - 127          # binade of |x| (normal float32)
    e = np.maximum(e, -6)                                     # subnormal e4m3 share the 2^-9 quantum
    q = np.ldexp(np.float32(1.0), e - 3).astype(np.float32)
    r = (np.rint(a / q) * q).astype(np.float32)               # RNE to the e4m3 grid of the binade
    rb = r.view(np.int32)
    re = ((rb >> 23) & 0xFF).astype(np.int32) - 127
    normal = r >= np.float32(2.0 ** -6)
    mant = (rb >> 20) & 0x7                                    # top 3 mantissa bits
    code_n = ((re + 7) << 3) | mant
    code_s = np.rint(np.minimum(r, np.float32(1.0)) * np.float32(512.0)).astype(np.int32)  # subnormal: r = code * 2^-9
    code = np.where(normal, code_n, code_s)
    code = np.where((a > 464.0) | np.isnan(x), 0x7F, code).astype(np.uint8)
    return np.where(neg, code | np.uint8(0x80), code).astype(np.uint8)


def e4m3_encode_table(x: np.ndarray) -> np.ndarray:
    """Nearest-value search over the 127 positive codes (slow; pins ``e4m3_encode``)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    neg = np.signbit(x)
    hi = np.searchsorted(_E4M3_POS, a, side='left')          # first value >= a
    hi_c = np.minimum(hi, 126)
    lo_c = np.maximum(hi - 1, 0)
    lo_v, hi_v = _E4M3_POS[lo_c], _E4M3_POS[hi_c]
    d_lo, d_hi = a - lo_v, hi_v - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi_c % 2 == 0))
    code = np.where(pick_hi, hi_c, lo_c)
    code = np.where(a >= _E4M3_POS[126], 126, code)           # saturate region start
    code = code.astype(np.uint8)
    code = np.where(a > 464.0, np.uint8(0x7F), code)           # overflow -> NaN
    code = np.where(np.isnan(x), np.uint8(0x7F), code)
    code = np.where(neg, code | np.uint8(0x80), code)
    return code.astype(np.uint8)


# ---------------------------------------------------------------- FP4 E2M1
E2M1_POS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """4-bit codes (low nibble of uint8/int8) -> float32. -0 decodes to +0."""
    c = np.asarray(codes).astype(np.uint8) & 0xF
    v = E2M1_POS[c & 0x7]
    return np.where((c & 0x8) != 0, -v, v).astype(np.float32)


def e2m1_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> 4-bit codes (uint8), nearest with ties to even mantissa.

    Magnitudes above 6 saturate to 6; negative values that round to 0 get a +0
    code. Midpoints 0.25, 1.25, 2.5, 5.0 round down (to the even code) and
    0.75, 1.75, 3.5 round up, exactly as ``deep_gemm/utils/math.py:84-96``
    lists its boundaries.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    hi = np.searchsorted(E2M1_POS.astype(np.float64), a, side='left')
    hi_c = np.minimum(hi, 7)
    lo_c = np.maximum(hi - 1, 0)
    lo_v, hi_v = E2M1_POS[lo_c].astype(np.float64), E2M1_POS[hi_c].astype(np.float64)
    d_lo, d_hi = a - lo_v, hi_v - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi_c % 2 == 0))
    code = np.where(pick_hi, hi_c, lo_c)
    code = np.where(a >= 6.0, 7, code).astype(np.uint8)
    sign = (x < 0) & (code != 0)
    return (code | (sign.astype(np.uint8) << 3)).astype(np.uint8)


def e2m1_pack(codes: np.ndarray) -> np.ndarray:
    """[..., K] 4-bit codes -> [..., K/2] bytes; element 2i in the low nibble."""
    c = np.asarray(codes, dtype=np.uint8)
    assert c.shape[-1] % 2 == 0
    return ((c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)).astype(np.uint8)


def e2m1_unpack(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed).astype(np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = (p >> 4) & 0xF
    return out


# ---------------------------------------------------------------- UE8M0
def f32_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.int32)


def bits_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.int32).view(np.float32)


def ceil_to_ue8m0(x: np.ndarray) -> np.ndarray:
    """Smallest power of two >= |x| (as float32), exponent clamped to [1, 254].

    Restates ``deep_gemm/utils/math.py:13-16``: bump the biased exponent by one
    when any mantissa bit is set.
    """
    bits = f32_bits(np.abs(np.asarray(x, dtype=np.float32)))
    exp = ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0).astype(np.int32)
    return bits_f32(np.clip(exp, 1, 254).astype(np.int32) << 23)


def ue8m0_from_pow2_f32(x: np.ndarray) -> np.ndarray:
    """Power-of-two float32 -> UE8M0 byte (the biased exponent field)."""
    b = f32_bits(x)
    assert (b >= 0).all() and ((b & 0x7FFFFF) == 0).all(), 'SF must be a non-negative power of two'
    return ((b >> 23) & 0xFF).astype(np.uint8)


def ue8m0_to_f32(e: np.ndarray) -> np.ndarray:
    return bits_f32(np.asarray(e, dtype=np.uint8).astype(np.int32) << 23)
