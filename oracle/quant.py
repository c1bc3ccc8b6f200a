"""Caller-side quantizers restated in numpy (the GEMM's input contract).

TEST INFRASTRUCTURE: see ``oracle/__init__.py``.

Inputs are float32 arrays whose values are bfloat16-representable (the reference
draws ``randn`` in bf16 before casting, ``tests/generators.py:357-358``). Every
step is done in float32 with IEEE rounding, in the reference's order:

    amax = max|x| over the group, clamped below at 1e-4   (float32)
    sf   = amax * fl32(1 / 448) (or 1 / 6 for FP4)        (float32 product)
    sf   = ceil_to_ue8m0(sf)    when use_ue8m0
    q    = cast(x * (1 / sf))   (float32 reciprocal, float32 product, RNE cast)

The reference writes ``sf = amax / 448.0`` (``/ 6.0`` for FP4) and runs it on
the GPU. PyTorch's true-divide kernel for CUDA/ROCm, when the divisor is a
Python scalar, multiplies by the scalar's float32 reciprocal instead of
dividing, so the reference's scales are ``amax * fl32(1/448)``. That product
and the correctly rounded quotient differ by one ulp for about half of all
float32 amax values (torch on the CPU does divide, and gives the other one).
``scale_from_amax`` restates the GPU behaviour.
``tests/test_quant_pin_gpu.py`` pins it against torch's own ``amax / 448.0`` and
``/ 6.0`` on the GPU over 3.8e5 amax values, 1e5 of them values where the
two roundings differ, and pins the reciprocal and cast steps with the
reference's whole torch sequence on the GPU.

Functions and the reference lines they follow:

* ``per_token_cast_to_fp8``  -- ``deep_gemm/utils/math.py:26-49`` (1 x gran_k groups)
* ``per_block_cast_to_fp8``  -- ``deep_gemm/utils/math.py:62-72`` (gran_k x gran_k blocks)
* ``per_token_cast_to_fp4``  -- ``deep_gemm/utils/math.py:99-125`` (e2m1, packed 2/byte)
* ``bf16_round``             -- float32 -> bfloat16 RNE (as ``__float22bfloat162_rn``,
  ``impls/sm90_fp8_gemm_1d2d.cuh:415``)

Pinned by ``tests/test_oracle.py``: group invariants (the group maximum lands
exactly on +-448 / +-6 when sf is not rounded up, |q| <= 448, the reconstruction
error bound of half an e4m3 ulp), brute-force per-element recomputation on tiny
inputs, and bitwise agreement with torch's own float8_e4m3fn cast pipeline.
"""
import numpy as np

from . import fp8


E4M3_MAX = 448.0
E2M1_MAX = 6.0


def _align(x: int, y: int) -> int:
    return (x + y - 1) // y * y


def scale_from_amax(amax: np.ndarray, max_code: float) -> np.ndarray:
    """sf = amax / max_code as torch computes it on the GPU (``deep_gemm/utils/math.py:36,69,111``):
    amax times the float32 reciprocal of the Python scalar, one float32 rounding."""
    inv = np.float32(1.0) / np.float32(max_code)
    return (np.asarray(amax, dtype=np.float32) * inv).astype(np.float32)


def _recip_f32(sf: np.ndarray) -> np.ndarray:
    return (np.float32(1.0) / sf.astype(np.float32)).astype(np.float32)


def per_token_cast_to_fp8(x: np.ndarray, use_ue8m0: bool, gran_k: int = 128):
    """x [m, n] -> (e4m3 codes uint8 [m, n], sf float32 [m, ceil(n/gran_k)])."""
    x = np.asarray(x, dtype=np.float32)
    assert x.ndim == 2
    m, n = x.shape
    pn = _align(n, gran_k)
    xp = np.zeros((m, pn), dtype=np.float32)
    xp[:, :n] = x
    xv = xp.reshape(m, pn // gran_k, gran_k)
    amax = np.maximum(np.abs(xv).max(axis=2), np.float32(1e-4)).astype(np.float32)
    sf = scale_from_amax(amax, E4M3_MAX)
    if use_ue8m0:
        sf = fp8.ceil_to_ue8m0(sf)
    scaled = (xv * _recip_f32(sf)[:, :, None]).astype(np.float32)
    q = fp8.e4m3_encode(scaled).reshape(m, pn)[:, :n]
    return np.ascontiguousarray(q), sf


def per_block_cast_to_fp8(x: np.ndarray, use_ue8m0: bool, gran_k: int = 128):
    """x [m, n] -> (codes [m, n], sf float32 [ceil(m/g), ceil(n/g)])."""
    x = np.asarray(x, dtype=np.float32)
    assert x.ndim == 2
    m, n = x.shape
    pm, pn = _align(m, gran_k), _align(n, gran_k)
    xp = np.zeros((pm, pn), dtype=np.float32)
    xp[:m, :n] = x
    xv = xp.reshape(pm // gran_k, gran_k, pn // gran_k, gran_k)
    amax = np.maximum(np.abs(xv).max(axis=(1, 3)), np.float32(1e-4)).astype(np.float32)
    sf = scale_from_amax(amax, E4M3_MAX)
    if use_ue8m0:
        sf = fp8.ceil_to_ue8m0(sf)
    scaled = (xv * _recip_f32(sf)[:, None, :, None]).astype(np.float32)
    q = fp8.e4m3_encode(scaled).reshape(pm, pn)[:m, :n]
    return np.ascontiguousarray(q), sf


def per_token_cast_to_fp4(x: np.ndarray, use_ue8m0: bool, gran_k: int = 128):
    """x [m, n] -> (packed e2m1 uint8 [m, n/2], sf float32 [m, ceil(n/gran_k)])."""
    x = np.asarray(x, dtype=np.float32)
    m, n = x.shape
    assert n % 2 == 0
    pn = _align(n, gran_k)
    xp = np.zeros((m, pn), dtype=np.float32)
    xp[:, :n] = x
    xv = xp.reshape(m, pn // gran_k, gran_k)
    amax = np.maximum(np.abs(xv).max(axis=2), np.float32(1e-4)).astype(np.float32)
    sf = scale_from_amax(amax, E2M1_MAX)
    if use_ue8m0:
        sf = fp8.ceil_to_ue8m0(sf)
    scaled = (xv * _recip_f32(sf)[:, :, None]).astype(np.float32)
    codes = fp8.e2m1_encode(scaled).reshape(m, pn)
    packed = fp8.e2m1_pack(codes)[:, :n // 2]
    return np.ascontiguousarray(packed), sf


def dequant_per_token(q: np.ndarray, sf: np.ndarray, gran_k: int = 128) -> np.ndarray:
    """codes [.., m, k] with sf [.., m, ceil(k/g)] -> float32 (fp32 product)."""
    v = fp8.e4m3_decode(q)
    k = v.shape[-1]
    idx = np.arange(k) // gran_k
    return (v * sf[..., idx]).astype(np.float32)


def dequant_per_block(q: np.ndarray, sf: np.ndarray, gran: int = 128) -> np.ndarray:
    """codes [.., n, k] with sf [.., ceil(n/g), ceil(k/g)] -> float32."""
    v = fp8.e4m3_decode(q)
    n, k = v.shape[-2:]
    rows = np.arange(n) // gran
    cols = np.arange(k) // gran
    s = sf[..., rows, :][..., :, cols]
    return (v * s).astype(np.float32)


def dequant_fp4(packed: np.ndarray, sf: np.ndarray, gran_k: int) -> np.ndarray:
    """packed e2m1 [.., mn, k/2] with sf [.., mn, ceil(k/gran_k)] -> float32."""
    v = fp8.e2m1_decode(fp8.e2m1_unpack(packed))
    k = v.shape[-1]
    idx = np.arange(k) // gran_k
    return (v * sf[..., idx]).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32 values."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bfloat16 bit patterns (RNE)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)
