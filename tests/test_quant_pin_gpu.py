"""Pins the oracle's quantizer arithmetic against torch on the GPU.

The reference quantizes with torch ops on the GPU (deep_gemm/utils/math.py:26-49,
62-72, 99-125): ``sf = x_amax / 448.0`` (``/ 6.0`` for FP4), then
``x * (1.0 / sf)`` cast to e4m3 (or the e2m1 boundary loop). The oracle
(oracle/quant.py) restates those steps in numpy. Its scale step is
``amax * fl32(1/448)``, a claim about torch's GPU division kernel (PyTorch's
true-divide with a Python-scalar divisor multiplies by the scalar's float32
reciprocal); the correctly rounded quotient, which torch on the CPU computes,
differs from it in the last bit for about half of all amax values. These tests
run torch's own GPU operations and compare bit patterns with the oracle:

  * the scale step over 3.8e5 amax values: every positive float32 exponent
    range the quantizers meet, values drawn from real bf16 groups, and 1e5
    values chosen where the correctly rounded quotient and the reciprocal
    product differ (so a wrong rounding choice cannot pass);
  * the reciprocal step ``1.0 / sf`` over the same scales;
  * the reference's whole per-token, per-block and FP4 sequences, written as the
    torch ops of deep_gemm/utils/math.py and run on the GPU, against the oracle's
    quantizers.
"""
import numpy as np
import pytest
import torch

from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'


def _amax_values():
    rng = np.random.default_rng(2024)
    lo = np.float32(1e-4).view(np.uint32)
    hi = np.float32(1e30).view(np.uint32)
    uniform_bits = rng.integers(lo, hi, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # amax of real 1x128 groups of bf16 randn (what the GEMM inputs see), at several scales
    x = gen.randn_bf16((1000, 128 * 20), 5).reshape(-1, 128)
    data = np.concatenate([np.abs(x).max(axis=1) * np.float32(s) for s in (1e-3, 1.0, 37.0, 1e4)])
    data = np.maximum(data, np.float32(1e-4)).astype(np.float32)
    return np.concatenate([uniform_bits, data])


def _disagreeing(max_code, count):
    """amax values whose correctly rounded quotient amax / max_code differs from
    fl32(amax * fl32(1 / max_code)). The float64 quotient rounded to float32 is
    the correctly rounded one: a float32 divided by 448 = 7 * 64 or 6 = 3 * 2 has
    a periodic binary expansion, so it never lies within 2^-53 of a float32
    rounding boundary and the double rounding is exact."""
    rng = np.random.default_rng(int(max_code))
    lo = np.float32(1e-4).view(np.uint32)
    hi = np.float32(1e30).view(np.uint32)
    out = []
    while sum(len(o) for o in out) < count:
        a = rng.integers(lo, hi, size=4 * count, dtype=np.uint64).astype(np.uint32).view(np.float32)
        cr = (a.astype(np.float64) / max_code).astype(np.float32)
        rm = (a * (np.float32(1.0) / np.float32(max_code))).astype(np.float32)
        out.append(a[cr.view(np.uint32) != rm.view(np.uint32)])
    return np.concatenate(out)[:count]


@pytest.mark.parametrize('max_code', [448.0, 6.0])
def test_scale_step_matches_torch_gpu_division(max_code):
    amax = np.concatenate([_amax_values(), _disagreeing(max_code, 100_000)])
    cr = (amax.astype(np.float64) / max_code).astype(np.float32)
    oracle = oquant.scale_from_amax(amax, max_code)
    n_differ = int((cr.view(np.uint32) != oracle.view(np.uint32)).sum())
    # torch on the GPU, exactly as the reference writes it: a float32 tensor / a Python float
    t = torch.from_numpy(amax).to(DEV) / max_code
    got = t.cpu().numpy()
    mism = got.view(np.uint32) != oracle.view(np.uint32)
    print(f'/ {max_code}: {amax.size} amax values, correctly rounded quotient differs from the '
          f'reciprocal product on {n_differ}; torch GPU vs oracle mismatches: {int(mism.sum())}', flush=True)
    assert n_differ >= 100_000          # the set discriminates between the two roundings
    assert not mism.any(), amax[mism][:8]


@pytest.mark.parametrize('max_code', [448.0, 6.0])
def test_reciprocal_step_matches_torch_gpu(max_code):
    sf = oquant.scale_from_amax(np.concatenate([_amax_values(), _disagreeing(max_code, 20_000)]), max_code)
    got = (1.0 / torch.from_numpy(sf).to(DEV)).cpu().numpy()
    want = oquant._recip_f32(sf)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _ref_per_token_fp8(x, use_ue8m0, gran_k=128):
    """deep_gemm/utils/math.py:26-49 as torch ops (the caller's tensor is bf16)."""
    m, n = x.shape
    pn = (n + gran_k - 1) // gran_k * gran_k
    xp = torch.zeros((m, pn), dtype=x.dtype, device=x.device)
    xp[:, :n] = x
    xv = xp.view(m, pn // gran_k, gran_k)
    amax = xv.abs().float().amax(dim=2).view(m, pn // gran_k).clamp(1e-4)
    sf = amax / 448.0
    if use_ue8m0:
        sf = _ref_ceil_to_ue8m0(sf)
    q = (xv * (1.0 / sf.unsqueeze(2))).to(torch.float8_e4m3fn).view(m, pn)[:, :n].contiguous()
    return q, sf


def _ref_ceil_to_ue8m0(x):
    """deep_gemm/utils/math.py:13-16 as torch ops."""
    bits = x.abs().float().view(torch.int)
    exp = ((bits >> 23) & 0xFF) + (bits & 0x7FFFFF).bool().int()
    return (exp.clamp(1, 254) << 23).view(torch.float)


def _ref_per_block_fp8(x, use_ue8m0, gran_k=128):
    """deep_gemm/utils/math.py:62-72 as torch ops."""
    m, n = x.shape
    pm, pn = (m + gran_k - 1) // gran_k * gran_k, (n + gran_k - 1) // gran_k * gran_k
    xp = torch.zeros((pm, pn), dtype=x.dtype, device=x.device)
    xp[:m, :n] = x
    xv = xp.view(-1, gran_k, pn // gran_k, gran_k)
    amax = xv.abs().float().amax(dim=(1, 3), keepdim=True).clamp(1e-4)
    sf = amax / 448.0
    if use_ue8m0:
        sf = _ref_ceil_to_ue8m0(sf)
    q = (xv * (1.0 / sf)).to(torch.float8_e4m3fn)
    return q.view_as(xp)[:m, :n].contiguous(), sf.view(xv.size(0), xv.size(2))


def _ref_per_token_fp4(x, use_ue8m0, gran_k):
    """deep_gemm/utils/math.py:84-125 as torch ops (the e2m1 boundary loop, two codes per byte)."""
    m, n = x.shape
    pn = (n + gran_k - 1) // gran_k * gran_k
    xp = torch.zeros((m, pn), dtype=x.dtype, device=x.device)
    xp[:, :n] = x
    xv = xp.view(m, -1, gran_k)
    amax = xv.abs().float().amax(dim=2).clamp_min(1e-4)
    sf = amax / 6.0
    if use_ue8m0:
        sf = _ref_ceil_to_ue8m0(sf)
    xs = xv * (1.0 / sf.unsqueeze(2))
    ax = xs.abs()
    code = torch.zeros_like(xs, dtype=torch.uint8)
    for boundary, round_up in zip((0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0),
                                  (False, True, False, True, False, True, False)):
        code += (ax >= boundary if round_up else ax > boundary).to(torch.uint8)
    sign = (xs < 0) & (code != 0)
    code = (code | (sign.to(torch.uint8) << 3)).view(m, pn)
    c2 = code.view(m, pn // 2, 2)
    packed = (c2[:, :, 0] & 0x0F) | ((c2[:, :, 1] & 0x0F) << 4)
    return packed[:, :n // 2].contiguous(), sf


@pytest.mark.parametrize('use_ue8m0', [False, True])
def test_reference_torch_sequences_on_gpu_match_oracle(use_ue8m0):
    # several magnitudes, ragged shapes (padding of the last group / block)
    for seed, (m, n), scale in [(1, (300, 7168), 1.0), (2, (129, 1000), 1e-3), (3, (64, 640), 3e3)]:
        a = gen.randn_bf16((m, n), seed) * np.float32(scale)
        a = torch.from_numpy(a).bfloat16().float().numpy()   # still bf16-representable after scaling
        x = torch.from_numpy(a).bfloat16().to(DEV)
        q, sf = _ref_per_token_fp8(x, use_ue8m0)
        oq, osf = oquant.per_token_cast_to_fp8(a, use_ue8m0=use_ue8m0)
        assert np.array_equal(sf.cpu().numpy().view(np.uint32), osf.view(np.uint32)), (seed, 'per-token sf')
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq), (seed, 'per-token codes')
        q, sf = _ref_per_block_fp8(x, use_ue8m0)
        oq, osf = oquant.per_block_cast_to_fp8(a, use_ue8m0=use_ue8m0)
        assert np.array_equal(sf.cpu().numpy().view(np.uint32), osf.view(np.uint32)), (seed, 'per-block sf')
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq), (seed, 'per-block codes')
        for gk in (32, 128):
            q, sf = _ref_per_token_fp4(x, use_ue8m0, gk)
            oq, osf = oquant.per_token_cast_to_fp4(a, use_ue8m0=use_ue8m0, gran_k=gk)
            assert np.array_equal(sf.cpu().numpy().view(np.uint32), osf.view(np.uint32)), (seed, gk, 'fp4 sf')
            assert np.array_equal(q.cpu().numpy().view(np.uint8), oq), (seed, gk, 'fp4 codes')
