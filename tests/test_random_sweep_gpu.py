"""Seeded random sweep of the FP32-scale GEMM entry points against the FP64 oracle.

The fixed-shape parity tests vary one axis at a time; here every case draws its
own combination: the layout (dense, m-grouped contiguous, masked), M from 1 to
700 (so the tiny-M, weight-streaming and tiled kernels all run), N a multiple of
8 or 16, K a multiple of 128 or with a 16-byte K tail, BF16 or FP32 D with no C,
a separate C or C in place, K- or MN-major SFA, D as a view into a wider row
pitch, empty experts, and masked_m anywhere from 0 to max_m.

Bars: calc_diff < 1e-3 (the reference's, tests/generators.py:69-74); every
output within one BF16 ulp (FP32 D: 2^-22 relative) of the FP64 oracle plus an
accumulation term of 2^-15 x sum_k |a_mk b_nk| (+ |C|); cells outside the output
(padding rows, rows at or past masked_m, columns past N in a wider pitch) keep
their sentinel bits; a rerun is bitwise identical (tests/test_fp8_fp4.py:72-82).

The accumulation term is stated against sum |a b|, not |D|: the FP8 MFMA sums its
products at less than FP32 precision, which is why the recipe promotes to FP32
every 128 K. Measured on gfx950 (412 x 464, FP32 D, with and without C): the
largest error is 1.7e-3 at K = 256, on an output whose two K-block partial sums
are -3.7 and -8.2 and whose sum |a b| is 160 (2^-16.5 of it); FP32 additions of
the block's 128 products would stay below about 128 x 2^-24 x 16 = 1.2e-4. At
K = 2048 the largest is 2^-18.6 x sum |a b|. The bar leaves a factor of 2.8 over
the K = 256 figure.
"""
import random

import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'
S16 = 0x7F7B            # bf16 sentinel bits (a large finite value)
S32 = 0x7F7B7F7B        # f32 sentinel bits (finite)
N_DENSE, N_CONTIG, N_MASKED = 20, 10, 10


def _k(rnd, max_blocks):
    """A multiple of 128 (most cases) or of 16 (a K tail), at most max_blocks blocks."""
    if rnd.random() < 0.7:
        return 128 * rnd.randint(1, max_blocks)
    return 16 * rnd.randint(1, 8 * max_blocks)


def _sentinel(shape, f32):
    if f32:
        return torch.full(shape, S32, dtype=torch.int32, device=DEV).view(torch.float32)
    return torch.full(shape, S16, dtype=torch.int16, device=DEV).view(torch.bfloat16)


def _bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16)


def _untouched(t):
    return bool((_bits(t) == (S32 if t.dtype == torch.float32 else S16)).all())


def _sfa(sfa_np, mn_major):
    t = gen.to_dev(np.asarray(sfa_np, dtype=np.float32))
    return deep_gemm.get_mn_major_tma_aligned_tensor(t) if mn_major else t


def _check(name, out, ref, s_abs, f32):
    """`s_abs`: sum_k |a_mk b_nk| (+ |C_mn|) for every output, from the same oracle."""
    diff = ogemm.calc_diff(out, ref)
    rel = ogemm.max_rel_err(out, ref)
    acc = float((np.abs(out - ref) / np.maximum(s_abs, 1e-30)).max()) if out.size else 0.0
    print(f'[{name}] {deep_gemm.get_last_config()} calc_diff={diff:.3e} max_rel_err={rel:.3e} '
          f'max |err| / sum|ab| = 2^{np.log2(max(acc, 2.0 ** -60)):.1f}', flush=True)
    assert diff < 1e-3, diff
    tol = np.abs(ref) * (2.0 ** -22 if f32 else 2.0 ** -8) + 2.0 ** -15 * s_abs
    bad = np.abs(out - ref) > tol
    assert not bad.any(), f'{int(bad.sum())} outputs further from the FP64 oracle than the bound'


def _rerun_identical(call, d):
    first = d.clone()
    call()
    torch.cuda.synchronize()
    assert torch.equal(_bits(d), _bits(first)), 'rerun not bitwise identical'


@pytest.mark.parametrize('idx', range(N_DENSE))
def test_random_dense(idx):
    rnd = random.Random(7000 + idx)
    m = rnd.choice([rnd.randint(1, 16), rnd.randint(17, 64), rnd.randint(65, 700)])
    n = 8 * rnd.randint(1, 192)
    k = _k(rnd, 24)
    out = rnd.choice(['bf16', 'bf16+c', 'bf16+c=d', 'f32', 'f32+c', 'f32+c=d'])
    mn_major = rnd.random() < 0.5
    pad = 8 * rnd.randint(1, 4) if rnd.random() < 0.4 else 0
    print(f'random dense #{idx}: m={m} n={n} k={k} out={out} sfa_mn_major={mn_major} pitch_pad={pad}', flush=True)
    f32 = out.startswith('f32')
    x = gen.dense_inputs(m, n, k, seed=7000 + idx)
    c_np = gen.randn_bf16((m, n), 9500 + idx) if '+c' in out else None   # BF16 values: exact in either dtype
    a_deq, b_deq = oquant.dequant_per_token(x['qa'], x['sfa']), oquant.dequant_per_block(x['qb'], x['sfb'])
    ref = ogemm.gemm_nt(a_deq, b_deq, c_np)
    s_abs = ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq), None if c_np is None else np.abs(c_np))

    buf = _sentinel((m, n + pad), f32)
    d = buf[:, :n]
    c, c0 = None, None
    if c_np is not None:
        c0 = gen.to_dev(c_np.astype(np.float32)).to(torch.float32 if f32 else torch.bfloat16)
        c = d if out.endswith('=d') else c0
    a = (gen.to_dev(x['qa'], torch.float8_e4m3fn), _sfa(x['sfa'], mn_major))
    b = (gen.to_dev(x['qb'], torch.float8_e4m3fn), gen.to_dev(x['sfb']))

    def call():
        if c is d:
            d.copy_(c0)   # in place: D starts as C on every call
        deep_gemm.fp8_gemm_nt(a, b, d, c=c)

    call()
    torch.cuda.synchronize()
    _check(f'dense #{idx}', d.float().cpu().numpy(), ref, s_abs, f32)
    if pad:
        assert _untouched(buf[:, n:]), 'columns past N in the row pitch were written'
    _rerun_identical(call, d)


@pytest.mark.parametrize('idx', range(N_CONTIG))
def test_random_contiguous(idx):
    rnd = random.Random(8000 + idx)
    g = rnd.randint(1, 6)
    ms = [rnd.choice([0, rnd.randint(1, 64), rnd.randint(65, 400)]) for _ in range(g)]
    if not any(ms):
        ms[rnd.randrange(g)] = rnd.randint(1, 300)
    al = deep_gemm.get_mk_alignment_for_contiguous_layout()
    aligned = [(mi + al - 1) // al * al for mi in ms]
    n = 16 * rnd.randint(1, 48)
    k = _k(rnd, 12)
    mn_major = rnd.random() < 0.5
    print(f'random contiguous #{idx}: ms={ms} aligned={aligned} n={n} k={k} sfa_mn_major={mn_major}', flush=True)
    x = gen.contiguous_inputs(ms, aligned, n, k, seed=8000 + idx)
    a_deq = oquant.dequant_per_token(x['qa'], x['sfa'])
    b_deq = np.stack([oquant.dequant_per_block(x['qb'][i], x['sfb'][i]) for i in range(g)])
    ref, valid = ogemm.gemm_contiguous(a_deq, b_deq, x['m_indices'])
    s_abs, _ = ogemm.gemm_contiguous(np.abs(a_deq), np.abs(b_deq), x['m_indices'])
    a = (gen.to_dev(x['qa'], torch.float8_e4m3fn), _sfa(x['sfa'], mn_major))
    b = (gen.to_dev(x['qb'], torch.float8_e4m3fn), gen.to_dev(x['sfb']))
    mi = gen.to_dev(x['m_indices'])
    d = _sentinel((sum(aligned), n), False)

    def call():
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, b, d, mi)

    call()
    torch.cuda.synchronize()
    out = d.float().cpu().numpy()
    _check(f'contiguous #{idx}', out[valid], ref[valid], s_abs[valid], False)
    assert _untouched(d[torch.from_numpy(~valid).to(DEV)]), 'padding rows were written'
    _rerun_identical(call, d)


def _masked_inputs(masked_m, max_m, n, k, seed):
    """As generators.masked_inputs, for a given masked_m (SFA rows >= masked_m
    zeroed, as the reference's generators.py:476-478 does)."""
    g = len(masked_m)
    a = gen.randn_bf16((g, max_m, k), seed)
    b = gen.randn_bf16((g, n, k), seed + 1)
    qa = np.empty((g, max_m, k), dtype=np.uint8)
    sfa = np.empty((g, max_m, (k + 127) // 128), dtype=np.float32)
    qb = np.empty((g, n, k), dtype=np.uint8)
    sfb = np.empty((g, (n + 127) // 128, (k + 127) // 128), dtype=np.float32)
    for i in range(g):
        qa[i], sfa[i] = oquant.per_token_cast_to_fp8(a[i], use_ue8m0=False)
        qb[i], sfb[i] = oquant.per_block_cast_to_fp8(b[i], use_ue8m0=False)
        sfa[i, masked_m[i]:] = 0.0
    return qa, sfa, qb, sfb


@pytest.mark.parametrize('idx', range(N_MASKED))
def test_random_masked(idx):
    rnd = random.Random(9000 + idx)
    g = rnd.randint(1, 8)
    max_m = rnd.choice([16, 32, 64, 128, 192, 256, 320])
    masked_m = np.array([rnd.choice([0, max_m, rnd.randint(1, max_m), rnd.randint(1, max_m)]) for _ in range(g)],
                        dtype=np.int32)
    n = 16 * rnd.randint(1, 64)
    k = _k(rnd, 16)
    expected_m = rnd.randint(1, max_m)
    mn_major = rnd.random() < 0.5
    print(f'random masked #{idx}: masked_m={masked_m.tolist()} max_m={max_m} n={n} k={k} expected_m={expected_m} '
          f'sfa_mn_major={mn_major}', flush=True)
    qa, sfa, qb, sfb = _masked_inputs(masked_m, max_m, n, k, seed=9000 + idx)
    a_deq = np.stack([oquant.dequant_per_token(qa[i], sfa[i]) for i in range(g)])
    b_deq = np.stack([oquant.dequant_per_block(qb[i], sfb[i]) for i in range(g)])
    ref, valid = ogemm.gemm_masked(a_deq, b_deq, masked_m)
    s_abs, _ = ogemm.gemm_masked(np.abs(a_deq), np.abs(b_deq), masked_m)
    a = (gen.to_dev(qa, torch.float8_e4m3fn), _sfa(sfa, mn_major))
    b = (gen.to_dev(qb, torch.float8_e4m3fn), gen.to_dev(sfb))
    mm = gen.to_dev(masked_m)
    d = _sentinel((g, max_m, n), False)

    def call():
        deep_gemm.m_grouped_fp8_gemm_nt_masked(a, b, d, mm, expected_m=expected_m)

    call()
    torch.cuda.synchronize()
    out = d.float().cpu().numpy()
    if valid.any():
        _check(f'masked #{idx}', out[valid], ref[valid], s_abs[valid], False)
    assert _untouched(d[torch.from_numpy(~valid).to(DEV)]), 'rows at or past masked_m were written'
    _rerun_identical(call, d)
