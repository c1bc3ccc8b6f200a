"""Seeded random shapes through the default routing, against the CPU oracle.

The fixed-shape tests pin each kernel and route; this sweep draws dense,
contiguous and masked calls of random sizes (ragged M and N, K tails, empty and
one-row groups, masked_m from 0 to max_m) and runs them under a reduced CU
count (set_num_sms), so that the route choice and the persistent walks see many
tiles per workgroup at sizes the oracle finishes in about a second. Bars:
calc_diff < 1e-3; each written output within one BF16 ulp of the oracle plus
2^-14 of its absolute dot product sum_k |a_k b_k| (the FP8 MFMA's own
accumulation error, measured up to 1.5e-5 = 2^-16 of that sum inside one 128-K
block, so a bound in terms of the output's magnitude alone fails at K = 128);
unwritten rows keep the sentinel.
"""
import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'
SENTINEL = 0x7F7B


def _dev8(x):
    return gen.to_dev(x, torch.float8_e4m3fn)


def _f32(x):
    return gen.to_dev(np.asarray(x, dtype=np.float32))


def _sentinel(shape):
    return torch.full(shape, SENTINEL, dtype=torch.int16, device=DEV).view(torch.bfloat16)


def _check(name, out_t, ref, absdot, written):
    out = out_t.float().cpu().numpy().reshape(ref.shape)
    w = written.reshape(ref.shape[:-1]) if written is not None else np.ones(ref.shape[:-1], bool)
    diff = ogemm.calc_diff(out[w], ref[w]) if w.any() else 0.0
    print(f'[{name}] calc_diff={diff:.3e} rows={int(w.sum())}', flush=True)
    assert diff < 1e-3
    tol = np.abs(ref[w]) * 2.0 ** -8 + 2.0 ** -14 * absdot[w]
    assert np.all(np.abs(out[w] - ref[w]) <= tol)
    untouched = out_t.view(torch.int16).reshape(ref.shape)[torch.from_numpy(~w).to(out_t.device)]
    assert bool((untouched == SENTINEL).all())


def _draw_k(rng):
    # mostly whole 128-K blocks; sometimes a tail (K % 16 == 0 is the FP32-scale path's rule)
    return int(rng.integers(1, 13)) * 128 if rng.random() < 0.75 else int(rng.integers(1, 96)) * 16


@pytest.mark.parametrize('seed', range(8))
def test_random_dense(seed):
    rng = np.random.default_rng(1000 + seed)
    m, n, k = int(rng.integers(1, 1025)), int(rng.integers(1, 2049)), _draw_k(rng)
    num_sms = int(rng.choice([8, 16, 64]))
    print(f'random dense seed={seed} m={m} n={n} k={k} num_sms={num_sms}', flush=True)
    x = gen.dense_inputs(m, n, k, seed=2000 + seed)
    a, b = (_dev8(x['qa']), _f32(x['sfa'])), (_dev8(x['qb']), _f32(x['sfb']))
    old = deep_gemm.get_num_sms()
    try:
        deep_gemm.set_num_sms(num_sms)
        # D rows on a 16-byte pitch (the library's rule); ragged N leaves columns
        # past N in the pitch, which must keep the sentinel
        pitch = (n + 7) // 8 * 8
        d_full = _sentinel((m, pitch))
        d = d_full[:, :n]
        deep_gemm.fp8_gemm_nt(a, b, d)
        torch.cuda.synchronize()
        print(deep_gemm.get_last_config(), flush=True)
    finally:
        deep_gemm.set_num_sms(old)
    a_deq, b_deq = oquant.dequant_per_token(x['qa'], x['sfa']), oquant.dequant_per_block(x['qb'], x['sfb'])
    ref, absdot = ogemm.gemm_nt(a_deq, b_deq), ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq))
    _check(f'dense {m}x{n}x{k}', d.contiguous(), ref, absdot, None)
    assert bool((d_full[:, n:].contiguous().view(torch.int16) == SENTINEL).all())


@pytest.mark.parametrize('seed', range(8))
def test_random_contiguous(seed):
    rng = np.random.default_rng(3000 + seed)
    g = int(rng.integers(1, 9))
    ms = [int(v) for v in rng.integers(0, 700, size=g)]
    if g > 1:
        ms[int(rng.integers(0, g))] = int(rng.choice([0, 1]))   # an empty or one-row group
    n, k = int(rng.integers(1, 17)) * 128, _draw_k(rng)
    aligned = [(mi + 127) // 128 * 128 for mi in ms]
    if sum(aligned) == 0:
        ms[0], aligned[0] = 1, 128
    num_sms = int(rng.choice([8, 16, 64]))
    print(f'random contiguous seed={seed} ms={ms} n={n} k={k} num_sms={num_sms}', flush=True)
    x = gen.contiguous_inputs(ms, aligned, n, k, seed=4000 + seed)
    a, b = (_dev8(x['qa']), _f32(x['sfa'])), (_dev8(x['qb']), _f32(x['sfb']))
    layout = gen.to_dev(x['m_indices'])
    old = deep_gemm.get_num_sms()
    try:
        deep_gemm.set_num_sms(num_sms)
        d = _sentinel((sum(aligned), n))
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, b, d, layout)
        torch.cuda.synchronize()
        print(deep_gemm.get_last_config(), flush=True)
    finally:
        deep_gemm.set_num_sms(old)
    b_deq = np.stack([oquant.dequant_per_block(x['qb'][i], x['sfb'][i]) for i in range(g)])
    a_deq = oquant.dequant_per_token(x['qa'], x['sfa'])
    ref, written = ogemm.gemm_contiguous(a_deq, b_deq, x['m_indices'])
    absdot, _ = ogemm.gemm_contiguous(np.abs(a_deq), np.abs(b_deq), x['m_indices'])
    _check(f'contiguous g={g} n={n} k={k}', d, ref, absdot, written)


@pytest.mark.parametrize('seed', range(8))
def test_random_masked(seed):
    rng = np.random.default_rng(5000 + seed)
    g = int(rng.integers(1, 7))
    max_m = int(rng.choice([64, 256, 512, 1024]))
    n, k = int(rng.integers(1, 17)) * 128, int(rng.integers(1, 13)) * 128
    masked = [int(v) for v in rng.integers(0, max_m + 1, size=g)]
    masked[int(rng.integers(0, g))] = int(rng.choice([0, 1, max_m]))
    expected_m = int(rng.choice([16, 128, 200, max(1, max_m // 2)]))
    num_sms = int(rng.choice([8, 16, 64]))
    print(f'random masked seed={seed} g={g} max_m={max_m} masked_m={masked} expected_m={expected_m} n={n} k={k} '
          f'num_sms={num_sms}', flush=True)
    x = gen.masked_inputs(g, max_m, n, k, seed=6000 + seed)
    x['masked_m'][:] = masked
    a, b = (_dev8(x['qa']), _f32(x['sfa'])), (_dev8(x['qb']), _f32(x['sfb']))
    mm = gen.to_dev(x['masked_m'])
    old = deep_gemm.get_num_sms()
    try:
        deep_gemm.set_num_sms(num_sms)
        d = _sentinel((g, max_m, n))
        deep_gemm.m_grouped_fp8_gemm_nt_masked(a, b, d, mm, expected_m=expected_m)
        torch.cuda.synchronize()
        print(deep_gemm.get_last_config(), flush=True)
    finally:
        deep_gemm.set_num_sms(old)
    a_deq = np.stack([oquant.dequant_per_token(x['qa'][i], x['sfa'][i]) for i in range(g)])
    b_deq = np.stack([oquant.dequant_per_block(x['qb'][i], x['sfb'][i]) for i in range(g)])
    ref, written = ogemm.gemm_masked(a_deq, b_deq, x['masked_m'])
    absdot, _ = ogemm.gemm_masked(np.abs(a_deq), np.abs(b_deq), x['masked_m'])
    _check(f'masked g={g} max_m={max_m} n={n} k={k}', d, ref, absdot, written)
