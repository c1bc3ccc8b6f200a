"""Parity at the reference's own test shapes (tests/generators.py:121-216 of the
reference), run at their full sizes on the GPU.

* dense (enumerate_normal, generators.py:121-174, as the FP8 path runs it):
  forward M in {1, 128, 4096} over the seven (N, K) of bf16_output_nk; backward
  at M = 4096: Dgrad (M, K, N) with BF16 out, Wgrad (N, M, K) through the 1D1D
  recipe accumulating into FP32 C, and Wgrad with BF16 out (per-block B);
* m-grouped contiguous (generators.py:190-202, 378-413): (G, m) in {(4, 8192),
  (8, 4096)} over four (N, K), segment sizes int(m * U(0.7, 1.3)) aligned to
  the M alignment, in the m_indices and the psum layout;
* m-grouped masked (generators.py:205-216, 447-485): max_m = 4096, (G, m) in
  {(32, 192), (6, 1024), (32, 20), (6, 20)} over the same four (N, K), masked_m =
  int(m * U(0.7, 1.3)), expected_m = int(1.2 m) (tests/test_fp8_fp4.py:187), in the
  masked layout and through the psum layout of the contiguous GEMM.

Inputs are random on the device (a seeded device generator), rounded to bf16 and
quantized by the product quantizers, which other tests pin bit for bit to the
oracle. Checks per case: a seeded sample of rows x columns against the FP64
oracle (calc_diff < 1e-3, the reference's FP8 bar, and the elementwise bound of
one output ulp plus 2^-15 x sum |a b|, the FP8 MFMA's accumulation error as
tests/test_random_sweep_gpu.py measures it), every output that must be written
is written and every row that must not be is left alone (sentinel), one expert
equal to a dense call on its rows, and bitwise-identical reruns (the reference
runs 20, tests/test_fp8_fp4.py:81-85,141-144).
"""
import random

import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'
SENTINEL = 0x7F7B
SAMPLE_ROWS = 192
SAMPLE_COLS = 768
RERUNS = 20

BF16_NK = [(2112, 7168), (576, 7168), (24576, 1536), (32768, 512), (7168, 16384), (4096, 7168), (7168, 2048)]
GROUPED_NK = [(6144, 7168), (7168, 3072), (4096, 4096), (4096, 2048)]


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def sentinel_bf16(shape):
    return torch.full(shape, SENTINEL, dtype=torch.int16, device=DEV).view(torch.bfloat16)


def randn_bf16(shape, gen):
    return torch.randn(shape, generator=gen, device=DEV, dtype=torch.float32).bfloat16()


def dev_gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def quant_a(x):
    return deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=False)


def quant_b(x):
    return deep_gemm.per_block_cast_to_fp8(x, use_ue8m0=False)


def pick(n, must, count, rng):
    must = [v for v in must if 0 <= v < n]
    extra = rng.choice(n, size=min(n, max(0, count - len(must))), replace=False)
    return np.unique(np.concatenate([np.asarray(must, dtype=np.int64), extra.astype(np.int64)]))


def edge_cols(n):
    return [0, 1, 127, 128, 255, 256, n // 2, n - 2, n - 1]


def oracle_sample(a, b, rows, cols, b_per_block=True, c=None):
    """FP64 oracle of D[rows][:, cols] from the codes and scales on the device, and
    sum_k |a b| (+ |C|) of the same outputs. Per-block B scales are the per-row
    scales of their 128-row block."""
    r = torch.from_numpy(rows).to(DEV)
    cc = torch.from_numpy(cols).to(DEV)
    a_deq = oquant.dequant_per_token(u8(a[0][r]), a[1][r].cpu().numpy())
    sfb = b[1][cc // 128] if b_per_block else b[1][cc]
    b_deq = oquant.dequant_per_token(u8(b[0][cc]), sfb.cpu().numpy())
    c_s = None if c is None else c[r][:, cc].cpu().numpy()
    return (ogemm.gemm_nt(a_deq, b_deq, c_s),
            ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq), None if c_s is None else np.abs(c_s)))


def check(name, out, ref, s_abs, out_f32=False):
    diff = ogemm.calc_diff(out, ref)
    rel = ogemm.max_rel_err(out, ref)
    acc = float((np.abs(out - ref) / np.maximum(s_abs, 1e-30)).max())
    print(f'[{name}] sample={out.shape} calc_diff={diff:.3e} max_rel_err={rel:.3e} '
          f'max |err| / sum|ab| = 2^{np.log2(max(acc, 2.0 ** -60)):.1f}', flush=True)
    assert diff < 1e-3, diff
    tol = np.abs(ref) * (2.0 ** -22 if out_f32 else 2.0 ** -8) + 2.0 ** -15 * s_abs
    bad = np.abs(out - ref) > tol
    assert not bad.any(), f'{int(bad.sum())} sampled outputs further from the FP64 oracle than the bound'


def rerun_identical(call, d, view=torch.int16):
    first = d.clone()
    for _ in range(RERUNS):
        call()
    torch.cuda.synchronize()
    assert torch.equal(d.view(view), first.view(view)), 'reruns not bitwise identical'


# ------------------------------------------------------------------ dense

def _dense_cases():
    cases = []
    for m in (1, 128, 4096):
        for n, k in BF16_NK:
            cases.append(('fwd', m, n, k))
    for n, k in BF16_NK:
        cases.append(('dgrad', 4096, k, n))
        cases.append(('wgrad_f32', n, 4096, k))
        cases.append(('wgrad_bf16', n, 4096, k))
    return cases


@pytest.mark.parametrize('kind,m,n,k', _dense_cases())
def test_reference_dense_shape(kind, m, n, k):
    print(f'reference dense {kind} M={m} N={n} K={k}', flush=True)
    seed = m * 7 + n * 3 + k
    gen = dev_gen(seed)
    rng = np.random.default_rng(seed)
    a = quant_a(randn_bf16((m, k), gen))
    one_d = kind == 'wgrad_f32'
    b = quant_a(randn_bf16((n, k), gen)) if one_d else quant_b(randn_bf16((n, k), gen))
    if one_d:
        c = torch.randn((m, n), generator=gen, device=DEV, dtype=torch.float32)
        d = torch.full((m, n), float('nan'), device=DEV)

        def call():
            deep_gemm.fp8_gemm_nt(a, b, d, c=c, recipe=(1, 1, 128))
    else:
        c = None
        d = sentinel_bf16((m, n))

        def call():
            deep_gemm.fp8_gemm_nt(a, b, d)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    if one_d:
        assert not bool(torch.isnan(d).any()), 'outputs left unwritten'
    else:
        assert not bool((d.view(torch.int16) == SENTINEL).any()), 'outputs left unwritten'
    rows = pick(m, [0, 1, 127, 128, 255, 256, m // 2, m - 1], SAMPLE_ROWS, rng)
    cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
    ref, s_abs = oracle_sample(a, b, rows, cols, b_per_block=not one_d, c=c)
    out = d[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy()
    check(f'{kind} {m}x{n}x{k}', out, ref, s_abs, out_f32=one_d)
    rerun_identical(call, d, torch.int32 if one_d else torch.int16)


# ------------------------------------------------------------------ m-grouped contiguous

def _grouped_b(g, n, k, gen):
    bq = torch.empty((g, n, k), dtype=torch.float8_e4m3fn, device=DEV)
    bs = torch.empty((g, (n + 127) // 128, (k + 127) // 128), device=DEV)
    for i in range(g):
        bq[i], bs[i] = quant_b(randn_bf16((n, k), gen))
    return bq, bs


def _segment_sizes(g, expected, seed):
    rnd = random.Random(seed)
    return [int(expected * rnd.uniform(0.7, 1.3)) for _ in range(g)]


@pytest.mark.parametrize('layout', ['m_indices', 'psum', 'psum_zero_padding'])
@pytest.mark.parametrize('n,k', GROUPED_NK)
@pytest.mark.parametrize('g,expected', [(4, 8192), (8, 4096)])
def test_reference_contiguous_shape(g, expected, n, k, layout):
    """psum without zero padding is what the reference runs on its FP8 path
    (generators.py:196-201); with it, the gap rows must be zero
    (tests/utils.py:9-18)."""
    psum = layout != 'm_indices'
    zero_pad = layout == 'psum_zero_padding'
    print(f'reference contiguous G={g} m={expected} N={n} K={k} layout={layout}', flush=True)
    seed = g * 1000 + n + k + int(psum) + int(zero_pad)
    gen = dev_gen(seed)
    rng = np.random.default_rng(seed)
    align = deep_gemm.get_mk_alignment_for_contiguous_layout()
    ms = _segment_sizes(g, expected, seed)
    aligned = [(x + align - 1) // align * align for x in ms]
    starts = np.concatenate([[0], np.cumsum(aligned)[:-1]]).astype(np.int64)
    m = int(sum(aligned))
    valid = np.zeros(m, dtype=bool)
    m_idx = np.full(m, -1, dtype=np.int32)
    for i, (s, mi) in enumerate(zip(starts, ms)):
        valid[s:s + mi] = True
        m_idx[s:s + mi] = i
    x = randn_bf16((m, k), gen)
    x[torch.from_numpy(~valid).to(DEV)] = 0          # zero padding rows (generators.py:402-406)
    a = quant_a(x)
    bq, bs = _grouped_b(g, n, k, gen)
    layout = torch.from_numpy(starts + np.asarray(ms) if psum else m_idx).to(torch.int32).to(DEV)
    d = sentinel_bf16((m, n))

    def call():
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, (bq, bs), d, layout, use_psum_layout=psum,
                                                   ensure_zero_padding=zero_pad)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    valid_dev = torch.from_numpy(valid).to(DEV)
    dv = d.view(torch.int16)
    if zero_pad:
        assert bool((dv[~valid_dev] == 0).all()), 'psum padding rows not zero'
    else:
        assert bool((dv[~valid_dev] == SENTINEL).all()), 'padding rows touched'
    assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'
    cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
    outs, refs, sabs = [], [], []
    for e in range(g):
        s, mi = int(starts[e]), ms[e]
        rows = s + pick(mi, [0, 1, mi - 1], SAMPLE_ROWS // g, rng)
        ref, s_abs = oracle_sample(a, (bq[e], bs[e]), rows, cols)
        refs.append(ref), sabs.append(s_abs)
        outs.append(d[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy())
    check(f'contiguous G={g} {n}x{k} {layout}', np.concatenate(outs), np.concatenate(refs), np.concatenate(sabs))
    e = g - 1
    s, mi = int(starts[e]), ms[e]
    dd = torch.empty((mi, n), dtype=torch.bfloat16, device=DEV)
    generators.dense_call_same_order(deep_gemm, (a[0][s:s + mi], a[1][s:s + mi]), (bq[e], bs[e]), dd)
    assert torch.equal(dd.view(torch.int16), d[s:s + mi].view(torch.int16)), f'expert {e} differs from a dense call'
    rerun_identical(call, d)


# ------------------------------------------------------------------ m-grouped masked

@pytest.mark.parametrize('psum', [False, True])
@pytest.mark.parametrize('n,k', GROUPED_NK)
@pytest.mark.parametrize('g,expected', [(32, 192), (6, 1024), (32, 20), (6, 20)])
def test_reference_masked_shape(g, expected, n, k, psum):
    max_m = 4096
    expected_m = int(expected * 1.2)
    print(f'reference masked G={g} m={expected} max_m={max_m} N={n} K={k} psum={psum}', flush=True)
    seed = g * 1000 + expected + n + k + int(psum)
    gen = dev_gen(seed)
    rng = np.random.default_rng(seed)
    masked = _segment_sizes(g, expected, seed)
    assert max(masked) <= max_m
    bq, bs = _grouped_b(g, n, k, gen)
    align = deep_gemm.get_mk_alignment_for_contiguous_layout()
    sfk = (k + 127) // 128
    if psum:
        # the same experts in the psum layout: expert e's rows start at align(psum[e - 1])
        starts, ends, acc = [], [], 0
        for mm in masked:
            starts.append(acc)
            ends.append(acc + mm)
            acc = (acc + mm + align - 1) // align * align
        m = acc
        x = torch.zeros((m, k), dtype=torch.bfloat16, device=DEV)
        for s, mm in zip(starts, masked):
            x[s:s + mm] = randn_bf16((mm, k), gen)
        a = quant_a(x)
        a_rows = [(a[0][s:s + mm], a[1][s:s + mm]) for s, mm in zip(starts, masked)]
        layout = torch.tensor(ends, dtype=torch.int32, device=DEV)
        d = sentinel_bf16((m, n))
        valid = np.zeros(m, dtype=bool)
        for s, mm in zip(starts, masked):
            valid[s:s + mm] = True
        d_rows = [d[s:s + mm] for s, mm in zip(starts, masked)]

        def call():
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, (bq, bs), d, layout, use_psum_layout=True,
                                                       expected_m_for_psum_layout=expected_m)
    else:
        aq = torch.zeros((g, max_m, k), dtype=torch.float8_e4m3fn, device=DEV)
        as_ = torch.zeros((g, max_m, sfk), device=DEV)     # SFA past masked_m is zero (generators.py:476-478)
        for e, mm in enumerate(masked):
            aq[e, :mm], as_[e, :mm] = quant_a(randn_bf16((mm, k), gen))
        a = (aq, as_)
        a_rows = [(aq[e, :mm], as_[e, :mm]) for e, mm in enumerate(masked)]
        layout = torch.tensor(masked, dtype=torch.int32, device=DEV)
        d = sentinel_bf16((g, max_m, n))
        valid = np.arange(max_m)[None, :] < np.asarray(masked)[:, None]
        d_rows = [d[e, :mm] for e, mm in enumerate(masked)]

        def call():
            deep_gemm.m_grouped_fp8_gemm_nt_masked(a, (bq, bs), d, layout, expected_m)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    valid_dev = torch.from_numpy(valid).to(DEV)
    dv = d.view(torch.int16)
    # through the psum layout the gaps are zeroed (ensure_zero_padding defaults to
    # true, csrc/apis/gemm.hpp:877); in the masked layout rows past masked_m are untouched
    assert bool((dv[~valid_dev] == (0 if psum else SENTINEL)).all()), 'rows past masked_m touched'
    assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'
    cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
    experts = sorted({0, g - 1, *rng.choice(g, size=min(g, 4), replace=False).tolist()})
    outs, refs, sabs = [], [], []
    cols_dev = torch.from_numpy(cols).to(DEV)
    for e in experts:
        mm = masked[e]
        rows = pick(mm, [0, 1, mm - 1], max(8, SAMPLE_ROWS // len(experts)), rng)
        ref, s_abs = oracle_sample(a_rows[e], (bq[e], bs[e]), rows, cols)
        refs.append(ref), sabs.append(s_abs)
        outs.append(d_rows[e][torch.from_numpy(rows).to(DEV)][:, cols_dev].float().cpu().numpy())
    check(f'masked G={g} m={expected} {n}x{k} psum={psum}', np.concatenate(outs), np.concatenate(refs),
          np.concatenate(sabs))
    e = g - 1
    dd = torch.empty((masked[e], n), dtype=torch.bfloat16, device=DEV)
    generators.dense_call_same_order(deep_gemm, a_rows[e], (bq[e], bs[e]), dd)
    assert torch.equal(dd.view(torch.int16), d_rows[e].view(torch.int16)), f'expert {e} differs from a dense call'
    rerun_identical(call, d)


# ------------------------------------------------------------------ past 2^31 bytes

def _quantized(rows, k, gen, per_block, chunk=8192):
    """A seeded [rows, k] operand quantized on the device chunk by chunk: e4m3
    codes and K-major FP32 SFs (per token, or per 128 x 128 block)."""
    q = torch.empty((rows, k), dtype=torch.float8_e4m3fn, device=DEV)
    sf = torch.empty(((rows + 127) // 128 if per_block else rows, (k + 127) // 128), device=DEV)
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        qc, sc = (quant_b if per_block else quant_a)(randn_bf16((r1 - r0, k), gen))
        q[r0:r1] = qc
        if per_block:
            sf[r0 // 128:(r1 + 127) // 128] = sc
        else:
            sf[r0:r1] = sc
        del qc, sc
    return q, sf


@pytest.mark.parametrize('case', ['dense_d', 'dense_a', 'contiguous_d', 'masked_b'])
def test_past_2gib(case):
    """Operands and outputs of more than 2^31 bytes (the maximum sizes of one
    call): D of 2.2 GB (dense, and m-grouped contiguous), A of 2.2 GB, and a
    masked B whose last expert starts at byte 2^31. Sampled rows on both sides
    of the 2^31-byte boundary against the FP64 oracle, every output written,
    padding rows untouched, and a bitwise-identical rerun."""
    print(f'past 2 GiB: {case}', flush=True)
    gen = dev_gen(31 + len(case))
    rng = np.random.default_rng(31)
    if case in ('dense_d', 'dense_a'):
        m, n, k = (65536, 16896, 512) if case == 'dense_d' else (266240, 256, 8192)
        a = _quantized(m, k, gen, False)
        b = _quantized(n, k, gen, True)
        d = sentinel_bf16((m, n))
        edge = (2 ** 31) // (n * 2) if case == 'dense_d' else (2 ** 31) // k   # first row past byte 2^31
        print(f'  A {m * k / 2 ** 30:.2f} GiB, D {m * n * 2 / 2 ** 30:.2f} GiB, first row past 2^31 bytes: {edge}',
              flush=True)

        def call():
            deep_gemm.fp8_gemm_nt(a, b, d)
        call()
        torch.cuda.synchronize()
        print(f'  {deep_gemm.get_last_config()}', flush=True)
        assert not bool((d.view(torch.int16) == SENTINEL).any()), 'outputs left unwritten'
        rows = pick(m, [0, 1, edge - 1, edge, edge + 1, m - 2, m - 1], SAMPLE_ROWS, rng)
        cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
        ref, s_abs = oracle_sample(a, b, rows, cols)
        out = d[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy()
        check(f'{case} {m}x{n}x{k}', out, ref, s_abs)
        rerun_identical(call, d)
    elif case == 'contiguous_d':
        n, k = 16896, 512
        ms = [16379, 16484, 16000, 16401]
        aligned = [(x + 127) // 128 * 128 for x in ms]
        m_pad = sum(aligned)
        starts = np.concatenate([[0], np.cumsum(aligned)[:-1]])
        layout = torch.full((m_pad,), -1, dtype=torch.int32, device=DEV)
        for e, (s, mi) in enumerate(zip(starts, ms)):
            layout[int(s):int(s) + mi] = e
        a = _quantized(m_pad, k, gen, False)
        bq = torch.empty((len(ms), n, k), dtype=torch.float8_e4m3fn, device=DEV)
        bs = torch.empty((len(ms), (n + 127) // 128, k // 128), device=DEV)
        for e in range(len(ms)):
            bq[e], bs[e] = _quantized(n, k, gen, True)
        d = sentinel_bf16((m_pad, n))
        edge = (2 ** 31) // (n * 2)
        print(f'  D {m_pad * n * 2 / 2 ** 30:.2f} GiB, first row past 2^31 bytes: {edge}', flush=True)

        def call():
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, (bq, bs), d, layout)
        call()
        torch.cuda.synchronize()
        print(f'  {deep_gemm.get_last_config()}', flush=True)
        valid_dev = layout >= 0
        dv = d.view(torch.int16)
        assert bool((dv[~valid_dev] == SENTINEL).all()), 'padding rows touched'
        assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'
        cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
        outs, refs, sabs = [], [], []
        for e in (0, len(ms) - 1):
            s, mi = int(starts[e]), ms[e]
            must = [0, 1, mi - 1] + ([edge - s - 1, edge - s, edge - s + 1] if e else [])
            rows = s + pick(mi, must, SAMPLE_ROWS // 2, rng)
            ref, s_abs = oracle_sample(a, (bq[e], bs[e]), rows, cols)
            refs.append(ref), sabs.append(s_abs)
            outs.append(d[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy())
        check(f'{case} G={len(ms)} {n}x{k}', np.concatenate(outs), np.concatenate(refs), np.concatenate(sabs))
        rerun_identical(call, d)
    else:
        g, max_m, n, k = 9, 64, 16384, 16384   # expert 8 of B starts at byte 8 * n * k = 2^31
        masked = [64, 1, 33, 0, 64, 17, 64, 50, 61]
        aq = torch.empty((g, max_m, k), dtype=torch.float8_e4m3fn, device=DEV)
        asf = torch.empty((g, max_m, k // 128), device=DEV)
        bq = torch.empty((g, n, k), dtype=torch.float8_e4m3fn, device=DEV)
        bs = torch.empty((g, n // 128, k // 128), device=DEV)
        for e in range(g):
            aq[e], asf[e] = _quantized(max_m, k, gen, False)
            bq[e], bs[e] = _quantized(n, k, gen, True)
        print(f'  B {g * n * k / 2 ** 30:.2f} GiB; expert {g - 1} starts at byte {(g - 1) * n * k}', flush=True)
        mm = torch.tensor(masked, dtype=torch.int32, device=DEV)
        d = sentinel_bf16((g, max_m, n))

        def call():
            deep_gemm.m_grouped_fp8_gemm_nt_masked((aq, asf), (bq, bs), d, mm, expected_m=48)
        call()
        torch.cuda.synchronize()
        print(f'  {deep_gemm.get_last_config()}', flush=True)
        valid = np.arange(max_m)[None, :] < np.asarray(masked)[:, None]
        valid_dev = torch.from_numpy(valid).to(DEV)
        dv = d.view(torch.int16)
        assert bool((dv[~valid_dev] == SENTINEL).all()), 'rows past masked_m touched'
        assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'
        cols = pick(n, edge_cols(n), SAMPLE_COLS, rng)
        outs, refs, sabs = [], [], []
        for e in (0, g - 2, g - 1):
            rows = np.arange(masked[e])
            ref, s_abs = oracle_sample((aq[e], asf[e]), (bq[e], bs[e]), rows, cols)
            refs.append(ref), sabs.append(s_abs)
            outs.append(d[e][torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].float().cpu().numpy())
        check(f'{case} G={g} {n}x{k}', np.concatenate(outs), np.concatenate(refs), np.concatenate(sabs))
        rerun_identical(call, d)
