"""Parity at the benchmark workloads: BASELINE configs 2-5 at their full sizes.

The inputs are built by bench.py's own operand builders (same seeds, same
shapes, same device quantizers), so every workload the benchmark times is a
workload checked here. For each launch:

  * the quantized codes and scales are copied back to the host and a seeded
    sample of about 512 output rows is compared with the FP64 oracle
    (FP32 dequantize-then-matmul, oracle/gemm.py): calc_diff < 1e-3 (the
    reference's bar, tests/generators.py:69-74), and every sampled output within
    one BF16 ulp (FP32 outputs: within the FP32 accumulation error) of the
    oracle. The sample always holds the first and last rows, the rows around
    tile edges, the first and last row of every contiguous segment and rows 0
    and masked_m - 1 of every masked expert;
  * full-size properties: every output row that must be written is written,
    padding rows (m_indices = -1) and rows >= masked_m keep a sentinel bit
    pattern, a contiguous segment / masked expert equals a dense call on its
    rows bit for bit, and 20 reruns are bitwise identical
    (reference tests/test_fp8_fp4.py:26-238).

calc_diff and the max relative error of every launch are printed.
"""
import numpy as np
import pytest
import torch

import bench
import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'
SENTINEL = 0x7F7B   # bf16 bit pattern written before each call (a large finite value)
SAMPLE = 512
RERUNS = 20


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def host(t):
    return t.float().cpu().numpy()


def sentinel_bf16(shape):
    return torch.full(shape, SENTINEL, dtype=torch.int16, device=DEV).view(torch.bfloat16)


def sample_rows(m, must, seed):
    rng = np.random.default_rng(seed)
    must = [r for r in must if 0 <= r < m]
    extra = rng.choice(m, size=min(m, max(0, SAMPLE - len(must))), replace=False)
    return np.unique(np.concatenate([np.asarray(must, dtype=np.int64), extra.astype(np.int64)]))


def check_rows(name, out, ref, k, out_f32=False, ab_max=None):
    """out / ref [rows, N]: calc_diff < 1e-3 and an elementwise bound. BF16
    outputs: one BF16 ulp (2^-8 relative) plus the FP32 accumulation error
    2^-20 sqrt(K) max|ref|; FP32 outputs: that accumulation error plus one FP32
    rounding of the result."""
    diff = ogemm.calc_diff(out, ref)
    rel = ogemm.max_rel_err(out, ref)
    print(f'[{name}] rows={out.shape[0]} calc_diff={diff:.3e} max_rel_err={rel:.3e}', flush=True)
    assert diff < 1e-3, diff
    scale = np.abs(ref).max() if ab_max is None else ab_max
    acc = 2.0 ** -20 * np.sqrt(k) * scale
    tol = np.abs(ref) * (2.0 ** -22 if out_f32 else 2.0 ** -8) + acc
    bad = np.abs(out - ref) > tol
    assert not bad.any(), f'{int(bad.sum())} outputs further from the FP64 oracle than the bound'
    return diff, rel


def rerun_identical(call, d):
    first = d.clone()
    for _ in range(RERUNS):
        call()
    torch.cuda.synchronize()
    assert torch.equal(d.view(torch.int16), first.view(torch.int16)), 'reruns not bitwise identical'


# ------------------------------------------------------------------ config 2

@pytest.fixture(scope='module')
def dense_ops():
    return bench.dense_operands(False, DEV)


@pytest.mark.parametrize('idx', range(len(bench.DENSE_NK)))
def test_cfg2_dense_bf16(dense_ops, idx):
    op = dense_ops[idx]
    m, n, k = op['m'], op['n'], op['k']
    print(f'cfg2 dense bf16 M={m} N={n} K={k}', flush=True)
    d = sentinel_bf16((m, n))

    def call():
        deep_gemm.fp8_gemm_nt(op['a'], op['b'], d)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    assert not bool((d.view(torch.int16) == SENTINEL).any()), 'outputs left unwritten'
    rows = sample_rows(m, [0, 1, 127, 128, 255, 256, m // 2, m - 1], seed=idx)
    qa, sfa = u8(op['a'][0])[rows], op['a'][1].cpu().numpy()[rows]
    ref = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa),
                        oquant.dequant_per_block(u8(op['b'][0]), op['b'][1].cpu().numpy()))
    check_rows(f'cfg2 {op["name"]}', host(d)[rows], ref, k)
    rerun_identical(call, d)


@pytest.fixture(scope='module')
def dense_acc_ops():
    return bench.dense_operands(True, DEV)


@pytest.mark.parametrize('idx', range(len(bench.DENSE_NK)))
def test_cfg2_dense_f32_c_accumulate(dense_acc_ops, idx):
    """D = C + A.B^T with FP32 C and D, in place (as bench.py runs it) and out of
    place: both equal bitwise and the oracle's C + A.B^T."""
    op = dense_acc_ops[idx]
    m, n, k = op['m'], op['n'], op['k']
    print(f'cfg2 dense f32 C-accumulate M={m} N={n} K={k}', flush=True)
    c = op['c']
    d_in = c.clone()
    deep_gemm.fp8_gemm_nt(op['a'], op['b'], d_in, c=d_in)
    d_out = torch.empty_like(c)

    def call():
        deep_gemm.fp8_gemm_nt(op['a'], op['b'], d_out, c=c)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    assert torch.equal(d_in.view(torch.int32), d_out.view(torch.int32)), 'in-place and out-of-place C differ'
    rows = sample_rows(m, [0, 1, 127, 128, 255, 256, m // 2, m - 1], seed=100 + idx)
    qa, sfa = u8(op['a'][0])[rows], op['a'][1].cpu().numpy()[rows]
    ab = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa),
                       oquant.dequant_per_block(u8(op['b'][0]), op['b'][1].cpu().numpy()))
    c_rows = c.cpu().numpy()[rows]
    check_rows(f'cfg2 acc {op["name"]}', d_out.cpu().numpy()[rows], ab + c_rows, k, out_f32=True,
               ab_max=np.abs(ab).max() + np.abs(c_rows).max())
    rerun_identical(call, d_out)


# ------------------------------------------------------------------ config 3

@pytest.fixture(scope='module')
def contiguous_ops():
    return bench.contiguous_operands(DEV)


@pytest.mark.parametrize('idx', [0, 1])
def test_cfg3_contiguous(contiguous_ops, idx):
    ops = contiguous_ops
    op = ops['shapes'][idx]
    n, k, m_pad = op['n'], op['k'], ops['m_pad']
    ms, aligned = ops['ms'], ops['aligned']
    print(f'cfg3 contiguous tokens/expert={ms} M_pad={m_pad} N={n} K={k}', flush=True)
    idx_dev = ops['m_indices']
    m_idx = idx_dev.cpu().numpy()
    d = sentinel_bf16((m_pad, n))

    def call():
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(op['a'], op['b'], d, idx_dev)
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    valid = m_idx >= 0
    dv = d.view(torch.int16)
    valid_dev = torch.from_numpy(valid).to(DEV)
    assert bool((dv[~valid_dev] == SENTINEL).all()), 'padding rows touched'
    assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'

    starts = np.concatenate([[0], np.cumsum(aligned)[:-1]]).astype(np.int64)
    must = []
    for s, mi in zip(starts, ms):
        if mi:
            must += [s, s + mi - 1]
    rng = np.random.default_rng(7 + idx)
    pool = np.flatnonzero(valid)
    rows = np.unique(np.concatenate([np.asarray(must, dtype=np.int64),
                                     rng.choice(pool, size=SAMPLE - len(must), replace=False)]))
    # expert of each sampled row: the contiguous-layout rule of the reference
    # (block expert = max(0, m_indices[block start]), block = 128 rows)
    experts = ogemm.contiguous_expert_of_block(m_idx, 128)[rows // 128]
    assert np.array_equal(experts, m_idx[rows]), 'segments are not aligned to 128-row blocks'
    qa, sfa = u8(op['a'][0])[rows], op['a'][1].cpu().numpy()[rows]
    a_deq = oquant.dequant_per_token(qa, sfa)
    ref = np.empty((rows.size, n))
    bq, bs = op['b']
    for e in np.unique(experts):
        sel = experts == e
        ref[sel] = ogemm.gemm_nt(a_deq[sel], oquant.dequant_per_block(u8(bq[e]), bs[e].cpu().numpy()))
    check_rows(f'cfg3 {op["name"]}', host(d)[rows], ref, k)

    # the largest and the smallest non-empty segment equal a dense call on their rows
    nonempty = [i for i, mi in enumerate(ms) if mi]
    for e in {max(nonempty, key=lambda i: ms[i]), min(nonempty, key=lambda i: ms[i])}:
        s, mi = int(starts[e]), ms[e]
        dd = torch.empty((mi, n), dtype=torch.bfloat16, device=DEV)
        gen.dense_call_same_order(deep_gemm, (op['a'][0][s:s + mi], op['a'][1][s:s + mi]), (bq[e], bs[e]), dd)
        assert torch.equal(dd.view(torch.int16), d[s:s + mi].view(torch.int16)), f'segment {e}'
    rerun_identical(call, d)


# ------------------------------------------------------------------ config 4

@pytest.fixture(scope='module')
def masked_ops():
    return bench.masked_operands(DEV)


@pytest.mark.parametrize('idx', [0, 1])
def test_cfg4_masked(masked_ops, idx):
    ops = masked_ops
    op = ops['shapes'][idx]
    g, max_m, n, k = ops['num_groups'], ops['max_m'], op['n'], op['k']
    masked = ops['masked_m']
    print(f'cfg4 masked masked_m={masked.tolist()} N={n} K={k}', flush=True)
    d = sentinel_bf16((g, max_m, n))

    def call():
        deep_gemm.m_grouped_fp8_gemm_nt_masked(op['a'], op['b'], d, ops['masked_m_dev'], ops['expected_m'])
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    valid = np.arange(max_m)[None, :] < masked[:, None]
    valid_dev = torch.from_numpy(valid).to(DEV)
    dv = d.view(torch.int16)
    assert bool((dv[~valid_dev] == SENTINEL).all()), 'rows >= masked_m touched'
    assert not bool((dv[valid_dev] == SENTINEL).any()), 'valid outputs left unwritten'

    rng = np.random.default_rng(17 + idx)
    per = SAMPLE // g
    aq, as_ = op['a']
    bq, bs = op['b']
    outs, refs = [], []
    for e in range(g):
        mm = int(masked[e])
        rows = np.unique(np.concatenate([[0, mm - 1], rng.choice(mm, size=min(mm, per - 2), replace=False)]))
        a_deq = oquant.dequant_per_token(u8(aq[e])[rows], as_[e].cpu().numpy()[rows])
        refs.append(ogemm.gemm_nt(a_deq, oquant.dequant_per_block(u8(bq[e]), bs[e].cpu().numpy())))
        outs.append(host(d[e])[rows])
    check_rows(f'cfg4 {op["name"]}', np.concatenate(outs), np.concatenate(refs), k)

    # two experts equal a dense call on their valid rows
    for e in (0, g - 1):
        mm = int(masked[e])
        dd = torch.empty((mm, n), dtype=torch.bfloat16, device=DEV)
        gen.dense_call_same_order(deep_gemm, (aq[e][:mm], as_[e][:mm]), (bq[e], bs[e]), dd)
        assert torch.equal(dd.view(torch.int16), d[e, :mm].view(torch.int16)), f'expert {e}'
    rerun_identical(call, d)


# ------------------------------------------------------------------ config 5

def test_cfg5_fp8_fp4():
    op = bench.fp8fp4_operands(DEV)
    m, n, k = op['m'], op['n'], op['k']
    print(f'cfg5 fp8 x fp4 M={m} N={n} K={k}', flush=True)
    d = sentinel_bf16((m, n))

    def call():
        deep_gemm.fp8_fp4_gemm_nt(op['a'], op['b'], d, recipe_a=(1, 128), recipe_b=(1, 32))
    call()
    torch.cuda.synchronize()
    print(f'  {deep_gemm.get_last_config()}', flush=True)
    assert not bool((d.view(torch.int16) == SENTINEL).any()), 'outputs left unwritten'
    rows = sample_rows(m, [0, 1, 127, 128, 255, 256, m // 2, m - 1], seed=5)
    ref = ogemm.fp8_fp4_gemm_nt(u8(op['a'][0])[rows], op['sfa_f32'].cpu().numpy()[rows], u8(op['b'][0]),
                                op['sfb_f32'].cpu().numpy(), 128, 32)
    check_rows('cfg5 fp8xfp4', host(d)[rows], ref, k)
    rerun_identical(call, d)
