"""Seeded random sweep of the GEMM entry points against the FP64 oracle.

The fixed-shape parity tests vary one axis at a time; here every case draws its
own combination. FP32-scale (1D2D) recipe: the layout (dense, m-grouped
contiguous, masked), M from 1 to 700 (so the tiny-M, weight-streaming and tiled
kernels all run), N a multiple of 8 or 16, K a multiple of 128 or with a 16-byte
K tail, BF16 or FP32 D with no C, a separate C or C in place, K- or MN-major SFA,
D as a view into a wider row pitch, empty experts, and masked_m anywhere from 0
to max_m. UE8M0 path: e4m3 or e2m1 operands, 1 x 32 or 1 x 128 power-of-two
scales, packed words or FP32 SFs, the three layouts, BF16 or FP32 D and C. 1D1D
recipe: dense and K-grouped (empty groups), C in place or separate, K- or
MN-major SFs.

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
K = 2048 the largest is 2^-18.6 x sum |a b|. Over the whole sweep the largest is
2^-16.1 (a 1D1D call with one K block), so the bar leaves a factor of 2.1.
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


# ------------------------------------------------ UE8M0 path (power-of-two scales)

N_UE8M0, N_1D1D = 15, 8


def _ue8m0_operand(x, fp4, gran):
    """Codes, power-of-two FP32 SFs and dequantized values of one operand (rows x K)."""
    if fp4:
        q, sf = oquant.per_token_cast_to_fp4(x, use_ue8m0=True, gran_k=gran)
        return q, sf, oquant.dequant_fp4(q, sf, gran)
    q, sf = oquant.per_token_cast_to_fp8(x, use_ue8m0=True, gran_k=gran)
    return q, sf, oquant.dequant_per_token(q, sf, gran)


def _ue8m0_grouped(x, fp4, gran):
    parts = [_ue8m0_operand(x[i], fp4, gran) for i in range(x.shape[0])]
    return tuple(np.stack([p[j] for p in parts]) for j in range(3))


def _codes(q, fp4):
    return gen.to_dev(q, torch.int8) if fp4 else gen.to_dev(q, torch.float8_e4m3fn)


def _ue8m0_sf(sf, packed):
    t = gen.to_dev(np.asarray(sf, dtype=np.float32))
    return deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(t) if packed else t


@pytest.mark.parametrize('idx', range(N_UE8M0))
def test_random_ue8m0(idx):
    rnd = random.Random(10000 + idx)
    layout = rnd.choice(['dense', 'dense', 'dense', 'masked', 'contiguous'])
    a_fp4 = layout == 'dense' and rnd.random() < 0.3
    b_fp4 = rnd.random() < 0.7
    gka = 32 if a_fp4 else rnd.choice([32, 128])
    gkb = 32 if b_fp4 else rnd.choice([32, 128])
    # FP8 x FP8 with two 1 x 128 FP32 SFs is the 1D1D recipe, not this path: pass packed words
    packed = layout != 'dense' or (not a_fp4 and not b_fp4 and gka == gkb == 128) or rnd.random() < 0.6
    n = 16 * rnd.randint(1, 48)
    k = 128 * rnd.randint(1, 16)
    rec = dict(recipe_a=(1, gka), recipe_b=(1, gkb))
    tag = f'a_fp4={a_fp4} b_fp4={b_fp4} gran_k=({gka},{gkb}) packed={packed} n={n} k={k}'
    seed = 10000 + idx
    if layout == 'dense':
        m = rnd.choice([rnd.randint(1, 32), rnd.randint(33, 600)])
        out = rnd.choice(['bf16', 'bf16+c', 'f32', 'f32+c', 'f32+c=d'])
        print(f'random ue8m0 dense #{idx}: m={m} {tag} out={out}', flush=True)
        f32 = out.startswith('f32')
        qa, sfa, a_deq = _ue8m0_operand(gen.randn_bf16((m, k), seed), a_fp4, gka)
        qb, sfb, b_deq = _ue8m0_operand(gen.randn_bf16((n, k), seed + 1), b_fp4, gkb)
        c_np = gen.randn_bf16((m, n), seed + 2) if '+c' in out else None
        ref = ogemm.gemm_nt(a_deq, b_deq, c_np)
        s_abs = ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq), None if c_np is None else np.abs(c_np))
        valid = np.ones((m, n), dtype=bool)
        d = _sentinel((m, n), f32)
        c, c0 = None, None
        if c_np is not None:
            c0 = gen.to_dev(c_np.astype(np.float32)).to(d.dtype)
            c = d if out.endswith('=d') else c0
        a = (_codes(qa, a_fp4), _ue8m0_sf(sfa, packed))
        b = (_codes(qb, b_fp4), _ue8m0_sf(sfb, packed))

        def call():
            if c is d:
                d.copy_(c0)
            deep_gemm.fp8_fp4_gemm_nt(a, b, d, c=c, **rec)
    elif layout == 'masked':
        g = rnd.randint(1, 6)
        max_m = rnd.choice([32, 64, 128, 256, 320])
        masked_m = np.array([rnd.choice([0, max_m, rnd.randint(1, max_m), rnd.randint(1, max_m)])
                             for _ in range(g)], dtype=np.int32)
        expected_m = rnd.randint(1, max_m)
        print(f'random ue8m0 masked #{idx}: masked_m={masked_m.tolist()} max_m={max_m} expected_m={expected_m} {tag}',
              flush=True)
        f32 = False
        qa, sfa, a_deq = _ue8m0_grouped(gen.randn_bf16((g, max_m, k), seed), False, gka)
        qb, sfb, b_deq = _ue8m0_grouped(gen.randn_bf16((g, n, k), seed + 1), b_fp4, gkb)
        ref, valid = ogemm.gemm_masked(a_deq, b_deq, masked_m)
        s_abs, _ = ogemm.gemm_masked(np.abs(a_deq), np.abs(b_deq), masked_m)
        d = _sentinel((g, max_m, n), False)
        a = (_codes(qa, False), _ue8m0_sf(sfa, True))
        b = (_codes(qb, b_fp4), _ue8m0_sf(sfb, True))
        mm = gen.to_dev(masked_m)

        def call():
            deep_gemm.m_grouped_fp8_fp4_gemm_nt_masked(a, b, d, mm, expected_m, **rec)
    else:
        g = rnd.randint(1, 5)
        ms = [rnd.choice([0, rnd.randint(1, 64), rnd.randint(65, 400)]) for _ in range(g)]
        if not any(ms):
            ms[rnd.randrange(g)] = rnd.randint(1, 300)
        aligned = [(mi + 127) // 128 * 128 for mi in ms]
        print(f'random ue8m0 contiguous #{idx}: ms={ms} {tag}', flush=True)
        f32 = False
        m_pad = sum(aligned)
        m_indices = np.full(m_pad, -1, np.int32)
        x_a = gen.randn_bf16((m_pad, k), seed)
        start = 0
        for i, (mi, ai) in enumerate(zip(ms, aligned)):
            m_indices[start:start + mi] = i
            x_a[start + mi:start + ai] = 0.0
            start += ai
        qa, sfa, a_deq = _ue8m0_operand(x_a, False, gka)
        qb, sfb, b_deq = _ue8m0_grouped(gen.randn_bf16((g, n, k), seed + 1), b_fp4, gkb)
        ref, valid = ogemm.gemm_contiguous(a_deq, b_deq, m_indices)
        s_abs, _ = ogemm.gemm_contiguous(np.abs(a_deq), np.abs(b_deq), m_indices)
        d = _sentinel((m_pad, n), False)
        a = (_codes(qa, False), _ue8m0_sf(sfa, True))
        b = (_codes(qb, b_fp4), _ue8m0_sf(sfb, True))
        mi_dev = gen.to_dev(m_indices)

        def call():
            deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous(a, b, d, mi_dev, **rec)

    call()
    torch.cuda.synchronize()
    out = d.float().cpu().numpy()
    if valid.any():
        _check(f'ue8m0 {layout} #{idx}', out[valid], ref[valid], s_abs[valid], f32)
    if not valid.all():
        assert _untouched(d[torch.from_numpy(~valid).to(DEV)]), 'rows outside the layout were written'
    _rerun_identical(call, d)


# ------------------------------------------------ 1D1D recipe: dense and K-grouped

def _sf_view(sf, mn_major):
    """FP32 SFs on the device, K-major or as the .T view of an MN-major array
    (strides (1, mn)), the form the reference's generators hand over."""
    if mn_major:
        return gen.to_dev(np.ascontiguousarray(np.asarray(sf, dtype=np.float32).T)).t()
    return gen.to_dev(np.asarray(sf, dtype=np.float32))


@pytest.mark.parametrize('idx', range(N_1D1D))
def test_random_1d1d(idx):
    rnd = random.Random(11000 + idx)
    m = rnd.randint(1, 600)
    n = 16 * rnd.randint(1, 48)
    inplace = rnd.random() < 0.5
    mn_major = rnd.random() < 0.5
    seed = 11000 + idx
    if idx % 2 == 0:
        k = 128 * rnd.randint(1, 16)
        print(f'random 1d1d dense #{idx}: m={m} n={n} k={k} inplace={inplace} sf_mn_major={mn_major}', flush=True)
        qa, sfa = oquant.per_token_cast_to_fp8(gen.randn_bf16((m, k), seed), use_ue8m0=False)
        qb, sfb = oquant.per_token_cast_to_fp8(gen.randn_bf16((n, k), seed + 1), use_ue8m0=False)
        a_deq, b_deq = oquant.dequant_per_token(qa, sfa), oquant.dequant_per_token(qb, sfb)
        c_np = gen.randn_bf16((m, n), seed + 2) * 8
        ref = ogemm.gemm_nt(a_deq, b_deq, c_np)
        s_abs = ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq), np.abs(c_np))
        c0 = gen.to_dev(c_np.astype(np.float32))
        d = c0.clone() if inplace else _sentinel((m, n), True)
        c = d if inplace else c0
        a = (gen.to_dev(qa, torch.float8_e4m3fn), _sf_view(sfa, mn_major))
        b = (gen.to_dev(qb, torch.float8_e4m3fn), _sf_view(sfb, mn_major))

        def call():
            if inplace:
                d.copy_(c0)
            deep_gemm.fp8_gemm_nt(a, b, d, c=c, recipe=(1, 1, 128))
    else:
        g = rnd.randint(1, 6)
        ks = [rnd.choice([0, 128 * rnd.randint(1, 8)]) for _ in range(g)]
        if not any(ks):
            ks[rnd.randrange(g)] = 128 * rnd.randint(1, 8)
        print(f'random 1d1d k-grouped #{idx}: ks={ks} m={m} n={n} inplace={inplace} sf_mn_major={mn_major}',
              flush=True)
        qa_g, sa_g, qb_g, sb_g = [], [], [], []
        for i, kg in enumerate(ks):
            if kg:
                qa, sfa = oquant.per_token_cast_to_fp8(gen.randn_bf16((m, kg), seed + 2 * i), use_ue8m0=False)
                qb, sfb = oquant.per_token_cast_to_fp8(gen.randn_bf16((n, kg), seed + 2 * i + 1), use_ue8m0=False)
                qa_g.append(qa.reshape(-1)), sa_g.append(sfa), qb_g.append(qb.reshape(-1)), sb_g.append(sfb)
        qa, qb = np.concatenate(qa_g), np.concatenate(qb_g)
        sfa, sfb = np.concatenate(sa_g, axis=1), np.concatenate(sb_g, axis=1)
        c_np = gen.randn_bf16((g, m, n), seed + 99) * 8
        ref = ogemm.gemm_k_grouped(qa, sfa, qb, sfb, ks, c_np, oquant.dequant_per_token)
        s_abs = ogemm.gemm_k_grouped(qa, sfa, qb, sfb, ks, np.abs(c_np),
                                     lambda q, s: np.abs(oquant.dequant_per_token(q, s)))
        c0 = gen.to_dev(c_np.astype(np.float32))
        d = c0.clone() if inplace else _sentinel((g, m, n), True)
        c = d if inplace else c0
        a = (gen.to_dev(qa, torch.float8_e4m3fn), _sf_view(sfa, mn_major))
        b = (gen.to_dev(qb, torch.float8_e4m3fn), _sf_view(sfb, mn_major))
        layout = torch.tensor(ks, dtype=torch.int32, device=DEV)

        def call():
            if inplace:
                d.copy_(c0)
            deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, ks, layout, c)

    call()
    torch.cuda.synchronize()
    _check(f'1d1d #{idx}', d.cpu().numpy(), ref, s_abs, True)
    _rerun_identical(call, d)
