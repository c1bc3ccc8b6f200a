"""Pins for the CPU oracle (CPU only).

The reference holds no golden vectors (its tests draw CUDA randn at run time,
tests/generators.py:350-485), so each oracle function is pinned by checks that
do not restate it: torch's own float8 cast, brute-force loops, closed forms,
invariants of the quantization recipe, and the committed fixtures under
tests/golden/ (regression vectors written by tests/golden/make_golden.py).
"""
import os

import numpy as np
import pytest
import torch

from oracle import fp8, gemm as ogemm, quant as oquant

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


# ----------------------------------------------------------------- codecs

def test_e4m3_table_matches_torch_view():
    codes = np.arange(256, dtype=np.uint8)
    tv = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    mine = fp8.e4m3_decode(codes)
    assert np.array_equal(np.isnan(tv), np.isnan(mine))
    ok = ~np.isnan(tv)
    assert np.array_equal(tv[ok], mine[ok])


def test_e4m3_table_closed_forms():
    t = fp8.E4M3_TABLE
    assert t[0x00] == 0.0 and t[0x01] == 2.0 ** -9 and t[0x07] == 7 * 2.0 ** -9
    assert t[0x08] == 2.0 ** -6 and t[0x38] == 1.0 and t[0x7E] == 448.0 and np.isnan(t[0x7F])
    assert t[0xB8] == -1.0 and t[0x80] == 0.0 and np.isnan(t[0xFF])
    assert np.all(np.diff(t[:127]) > 0)


def _probe_values():
    rng = np.random.default_rng(0)
    pos = fp8.E4M3_TABLE[:127]
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    return np.concatenate([
        mids, -mids, pos.astype(np.float32), np.nextafter(mids, 0).astype(np.float32),
        np.nextafter(mids, 1e4).astype(np.float32), (rng.standard_normal(200_000) * 100).astype(np.float32),
        (rng.standard_normal(50_000) * 1e-2).astype(np.float32),
        np.array([448.5, 463.9, 464.0, 464.01, 479.0, 480.0, 1e4, -500.0, 0.0, -0.0, 1e-30, 2.0 ** -10],
                 dtype=np.float32)])


def test_e4m3_encode_matches_torch():
    v = _probe_values()
    t = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.e4m3_encode(v), t)


def test_e4m3_encode_matches_table_search():
    v = _probe_values()
    assert np.array_equal(fp8.e4m3_encode(v), fp8.e4m3_encode_table(v))


def test_e2m1_reference_boundaries():
    # deep_gemm/utils/math.py:89-93: (boundary, rounds-up-at-tie)
    for b, up in ((0.25, False), (0.75, True), (1.25, False), (1.75, True), (2.5, False), (3.5, True), (5.0, False)):
        below = fp8.e2m1_decode(fp8.e2m1_encode(np.array([b], np.float32)))[0]
        lo = fp8.E2M1_POS[fp8.E2M1_POS < b].max()
        hi = fp8.E2M1_POS[fp8.E2M1_POS > b].min()
        assert below == (hi if up else lo), b


def test_e2m1_nearest_brute_force():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20_000) * 3).astype(np.float32)
    codes = fp8.e2m1_encode(x)
    vals = fp8.e2m1_decode(codes)
    grid = np.concatenate([-fp8.E2M1_POS[::-1], fp8.E2M1_POS])
    best = np.abs(x[:, None].clip(-6, 6) - grid[None, :]).min(axis=1)
    assert np.allclose(np.abs(x.clip(-6, 6) - vals), best)
    assert np.array_equal(fp8.e2m1_unpack(fp8.e2m1_pack(codes[:20_000].reshape(100, 200))), codes.reshape(100, 200))


def test_ceil_to_ue8m0_closed_forms():
    x = np.array([1.0, 1.5, 2.0, 3.0, 0.75, 2.0 ** -130, 1e38 * 3], dtype=np.float32)
    want = np.array([1.0, 2.0, 2.0, 4.0, 1.0, 2.0 ** -126, 2.0 ** 127], dtype=np.float32)
    assert np.array_equal(fp8.ceil_to_ue8m0(x), want)
    assert np.array_equal(fp8.ue8m0_from_pow2_f32(want[:5]), np.array([127, 128, 128, 129, 127], np.uint8))


# ----------------------------------------------------------------- quantizers

def _bf16_vals(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).bfloat16().float().numpy()


def test_per_token_invariants():
    x = _bf16_vals((16, 300), 2)
    q, sf = oquant.per_token_cast_to_fp8(x, use_ue8m0=False, gran_k=128)
    assert q.shape == (16, 300) and sf.shape == (16, 3)
    v = fp8.e4m3_decode(q)
    assert np.all(np.abs(v) <= 448)
    for r in range(16):
        for g in range(3):
            seg = x[r, g * 128:(g + 1) * 128]
            amax = max(np.abs(seg).max(), np.float32(1e-4))
            assert sf[r, g] == np.float32(np.float32(amax) * np.float32(1.0 / 448.0))
            j = np.argmax(np.abs(seg))
            assert abs(v[r, g * 128 + j]) == 448.0           # the group maximum lands on the grid edge
    # reconstruction error <= half an e4m3 ulp (relative 2^-4) or half the subnormal quantum
    rec = oquant.dequant_per_token(q, sf)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, sf[:, np.arange(300) // 128] * 2.0 ** -10) * 1.0001
    assert np.all(np.abs(rec - x) <= bound)


def test_per_token_brute_force_tiny():
    x = _bf16_vals((3, 256), 3)
    q, sf = oquant.per_token_cast_to_fp8(x, use_ue8m0=True)
    for r in range(3):
        for g in range(2):
            seg = x[r, g * 128:(g + 1) * 128]
            s = np.float32(max(float(np.abs(seg).max()), 1e-4)) * np.float32(1.0 / 448.0)
            s = np.float32(2.0 ** np.ceil(np.log2(np.float64(s))))        # power of two >= s
            assert sf[r, g] == s
            recip = np.float32(1.0) / s
            for j in range(128):
                val = np.float32(seg[j] * recip)
                # nearest e4m3 value by exhaustive search, ties to the even code
                d = np.abs(fp8.E4M3_TABLE[:127] - abs(float(val)))
                ties = [int(i) for i in np.flatnonzero(d == d.min())]
                c = ties[0] if len(ties) == 1 else [i for i in ties if i % 2 == 0][0]
                if val < 0 and c:
                    c |= 0x80
                assert q[r, g * 128 + j] == c


def test_per_block_invariants():
    x = _bf16_vals((200, 260), 4)
    q, sf = oquant.per_block_cast_to_fp8(x, use_ue8m0=False)
    assert sf.shape == (2, 3)
    for bi in range(2):
        for bj in range(3):
            blk = x[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            assert sf[bi, bj] == np.float32(np.float32(np.abs(blk).max()) * np.float32(1.0 / 448.0))
    rec = oquant.dequant_per_block(q, sf)
    assert np.all(np.abs(rec - x) <= np.maximum(np.abs(x) * 2.0 ** -4, 2.0 ** -10) * 1.0001)


def test_per_token_fp4_invariants():
    x = _bf16_vals((8, 128), 5)
    p, sf = oquant.per_token_cast_to_fp4(x, use_ue8m0=True, gran_k=32)
    assert p.shape == (8, 64) and sf.shape == (8, 4)
    assert np.all(fp8.f32_bits(sf) & 0x7FFFFF == 0)
    v = fp8.e2m1_decode(fp8.e2m1_unpack(p))
    assert np.all(np.abs(v) <= 6)
    rec = oquant.dequant_fp4(p, sf, 32)
    # each value lands on the nearest representable point of its group's grid
    for r in range(8):
        for g in range(4):
            s = sf[r, g]
            seg = x[r, g * 32:(g + 1) * 32] / s
            grid = np.concatenate([-fp8.E2M1_POS, fp8.E2M1_POS]) * s
            best = np.abs(x[r, g * 32:(g + 1) * 32, None] - grid[None]).min(axis=1)
            assert np.allclose(np.abs(rec[r, g * 32:(g + 1) * 32] - x[r, g * 32:(g + 1) * 32]), best, atol=0)
            assert np.all(np.abs(seg) <= 6.0 + 1e-6)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(6)
    v = (rng.standard_normal(100_000) * 1e3).astype(np.float32)
    t = torch.from_numpy(v).bfloat16().float().numpy()
    assert np.array_equal(oquant.bf16_round(v), t)


# ----------------------------------------------------------------- GEMMs

def test_gemm_nt_triple_loop():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    b = rng.standard_normal((4, 5)).astype(np.float32)
    c = rng.standard_normal((3, 4))
    d = ogemm.gemm_nt(a, b, c)
    for i in range(3):
        for j in range(4):
            s = c[i, j]
            for k in range(5):
                s += float(a[i, k]) * float(b[j, k])
            assert abs(d[i, j] - s) < 1e-12


def test_k_grouped_brute_force_tiny():
    """gemm_k_grouped against scalar loops over the flat layout: group g's A_g is the
    [M, K_g] row-major block at element offset sum_{j<g} K_j * M, its scales the
    K-block columns of the same slice; an empty group leaves C as it is."""
    rng = np.random.default_rng(11)
    ks, m, n = [128, 0, 256], 3, 2
    sum_k = sum(ks)
    a = rng.integers(0, 256, size=sum_k * m).astype(np.uint8)
    b = rng.integers(0, 256, size=sum_k * n).astype(np.uint8)
    a[(a & 0x7F) == 0x7F] = 0                       # no NaN codes
    b[(b & 0x7F) == 0x7F] = 0
    sfa = rng.uniform(0.5, 2.0, size=(m, sum_k // 128)).astype(np.float32)
    sfb = rng.uniform(0.5, 2.0, size=(n, sum_k // 128)).astype(np.float32)
    c = rng.standard_normal((len(ks), m, n))
    d = ogemm.gemm_k_grouped(a, sfa, b, sfb, ks, c, oquant.dequant_per_token)
    val = fp8.E4M3_TABLE
    off = 0
    for g, k in enumerate(ks):
        for i in range(m):
            for j in range(n):
                s = c[g, i, j]
                for kk in range(k):
                    kb = (off + kk) // 128
                    av = np.float32(val[a[off * m + i * k + kk]]) * sfa[i, kb]
                    bv = np.float32(val[b[off * n + j * k + kk]]) * sfb[j, kb]
                    s += float(av) * float(bv)
                assert abs(d[g, i, j] - s) <= 1e-9 * max(1.0, abs(s))
        off += k
    assert np.array_equal(d[1], c[1])


def test_k_grouped_single_group_is_dense():
    rng = np.random.default_rng(12)
    m, n, k = 5, 4, 384
    qa = rng.integers(0, 0x7E, size=(m, k)).astype(np.uint8)
    qb = rng.integers(0, 0x7E, size=(n, k)).astype(np.uint8)
    sfa = rng.uniform(0.1, 1.0, size=(m, 3)).astype(np.float32)
    sfb = rng.uniform(0.1, 1.0, size=(n, 3)).astype(np.float32)
    c = rng.standard_normal((1, m, n))
    d = ogemm.gemm_k_grouped(qa.reshape(-1), sfa, qb.reshape(-1), sfb, [k], c, oquant.dequant_per_token)
    ref = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_token(qb, sfb), c[0])
    assert np.array_equal(d[0], ref)


def test_gemm_closed_form_ones():
    """A all 1.0 with SF 2, B all 0.5 with SF 0.25, K = 256: every D = 256 * 2 * 0.125 = 64."""
    m, n, k = 5, 130, 256
    qa = np.full((m, k), 0x38, np.uint8)                 # e4m3 1.0
    qb = np.full((n, k), 0x30, np.uint8)                 # e4m3 0.5
    sfa = np.full((m, 2), 2.0, np.float32)
    sfb = np.full((2, 2), 0.25, np.float32)
    d = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_block(qb, sfb))
    assert np.all(d == 64.0)


def test_gemm_single_k_block_exact():
    """Only K block 1 non-zero, power-of-two scales: D is exactly the integer-valued product sum."""
    rng = np.random.default_rng(8)
    m, n, k = 4, 6, 384
    qa = np.zeros((m, k), np.uint8)
    qb = np.zeros((n, k), np.uint8)
    ia = rng.integers(-4, 5, size=(m, 128))
    ib = rng.integers(-4, 5, size=(n, 128))
    qa[:, 128:256] = fp8.e4m3_encode(ia.astype(np.float32))
    qb[:, 128:256] = fp8.e4m3_encode(ib.astype(np.float32))
    sfa = np.full((m, 3), 0.5, np.float32)
    sfb = np.full((1, 3), 4.0, np.float32)
    d = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_block(qb, sfb))
    assert np.array_equal(d, (ia @ ib.T) * 2.0)


def test_gemm_transposition_and_linearity():
    rng = np.random.default_rng(9)
    a = rng.standard_normal((7, 33)).astype(np.float32)
    b = rng.standard_normal((5, 33)).astype(np.float32)
    c = rng.standard_normal((7, 5))
    assert np.allclose(ogemm.gemm_nt(a, b, c) - c, ogemm.gemm_nt(b, a).T)
    assert np.allclose(ogemm.gemm_nt(2 * a, b), 2 * ogemm.gemm_nt(a, b))


def test_contiguous_rules_brute_force():
    block_m = 4
    m_indices = np.array([0, 0, 0, -1, 2, 2, 2, 2, -1, -1, -1, -1, 1, -1, -1, -1], np.int32)
    assert list(ogemm.contiguous_expert_of_block(m_indices, block_m)) == [0, 2, 0, 1]
    rng = np.random.default_rng(10)
    a = rng.standard_normal((16, 8)).astype(np.float32)
    b = rng.standard_normal((3, 6, 8)).astype(np.float32)
    d, valid = ogemm.gemm_contiguous(a, b, m_indices, block_m)
    for r in range(16):
        if m_indices[r] < 0:
            assert not valid[r] and np.all(np.isnan(d[r]))
        else:
            e = max(0, m_indices[r // block_m * block_m])
            assert np.allclose(d[r], a[r].astype(np.float64) @ b[e].astype(np.float64).T)


def test_masked_rules_brute_force():
    rng = np.random.default_rng(11)
    a = rng.standard_normal((3, 5, 8)).astype(np.float32)
    b = rng.standard_normal((3, 4, 8)).astype(np.float32)
    mm = np.array([0, 5, 2], np.int32)
    d, valid = ogemm.gemm_masked(a, b, mm)
    for g in range(3):
        for r in range(5):
            assert valid[g, r] == (r < mm[g])
            if r < mm[g]:
                assert np.allclose(d[g, r], a[g, r].astype(np.float64) @ b[g].astype(np.float64).T)
            else:
                assert np.all(np.isnan(d[g, r]))


@pytest.mark.parametrize('seed', range(6))
def test_psum_rules_brute_force(seed):
    """psum_blocks / gemm_psum against the layout's own definition, row by row: the
    reference's generator puts group i's rows at [align(psum[i-1]), psum[i]) with
    psum[i] = align(psum[i-1]) + m_i (tests/generators.py:422-431,459), and its
    zero-padding check wants rows [psum[i], align(psum[i])) zero (tests/utils.py:9-18)."""
    rng = np.random.default_rng(40 + seed)
    align = 4
    counts = rng.integers(0, 11, size=int(rng.integers(1, 6)))
    counts[rng.integers(0, len(counts))] = 0           # an empty group somewhere
    psum, prev = [], 0
    for c in counts:
        prev = (prev + align - 1) // align * align + int(c)
        psum.append(prev)
    m = (psum[-1] + align - 1) // align * align + align   # a spare block past the last group
    owner = np.full(m, -1)
    start = 0
    for i, end in enumerate(psum):
        owner[start:end] = i
        start = (end + align - 1) // align * align
    # walk coverage: each owned row once, with its group; no other row
    seen = np.full(m, -1)
    for g, mb, row_end in ogemm.psum_blocks(psum, align):
        for r in range(mb * align, min((mb + 1) * align, row_end)):
            assert seen[r] == -1, 'row computed twice'
            seen[r] = g
    assert np.array_equal(seen, owner), (psum, seen, owner)
    a = rng.standard_normal((m, 8)).astype(np.float32)
    b = rng.standard_normal((len(psum), 3, 8)).astype(np.float32)
    for zero_pad in (False, True):
        d, written = ogemm.gemm_psum(a, b, psum, align, align, zero_pad)
        for r in range(m):
            pad = any(e <= r < (e + align - 1) // align * align for e in psum) and owner[r] < 0
            if owner[r] >= 0:
                assert written[r] and np.allclose(d[r], a[r].astype(np.float64) @ b[owner[r]].astype(np.float64).T)
            elif pad and zero_pad:
                assert written[r] and np.all(d[r] == 0.0)
            else:
                assert not written[r] and np.all(np.isnan(d[r]))


def test_psum_rejects_overlapping_groups():
    with pytest.raises(AssertionError):
        ogemm.psum_blocks([5, 6], 4)    # group 1 would start at align(5) = 8 > 6


@pytest.mark.parametrize('seed', range(4))
def test_moe_dispatch_against_stable_sort(seed):
    """oracle.moe.dispatch_rows against an independent construction: a stable
    sort of the flattened (token, slot) expert ids gives each expert's entries in
    token-then-slot order; segments start at aligned offsets; psum ends cover
    exactly the rows oracle.gemm.psum_blocks walks; masked keeps the first max_m
    entries of each expert."""
    from oracle import moe as omoe
    rng = np.random.default_rng(90 + seed)
    t_n, k, e_n, align = int(rng.integers(1, 40)), int(rng.integers(1, 5)), int(rng.integers(1, 7)), 8
    idx = rng.integers(-1, e_n, size=(t_n, k))
    flat = idx.reshape(-1)
    order = np.argsort(np.where(flat >= 0, flat, e_n), kind='stable')   # not-routed entries last
    counts = np.array([(flat == e).sum() for e in range(e_n)])
    starts = np.concatenate([[0], np.cumsum([(c + align - 1) // align * align for c in counts])])[:-1]
    want = np.full(flat.size, -1)
    r = 0
    for e in range(e_n):
        for i in range(counts[e]):
            want[order[r]] = starts[e] + i
            r += 1
    pos, m_idx, rows = omoe.dispatch_rows(idx, e_n, 'contiguous', align)
    assert np.array_equal(pos.reshape(-1), want)
    assert rows == sum((c + align - 1) // align * align for c in counts)
    assert np.all(starts % align == 0)
    for e in range(e_n):
        assert np.all(m_idx[starts[e]:starts[e] + counts[e]] == e)
    assert (m_idx >= 0).sum() == counts.sum()
    pos_p, psum, rows_p = omoe.dispatch_rows(idx, e_n, 'psum', align)
    assert np.array_equal(pos_p, pos) and rows_p == rows
    covered = {}
    for g, mb, row_end in ogemm.psum_blocks(psum, align):
        for row in range(mb * align, min((mb + 1) * align, row_end)):
            covered[row] = g
    assert covered == {int(want[i]): int(flat[i]) for i in range(flat.size) if want[i] >= 0}
    max_m = 3
    pos_m, mm, _ = omoe.dispatch_rows(idx, e_n, 'masked', max_m=max_m)
    assert np.array_equal(mm, np.minimum(counts, max_m))
    for e in range(e_n):
        ent = [i for i in order[:counts.sum()] if flat[i] == e]
        for r_, i in enumerate(ent):
            assert pos_m.reshape(-1)[i] == (e * max_m + r_ if r_ < max_m else -1)


def test_moe_dispatch_copies_rows_and_zero_padding():
    from oracle import moe as omoe
    rng = np.random.default_rng(5)
    t_n, k, e_n, kk = 12, 2, 3, 256
    idx = rng.integers(0, e_n, size=(t_n, k))
    codes = rng.integers(0, 256, size=(t_n, kk)).astype(np.uint8)
    sf = rng.random((t_n, 2)).astype(np.float32)
    w = rng.random((t_n, k)).astype(np.float32)
    out = omoe.dispatch(codes, sf, idx, e_n, 'contiguous', alignment=8, topk_weights=w)
    for t in range(t_n):
        for j in range(k):
            p = out['pos'][t, j]
            assert np.array_equal(out['a'][p], codes[t]) and np.array_equal(out['sf'][p], sf[t])
            assert out['weights'][p] == w[t, j]
    pad = out['layout'] < 0
    assert np.all(out['a'][pad] == 0) and np.all(out['sf'][pad] == 0) and np.all(out['weights'][pad] == 0)


def test_exp_f32_within_1_5_ulp_of_float64():
    """The float32 exp restatement (the device kernels run the same steps): within
    1.5 ulp of float64 exp over 4 million uniform arguments in [-87, 88], 2 million
    in [-1, 1] and every 7th float32 of [0.5, 1); exact at 0; finite at both ends
    of its domain."""
    from oracle import moe as omoe
    rng = np.random.default_rng(61)
    xs = np.concatenate([rng.uniform(-87, 88, 4_000_000).astype(np.float32),
                         np.linspace(-1, 1, 2_000_001, dtype=np.float32),
                         (np.arange(0, 2 ** 23, 7, dtype=np.uint32) | np.uint32(0x3f000000)).view(np.float32)])
    got = omoe.exp_f32(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulps = np.abs(got - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulps.max() <= 1.5, ulps.max()
    assert omoe.exp_f32(np.float32(0.0)) == np.float32(1.0)
    ends = omoe.exp_f32(np.array([-87.0, 88.0], np.float32))
    assert np.all(np.isfinite(ends)) and np.all(ends > 0)


def test_silu_f32_special_values():
    """silu(0) = 0; silu(g) = g for g > 87 (1 + exp(-g) rounds to 1); -0 for
    g < -88 (exp(-g) overflows); NaN in, NaN out; and within 2 ulp (relative
    2.4e-7) of the float64 closed form on a million normal samples."""
    from scipy.special import expit
    from oracle import moe as omoe
    g = np.array([0.0, 87.5, 100.0, -88.5, -1e4, np.nan], np.float32)
    s = omoe.silu_f32(g)
    assert s[0] == 0.0 and s[1] == np.float32(87.5) and s[2] == np.float32(100.0)
    assert s[3] == 0.0 and np.signbit(s[3]) and s[4] == 0.0 and np.isnan(s[5])
    x = (np.random.default_rng(62).standard_normal(1_000_000) * 8).astype(np.float32)
    ref = x.astype(np.float64) * expit(x.astype(np.float64))
    rel = np.abs(omoe.silu_f32(x).astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() < 2.4e-7, rel.max()


def test_moe_swiglu_closed_forms():
    from scipy.special import expit
    from oracle import moe as omoe
    rng = np.random.default_rng(6)
    x = gen_bf16((7, 64), rng)
    w = rng.random(7).astype(np.float32)
    y = omoe.swiglu_apply_weight(x, w)
    assert y.dtype == np.float32
    g, u = x[:, :32].astype(np.float64), x[:, 32:].astype(np.float64)
    # three float32 roundings after silu's (division, * up, * w): within 4 ulp
    assert np.allclose(y, g * expit(g) * u * w[:, None].astype(np.float64), rtol=5e-7, atol=0)
    # the steps themselves: silu, then * up, then * w, each rounded to float32
    step = ((omoe.silu_f32(x[:, :32]) * x[:, 32:]).astype(np.float32) * w[:, None]).astype(np.float32)
    assert np.array_equal(y, step)
    z = omoe.swiglu_apply_weight(np.concatenate([np.zeros((1, 4)), np.full((1, 4), 3.0)], axis=1))
    assert np.all(z == 0.0)                      # silu(0) = 0
    c = omoe.swiglu_apply_weight(np.array([[50.0, -50.0, 2.0, 2.0]]), clamp=7.0)
    assert np.allclose(c, [[7.0 / (1 + np.exp(-7.0)) * 2.0, -50.0 / (1 + np.exp(50.0)) * 2.0]])
    q, sf = omoe.swiglu_apply_weight_to_fp8(x, w, gran_k=32)
    qq, ss = oquant.per_token_cast_to_fp8(omoe.swiglu_apply_weight(x, w).astype(np.float32), False, 32)
    assert np.array_equal(q, qq) and np.array_equal(sf, ss)


def test_moe_combine_exact_sums_and_slot_order():
    """Where every product and partial sum is exactly representable (bf16 values
    times power-of-two weights, small magnitudes) combine equals the exact sum;
    and the float32 accumulation runs in slot order: with rows 2^24, -2^24 and 1,
    slots (0, 1, 2) give (2^24 - 2^24) + 1 = 1, slots (0, 2, 1) give
    (2^24 + 1) - 2^24 = 0 (2^24 + 1 rounds to 2^24 in float32)."""
    from oracle import moe as omoe
    rng = np.random.default_rng(63)
    t_n, k, rows, n = 6, 4, 20, 16
    y = (rng.integers(-64, 64, size=(rows, n)) / 8.0).astype(np.float32)      # exact in bf16
    pos = rng.integers(-1, rows, size=(t_n, k))
    w = (2.0 ** rng.integers(-3, 3, size=(t_n, k))).astype(np.float32)
    exact = np.zeros((t_n, n))
    for t in range(t_n):
        for j in range(k):
            if pos[t, j] >= 0:
                exact[t] += w[t, j] * y[pos[t, j]].astype(np.float64)
    out = omoe.combine(y, pos, w)
    assert np.array_equal(out, oquant.bf16_round(exact.astype(np.float32)))
    yy = np.array([[2.0 ** 24], [-2.0 ** 24], [1.0]], np.float32)
    assert omoe.combine(yy, np.array([[0, 1, 2]]))[0, 0] == 1.0
    assert omoe.combine(yy, np.array([[0, 2, 1]]))[0, 0] == 0.0


def test_moe_combine_against_vectorized_sum():
    from oracle import moe as omoe
    rng = np.random.default_rng(7)
    t_n, k, rows, n = 9, 3, 40, 24
    y = oquant.bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    pos = rng.integers(-1, rows, size=(t_n, k))
    w = rng.random((t_n, k)).astype(np.float32)
    for wts in (None, w):
        acc = np.zeros((t_n, n), np.float32)
        for j in range(k):                        # slot order, float32 rounding after each step
            term = y[np.maximum(pos[:, j], 0)]
            if wts is not None:
                term = (wts[:, j:j + 1] * term).astype(np.float32)
            acc = np.where(pos[:, j:j + 1] >= 0, (acc + term).astype(np.float32), acc)
        assert np.array_equal(omoe.combine(y, pos, wts), oquant.bf16_round(acc))


def gen_bf16(shape, rng):
    return oquant.bf16_round(rng.standard_normal(shape).astype(np.float32))


def test_calc_diff_closed_forms():
    x = np.random.default_rng(12).standard_normal(1000)
    assert ogemm.calc_diff(x, x) == pytest.approx(0.0, abs=1e-15)
    assert ogemm.calc_diff(x, -x) == pytest.approx(2.0)
    assert ogemm.calc_diff(x, np.zeros_like(x)) == pytest.approx(1.0)
    assert ogemm.calc_diff(x, 2 * x) == pytest.approx(1 - 4 / 5)
    assert ogemm.calc_diff(np.zeros(3), np.zeros(3)) == 0.0


def test_sf_layout_restatements():
    rng = np.random.default_rng(13)
    sf = rng.standard_normal((2, 5, 3)).astype(np.float32)
    storage, view, strides = ogemm.mn_major_tma_aligned(sf)
    assert storage.shape == (2, 3, 8) and strides == (24, 1, 8)
    assert np.array_equal(view, sf)
    e = rng.integers(100, 140, size=(5, 6))
    pow2 = fp8.ue8m0_to_f32(e.astype(np.uint8))
    packed = ogemm.pack_ue8m0_mn_major(pow2)          # [1, 2, 8]
    assert packed.shape == (1, 2, 8)
    for r in range(5):
        for w in range(2):
            word = int(packed[0, w, r]) & 0xFFFFFFFF
            for j in range(4):
                kk = 4 * w + j
                assert (word >> (8 * j)) & 0xFF == (e[r, kk] if kk < 6 else 0)
    assert np.all(packed[0, :, 5:] == 0)


# ----------------------------------------------------------------- fixtures

def _fixture(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f'{name} not generated')
    return np.load(path, allow_pickle=False)


def test_golden_dense_reproduces():
    f = _fixture('dense_fp8_small.npz')
    qa, sfa = oquant.per_token_cast_to_fp8(f['a'], use_ue8m0=False)
    qb, sfb = oquant.per_block_cast_to_fp8(f['b'], use_ue8m0=False)
    assert np.array_equal(qa, f['qa']) and np.array_equal(sfa, f['sfa'])
    assert np.array_equal(qb, f['qb']) and np.array_equal(sfb, f['sfb'])
    d = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_block(qb, sfb))
    assert np.array_equal(d, f['d'])
    assert np.array_equal(oquant.bf16_bits(d.astype(np.float32)), f['d_bf16_bits'])


def test_golden_fp8_fp4_reproduces():
    f = _fixture('fp8_fp4_small.npz')
    qa, sfa = oquant.per_token_cast_to_fp8(f['a'], use_ue8m0=True, gran_k=128)
    qb, sfb = oquant.per_token_cast_to_fp4(f['b'], use_ue8m0=True, gran_k=32)
    assert np.array_equal(qa, f['qa']) and np.array_equal(sfa, f['sfa'])
    assert np.array_equal(qb, f['qb']) and np.array_equal(sfb, f['sfb'])
    d = ogemm.fp8_fp4_gemm_nt(qa, sfa, qb, sfb, 128, 32)
    assert np.array_equal(d, f['d'])
