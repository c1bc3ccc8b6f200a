"""GPU parity of the fused L1 grouped GEMM (SwiGLU x routing weight -> FP8 in the
epilogue) against the unfused pipeline it replaces: the plain m-grouped GEMM with
the standard [gate | up] weight, BF16 D, then moe_swiglu_apply_weight_to_fp8.

Bar: bit for bit. Every stored row's e4m3 codes and FP32 scale must equal the
unfused pipeline's; rows the GEMM leaves untouched (m_indices -1, rows >=
masked_m, psum padding without ensure_zero_padding) must keep their sentinel
bytes; psum padding rows with ensure_zero_padding must hold zero codes and the
scale of an all-zero row. The unfused pipeline itself is pinned against the
oracle by tests/test_moe_gpu.py, and a whole MoE layer on the fused path is
checked against the oracle's FP64 pipeline to calc_diff < 1e-3 here.
"""
import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators as gen
from test_moe_gpu import _layer_oracle, _routing, _x

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'
SENTINEL = 0x5A        # q bytes the kernels must not touch
SF_SENTINEL = -7.25    # sf values likewise


def _weights(g, n, k, seed):
    """Per-expert e4m3 weights [g, n, k] with 128 x 128 FP32 scales (oracle quantizer)."""
    qb = np.empty((g, n, k), np.uint8)
    sfb = np.empty((g, n // 128, (k + 127) // 128), np.float32)
    for e in range(g):
        qb[e], sfb[e] = oquant.per_block_cast_to_fp8(gen.randn_bf16((n, k), seed + e), use_ue8m0=False)
    return gen.to_dev(qb, torch.float8_e4m3fn), gen.to_dev(sfb)


def _alloc_out(rows_shape, inter):
    q = torch.full(rows_shape + (inter,), SENTINEL, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    sf = torch.full(rows_shape + (inter // 128,), SF_SENTINEL, dtype=torch.float32, device=DEV)
    return q, sf


def _psum_layout(ms, align):
    ends, starts, acc = [], [], 0
    for mi in ms:
        starts.append(acc)
        ends.append(acc + mi)
        acc = (acc + mi + align - 1) // align * align
    return np.array(starts), np.array(ends, np.int32), acc


def _check_rows(q, sf, rq, rsf, stored, zero=None):
    """stored / zero: boolean row masks over the flattened rows."""
    qh = q.view(torch.uint8).reshape(-1, q.shape[-1]).cpu().numpy()
    sh = sf.reshape(-1, sf.shape[-1]).cpu().numpy()
    rqh = rq.view(torch.uint8).reshape(-1, rq.shape[-1]).cpu().numpy()
    rsh = rsf.reshape(-1, rsf.shape[-1]).cpu().numpy()
    zero = np.zeros_like(stored) if zero is None else zero
    assert np.array_equal(qh[stored], rqh[stored]), 'codes of stored rows'
    assert np.array_equal(sh[stored].view(np.int32), rsh[stored].view(np.int32)), 'scales of stored rows'
    if zero.any():
        assert np.all(qh[zero] == 0)
        assert np.all(sh[zero] == np.float32(np.float32(1e-4) * np.float32(1.0 / 448.0)))
    rest = ~(stored | zero)
    assert np.all(qh[rest] == SENTINEL), 'untouched rows'
    assert np.all(sh[rest] == np.float32(SF_SENTINEL)), 'untouched scales'


def test_transform_weights_round_trip():
    """The fused layout is a block permutation: interleaved rows [256j, +128) are gate
    block j and [256j + 128, +128) up block j, and SF rows follow the blocks."""
    g, inter, k = 3, 384, 256
    b = (gen.to_dev(np.random.default_rng(1).integers(0, 126, (g, 2 * inter, k)).astype(np.uint8),
                    torch.float8_e4m3fn),
         gen.to_dev(np.random.default_rng(2).random((g, 2 * inter // 128, k // 128)).astype(np.float32)))
    bi, si = deep_gemm.transform_l1_weights_for_swiglu(b)
    torch.cuda.synchronize()
    src, dst = b[0].view(torch.uint8).cpu().numpy(), bi.view(torch.uint8).cpu().numpy()
    ssrc, sdst = b[1].cpu().numpy(), si.cpu().numpy()
    for j in range(inter // 128):
        assert np.array_equal(dst[:, 256 * j:256 * j + 128], src[:, 128 * j:128 * j + 128])
        assert np.array_equal(dst[:, 256 * j + 128:256 * j + 256], src[:, inter + 128 * j:inter + 128 * j + 128])
        assert np.array_equal(sdst[:, 2 * j], ssrc[:, j]) and np.array_equal(sdst[:, 2 * j + 1], ssrc[:, inter // 128 + j])


@pytest.mark.parametrize('tile', [None, (256, 256), (128, 256)])
@pytest.mark.parametrize('k,clamp,weighted', [(1024, None, True), (896, 5.0, True), (2048, None, False),
                                              (1040, None, True)])
def test_fused_contiguous_equals_unfused(tile, k, clamp, weighted):
    ms = [0, 300, 5, 128, 700, 1]
    g, inter = len(ms), 512
    aligned = [(x + 127) // 128 * 128 for x in ms]
    rows = sum(aligned)
    a_np = gen.randn_bf16((rows, k), 3)
    qa, sfa = oquant.per_token_cast_to_fp8(a_np, use_ue8m0=False)
    m_idx = np.full(rows, -1, np.int32)
    start = 0
    for e, (mi, ai) in enumerate(zip(ms, aligned)):
        m_idx[start:start + mi] = e
        start += ai
    a = (gen.to_dev(qa, torch.float8_e4m3fn), gen.to_dev(sfa))
    w_std = _weights(g, 2 * inter, k, 10)
    w_fused = deep_gemm.transform_l1_weights_for_swiglu(w_std)
    rw = gen.to_dev(np.random.default_rng(4).random(rows).astype(np.float32)) if weighted else None
    gl = gen.to_dev(m_idx)
    q, sf = _alloc_out((rows,), inter)
    if tile:
        deep_gemm.set_tile_override(*tile, variant=2)
    try:
        if tile == (256, 256) and k % 128:
            # no K-tail schedule for 256-row tiles: refused before any launch
            with pytest.raises(RuntimeError, match='128 x 256'):
                deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu(a, w_fused, (q, sf), gl, rw, clamp)
            return
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu(a, w_fused, (q, sf), gl, rw, clamp)
        cfg = deep_gemm.get_last_config()
    finally:
        deep_gemm.set_tile_override(0, 0)
    h = torch.zeros((rows, 2 * inter), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, w_std, h, gl)
    rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw, gl, clamp)
    torch.cuda.synchronize()
    print(cfg, flush=True)
    _check_rows(q, sf, rq, rsf, m_idx >= 0)


@pytest.mark.parametrize('align', [128, 256])
@pytest.mark.parametrize('zero_padding', [True, False])
def test_fused_psum_equals_unfused(align, zero_padding):
    ms = [130, 0, 257, 1, 64]
    g, inter, k = len(ms), 256, 1536
    starts, ends, rows = _psum_layout(ms, align)
    rows += 64   # rows past the last group stay untouched
    a_np = gen.randn_bf16((rows, k), 5)
    qa, sfa = oquant.per_token_cast_to_fp8(a_np, use_ue8m0=False)
    a = (gen.to_dev(qa, torch.float8_e4m3fn), gen.to_dev(sfa))
    w_std = _weights(g, 2 * inter, k, 20)
    w_fused = deep_gemm.transform_l1_weights_for_swiglu(w_std)
    rw = gen.to_dev(np.random.default_rng(6).random(rows).astype(np.float32))
    gl = gen.to_dev(ends)
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(align)
    try:
        q, sf = _alloc_out((rows,), inter)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu(a, w_fused, (q, sf), gl, rw, None, use_psum_layout=True,
                                                          ensure_zero_padding=zero_padding)
        print(deep_gemm.get_last_config(), flush=True)
        h = torch.zeros((rows, 2 * inter), dtype=torch.bfloat16, device=DEV)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, w_std, h, gl, use_psum_layout=True, ensure_zero_padding=True)
        rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw, None, None)
        torch.cuda.synchronize()
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    stored = np.zeros(rows, bool)
    zero = np.zeros(rows, bool)
    for s, e in zip(starts, ends):
        stored[s:e] = True
        if zero_padding:
            zero[e:(e + align - 1) // align * align] = True
    _check_rows(q, sf, rq, rsf, stored, zero)


@pytest.mark.parametrize('tile', [None, (256, 256), (128, 256)])
@pytest.mark.parametrize('masked_m', [[0, 1, 97, 160], [161, 300, 5, 64]])
def test_fused_masked_equals_unfused(tile, masked_m):
    g, max_m, inter, k = len(masked_m), 320, 512, 1024
    qa = np.empty((g, max_m, k), np.uint8)
    sfa = np.empty((g, max_m, k // 128), np.float32)
    for e in range(g):
        qa[e], sfa[e] = oquant.per_token_cast_to_fp8(gen.randn_bf16((max_m, k), 30 + e), use_ue8m0=False)
    a = (gen.to_dev(qa, torch.float8_e4m3fn), gen.to_dev(sfa))
    w_std = _weights(g, 2 * inter, k, 40)
    w_fused = deep_gemm.transform_l1_weights_for_swiglu(w_std)
    rw = gen.to_dev(np.random.default_rng(7).random((g, max_m)).astype(np.float32))
    mm = gen.to_dev(np.array(masked_m, np.int32))
    q, sf = _alloc_out((g, max_m), inter)
    if tile:
        deep_gemm.set_tile_override(*tile, variant=2)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu(a, w_fused, (q, sf), mm, expected_m=128, row_weights=rw)
        cfg = deep_gemm.get_last_config()
    finally:
        deep_gemm.set_tile_override(0, 0)
    h = torch.zeros((g, max_m, 2 * inter), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_gemm_nt_masked(a, w_std, h, mm, expected_m=128)
    rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(g * max_m, -1), rw.view(-1))
    torch.cuda.synchronize()
    print(cfg, flush=True)
    stored = (np.arange(max_m)[None, :] < np.array(masked_m)[:, None]).reshape(-1)
    _check_rows(q, sf, rq.view(g, max_m, -1), rsf.view(g, max_m, -1), stored)


@pytest.mark.parametrize('masked_m', [[0, 1, 300, 1024], [200, 513, 7, 256]])
def test_fused_masked_sparse_persistent(masked_m):
    """Masked groups far below max_m (expected_m 200 of 1024) run the persistent
    group walk (variant 4) on the fused path too: the same bits as the unfused
    pipeline, rows past masked_m untouched."""
    g, max_m, inter, k = len(masked_m), 1024, 512, 1024
    qa = np.empty((g, max_m, k), np.uint8)
    sfa = np.empty((g, max_m, k // 128), np.float32)
    for e in range(g):
        qa[e], sfa[e] = oquant.per_token_cast_to_fp8(gen.randn_bf16((max_m, k), 60 + e), use_ue8m0=False)
    a = (gen.to_dev(qa, torch.float8_e4m3fn), gen.to_dev(sfa))
    w_std = _weights(g, 2 * inter, k, 70)
    w_fused = deep_gemm.transform_l1_weights_for_swiglu(w_std)
    rw = gen.to_dev(np.random.default_rng(8).random((g, max_m)).astype(np.float32))
    mm = gen.to_dev(np.array(masked_m, np.int32))
    q, sf = _alloc_out((g, max_m), inter)
    deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu(a, w_fused, (q, sf), mm, expected_m=200, row_weights=rw)
    cfg = deep_gemm.get_last_config()
    h = torch.zeros((g, max_m, 2 * inter), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_gemm_nt_masked(a, w_std, h, mm, expected_m=200)
    rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(g * max_m, -1), rw.view(-1))
    torch.cuda.synchronize()
    print(cfg, flush=True)
    assert 'v4' in cfg
    stored = (np.arange(max_m)[None, :] < np.array(masked_m)[:, None]).reshape(-1)
    _check_rows(q, sf, rq.view(g, max_m, -1), rsf.view(g, max_m, -1), stored)


def test_fused_reruns_bitwise():
    """The fused launches are deterministic: 10 reruns of each kernel give the same bytes."""
    ms = [500, 37, 260]
    g, inter, k = len(ms), 1024, 2048
    aligned = [(x + 127) // 128 * 128 for x in ms]
    rows = sum(aligned)
    qa, sfa = oquant.per_token_cast_to_fp8(gen.randn_bf16((rows, k), 8), use_ue8m0=False)
    m_idx = np.concatenate([np.r_[np.full(mi, e), np.full(ai - mi, -1)] for e, (mi, ai) in
                            enumerate(zip(ms, aligned))]).astype(np.int32)
    a = (gen.to_dev(qa, torch.float8_e4m3fn), gen.to_dev(sfa))
    w = deep_gemm.transform_l1_weights_for_swiglu(_weights(g, 2 * inter, k, 50))
    first = None
    for _ in range(10):
        q, sf = _alloc_out((rows,), inter)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu(a, w, (q, sf), gen.to_dev(m_idx))
        cur = (q.view(torch.uint8).clone(), sf.view(torch.int32).clone())
        if first is None:
            first = cur
        assert torch.equal(cur[0], first[0]) and torch.equal(cur[1], first[1])


def test_fused_config3_full_size():
    """Config 3's gate/up launch at full size (8 experts, 32768 tokens, Dirichlet(1)
    segments, N = 4096 = 2 x 2048, K = 7168): fused == unfused bit for bit over every
    stored row, padding rows untouched. Config 4's gate/up launch (16 experts,
    max_m 256, masked_m ~ U[96, 160], N = 4096, K = 7168) likewise."""
    torch.manual_seed(0)
    ms, aligned = gen.contiguous_sizes(8, 32768, seed=3)
    rows, inter, k = sum(aligned), 2048, 7168
    m_idx = np.concatenate([np.r_[np.full(mi, e), np.full(ai - mi, -1)] for e, (mi, ai) in
                            enumerate(zip(ms, aligned))]).astype(np.int32)
    x = torch.randn((rows, k), device=DEV).bfloat16()
    qa, sfa = deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=False)
    wq = torch.empty((8, 2 * inter, k), dtype=torch.float8_e4m3fn, device=DEV)
    ws = torch.empty((8, 2 * inter // 128, k // 128), dtype=torch.float32, device=DEV)
    for e in range(8):
        wq[e], ws[e] = deep_gemm.per_block_cast_to_fp8(torch.randn((2 * inter, k), device=DEV).bfloat16(), False)
    wf = deep_gemm.transform_l1_weights_for_swiglu((wq, ws))
    rw = torch.rand((rows,), device=DEV)
    gl = gen.to_dev(m_idx)
    q, sf = _alloc_out((rows,), inter)
    deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu((qa, sfa), wf, (q, sf), gl, rw)
    cfg = deep_gemm.get_last_config()
    print(cfg, flush=True)
    assert 'v4' in cfg   # eight rounds of 256 x 256 tiles: persistent workgroups
    h = torch.empty((rows, 2 * inter), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_gemm_nt_contiguous((qa, sfa), (wq, ws), h, gl)
    rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw, gl)
    valid = gl >= 0
    assert torch.equal(q.view(torch.uint8)[valid], rq.view(torch.uint8)[valid])
    assert torch.equal(sf.view(torch.int32)[valid], rsf.view(torch.int32)[valid])
    assert bool((q.view(torch.uint8)[~valid] == SENTINEL).all()) and bool((sf[~valid] == SF_SENTINEL).all())

    g, max_m = 16, 256
    masked_m = torch.from_numpy(np.random.default_rng(4).integers(96, 161, size=g).astype(np.int32)).to(DEV)
    xa = torch.randn((g * max_m, k), device=DEV).bfloat16()
    qa, sfa = deep_gemm.per_token_cast_to_fp8(xa, use_ue8m0=False)
    qa, sfa = qa.view(g, max_m, k), sfa.view(g, max_m, -1)
    wq = torch.empty((g, 2 * inter, k), dtype=torch.float8_e4m3fn, device=DEV)
    ws = torch.empty((g, 2 * inter // 128, k // 128), dtype=torch.float32, device=DEV)
    for e in range(g):
        wq[e], ws[e] = deep_gemm.per_block_cast_to_fp8(torch.randn((2 * inter, k), device=DEV).bfloat16(), False)
    wf = deep_gemm.transform_l1_weights_for_swiglu((wq, ws))
    rw = torch.rand((g, max_m), device=DEV)
    q, sf = _alloc_out((g, max_m), inter)
    deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu((qa, sfa), wf, (q, sf), masked_m, 128, rw)
    print(deep_gemm.get_last_config(), flush=True)
    h = torch.empty((g, max_m, 2 * inter), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_gemm_nt_masked((qa, sfa), (wq, ws), h, masked_m, 128)
    rq, rsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(g * max_m, -1), rw.view(-1))
    valid = (torch.arange(max_m, device=DEV)[None, :] < masked_m[:, None]).reshape(-1)
    qf, sff = q.view(torch.uint8).view(g * max_m, -1), sf.view(g * max_m, -1)
    assert torch.equal(qf[valid], rq.view(torch.uint8)[valid])
    assert torch.equal(sff.view(torch.int32)[valid], rsf.view(torch.int32)[valid])
    assert bool((qf[~valid] == SENTINEL).all()) and bool((sff[~valid] == SF_SENTINEL).all())


def test_moe_layer_fused_end_to_end():
    """The one-GPU MoE layer of tests/test_moe_gpu.py with the fused L1 on each
    layout: the same bits as the unfused layer, and calc_diff < 1e-3 against the
    oracle's FP64 pipeline."""
    t, k, e, hidden, inter = 256, 2, 8, 2048, 1024
    idx, w = _routing(t, k, e, seed=31, unrouted=0.05)
    q, sf = _x(t, hidden, 32)
    l1 = (np.empty((e, 2 * inter, hidden), np.uint8), np.empty((e, 2 * inter // 128, hidden // 128), np.float32))
    l2 = (np.empty((e, hidden, inter), np.uint8), np.empty((e, hidden // 128, inter // 128), np.float32))
    for ei in range(e):
        l1[0][ei], l1[1][ei] = oquant.per_block_cast_to_fp8(gen.randn_bf16((2 * inter, hidden), 40 + ei), False)
        l2[0][ei], l2[1][ei] = oquant.per_block_cast_to_fp8(gen.randn_bf16((hidden, inter), 60 + ei), False)
    w1 = (gen.to_dev(l1[0], torch.float8_e4m3fn), gen.to_dev(l1[1]))
    w1f = deep_gemm.transform_l1_weights_for_swiglu(w1)
    w2 = (gen.to_dev(l2[0], torch.float8_e4m3fn), gen.to_dev(l2[1]))
    x = (gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf))
    idx_d, w_d = gen.to_dev(idx), gen.to_dev(w)
    outs = {}
    for layout in ('contiguous', 'psum', 'masked'):
        max_m = 256 if layout == 'masked' else None
        a, a_sf, gl, pos, rw = deep_gemm.moe_dispatch(x, idx_d, e, layout=layout, max_m=max_m, topk_weights=w_d)
        for fused in (False, True):
            if layout == 'masked':
                if fused:
                    hq = torch.zeros((e, max_m, inter), dtype=torch.float8_e4m3fn, device=DEV)
                    hsf = torch.zeros((e, max_m, inter // 128), dtype=torch.float32, device=DEV)
                    deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu((a, a_sf), w1f, (hq, hsf), gl, t * k // e, rw)
                else:
                    h = torch.empty((e, max_m, 2 * inter), dtype=torch.bfloat16, device=DEV)
                    deep_gemm.m_grouped_fp8_gemm_nt_masked((a, a_sf), w1, h, gl, expected_m=t * k // e)
                    hq, hsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(e * max_m, 2 * inter), rw.view(-1))
                    hq, hsf = hq.view(e, max_m, inter), hsf.view(e, max_m, -1)
                y = torch.empty((e, max_m, hidden), dtype=torch.bfloat16, device=DEV)
                deep_gemm.m_grouped_fp8_gemm_nt_masked((hq, hsf), w2, y, gl, expected_m=t * k // e)
            else:
                psum = layout == 'psum'
                if fused:
                    # padding rows of the L2 input: zero codes (contiguous: written by
                    # nothing, so start from zeros; psum: the fused zero padding)
                    hq = torch.zeros((a.shape[0], inter), dtype=torch.float8_e4m3fn, device=DEV)
                    hsf = torch.zeros((a.shape[0], inter // 128), dtype=torch.float32, device=DEV)
                    deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu((a, a_sf), w1f, (hq, hsf), gl, rw,
                                                                      use_psum_layout=psum)
                else:
                    h = torch.empty((a.shape[0], 2 * inter), dtype=torch.bfloat16, device=DEV)
                    deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, a_sf), w1, h, gl, use_psum_layout=psum)
                    hq, hsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw, None if psum else gl)
                y = torch.empty((a.shape[0], hidden), dtype=torch.bfloat16, device=DEV)
                deep_gemm.m_grouped_fp8_gemm_nt_contiguous((hq, hsf), w2, y, gl, use_psum_layout=psum)
            outs[(layout, fused)] = deep_gemm.moe_combine(y, pos)
        torch.cuda.synchronize()
    ref = _layer_oracle(q, sf, idx, w, l1, l2)
    out = outs[('contiguous', True)].float().cpu().numpy()
    diff = ogemm.calc_diff(out, ref)
    print(f'fused moe layer calc_diff={diff:.3e} max_rel_err={ogemm.max_rel_err(out, ref):.3e}', flush=True)
    assert diff < 1e-3
    for key, val in outs.items():
        assert torch.equal(val.view(torch.int16), outs[('contiguous', False)].view(torch.int16)), key
