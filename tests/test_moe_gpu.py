"""GPU parity of the MoE plumbing (dispatch, SwiGLU -> FP8 cast, combine) and of a
whole one-GPU MoE layer built from it and the grouped GEMMs, against oracle/moe.py.

Bars: dispatch and combine are integer / copy / fixed-order float work and must
match the oracle bit for bit; the SwiGLU cast uses the device exp (a few ulps
from the float64 oracle), so its scales must agree to 4 ulps and its codes must
be equal or adjacent e4m3 codes (equal for >= 99.9%); the layer must match the
oracle's FP64 pipeline to calc_diff < 1e-3 (the reference's bar), and the three
layouts (contiguous, psum, masked) must give the same bits.
"""
import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import moe as omoe
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'


def _routing(t, k, e, seed, unrouted=0.1):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]) if k <= e else \
        rng.integers(0, e, size=(t, k))
    idx = np.where(rng.random((t, k)) < unrouted, -1, idx).astype(np.int32)
    w = rng.random((t, k)).astype(np.float32)
    return idx, w


def _x(t, kdim, seed):
    x = gen.randn_bf16((t, kdim), seed)
    q, sf = oquant.per_token_cast_to_fp8(x, use_ue8m0=False)
    return q, sf


@pytest.mark.parametrize('layout', ['contiguous', 'psum', 'masked'])
@pytest.mark.parametrize('t,k,e,kdim', [(1, 1, 4, 256), (100, 2, 8, 512), (1000, 8, 32, 1024), (300, 6, 256, 256),
                                         (4096, 8, 256, 512), (1024, 2, 1024, 128), (1025, 2, 1024, 128),
                                         (5000, 4, 64, 256), (20000, 2, 1024, 128), (70, 3, 5, 8320)])
def test_dispatch_vs_oracle(layout, t, k, e, kdim):
    """Dispatch against the oracle in all three layouts, from one token to
    config-scale calls (4096 tokens, top-8 over 256 experts). The last two cases
    cover the kernels' multi-round paths: 313 chunks of 64 tokens (the
    per-expert scan's 256-chunk rounds) over 1024 experts (every id bit in the
    ballot ranking), and rows of 8320 bytes with 65 scales (two 8 KB copy
    rounds, two 64-scale rounds)."""
    idx, w = _routing(t, k, e, seed=t + k + e)
    q, sf = _x(t, kdim, seed=t)
    max_m = 64 if layout == 'masked' else 0          # small enough that some experts overflow
    ref = omoe.dispatch(q, sf, idx, e, layout, alignment=128, max_m=max_m, topk_weights=w)
    for idx_dtype in (torch.int32, torch.int64):
        a, a_sf, gl, pos, rw = deep_gemm.moe_dispatch(
            (gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf)), torch.from_numpy(idx).to(idx_dtype).to(DEV), e,
            layout=layout, alignment=128, max_m=max_m or None, topk_weights=gen.to_dev(w))
        torch.cuda.synchronize()
        print(f'{deep_gemm.get_last_config()}', flush=True)
        assert np.array_equal(pos.cpu().numpy(), ref['pos'])
        a_h, sf_h, w_h = a.view(torch.uint8).cpu().numpy(), a_sf.cpu().numpy(), rw.cpu().numpy()
        if layout == 'masked':
            assert np.array_equal(gl.cpu().numpy(), ref['layout'])
            for ei in range(e):
                r = int(ref['layout'][ei])
                assert np.array_equal(a_h[ei, :r], ref['a'][ei, :r])
                assert np.array_equal(sf_h[ei, :r], ref['sf'][ei, :r])
                assert np.array_equal(w_h[ei, :r], ref['weights'][ei, :r])
        else:
            rows = ref['rows']
            assert np.array_equal(a_h[:rows], ref['a']) and np.array_equal(sf_h[:rows], ref['sf'])
            assert np.array_equal(w_h[:rows], ref['weights'])
            if layout == 'contiguous':
                m_idx = gl.cpu().numpy()
                assert np.array_equal(m_idx[:rows], ref['layout']) and np.all(m_idx[rows:] == -1)
            else:
                assert np.array_equal(gl.cpu().numpy(), ref['layout'])


def test_dispatch_empty_and_unrouted():
    e, kdim = 4, 256
    q, sf = _x(0, kdim, 1)
    a, a_sf, gl, pos, _ = deep_gemm.moe_dispatch((gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf)),
                                                 torch.zeros((0, 2), dtype=torch.int32, device=DEV), e)
    torch.cuda.synchronize()
    assert pos.numel() == 0 and bool((gl == -1).all())
    q, sf = _x(5, kdim, 2)
    idx = np.full((5, 2), -1, np.int32)
    idx[3, 1] = 7                                      # ids outside [0, E) are not routed either
    _, _, gl, pos, _ = deep_gemm.moe_dispatch((gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf)),
                                              gen.to_dev(idx), e, layout='psum')
    torch.cuda.synchronize()
    assert bool((pos == -1).all()) and bool((gl == 0).all())
    # int64 ids: 2^32 + e and -2^32 + e are outside [0, E) and stay unrouted (no
    # narrowing to e first); the oracle compares in int64 the same way
    idx64 = np.full((5, 2), -1, np.int64)
    idx64[0, 0], idx64[1, 1], idx64[2, 0], idx64[4, 1] = 2 ** 32 + 1, -(2 ** 32) + 2, 3, 2 ** 33
    ref = omoe.dispatch(q, sf, idx64, e, 'contiguous', alignment=128)
    _, _, gl, pos, _ = deep_gemm.moe_dispatch((gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf)),
                                              torch.from_numpy(idx64).to(DEV), e)
    torch.cuda.synchronize()
    assert np.array_equal(pos.cpu().numpy(), ref['pos'])
    assert int((pos >= 0).sum()) == 1 and int(pos[2, 0]) == 0


@pytest.mark.parametrize('gran,clamp', [(128, None), (32, None), (128, 7.0)])
def test_swiglu_cast_vs_oracle(gran, clamp):
    m, i = 300, 1024
    x = gen.randn_bf16((m, 2 * i), 11) * np.float32(3.0)
    x = oquant.bf16_round(x)
    rng = np.random.default_rng(12)
    w = rng.random(m).astype(np.float32)
    layout = np.where(rng.random(m) < 0.1, -1, 0).astype(np.int32)
    q, sf = deep_gemm.moe_swiglu_apply_weight_to_fp8(torch.from_numpy(x).bfloat16().to(DEV), gen.to_dev(w),
                                                     gen.to_dev(layout), clamp, gran)
    torch.cuda.synchronize()
    # rows marked padding are written as +0 codes (a product with 0 would give -0 for negative x)
    rq, rsf = omoe.swiglu_apply_weight_to_fp8(np.where((layout >= 0)[:, None], x, 0.0), w, clamp, gran)
    gq, gsf = q.view(torch.uint8).cpu().numpy(), sf.cpu().numpy()
    print(f'swiglu gran={gran} clamp={clamp}: codes equal {np.mean(gq == rq):.6f}, '
          f'scales equal {np.mean(gsf.view(np.int32) == rsf.view(np.int32)):.6f}', flush=True)
    # bit-exact: the kernel runs the oracle's float32 steps, exp included
    assert np.array_equal(gq, rq)
    assert np.array_equal(gsf.view(np.int32), rsf.view(np.int32))
    pad = layout < 0
    assert np.all(gq[pad] == 0)


def test_combine_slot_order():
    """The float32 sums run in slot order: rows 2^24, -2^24 and 1 give 1 for
    slots (0, 1, 2) and 0 for (0, 2, 1), as the oracle's do."""
    y = np.repeat(np.array([[2.0 ** 24], [-2.0 ** 24], [1.0]], np.float32), 8, axis=1)
    pos = np.array([[0, 1, 2], [0, 2, 1]], np.int32)
    out = deep_gemm.moe_combine(torch.from_numpy(y).bfloat16().to(DEV), gen.to_dev(pos), None)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.array_equal(got, omoe.combine(y, pos)) and np.all(got[0] == 1.0) and np.all(got[1] == 0.0)


@pytest.mark.parametrize('weighted', [False, True])
@pytest.mark.parametrize('masked', [False, True])
def test_combine_vs_oracle(weighted, masked):
    t, k, n, rows = 200, 4, 768, 1000
    rng = np.random.default_rng(21)
    y = oquant.bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    pos = rng.integers(-1, rows, size=(t, k)).astype(np.int32)
    w = rng.random((t, k)).astype(np.float32) if weighted else None
    ref = omoe.combine(y, pos, w)
    yd = torch.from_numpy(y).bfloat16().to(DEV)
    if masked:   # the same rows viewed as [E, max_m, N]
        yd = yd.view(10, 100, n)
    out = deep_gemm.moe_combine(yd, gen.to_dev(pos), gen.to_dev(w) if weighted else None)
    torch.cuda.synchronize()
    assert np.array_equal(out.float().cpu().numpy(), ref)


def test_combine_skips_rows_past_y():
    """pos entries at or past y's row count (E * max_m for a 3-D y) are skipped, as
    negative ones are: the result equals the oracle's combine with them set to -1."""
    t, k, n, rows = 64, 4, 256, 300
    rng = np.random.default_rng(22)
    y = oquant.bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    pos = rng.integers(-1, rows, size=(t, k)).astype(np.int32)
    pos[::3, 1] = rows                      # one past the end
    pos[::5, 2] = rows + 12345              # far past it
    pos[7, 0] = 2 ** 31 - 1
    w = rng.random((t, k)).astype(np.float32)
    ref = omoe.combine(y, np.where(pos >= rows, -1, pos), w)
    for yd in (torch.from_numpy(y).bfloat16().to(DEV), torch.from_numpy(y).bfloat16().to(DEV).view(3, 100, n)):
        out = deep_gemm.moe_combine(yd, gen.to_dev(pos), gen.to_dev(w))
        torch.cuda.synchronize()
        assert np.array_equal(out.float().cpu().numpy(), ref)


def _layer_oracle(q, sf, idx, w, l1, l2):
    """The MoE layer on the host: dispatch, L1 (FP64 dequantized GEMM, bf16 out),
    SwiGLU x weight -> FP8, L2, combine."""
    e = l1[0].shape[0]
    d = omoe.dispatch(q, sf, idx, e, 'contiguous', 128, topk_weights=w)
    a_deq = oquant.dequant_per_token(d['a'], d['sf'])
    h = np.zeros((d['rows'], l1[0].shape[1]), np.float32)
    for ei in range(e):
        rows = d['layout'] == ei
        if rows.any():
            h[rows] = oquant.bf16_round(ogemm.gemm_nt(a_deq[rows], oquant.dequant_per_block(l1[0][ei], l1[1][ei])))
    hq, hsf = omoe.swiglu_apply_weight_to_fp8(np.where((d['layout'] >= 0)[:, None], h, 0.0), d['weights'])
    h_deq = oquant.dequant_per_token(hq, hsf)
    y = np.zeros((d['rows'], l2[0].shape[1]), np.float32)
    for ei in range(e):
        rows = d['layout'] == ei
        if rows.any():
            y[rows] = oquant.bf16_round(ogemm.gemm_nt(h_deq[rows], oquant.dequant_per_block(l2[0][ei], l2[1][ei])))
    return omoe.combine(y, d['pos'])


def test_moe_layer_end_to_end():
    """A one-GPU MoE layer (8 experts, top-2, hidden 2048, intermediate 1024):
    dispatch -> L1 grouped GEMM -> SwiGLU x weight -> FP8 -> L2 grouped GEMM ->
    combine, on the contiguous, psum and masked layouts. All three give the same
    bits, and match the host pipeline to calc_diff < 1e-3."""
    t, k, e, hidden, inter = 256, 2, 8, 2048, 1024
    idx, w = _routing(t, k, e, seed=31, unrouted=0.05)
    q, sf = _x(t, hidden, 32)
    l1 = (np.empty((e, 2 * inter, hidden), np.uint8), np.empty((e, 2 * inter // 128, hidden // 128), np.float32))
    l2 = (np.empty((e, hidden, inter), np.uint8), np.empty((e, hidden // 128, inter // 128), np.float32))
    for ei in range(e):
        l1[0][ei], l1[1][ei] = oquant.per_block_cast_to_fp8(gen.randn_bf16((2 * inter, hidden), 40 + ei), False)
        l2[0][ei], l2[1][ei] = oquant.per_block_cast_to_fp8(gen.randn_bf16((hidden, inter), 60 + ei), False)
    w1 = (gen.to_dev(l1[0], torch.float8_e4m3fn), gen.to_dev(l1[1]))
    w2 = (gen.to_dev(l2[0], torch.float8_e4m3fn), gen.to_dev(l2[1]))
    x = (gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf))
    idx_d, w_d = gen.to_dev(idx), gen.to_dev(w)
    outs = {}
    for layout in ('contiguous', 'psum', 'masked'):
        max_m = 256 if layout == 'masked' else None
        a, a_sf, gl, pos, rw = deep_gemm.moe_dispatch(x, idx_d, e, layout=layout, max_m=max_m, topk_weights=w_d)
        if layout == 'masked':
            h = torch.empty((e, max_m, 2 * inter), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_masked((a, a_sf), w1, h, gl, expected_m=t * k // e)
            hq, hsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(e * max_m, 2 * inter), rw.view(-1))
            y = torch.empty((e, max_m, hidden), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_masked((hq.view(e, max_m, inter), hsf.view(e, max_m, -1)), w2, y, gl,
                                                   expected_m=t * k // e)
        else:
            psum = layout == 'psum'
            h = torch.empty((a.shape[0], 2 * inter), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, a_sf), w1, h, gl, use_psum_layout=psum)
            # contiguous: m_indices marks the padding rows; psum: they are zero rows of A
            hq, hsf = deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw, None if psum else gl)
            y = torch.empty((a.shape[0], hidden), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous((hq, hsf), w2, y, gl, use_psum_layout=psum)
        outs[layout] = deep_gemm.moe_combine(y, pos)
        torch.cuda.synchronize()
    ref = _layer_oracle(q, sf, idx, w, l1, l2)
    out = outs['contiguous'].float().cpu().numpy()
    diff = ogemm.calc_diff(out, ref)
    print(f'moe layer calc_diff={diff:.3e} max_rel_err={ogemm.max_rel_err(out, ref):.3e}', flush=True)
    assert diff < 1e-3
    for layout in ('psum', 'masked'):
        assert torch.equal(outs[layout].view(torch.int16), outs['contiguous'].view(torch.int16)), layout
