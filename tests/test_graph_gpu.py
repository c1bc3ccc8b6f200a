"""HIP graph capture of the library's launches.

The library allocates nothing and records no memset, so a call made while a
stream captures is recorded as its kernels alone. Each test runs a call
eagerly, captures the same call into a graph, and replays it several times with
eager work (an overwrite of the outputs) and a synchronisation between
replays; every replay must reproduce the eager bits.
"""
import numpy as np
import pytest
import torch

import deep_gemm
import generators as gen

pytestmark = pytest.mark.gpu
DEV = 'cuda'
REPLAYS = 4


def e4m3(x):
    return gen.to_dev(x, torch.float8_e4m3fn)


def f32(x):
    return gen.to_dev(np.asarray(x, dtype=np.float32))


def bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32) if t.element_size() == 4 \
        else t.view(torch.uint8)


def replay_matches_eager(run, out, written=None):
    """run() writes `out` (the rows where `written` is true, else all of it);
    compare graph replays of it with one eager call. Rows it does not write
    must keep what the eager work between replays put there."""
    run()
    torch.cuda.synchronize()
    sel = (lambda t: t[written]) if written is not None else (lambda t: t)
    ref = bits(sel(out)).clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for i in range(REPLAYS):
        bits(out).fill_(0x5A + i)      # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(sel(out)), ref), f'replay {i} differs from the eager call'
        if written is not None:
            assert bool((bits(out[~written]) == 0x5A + i).all()), 'rows the call must not write were written'


def test_graph_dense_bf16_and_accumulate():
    print('graph dense m=520 n=768 k=1024', flush=True)
    m, n, k = 520, 768, 1024
    x = gen.dense_inputs(m, n, k, seed=21)
    a, b = (e4m3(x['qa']), f32(x['sfa'])), (e4m3(x['qb']), f32(x['sfb']))
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    replay_matches_eager(lambda: deep_gemm.fp8_gemm_nt(a, b, d), d)
    c = torch.randn((m, n), generator=torch.Generator().manual_seed(3)).to(DEV)
    d32 = torch.empty((m, n), dtype=torch.float32, device=DEV)
    replay_matches_eager(lambda: deep_gemm.fp8_gemm_nt(a, b, d32, c=c), d32)


def test_graph_grouped_contiguous_and_masked():
    print('graph contiguous g=4 / masked g=4', flush=True)
    ms, aligned = gen.contiguous_sizes(4, 900, seed=5)
    n, k = 512, 1024
    x = gen.contiguous_inputs(ms, aligned, n, k, seed=22)
    a, b = (e4m3(x['qa']), f32(x['sfa'])), (e4m3(x['qb']), f32(x['sfb']))
    idx = gen.to_dev(x['m_indices'])
    d = torch.zeros((sum(aligned), n), dtype=torch.bfloat16, device=DEV)
    # padding rows (m_indices == -1) are left untouched
    replay_matches_eager(lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a, b, d, idx), d, written=idx >= 0)

    y = gen.masked_inputs(4, 256, n, k, seed=23)
    a, b = (e4m3(y['qa']), f32(y['sfa'])), (e4m3(y['qb']), f32(y['sfb']))
    mm = gen.to_dev(y['masked_m'])
    dm = torch.zeros((4, 256, n), dtype=torch.bfloat16, device=DEV)
    # rows >= masked_m are left untouched
    valid = torch.arange(256, device=DEV)[None, :] < mm[:, None]
    replay_matches_eager(lambda: deep_gemm.m_grouped_fp8_gemm_nt_masked(a, b, dm, mm, 128), dm, written=valid)


def test_graph_fp8_fp4_packed():
    print('graph fp8xfp4 m=256 n=512 k=1024', flush=True)
    m, n, k = 256, 512, 1024
    x = gen.fp8_fp4_inputs(m, n, k, seed=24)
    sfa = deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(f32(x['sfa']))
    sfb = deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(f32(x['sfb']))
    a, b = (e4m3(x['qa']), sfa), (gen.to_dev(x['qb'], torch.int8), sfb)
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    replay_matches_eager(lambda: deep_gemm.fp8_fp4_gemm_nt(a, b, d, recipe_a=(1, 128), recipe_b=(1, 32)), d)


def test_graph_cast():
    print('graph per_token_cast m=300 k=1536', flush=True)
    xb = torch.from_numpy(gen.randn_bf16((300, 1536), 25)).bfloat16().to(DEV)
    q0, sf0 = deep_gemm.per_token_cast_to_fp8_mn_major(xb, use_ue8m0=False)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q, sf = deep_gemm.per_token_cast_to_fp8_mn_major(xb, use_ue8m0=False)
    for i in range(REPLAYS):
        q.view(torch.uint8).fill_(0x5A + i)
        sf.fill_(float(i))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
        assert torch.equal(sf.view(torch.int32), sf0.view(torch.int32))


def test_graph_split_calls():
    """Calls that run as two launches (a dense column split, a contiguous row
    split) capture as both kernels and replay bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(9)
    m, n, k = 4096, 7168, 4096
    a = deep_gemm.per_token_cast_to_fp8(torch.randn((m, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    b = deep_gemm.per_block_cast_to_fp8(torch.randn((n, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    print('graph dense split 4096x7168x4096', flush=True)
    replay_matches_eager(lambda: deep_gemm.fp8_gemm_nt(a, b, d), d)
    assert 'split_n=' in deep_gemm.get_last_config()

    ms, aligned = gen.contiguous_sizes(8, 8192, seed=7)   # 8832 rows: 35 M blocks, 2.2 rounds
    n, k = 4096, 4096
    m_pad = sum(aligned)
    layout_np = np.full(m_pad, -1, dtype=np.int32)
    start = 0
    for e, (mi, ai) in enumerate(zip(ms, aligned)):
        layout_np[start:start + mi] = e
        start += ai
    layout = gen.to_dev(layout_np)
    ca = deep_gemm.per_token_cast_to_fp8(torch.randn((m_pad, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    bq = torch.empty((8, n, k), dtype=torch.float8_e4m3fn, device=DEV)
    bs = torch.empty((8, n // 128, k // 128), device=DEV)
    for e in range(8):
        bq[e], bs[e] = deep_gemm.per_block_cast_to_fp8(torch.randn((n, k), generator=g, device=DEV).bfloat16(),
                                                       use_ue8m0=False)
    dc = torch.empty((m_pad, n), dtype=torch.bfloat16, device=DEV)
    print(f'graph contiguous split m_pad={m_pad}', flush=True)
    replay_matches_eager(lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous(ca, (bq, bs), dc, layout), dc,
                         written=torch.from_numpy(layout_np >= 0).to(DEV))
    assert 'split_m=' in deep_gemm.get_last_config()


def test_graph_persistent_call():
    """A call routed to persistent workgroups (config 2's 4096 x 24576 x 1536: six
    rounds of tiles) captures and replays bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(10)
    m, n, k = 4096, 24576, 1536
    a = deep_gemm.per_token_cast_to_fp8(torch.randn((m, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    b = deep_gemm.per_block_cast_to_fp8(torch.randn((n, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    print('graph persistent 4096x24576x1536', flush=True)
    replay_matches_eager(lambda: deep_gemm.fp8_gemm_nt(a, b, d), d)
    if deep_gemm.get_num_sms() >= 256:
        assert ' v4 ' in deep_gemm.get_last_config()


@pytest.mark.parametrize('layout', ['contiguous', 'masked'])
def test_graph_moe_layer(layout):
    """The one-GPU MoE layer captured whole (dispatch, the L1 GEMM with the fused
    SwiGLU x weight -> FP8 epilogue, the L2 GEMM, combine; the workspace and the
    intermediate tensors come from torch's graph pool): every replay reproduces
    the eager layer output, routing and dispatched rows bit for bit."""
    print(f'graph moe layer {layout}', flush=True)
    t, topk, e, hidden, inter = 300, 2, 8, 512, 256
    rng = np.random.default_rng(31)
    xq, xsf = deep_gemm.per_token_cast_to_fp8(
        torch.from_numpy(gen.randn_bf16((t, hidden), 32)).bfloat16().to(DEV), use_ue8m0=False)
    idx = torch.from_numpy(np.stack([rng.choice(e, size=topk, replace=False) for _ in range(t)]).astype(np.int32)).to(DEV)
    w = torch.from_numpy(rng.random((t, topk)).astype(np.float32)).to(DEV)
    w1 = torch.empty((e, 2 * inter, hidden), dtype=torch.float8_e4m3fn, device=DEV)
    w1s = torch.empty((e, 2 * inter // 128, hidden // 128), device=DEV)
    w2 = torch.empty((e, hidden, inter), dtype=torch.float8_e4m3fn, device=DEV)
    w2s = torch.empty((e, hidden // 128, inter // 128), device=DEV)
    for i in range(e):
        w1[i], w1s[i] = deep_gemm.per_block_cast_to_fp8(
            torch.from_numpy(gen.randn_bf16((2 * inter, hidden), 40 + i)).bfloat16().to(DEV), use_ue8m0=False)
        w2[i], w2s[i] = deep_gemm.per_block_cast_to_fp8(
            torch.from_numpy(gen.randn_bf16((hidden, inter), 60 + i)).bfloat16().to(DEV), use_ue8m0=False)
    w1f = deep_gemm.transform_l1_weights_for_swiglu((w1, w1s))
    max_m = 256

    def layer():
        if layout == 'contiguous':
            a, asf, gl, pos, rw = deep_gemm.moe_dispatch((xq, xsf), idx, e, 'contiguous', topk_weights=w)
            q = torch.empty((a.shape[0], inter), dtype=torch.float8_e4m3fn, device=DEV)
            qs = torch.empty((a.shape[0], inter // 128), device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu((a, asf), w1f, (q, qs), gl, rw)
            y = torch.empty((a.shape[0], hidden), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous((q, qs), (w2, w2s), y, gl)
        else:
            a, asf, gl, pos, rw = deep_gemm.moe_dispatch((xq, xsf), idx, e, 'masked', max_m=max_m, topk_weights=w)
            q = torch.empty((e, max_m, inter), dtype=torch.float8_e4m3fn, device=DEV)
            qs = torch.empty((e, max_m, inter // 128), device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu((a, asf), w1f, (q, qs), gl, 128, rw)
            y = torch.empty((e, max_m, hidden), dtype=torch.bfloat16, device=DEV)
            deep_gemm.m_grouped_fp8_gemm_nt_masked((q, qs), (w2, w2s), y, gl, 128)
        out = deep_gemm.moe_combine(y, pos)
        return out, gl, pos

    ref = [r.clone() for r in layer()]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = layer()
    for i in range(REPLAYS):
        for r in got:
            bits(r).fill_(0x5A + i)      # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for r, r0 in zip(got, ref):
            assert torch.equal(bits(r), bits(r0)), f'replay {i} differs from the eager layer'
