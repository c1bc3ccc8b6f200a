"""GPU parity of the 1D1D recipe (per-row 1x128 scales on both operands, FP32 D
accumulating into C): dense fp8_gemm_nt with recipe (1, 1, 128) and
k_grouped_fp8_gemm_nt_contiguous, against the oracle (oracle/gemm.py gemm_nt,
gemm_k_grouped), calc_diff < 1e-3 as the reference's FP8 bar
(tests/generators.py:69-74), plus bitwise determinism and the reference's
argument checks."""
import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def e4m3(x):
    return gen.to_dev(x, torch.float8_e4m3fn)


def f32(x):
    return gen.to_dev(np.asarray(x, dtype=np.float32))


def dense_1d1d(m, n, k, seed):
    a = gen.randn_bf16((m, k), seed)
    b = gen.randn_bf16((n, k), seed + 1)
    qa, sfa = oquant.per_token_cast_to_fp8(a, use_ue8m0=False)
    qb, sfb = oquant.per_token_cast_to_fp8(b, use_ue8m0=False)
    return qa, sfa, qb, sfb


@pytest.mark.parametrize('m,n,k,inplace', [(300, 520, 1024, True), (128, 256, 128, False), (1000, 2112, 2048, True),
                                           (77, 96, 384, False)])
def test_dense_1d1d_vs_oracle(m, n, k, inplace):
    print(f'1d1d dense m={m} n={n} k={k} inplace={inplace}', flush=True)
    qa, sfa, qb, sfb = dense_1d1d(m, n, k, m + n + k)
    c_np = np.random.default_rng(k).standard_normal((m, n)).astype(np.float32) * 4
    ref = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_token(qb, sfb), c_np)
    a, b = (e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb))
    c = f32(c_np)
    d = c if inplace else torch.full((m, n), float('nan'), device=DEV)
    deep_gemm.fp8_gemm_nt(a, b, d, c=c, recipe=(1, 1, 128))
    torch.cuda.synchronize()
    assert 'fp8_gemm_1d1d' in deep_gemm.get_last_config()
    out = d.cpu().numpy()
    diff = ogemm.calc_diff(out, ref)
    print(f'  calc_diff {diff:.3e} max_rel {ogemm.max_rel_err(out, ref):.3e}', flush=True)
    assert diff < 1e-3
    # bitwise determinism
    d2 = torch.empty_like(c)
    d3 = torch.empty_like(c)
    c2 = f32(c_np)
    deep_gemm.fp8_gemm_nt(a, b, d2, c=c2, recipe=(1, 1, 128))
    deep_gemm.fp8_gemm_nt(a, b, d3, c=c2, recipe=(1, 1, 128))
    assert torch.equal(d2.view(torch.int32), d3.view(torch.int32))


def test_dense_1d1d_argument_checks():
    qa, sfa, qb, sfb = dense_1d1d(64, 128, 256, 3)
    a, b = (e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb))
    d = torch.zeros((64, 128), device=DEV)
    with pytest.raises(RuntimeError, match='Assertion'):   # C is required
        deep_gemm.fp8_gemm_nt(a, b, d, recipe=(1, 1, 128))
    with pytest.raises(RuntimeError, match='Assertion'):   # FP32 D is required
        db = torch.zeros((64, 128), dtype=torch.bfloat16, device=DEV)
        deep_gemm.fp8_gemm_nt(a, b, db, c=db, recipe=(1, 1, 128))
    qa, sfa, qb, sfb = dense_1d1d(64, 128, 1000, 4)
    with pytest.raises(RuntimeError, match='Unsupported'):   # K % 128 != 0
        deep_gemm.fp8_gemm_nt((e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb)), d, c=d, recipe=(1, 1, 128))


def k_grouped_inputs(ks, m, n, seed):
    rng = np.random.default_rng(seed)
    qa_g, sa_g, qb_g, sb_g = [], [], [], []
    for i, k in enumerate(ks):
        if k == 0:
            continue
        qa, sfa = oquant.per_token_cast_to_fp8(gen.randn_bf16((m, k), seed + 2 * i), use_ue8m0=False)
        qb, sfb = oquant.per_token_cast_to_fp8(gen.randn_bf16((n, k), seed + 2 * i + 1), use_ue8m0=False)
        qa_g.append(qa.reshape(-1)), sa_g.append(sfa), qb_g.append(qb.reshape(-1)), sb_g.append(sfb)
    qa = np.concatenate(qa_g) if qa_g else np.zeros(0, np.uint8)
    qb = np.concatenate(qb_g) if qb_g else np.zeros(0, np.uint8)
    sfa = np.concatenate(sa_g, axis=1) if sa_g else np.zeros((m, 0), np.float32)
    sfb = np.concatenate(sb_g, axis=1) if sb_g else np.zeros((n, 0), np.float32)
    c = (rng.standard_normal((len(ks), m, n)) * 32).astype(np.float32)
    return qa, sfa, qb, sfb, c


@pytest.mark.parametrize('ks,m,n,mn_major_sf', [([256, 0, 512, 128], 256, 384, False),
                                                ([128, 384, 0, 256, 128], 200, 264, True),
                                                ([1024, 896], 768, 512, True)])
def test_k_grouped_vs_oracle(ks, m, n, mn_major_sf):
    print(f'k-grouped ks={ks} m={m} n={n} mn_major_sf={mn_major_sf}', flush=True)
    qa, sfa, qb, sfb, c_np = k_grouped_inputs(ks, m, n, sum(ks) + m)
    ref = ogemm.gemm_k_grouped(qa, sfa, qb, sfb, ks, c_np, oquant.dequant_per_token)
    sa_t, sb_t = f32(sfa), f32(sfb)
    if mn_major_sf:   # the reference generator hands over sf.T views (strides (1, mn))
        sa_t = f32(np.ascontiguousarray(sfa.T)).t()
        sb_t = f32(np.ascontiguousarray(sfb.T)).t()
    d = f32(c_np)
    layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
    deep_gemm.k_grouped_fp8_gemm_nt_contiguous((e4m3(qa), sa_t), (e4m3(qb), sb_t), d, ks, layout, d)
    torch.cuda.synchronize()
    assert 'k_grouped' in deep_gemm.get_last_config()
    out = d.cpu().numpy()
    diff = ogemm.calc_diff(out, ref)
    print(f'  calc_diff {diff:.3e} max_rel {ogemm.max_rel_err(out, ref):.3e}', flush=True)
    assert diff < 1e-3
    for i, k in enumerate(ks):
        if k == 0:
            assert np.array_equal(out[i], c_np[i])   # an empty group leaves C
    # 20 reruns bitwise identical (reference tests/test_fp8_fp4.py:287-298)
    first = None
    for _ in range(20):
        d2 = f32(c_np)
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous((e4m3(qa), sa_t), (e4m3(qb), sb_t), d2, ks, layout, d2)
        if first is None:
            first = d2
        else:
            assert torch.equal(d2.view(torch.int32), first.view(torch.int32))


def test_k_grouped_group_equals_dense_1d1d():
    """One group of a K-grouped call equals the dense 1D1D call on its slice, bit for bit."""
    ks, m, n = [384, 256], 256, 512
    qa, sfa, qb, sfb, c_np = k_grouped_inputs(ks, m, n, 5)
    d = f32(c_np)
    layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
    deep_gemm.k_grouped_fp8_gemm_nt_contiguous((e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb)), d, ks, layout, d)
    k1 = ks[1]
    a1 = qa[ks[0] * m:].reshape(m, k1)
    b1 = qb[ks[0] * n:].reshape(n, k1)
    dd = f32(c_np[1])
    deep_gemm.fp8_gemm_nt((e4m3(a1), f32(sfa[:, 3:])), (e4m3(b1), f32(sfb[:, 3:])), dd, c=dd, recipe=(1, 1, 128))
    torch.cuda.synchronize()
    assert torch.equal(dd.view(torch.int32), d[1].view(torch.int32))


def test_k_grouped_empty_and_checks():
    ks, m, n = [0, 0], 64, 128
    c_np = np.random.default_rng(1).standard_normal((2, m, n)).astype(np.float32)
    c = f32(c_np)
    d = torch.zeros_like(c)
    layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
    empty = torch.empty(0, dtype=torch.float8_e4m3fn, device=DEV)
    sf_a, sf_b = torch.empty((m, 0), device=DEV), torch.empty((n, 0), device=DEV)
    deep_gemm.k_grouped_fp8_gemm_nt_contiguous((empty, sf_a), (empty, sf_b), d, ks, layout, c)
    torch.cuda.synchronize()
    assert torch.equal(d, c)   # sum K = 0: D = C
    ks = [128, 256]
    qa, sfa, qb, sfb, c_np = k_grouped_inputs(ks, m, n, 2)
    a, b = (e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb))
    d = f32(c_np)
    layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match='Assertion'):   # recipe must be (1, 1, 128)
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, ks, layout, d, recipe=(1, 1, 32))
    with pytest.raises(RuntimeError, match='Assertion'):   # no psum layout on FP8 NT
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, ks, layout, d, use_psum_layout=True)
    with pytest.raises(RuntimeError, match='Assertion'):   # C is required
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, ks, layout)
    with pytest.raises(RuntimeError, match='Assertion'):   # K not a multiple of 128
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, [100, 284], layout, d)
    with pytest.raises(RuntimeError, match='Unsupported'):
        deep_gemm.k_grouped_fp8_gemm_tn_contiguous(a, b, d, ks, layout, d)


@pytest.mark.parametrize('kg', [False, True])
def test_1d1d_kernels_bitwise_equal(kg):
    """The 128 x 128 pipelined 1D1D kernel (variant 7, the default) and the 128-row
    streaming one (variant 6) compute the same bits."""
    outs = []
    for v, tile in [(7, (128, 128)), (6, (128, 256)), (6, (128, 192))]:
        deep_gemm.set_tile_override(tile[0], tile[1], variant=v)
        try:
            if kg:
                ks, m, n = [384, 0, 256, 128], 300, 456
                qa, sfa, qb, sfb, c_np = k_grouped_inputs(ks, m, n, 9)
                d = f32(c_np)
                layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
                deep_gemm.k_grouped_fp8_gemm_nt_contiguous((e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb)), d, ks,
                                                           layout, d)
            else:
                qa, sfa, qb, sfb = dense_1d1d(520, 600, 1152, 8)
                d = f32(np.random.default_rng(3).standard_normal((520, 600)))
                deep_gemm.fp8_gemm_nt((e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb)), d, c=d, recipe=(1, 1, 128))
            cfg = deep_gemm.get_last_config()
        finally:
            deep_gemm.set_tile_override(0, 0)
        torch.cuda.synchronize()
        assert f' v{v} ' in cfg, cfg
        outs.append(d)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32))


def test_k_grouped_chunked_group_order():
    """Eight groups whose tile count (8 x 6 = 48 tiles of 128 x 128) is a multiple of
    8: the launch walks the groups in chunks of 6 tiles, so each XCD holds a chunk
    of every group. Against the oracle, an empty group leaves C, and each group
    equals the dense 1D1D call on its slice bit for bit."""
    ks, m, n = [512, 0, 384, 1024, 128, 256, 640, 768], 1024, 768
    print(f'k-grouped chunked ks={ks} m={m} n={n}', flush=True)
    qa, sfa, qb, sfb, c_np = k_grouped_inputs(ks, m, n, 77)
    ref = ogemm.gemm_k_grouped(qa, sfa, qb, sfb, ks, c_np, oquant.dequant_per_token)
    d = f32(c_np)
    layout = torch.tensor(ks, dtype=torch.int32, device=DEV)
    deep_gemm.k_grouped_fp8_gemm_nt_contiguous((e4m3(qa), f32(sfa)), (e4m3(qb), f32(sfb)), d, ks, layout, d)
    torch.cuda.synchronize()
    out = d.cpu().numpy()
    diff = ogemm.calc_diff(out, ref)
    print(f'  calc_diff {diff:.3e}', flush=True)
    assert diff < 1e-3
    kb0 = 0
    for g, k in enumerate(ks):
        if k == 0:
            assert np.array_equal(out[g], c_np[g])
            continue
        off = sum(ks[:g])
        a_g = qa[off * m:(off + k) * m].reshape(m, k)
        b_g = qb[off * n:(off + k) * n].reshape(n, k)
        dd = f32(c_np[g])
        deep_gemm.fp8_gemm_nt((e4m3(a_g), f32(sfa[:, kb0:kb0 + k // 128])), (e4m3(b_g), f32(sfb[:, kb0:kb0 + k // 128])),
                              dd, c=dd, recipe=(1, 1, 128))
        torch.cuda.synchronize()
        assert torch.equal(dd.view(torch.int32), d[g].view(torch.int32)), f'group {g}'
        kb0 += k // 128
