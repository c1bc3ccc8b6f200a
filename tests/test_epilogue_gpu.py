"""GPU tests of the UE8M0-path epilogues: alpha / epilogue.Alpha, epilogue.Identity
and epilogue.FP8Quantization (reference csrc/jit_kernels/impls/epilogue_class.hpp:
19-124, deep_gemm/include/deep_gemm/epilogue/operators.cuh).

Bars:
  * Alpha scales the FP32 product with one multiply before C is added, so an FP32 D
    equals alpha * D(alpha = None) (+ C) computed in FP32 by torch, bit for bit, on
    both UE8M0 kernels; BF16 D equals that FP32 value rounded to BF16.
  * Identity gives the same bits as no epilogue.
  * FP8Quantization gives bitwise the oracle's per-32-column UE8M0 cast of the BF16
    D (the reference's definition of its fused epilogue, operators.cuh:65-69), with
    the scale bytes packed as the oracle packs MN-major UE8M0 words.
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
EP = deep_gemm.epilogue


def _operands(m, n, k, seed):
    """Config-5 operands: A e4m3 (1 x 128 UE8M0), B e2m1 (1 x 32 UE8M0), packed words."""
    qa, sfa = oquant.per_token_cast_to_fp8(gen.randn_bf16((m, k), seed), use_ue8m0=True, gran_k=128)
    qb, sfb = oquant.per_token_cast_to_fp4(gen.randn_bf16((n, k), seed + 1), use_ue8m0=True, gran_k=32)
    ref = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa, 128), oquant.dequant_fp4(qb, sfb, 32))
    pack = lambda s: deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(gen.to_dev(np.asarray(s, np.float32)))
    a = (gen.to_dev(qa, torch.float8_e4m3fn), pack(sfa))
    b = (gen.to_dev(qb, torch.int8), pack(sfb))
    return a, b, ref


def _each_kernel(fn):
    """fn() on the 128 x 128 UE8M0 kernel and on the pipelined 256 x 256 one."""
    outs = []
    try:
        for v, bm, bn in ((1, 128, 128), (2, 256, 256)):
            deep_gemm.set_tile_override(bm, bn, variant=v)
            outs.append(fn())
            print(deep_gemm.get_last_config(), flush=True)
    finally:
        deep_gemm.set_tile_override(0, 0)
    return outs


@pytest.mark.parametrize('m,n,k', [(384, 512, 512), (300, 520, 640)])
@pytest.mark.parametrize('alpha', [0.37, -2.5])
def test_alpha_dense(m, n, k, alpha):
    a, b, ref = _operands(m, n, k, seed=m + k)
    c = torch.from_numpy(gen.randn_bf16((m, n), 7)).to(DEV)

    def run(dtype, with_c, al, ep=None):
        d = torch.empty((m, n), dtype=dtype, device=DEV)
        deep_gemm.fp8_fp4_gemm_nt(a, b, d, c=c.to(dtype) if with_c else None, recipe_a=(1, 128),
                                  recipe_b=(1, 32), alpha=al, epilogue=ep)
        torch.cuda.synchronize()
        return d

    for plain, scaled, scaled_c, scaled_bf16, via_class, ident in _each_kernel(lambda: (
            run(torch.float32, False, None), run(torch.float32, False, alpha), run(torch.float32, True, alpha),
            run(torch.bfloat16, False, alpha), run(torch.float32, False, None, EP.Alpha(alpha)),
            run(torch.float32, False, None, EP.Identity()))):
        expect = plain * alpha          # one FP32 multiply, round to nearest even
        assert torch.equal(scaled, expect)
        assert torch.equal(via_class, expect)
        assert torch.equal(scaled_c, expect + c.float())
        assert torch.equal(scaled_bf16.view(torch.int16), expect.bfloat16().view(torch.int16))
        assert torch.equal(ident, plain)
        diff = ogemm.calc_diff(scaled_c.cpu().numpy(), alpha * ref + c.float().cpu().numpy())
        print(f'alpha={alpha} {m}x{n}x{k} calc_diff={diff:.3e}', flush=True)
        assert diff < 1e-6


def test_alpha_grouped():
    """epilogue.Alpha on the masked and contiguous UE8M0 layouts, against the oracle."""
    g, max_m, n, k = 3, 192, 256, 512
    alpha = 1.75
    qa, sfa, qb, sfb, refs = [], [], [], [], []
    for i in range(g):
        x_a, s_a = oquant.per_token_cast_to_fp8(gen.randn_bf16((max_m, k), 20 + i), use_ue8m0=True, gran_k=128)
        x_b, s_b = oquant.per_token_cast_to_fp4(gen.randn_bf16((n, k), 40 + i), use_ue8m0=True, gran_k=32)
        qa.append(x_a), sfa.append(s_a), qb.append(x_b), sfb.append(s_b)
        refs.append(ogemm.gemm_nt(oquant.dequant_per_token(x_a, s_a, 128), oquant.dequant_fp4(x_b, s_b, 32)))
    pack = lambda s: deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(gen.to_dev(np.asarray(s, np.float32)))
    a = (gen.to_dev(np.stack(qa), torch.float8_e4m3fn), pack(np.stack(sfa)))
    b = (gen.to_dev(np.stack(qb), torch.int8), pack(np.stack(sfb)))
    masked_m = torch.tensor([192, 77, 0], dtype=torch.int32, device=DEV)
    d = torch.zeros((g, max_m, n), dtype=torch.bfloat16, device=DEV)
    deep_gemm.m_grouped_fp8_fp4_gemm_nt_masked(a, b, d, masked_m, 128, recipe_a=(1, 128), recipe_b=(1, 32),
                                               epilogue=EP.Alpha(alpha))
    torch.cuda.synchronize()
    out = d.float().cpu().numpy()
    for i, mm in enumerate([192, 77, 0]):
        if mm:
            diff = ogemm.calc_diff(out[i, :mm], alpha * refs[i][:mm])
            print(f'masked alpha group {i} calc_diff={diff:.3e}', flush=True)
            assert diff < 1e-5
        assert not out[i, mm:].any()   # rows >= masked_m untouched (zeros here)
    # contiguous: three 192-row segments (128-aligned: 256 rows each, padding marked -1)
    rows = []
    idx = []
    for i in range(g):
        rows.append(np.concatenate([qa[i], np.zeros((64, k), np.uint8)]))
        idx += [i] * 192 + [-1] * 64
    s_rows = [np.concatenate([sfa[i], np.ones((64, k // 128), np.float32)]) for i in range(g)]
    a_c = (gen.to_dev(np.concatenate(rows), torch.float8_e4m3fn), pack(np.concatenate(s_rows)))
    layout = torch.tensor(idx, dtype=torch.int32, device=DEV)
    d_c = torch.zeros((g * 256, n), dtype=torch.bfloat16, device=DEV)
    d_i = torch.zeros_like(d_c)
    deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous(a_c, b, d_c, layout, recipe_a=(1, 128), recipe_b=(1, 32),
                                                   epilogue=EP.Alpha(alpha))
    deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous(a_c, b, d_i, layout, recipe_a=(1, 128), recipe_b=(1, 32),
                                                   epilogue=EP.Identity())
    torch.cuda.synchronize()
    out = d_c.float().cpu().numpy()
    for i in range(g):
        diff = ogemm.calc_diff(out[256 * i:256 * i + 192], alpha * refs[i])
        print(f'contiguous alpha group {i} calc_diff={diff:.3e}', flush=True)
        assert diff < 1e-5
    d_n = torch.zeros_like(d_c)
    deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous(a_c, b, d_n, layout, recipe_a=(1, 128), recipe_b=(1, 32))
    assert torch.equal(d_i.view(torch.int16), d_n.view(torch.int16))


@pytest.mark.parametrize('m,n,k', [(300, 520, 640), (256, 512, 1024), (64, 96, 0)])
def test_fp8_quantization(m, n, k):
    kk = max(k, 128)
    a, b, _ = _operands(m, n, kk, seed=3)
    if k == 0:   # (an empty problem returns before its scales are read)
        a = (a[0][:, :0], torch.zeros((m, 0), dtype=torch.int32, device=DEV))
        b = (b[0][:, :0], torch.zeros((n, 0), dtype=torch.int32, device=DEV))
    words = ((n + 31) // 32 + 3) // 4
    am = (m + 3) // 4 * 4
    d8 = torch.full((m, n), 0x7E, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    sfd = torch.empty_strided((m, words), (1, am), dtype=torch.int32, device=DEV).fill_(0x55)
    deep_gemm.fp8_fp4_gemm_nt(a, b, d8, recipe_a=(1, 128), recipe_b=(1, 32), epilogue=EP.FP8Quantization(sfd))
    torch.cuda.synchronize()
    if k == 0:
        assert not d8.view(torch.uint8).any() and not sfd.any()
        return
    d16 = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    deep_gemm.fp8_fp4_gemm_nt(a, b, d16, recipe_a=(1, 128), recipe_b=(1, 32))
    torch.cuda.synchronize()
    codes, sf = oquant.per_token_cast_to_fp8(d16.float().cpu().numpy(), use_ue8m0=True, gran_k=32)
    assert np.array_equal(d8.view(torch.uint8).cpu().numpy(), codes)
    packed = ogemm.pack_ue8m0_mn_major(sf)[0]          # [words, align(m, 4)]
    assert np.array_equal(sfd.cpu().numpy(), packed[:, :m].T)
    print(f'fp8 quantization {m}x{n}x{k}: codes and {words} SF words per row bit-exact', flush=True)


def test_fp32_scale_path_rejects_epilogues():
    """The FP32-scale path takes no alpha or epilogue class (reference csrc/apis/gemm.hpp:118-119)."""
    x = gen.dense_inputs(128, 256, 256, seed=1)
    a = (gen.to_dev(x['qa'], torch.float8_e4m3fn), gen.to_dev(x['sfa']))
    b = (gen.to_dev(x['qb'], torch.float8_e4m3fn), gen.to_dev(x['sfb']))
    d = torch.empty((128, 256), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match='need UE8M0 scales'):
        deep_gemm.fp8_gemm_nt(a, b, d, alpha=2.0)
    with pytest.raises(RuntimeError, match='need UE8M0 scales'):
        deep_gemm.fp8_gemm_nt(a, b, d, epilogue=EP.Identity())
