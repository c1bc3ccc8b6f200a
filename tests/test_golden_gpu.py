"""GPU results against the stored fixtures in tests/golden/ (written by
tests/golden/make_golden.py from the CPU oracle and checked against it by
tests/test_oracle.py): the stored quantized inputs go through the library, and
its outputs are compared with the stored FP64 results. The device quantizer must
reproduce the stored codes and scales bit for bit, and every dense kernel
family (the default route, the tiled kernels, the tiny-M and split-K decode
kernels, the UE8M0 scaled-MFMA kernels) must match the stored output within one
BF16 ulp plus 2^-15 x sum |a b|, the bound the other parity tests use."""
import os

import numpy as np
import pytest
import torch

import deep_gemm
from oracle import gemm as ogemm
from oracle import quant as oquant

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def _load(name):
    with np.load(os.path.join(GOLDEN, name)) as f:   # plain arrays (no pickles)
        return {k: f[k] for k in f.files}


def _dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.view(dtype) if dtype is not None else t).to(DEV)


def _check(out, ref, s_abs, what):
    diff = ogemm.calc_diff(out, ref)
    print(f'{what}: calc_diff {diff:.3e}', flush=True)
    assert diff < 1e-3
    assert np.all(np.abs(out - ref) <= np.abs(ref) * 2.0 ** -8 + 2.0 ** -15 * s_abs), what


def test_golden_dense():
    g = _load('dense_fp8_small.npz')
    m, k = g['qa'].shape
    n = g['qb'].shape[0]
    # the device quantizer reproduces the stored codes and scales
    q, sf = deep_gemm.per_token_cast_to_fp8(_dev(g['a']).bfloat16(), use_ue8m0=False)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), g['qa'])
    assert np.array_equal(sf.cpu().numpy().view(np.int32), g['sfa'].view(np.int32))
    a = (_dev(g['qa'], torch.float8_e4m3fn), _dev(g['sfa']))
    b = (_dev(g['qb'], torch.float8_e4m3fn), _dev(g['sfb']))
    s_abs = ogemm.gemm_nt(np.abs(oquant.dequant_per_token(g['qa'], g['sfa'])),
                          np.abs(oquant.dequant_per_block(g['qb'], g['sfb'])))
    for override in [(0, 0, 0), (128, 128, 2), (256, 128, 2), (128, 128, 1), (32, 32, 9), (16, 16, 8), (0, 0, 10),
                     (0, 3, 10)]:
        deep_gemm.set_tile_override(override[0], override[1], variant=override[2])
        try:
            d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
            deep_gemm.fp8_gemm_nt(a, b, d)
            cfg = deep_gemm.get_last_config()
        finally:
            deep_gemm.set_tile_override(0, 0)
        torch.cuda.synchronize()
        if override[2]:
            assert f' v{override[2]} ' in cfg, cfg
        _check(d.float().cpu().numpy(), g['d'], s_abs, f'golden dense [{cfg.split(" kind")[0]}]')


def test_golden_fp8_fp4():
    g = _load('fp8_fp4_small.npz')
    m, n = g['qa'].shape[0], g['qb'].shape[0]
    a = (_dev(g['qa'], torch.float8_e4m3fn), _dev(g['sfa']))
    b = (_dev(g['qb'], torch.int8), _dev(g['sfb']))
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    deep_gemm.fp8_fp4_gemm_nt(a, b, d, recipe_a=(1, 128), recipe_b=(1, 32))
    torch.cuda.synchronize()
    a_deq = oquant.dequant_per_token(g['qa'], g['sfa'], gran_k=128)
    b_deq = oquant.dequant_fp4(g['qb'], g['sfb'], gran_k=32)
    s_abs = ogemm.gemm_nt(np.abs(a_deq), np.abs(b_deq))
    _check(d.float().cpu().numpy(), g['d'], s_abs, f'golden fp8 x fp4 [{deep_gemm.get_last_config().split(" kind")[0]}]')
