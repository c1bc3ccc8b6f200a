"""The reference's testing helpers on the GPU (deep_gemm.testing, reference
deep_gemm/testing/bench.py:7-146): bench_kineto times each named kernel."""
import pytest
import torch

import deep_gemm
from deep_gemm.testing import bench, bench_kineto
import generators as gen

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'


def _gemm_call(m=512, n=1024, k=2048):
    x = gen.dense_inputs(m, n, k, seed=3)
    a = (gen.to_dev(x['qa'], torch.float8_e4m3fn), gen.to_dev(x['sfa']))
    b = (gen.to_dev(x['qb'], torch.float8_e4m3fn), gen.to_dev(x['sfb']))
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    return lambda: deep_gemm.fp8_gemm_nt(a, b, d)


def test_bench_kineto_times_named_kernels():
    call = _gemm_call()
    t = bench_kineto(call, 'fp8_gemm', num_tests=10)
    t_call = bench(call, num_warmups=2, num_tests=10, flush_cache=True)
    print(f'bench_kineto fp8_gemm: {t * 1e6:.1f} us, bench (whole call): {t_call * 1e6:.1f} us', flush=True)
    assert 0 < t < 1e-2
    assert t <= t_call * 1.5
    # a tuple gives a tuple; a name that matches no kernel gives 0
    both = bench_kineto(call, ('fp8_gemm', 'no_such_kernel_name'), num_tests=5)
    assert isinstance(both, tuple) and both[0] > 0 and both[1] == 0


def test_bench_kineto_rejects_ambiguous_names():
    ca = _gemm_call(256, 512, 1024)
    x = torch.randn(1 << 20, device=DEV)

    def two_kernels():
        ca()
        torch.neg(x)
    # 'k' is in the names of both kernels
    with pytest.raises(AssertionError):
        bench_kineto(two_kernels, 'k', num_tests=3)
    assert bench_kineto(two_kernels, 'k', num_tests=3, with_multiple_kernels=True) > 0


def test_bench_kineto_split_call_is_one_call():
    """A dense call split into two launches (4096 x 7168 x 4096: 256 x 256 tiles over
    the first columns, 256 x 192 over the rest) is timed as one call: the sum of its
    two kernels, not an ambiguity error, and about twice the per-launch average
    that with_multiple_kernels reports."""
    m, n, k = 4096, 7168, 4096
    g = torch.Generator(device=DEV).manual_seed(5)
    a = deep_gemm.per_token_cast_to_fp8(torch.randn((m, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    b = deep_gemm.per_block_cast_to_fp8(torch.randn((n, k), generator=g, device=DEV).bfloat16(), use_ue8m0=False)
    d = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)

    def call():
        deep_gemm.fp8_gemm_nt(a, b, d)
    call()
    assert 'split_n=' in deep_gemm.get_last_config()
    t = bench_kineto(call, 'gemm_', num_tests=10)
    t_avg = bench_kineto(call, 'gemm_', num_tests=10, with_multiple_kernels=True)
    t_call = bench(call, num_warmups=2, num_tests=10, flush_cache=True)
    print(f'split call: bench_kineto {t * 1e6:.1f} us, per launch {t_avg * 1e6:.1f} us, '
          f'whole call {t_call * 1e6:.1f} us', flush=True)
    assert 1.6 * t_avg < t < 2.4 * t_avg
    assert 0.5 * t_call < t <= 1.2 * t_call
