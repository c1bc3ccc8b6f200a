"""Timing helpers (reference deep_gemm/testing/bench.py:7-146), on HIP events.

MI355X has a 256 MB Infinity Cache in front of HBM, so the cache flush between
timed calls writes 512 MB (the reference flushes 256 MB for its L2).
"""
import torch

__all__ = ['bench', 'bench_kineto', 'get_arch_major']

_FLUSH_BYTES = 512 * 1024 * 1024


def get_arch_major() -> int:
    major, _ = torch.cuda.get_device_capability()
    return major


def bench(fn, num_warmups: int = 5, num_tests: int = 10, flush_cache: bool = False) -> float:
    """Average seconds per call of `fn`, timed with events on the current stream."""
    torch.cuda.synchronize()
    cache = torch.empty(_FLUSH_BYTES // 4, dtype=torch.int32, device='cuda') if flush_cache else None
    for _ in range(num_warmups):
        fn()
    start = [torch.cuda.Event(enable_timing=True) for _ in range(num_tests)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(num_tests)]
    for i in range(num_tests):
        if cache is not None:
            cache.zero_()
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(start, end)) / num_tests / 1e3


def bench_kineto(fn, kernel_names=None, num_tests: int = 30, suppress_kineto_output: bool = False,
                 trace_path=None, flush_l2: bool = True, with_multiple_kernels: bool = False):
    """Event-timed stand-in for the reference's kineto profiler helper: seconds per call of `fn`
    (kernel_names is accepted for signature compatibility)."""
    t = bench(fn, num_warmups=3, num_tests=num_tests, flush_cache=flush_l2)
    if isinstance(kernel_names, (tuple, list)):
        return [t] + [0.0] * (len(kernel_names) - 1)
    return t
