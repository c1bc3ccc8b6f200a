"""Timing helpers of the reference's deep_gemm.testing (deep_gemm/testing/bench.py:7-146).

`bench` times whole calls with HIP events on the current stream. `bench_kineto`
times named kernels: it runs the call under torch.profiler (kineto, which reads
the ROCm kernel trace on this stack) and returns, per requested name, the
average device time of the kernels whose names contain it, as the reference's
version does.

MI355X has a 256 MB Infinity Cache in front of HBM, so the cache flush between
timed calls covers 512 MB (the reference flushes 256 MB for its L2). The flush
reads the buffer: a zero fill would leave dirty lines whose write-back lands
inside the next timed kernel.
"""
import os

import torch

__all__ = ['bench', 'bench_kineto', 'get_arch_major']

_FLUSH_BYTES = 512 * 1024 * 1024


def get_arch_major() -> int:
    major, _ = torch.cuda.get_device_capability()
    return major


def _flush_buffer():
    return torch.ones(_FLUSH_BYTES // 4, dtype=torch.int32, device='cuda')


def bench(fn, num_warmups: int = 5, num_tests: int = 10, flush_cache: bool = False) -> float:
    """Average seconds per call of `fn`, timed with events on the current stream."""
    torch.cuda.synchronize()
    cache = _flush_buffer() if flush_cache else None
    for _ in range(num_warmups):
        fn()
    start = [torch.cuda.Event(enable_timing=True) for _ in range(num_tests)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(num_tests)]
    for i in range(num_tests):
        if cache is not None:
            torch.sum(cache, dtype=torch.int64)
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(start, end)) / num_tests / 1e3


def _device_time_us(evt) -> float:
    for attr in ('device_time_total', 'cuda_time_total'):
        v = getattr(evt, attr, None)
        if v is not None:
            return float(v)
    return 0.0


def bench_kineto(fn, kernel_names, num_tests: int = 30, suppress_kineto_output: bool = False,
                 trace_path=None, flush_l2: bool = True, with_multiple_kernels: bool = False, barrier=None):
    """Average device seconds per launch of each named kernel while `fn` runs.

    `kernel_names` is a string or a tuple of strings; a kernel matches a name when
    its symbol contains it. Returns a float for a string and a tuple for a tuple;
    a name no kernel matched gives 0. Unless `with_multiple_kernels`, a name that
    matches more than one distinct kernel is an error (as in the reference), except
    for one library call that runs as two launches (a column or row split): then
    each of its kernels ran once per call and the result is the call's time.
    `fn` runs once untraced, then `num_tests` times in the traced window, each
    after a cache flush (`flush_l2`) and a call of `barrier` when given.
    `suppress_kineto_output` is accepted for signature compatibility.
    """
    assert isinstance(kernel_names, (str, tuple))
    is_tuple = isinstance(kernel_names, tuple)
    names = kernel_names if is_tuple else (kernel_names,)
    if int(os.environ.get('DG_USE_NVIDIA_TOOLS', 0)):   # the reference skips profiling under external profilers
        return (1,) * len(names) if is_tuple else 1

    cache = _flush_buffer() if flush_l2 else None
    fn()
    torch.cuda.synchronize()
    schedule = torch.profiler.schedule(wait=0, warmup=1, active=1, repeat=1)
    prof = torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA], schedule=schedule)
    with prof:
        for _ in range(2):   # one warm-up window, one recorded window
            for _ in range(num_tests):
                if cache is not None:
                    torch.sum(cache, dtype=torch.int64)
                if barrier is not None:
                    barrier()
                fn()
            torch.cuda.synchronize()
            prof.step()
    if trace_path is not None:
        prof.export_chrome_trace(trace_path)

    averages = [e for e in prof.key_averages() if _device_time_us(e) > 0 and e.count > 0]
    times = []
    for name in names:
        hits = [e for e in averages if name in e.key]
        if not with_multiple_kernels and len(hits) > 1:
            # One library call can run as two launches of different tiles (a dense
            # column split or a contiguous row split): every matching kernel is then
            # one of this library's and ran once per call, and the call's time is the
            # sum of their averages. Any other ambiguity is an error, as in the reference.
            if all('dgm::' in e.key and e.count == num_tests for e in hits):
                times.append(sum(_device_time_us(e) / e.count for e in hits) / 1e6)
                continue
            raise AssertionError(f'kernel name {name!r} matches several kernels: {[e.key for e in hits]}')
        total_us = sum(_device_time_us(e) for e in hits)
        count = sum(e.count for e in hits)
        times.append(total_us / count / 1e6 if count else 0.0)
    return tuple(times) if is_tuple else times[0]
