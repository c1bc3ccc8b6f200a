"""Benchmark of the FP8 block-scaled GEMM hot path on one MI355X.

Default workload (the headline configuration): dense fp8_gemm_nt at M = 4096 over
the DeepSeek-V3 (N, K) sweep {(2112,7168), (24576,1536), (7168,16384),
(4096,7168), (7168,2048)}, e4m3 operands with 1x128 / 128x128 FP32 scales, BF16
output. One step = one call per shape (5 launches). `value` is total
algorithmic FLOPs / wall time of the timed steps (inputs resident in HBM).
The activation scales (SFA) are passed in the MN-major TMA-aligned layout the
reference's kernels consume (K-major for the decode shape, where the two are
equal; `--sfa-major` forces one; the library takes both).

Each launch has 8 rotating buffer sets (copies of its inputs and outputs) and
step s runs on set s % 8, so no launch finds its operands in L2 or the 256 MB
Infinity Cache. Steps are replayed from HIP graphs captured once (the library
launches into a capturing stream like any other), which takes the Python call
overhead out of the timed region; --eager launches from Python instead.

Other workloads (`--workload`): dense_acc (FP32 C += A.B^T), contiguous
(config 3, 8 experts, 32768 tokens), masked (config 4, 16 experts, max_m 256),
fp8fp4 (config 5), cast (the fused per-token FP8 activation cast that produces
A and its MN-major SFA for these GEMMs; HBM-bound, reported in GB/s), kgrouped
(k_grouped_fp8_gemm_nt_contiguous, the 1D1D weight-gradient GEMM), decode
(config 1's shape, 64 x 2112 x 7168, on the GPU), moe_l1 (the config 3 / 4
gate-up GEMMs with the fused SwiGLU x weight -> FP8 epilogue, beside the
unfused GEMM + cast), moe_dispatch (token rows -> the contiguous expert layout,
256 experts, top-8; HBM-bound, GB/s).

Prints one JSON line. `roofline` is computed from per-launch durations measured
live with HIP events on the launch stream; `cpu_baseline` times the oracle/
restatement on the host on a bounded sample (the FP32 dequantize-then-matmul
for the GEMMs, the numpy quantizer for the cast).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, 'deepgemm-amd_amd'))

PEAK_FP8_TFLOPS = 5000.0     # MI355X dense FP8 MFMA (AMD public spec: 2.5 PFLOP/s bf16 x2)
PEAK_FP4_TFLOPS = 10100.0
PEAK_HBM_GBS = 8000.0
DENSE_NK = [(2112, 7168), (24576, 1536), (7168, 16384), (4096, 7168), (7168, 2048)]
# Calibrated HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE passes,
# written by deep_gemm.testing.rocprof_summary), per workload.
PROFILE_NAMES = {'dense': 'fp8_gemm_nt_dense_m4096', 'dense_acc': 'fp8_gemm_nt_dense_acc_m4096',
                 'contiguous': 'm_grouped_fp8_gemm_nt_contiguous_e8_t32768',
                 'masked': 'm_grouped_fp8_gemm_nt_masked_e16_m256', 'fp8fp4': 'fp8_fp4_gemm_nt_m4096',
                 'cast': 'per_token_cast_to_fp8_bf16', 'kgrouped': 'k_grouped_fp8_gemm_nt_e8_m4096_n7168',
                 'decode': 'fp8_gemm_nt_m64_n2112_k7168', 'moe_l1': 'moe_l1_swiglu_e8_t32768_e16_m256',
                 'moe_dispatch': 'moe_dispatch_e256_top8'}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--workload', default='dense',
                    choices=['dense', 'dense_acc', 'contiguous', 'masked', 'fp8fp4', 'cast', 'kgrouped', 'decode',
                             'moe_l1', 'moe_dispatch'])
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-extras', action='store_true',
                    help='default workload only: skip the per-launch summaries of the other configurations')
    ap.add_argument('--rotate', type=int, default=8, help='rotating buffer sets per launch')
    ap.add_argument('--eager', action='store_true', help='launch from Python instead of replaying HIP graphs')
    ap.add_argument('--cpu-sample-m', type=int, default=512)
    ap.add_argument('--hbm-context', action='store_true',
                    help='masked workload: also time torch\'s own streaming read (sum) and copy over 1-4 GiB, '
                         'for context on the HBM roofline (not part of value)')
    ap.add_argument('--hipblaslt', action='store_true',
                    help='dense workload: also time the vendor FP8 GEMM (torch._scaled_mm -> hipBLASLt) on the same '
                         'shapes with per-tensor and row-wise scales, for context (not part of value)')
    ap.add_argument('--sfa-major', choices=['auto', 'mn', 'k'], default='auto',
                    help='SFA layout of the GEMM workloads: MN-major TMA-aligned (as the reference\'s kernels '
                         'consume it), K-major (as per_token_cast_to_fp8 returns it), or per launch the one its '
                         'kernel reads fastest (auto)')
    ap.add_argument('--calibrate-copy-mib', type=int, default=0,
                    help='first run torch.neg over this many MiB of float32 (a plain copy kernel of known '
                         'size, the reference for FETCH_SIZE / WRITE_SIZE counter passes)')
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def hbm_context(reps: int):
    """HBM rates of torch's own kernels on this GPU, timed as the launches are (a
    read flush, then one call between two events): a reduction (`sum`, read only)
    and a device copy (read + write) over 1, 2 and 4 GiB of float32."""
    import torch
    dev = 'cuda:0'
    stream = torch.cuda.current_stream()
    flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    out = {}
    for gib in (1, 2, 4):
        n = gib * 2 ** 30 // 4
        x = torch.randn(n, device=dev)
        y = torch.empty_like(x)
        x.sum()
        y.copy_(x)
        torch.cuda.synchronize()
        for name, fn, nbytes in (('sum_read', lambda: x.sum(), 4 * n), ('copy_read_write', lambda: y.copy_(x), 8 * n)):
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            for e0, e1 in evs:
                torch.sum(flush, dtype=torch.int64)
                e0.record(stream)
                fn()
                e1.record(stream)
            torch.cuda.synchronize()
            us = sum(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3 / reps
            out[f'{name}_{gib}gib_gbs'] = round(nbytes / us / 1e3, 1)
        del x, y
        torch.cuda.empty_cache()
    del flush
    return out


def hipblaslt_context(rot: int, reps: int):
    """The vendor library's FP8 GEMM on the dense shapes, timed as the headline is
    (flush, then `rot` back-to-back launches on rotating operand sets): torch's
    _scaled_mm (hipBLASLt on ROCm) with one per-tensor scale, and with row-wise
    scales (per row of A, per column of B, applied once in the epilogue). Neither
    has the per-128-K block scales of the path this library implements, so both
    do less work per output; the numbers are context for the roofline fraction."""
    import torch
    dev = 'cuda:0'
    stream = torch.cuda.current_stream()
    flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    out = {}
    m = 4096
    for mode in ('per_tensor', 'row_wise'):
        per, tot_us, tot_fl = {}, 0.0, 0
        for n, k in DENSE_NK:
            fns = []
            for _ in range(rot):
                a = torch.randn((m, k), device=dev, generator=gen).to(torch.float8_e4m3fn)
                b = torch.randn((n, k), device=dev, generator=gen).to(torch.float8_e4m3fn)
                if mode == 'per_tensor':
                    sa, sb = torch.ones((), device=dev), torch.ones((), device=dev)
                else:
                    sa, sb = torch.ones((m, 1), device=dev), torch.ones((1, n), device=dev)
                fns.append(lambda a=a, b=b, sa=sa, sb=sb: torch._scaled_mm(a, b.t(), scale_a=sa, scale_b=sb,
                                                                          out_dtype=torch.bfloat16))
            try:
                for f in fns:
                    f()
                torch.cuda.synchronize()
            except Exception as e:   # a torch build without this form: say so, time nothing
                out[mode] = {'error': f'{type(e).__name__}: {str(e)[:160]}'}
                break
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            for e0, e1 in evs:
                torch.sum(flush, dtype=torch.int64)
                e0.record(stream)
                for f in fns:
                    f()
                e1.record(stream)
            torch.cuda.synchronize()
            us = sum(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3 / (reps * rot)
            per[f'n{n}_k{k}'] = round(us, 2)
            tot_us += us
            tot_fl += 2 * m * n * k
            del fns
            torch.cuda.empty_cache()
        else:
            out[mode] = {'per_launch_us': per, 'step_us': round(tot_us, 1),
                         'tflops': round(tot_fl / tot_us / 1e6, 1),
                         'frac': round(tot_fl / tot_us / 1e6 / PEAK_FP8_TFLOPS, 4)}
    del flush
    return out


# ---------------------------------------------------------------- workloads

class Launch:
    """One launch of the workload with its algorithmic FLOPs and bytes. `mk()`
    returns a callable bound to a fresh copy of the launch's inputs and outputs
    (one rotating buffer set)."""

    def __init__(self, name, mk, flops, nbytes):
        self.name, self.mk, self.flops, self.nbytes = name, mk, flops, nbytes


def _twin(x):
    """Copy of a tensor (or of each tensor of a tuple) with the same strides."""
    import torch
    if isinstance(x, (tuple, list)):
        return tuple(_twin(t) for t in x)
    out = torch.empty_strided(tuple(x.shape), x.stride(), dtype=x.dtype, device=x.device)
    out.copy_(x)
    return out


def _quant_a(m, k, gen, dev):
    import torch
    import deep_gemm
    x = torch.randn((m, k), generator=gen).bfloat16().to(dev)
    return deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=False)


def _quant_b(n, k, gen, dev):
    import torch
    import deep_gemm
    x = torch.randn((n, k), generator=gen).bfloat16().to(dev)
    return deep_gemm.per_block_cast_to_fp8(x, use_ue8m0=False)


# SFA layout the GEMM workloads pass (the values are the same in both):
#   'mn'   the MN-major TMA-aligned layout, as the reference's kernels consume it
#          (its API transforms K-major SFA inside each call, and its benchmarks
#          time the GEMM kernel alone, tests/test_fp8_fp4.py:169,226) and as
#          per_token_cast_to_fp8_mn_major writes it in one pass;
#   'k'    the K-major layout per_token_cast_to_fp8 returns;
#   'auto' (default) per launch, the layout its kernel reads fastest: MN-major
#          for the dense, masked and contiguous kernels (3.5%, 6% and 3.5% faster
#          than K-major), K-major for the decode shape (no difference).
SFA_MAJOR = 'auto'


def _sfa(a, prefer):
    """(codes, SFA) in the layout SFA_MAJOR names ('auto': `prefer`)."""
    import deep_gemm
    major = prefer if SFA_MAJOR == 'auto' else SFA_MAJOR
    return (a[0], deep_gemm.get_mn_major_tma_aligned_tensor(a[1])) if major == 'mn' else a


def _sfa_name(prefer):
    return (prefer if SFA_MAJOR == 'auto' else SFA_MAJOR) + '-major'


# Operand builders: the exact seeded inputs of each configuration. The
# full-size parity tests (tests/test_configs_gpu.py) build their inputs through
# these same functions, so the bench workloads are the tested workloads.

def dense_operands(acc: bool, dev='cuda:0'):
    """Config 2: M = 4096 over DENSE_NK. A 1x128 and B 128x128 FP32-scale e4m3
    (the product quantizers, on the device); with `acc`, an FP32 C = 32 randn."""
    import torch
    gen = torch.Generator().manual_seed(0)
    m = 4096
    out = []
    for n, k in DENSE_NK:
        a = _quant_a(m, k, gen, dev)
        b = _quant_b(n, k, gen, dev)
        c = (torch.randn((m, n), generator=gen) * 32).to(dev) if acc else None
        out.append(dict(name=f'n{n}_k{k}', m=m, n=n, k=k, a=a, b=b, c=c))
    return out


def contiguous_operands(dev='cuda:0'):
    """Config 3: 8 experts, 32768 tokens ~ Multinomial(Dirichlet(1)), segments
    padded to the M alignment with m_indices = -1 and zero A rows."""
    import numpy as np
    import torch
    import deep_gemm
    gen = torch.Generator().manual_seed(0)
    rng = np.random.default_rng(0)
    g, total = 8, 32768
    ms = rng.multinomial(total, rng.dirichlet(np.ones(g)))
    align = deep_gemm.get_mk_alignment_for_contiguous_layout()
    aligned = [(int(x) + align - 1) // align * align for x in ms]
    m_pad = sum(aligned)
    idx_h = torch.full((m_pad,), -1, dtype=torch.int32)
    s = 0
    for i, (mi, ai) in enumerate(zip(ms, aligned)):
        idx_h[s:s + int(mi)] = i
        s += ai
    idx = idx_h.to(dev)
    shapes = []
    for n, k in [(4096, 7168), (7168, 2048)]:
        x = torch.randn((m_pad, k), generator=gen).bfloat16()
        x[idx_h < 0] = 0
        a = deep_gemm.per_token_cast_to_fp8(x.to(dev), use_ue8m0=False)
        bq = torch.empty((g, n, k), dtype=torch.float8_e4m3fn, device=dev)
        bs = torch.empty((g, (n + 127) // 128, (k + 127) // 128), device=dev)
        for i in range(g):
            bq[i], bs[i] = _quant_b(n, k, gen, dev)
        shapes.append(dict(name=f'n{n}_k{k}', n=n, k=k, a=a, b=(bq, bs)))
    return dict(num_groups=g, total=total, ms=[int(v) for v in ms], aligned=aligned, m_pad=m_pad,
                m_indices=idx, shapes=shapes)


def masked_operands(dev='cuda:0'):
    """Config 4: 16 experts, max_m = 256, masked_m ~ U{96..160}; SFA rows past
    masked_m are zero (reference tests/generators.py:476-478)."""
    import numpy as np
    import torch
    gen = torch.Generator().manual_seed(0)
    rng = np.random.default_rng(0)
    g, max_m = 16, 256
    masked = rng.integers(96, 161, size=g).astype(np.int32)
    shapes = []
    for n, k in [(4096, 7168), (7168, 2048)]:
        aq = torch.empty((g, max_m, k), dtype=torch.float8_e4m3fn, device=dev)
        as_ = torch.empty((g, max_m, (k + 127) // 128), device=dev)
        bq = torch.empty((g, n, k), dtype=torch.float8_e4m3fn, device=dev)
        bs = torch.empty((g, (n + 127) // 128, (k + 127) // 128), device=dev)
        for i in range(g):
            aq[i], as_[i] = _quant_a(max_m, k, gen, dev)
            as_[i, int(masked[i]):] = 0
            bq[i], bs[i] = _quant_b(n, k, gen, dev)
        shapes.append(dict(name=f'n{n}_k{k}', n=n, k=k, a=(aq, as_), b=(bq, bs)))
    return dict(num_groups=g, max_m=max_m, masked_m=masked, masked_m_dev=torch.from_numpy(masked).to(dev),
                expected_m=128, shapes=shapes)


def fp8fp4_operands(dev='cuda:0'):
    """Config 5: M = 4096, N = K = 7168; A e4m3 with 1x128 UE8M0 scales, B e2m1
    with 1x32 UE8M0 scales. Returns the FP32 (power-of-two) scales and their
    packed MN-major UE8M0 form, which the launches use."""
    import torch
    import deep_gemm
    gen = torch.Generator().manual_seed(0)
    m, n, k = 4096, 7168, 7168
    a = deep_gemm.per_token_cast_to_fp8(torch.randn((m, k), generator=gen).bfloat16().to(dev), use_ue8m0=True)
    b = deep_gemm.per_token_cast_to_fp4(torch.randn((n, k), generator=gen).bfloat16().to(dev), use_ue8m0=True,
                                        gran_k=32)
    # Scales in the kernel's packed MN-major UE8M0 form, transformed once up front
    # as for weights (the reference transforms FP32 SFs inside each call and times
    # the GEMM kernel alone, tests/test_fp8_fp4.py:84-86,100).
    packed_a = (a[0], deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(a[1]))
    packed_b = (b[0], deep_gemm.get_mn_major_tma_aligned_packed_ue8m0_tensor(b[1]))
    return dict(m=m, n=n, k=k, a=packed_a, b=packed_b, sfa_f32=a[1], sfb_f32=b[1])


def _dense_bytes(m, n, k, out_bytes):
    return m * k + n * k + 4 * m * ((k + 127) // 128) + 4 * ((n + 127) // 128) * ((k + 127) // 128) + out_bytes


def make_dense(acc: bool):
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    launches = []
    for op in dense_operands(acc, dev):
        m, n, k = op['m'], op['n'], op['k']
        op['a'] = _sfa(op['a'], 'mn')
        if acc:
            def mk(a=op['a'], b=op['b'], d=op['c']):
                a2, b2, d2 = _twin(a), _twin(b), _twin(d)
                return lambda: deep_gemm.fp8_gemm_nt(a2, b2, d2, c=d2)
            out_bytes = 8 * m * n
        else:
            def mk(a=op['a'], b=op['b'], m=m, n=n):
                a2, b2 = _twin(a), _twin(b)
                d2 = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
                return lambda: deep_gemm.fp8_gemm_nt(a2, b2, d2)
            out_bytes = 2 * m * n
        launches.append(Launch(op['name'], mk, 2 * m * n * k, _dense_bytes(m, n, k, out_bytes)))
    cfg = {'workload': 'fp8_gemm_nt M=4096 DeepSeek-V3 (N,K) sweep' + (' FP32 C-accumulate' if acc else ''),
           'm': 4096, 'nk': DENSE_NK, 'out': 'f32 (D=C+AB^T)' if acc else 'bf16',
           'recipe': '1x128 A / 128x128 B FP32 scales', 'sfa': _sfa_name('mn')}
    return launches, cfg


def make_decode():
    """Config 1's shape on the GPU: dense fp8_gemm_nt, A [64, 7168] (1x128 FP32
    scales), B [2112, 7168] (128x128 FP32 scales), BF16 D: a decode-sized call
    (the configuration the CPU baseline of the reference is quoted on)."""
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    gen = torch.Generator().manual_seed(1)
    m, n, k = 64, 2112, 7168
    a, b = _sfa(_quant_a(m, k, gen, dev), 'k'), _quant_b(n, k, gen, dev)

    def mk():
        a2, b2 = _twin(a), _twin(b)
        d2 = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        return lambda: deep_gemm.fp8_gemm_nt(a2, b2, d2)
    cfg = {'workload': 'fp8_gemm_nt M=64 N=2112 K=7168 (config 1 shape)', 'm': m, 'n': n, 'k': k, 'out': 'bf16',
           'sfa': _sfa_name('k')}
    return [Launch('m64_n2112_k7168', mk, 2 * m * n * k, _dense_bytes(m, n, k, 2 * m * n))], cfg


def make_contiguous():
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    ops = contiguous_operands(dev)
    g, m_pad, total, idx = ops['num_groups'], ops['m_pad'], ops['total'], ops['m_indices']
    launches = []
    for op in ops['shapes']:
        n, k = op['n'], op['k']

        def mk(a=_sfa(op['a'], 'mn'), b=op['b'], n=n):
            a2, b2 = _twin(a), _twin(b)
            d2 = torch.empty((m_pad, n), dtype=torch.bfloat16, device=dev)
            return lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a2, b2, d2, idx)
        nbytes = m_pad * k + g * n * k + 2 * m_pad * n + 4 * m_pad * ((k + 127) // 128) + \
            4 * g * ((n + 127) // 128) * ((k + 127) // 128) + 4 * m_pad
        launches.append(Launch(op['name'], mk, 2 * total * n * k, nbytes))
    cfg = {'workload': 'm_grouped_fp8_gemm_nt_contiguous 8 experts 32768 tokens Dirichlet(1)',
           'tokens_per_expert': ops['ms'], 'm_padded': m_pad, 'nk': [(4096, 7168), (7168, 2048)],
           'sfa': _sfa_name('mn')}
    return launches, cfg


def make_masked():
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    ops = masked_operands(dev)
    g, max_m, masked, mm = ops['num_groups'], ops['max_m'], ops['masked_m'], ops['masked_m_dev']
    sum_m = int(masked.sum())
    launches = []
    for op in ops['shapes']:
        n, k = op['n'], op['k']

        def mk(a=_sfa(op['a'], 'mn'), b=op['b'], n=n):
            a2, b2 = _twin(a), _twin(b)
            d2 = torch.empty((g, max_m, n), dtype=torch.bfloat16, device=dev)
            return lambda: deep_gemm.m_grouped_fp8_gemm_nt_masked(a2, b2, d2, mm, ops['expected_m'])
        nbytes = g * n * k + sum_m * k + 2 * sum_m * n + 4 * sum_m * ((k + 127) // 128) + \
            4 * g * ((n + 127) // 128) * ((k + 127) // 128)
        launches.append(Launch(op['name'], mk, 2 * sum_m * n * k, nbytes))
    cfg = {'workload': 'm_grouped_fp8_gemm_nt_masked 16 experts max_m=256 masked_m~U[96,160]',
           'masked_m': masked.tolist(), 'nk': [(4096, 7168), (7168, 2048)], 'sfa': _sfa_name('mn')}
    return launches, cfg


def make_fp8fp4():
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    op = fp8fp4_operands(dev)
    m, n, k = op['m'], op['n'], op['k']

    def mk():
        a2, b2 = _twin(op['a']), _twin(op['b'])
        d2 = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        return lambda: deep_gemm.fp8_fp4_gemm_nt(a2, b2, d2, recipe_a=(1, 128), recipe_b=(1, 32))
    nbytes = m * k + n * k // 2 + 4 * m * (k // 128) + 4 * n * (k // 32) + 2 * m * n
    cfg = {'workload': 'fp8_fp4_gemm_nt M=4096 N=K=7168, A e4m3 1x128 UE8M0, B e2m1 1x32 UE8M0', 'm': m, 'n': n,
           'k': k}
    return [Launch('m4096_n7168_k7168', mk, 2 * m * n * k, nbytes)], cfg


def make_kgrouped():
    """k_grouped_fp8_gemm_nt_contiguous, the reference's EP32 weight-gradient case
    (tests/generators.py:229-262): 8 groups, M = 4096, N = 7168, K_g ~ 4096 x U[0.7, 1.3]
    aligned to 128, FP32 D += A_g.B_g^T in place."""
    import numpy as np
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    rng = np.random.default_rng(0)
    g, m, n = 8, 4096, 7168
    ks = [int((4096 * rng.uniform(0.7, 1.3) + 127) // 128 * 128) for _ in range(g)]
    sum_k = sum(ks)
    torch.manual_seed(0)
    qa, sa, qb, sb = [], [], [], []
    for k in ks:   # per-group 1 x 128 casts of randn rows, on the device
        q, sf = deep_gemm.per_token_cast_to_fp8(torch.randn((m, k), device=dev, dtype=torch.bfloat16), False)
        qa.append(q.view(torch.uint8).reshape(-1)), sa.append(sf)
        q, sf = deep_gemm.per_token_cast_to_fp8(torch.randn((n, k), device=dev, dtype=torch.bfloat16), False)
        qb.append(q.view(torch.uint8).reshape(-1)), sb.append(sf)
    qa, qb = torch.cat(qa).view(torch.float8_e4m3fn), torch.cat(qb).view(torch.float8_e4m3fn)
    sfa, sfb = torch.cat(sa, dim=1), torch.cat(sb, dim=1)
    d0 = torch.randn((g, m, n), device=dev) * 32
    layout = torch.tensor(ks, dtype=torch.int32, device=dev)

    def mk():
        a2, b2, d2 = _twin((qa, sfa)), _twin((qb, sfb)), _twin(d0)
        return lambda: deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a2, b2, d2, ks, layout, d2)
    nbytes = sum_k * (m + n) + 4 * (m + n) * (sum_k // 128) + 8 * g * m * n
    cfg = {'workload': 'k_grouped_fp8_gemm_nt_contiguous 8 groups M=4096 N=7168 K_g~4096 (1D1D, FP32 D += )',
           'ks': ks}
    return [Launch(f'g{g}_m{m}_n{n}_sumk{sum_k}', mk, 2 * m * n * sum_k, nbytes)], cfg


def make_moe_l1():
    """The L1 (gate/up) grouped GEMM of the MoE layer with its SwiGLU x routing
    weight -> FP8 step, unfused (BF16 D through HBM, then the cast kernel) and
    fused (the step in the GEMM's epilogue), at the config 3 (contiguous, N = 4096
    = 2 x 2048, K = 7168) and config 4 (masked, same N and K) gate/up shapes. All
    four launches produce the same q and sf bits; FLOPs are the valid rows' GEMM
    FLOPs, bytes the fused job's (A, B, scales, q and sf)."""
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    c = contiguous_operands(dev)
    m = masked_operands(dev)
    co, mo = c['shapes'][0], m['shapes'][0]
    assert (co['n'], co['k']) == (4096, 7168) and (mo['n'], mo['k']) == (4096, 7168)
    co['a'], mo['a'] = _sfa(co['a'], 'mn'), _sfa(mo['a'], 'mn')
    n, k = co['n'], co['k']
    inter = n // 2
    m_pad, idx, total = c['m_pad'], c['m_indices'], c['total']
    g, max_m, mm, sum_m = m['num_groups'], m['max_m'], m['masked_m_dev'], int(m['masked_m'].sum())
    gen = torch.Generator().manual_seed(1)
    rw_c = torch.rand((m_pad,), generator=gen).to(dev)
    rw_m = torch.rand((g, max_m), generator=gen).to(dev)
    bf_c = deep_gemm.transform_l1_weights_for_swiglu(co['b'])
    bf_m = deep_gemm.transform_l1_weights_for_swiglu(mo['b'])
    sfk = (k + 127) // 128

    def out(rows_shape):
        return (torch.empty(rows_shape + (inter,), dtype=torch.float8_e4m3fn, device=dev),
                torch.empty(rows_shape + (inter // 128,), dtype=torch.float32, device=dev))

    def mk_c_unfused():
        a2, b2 = _twin(co['a']), _twin(co['b'])
        h = torch.empty((m_pad, n), dtype=torch.bfloat16, device=dev)
        q, sf = out((m_pad,))

        def run():
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous(a2, b2, h, idx)
            names[0] = deep_gemm.get_last_config()
            deep_gemm.moe_swiglu_apply_weight_to_fp8(h, rw_c, idx, out=(q, sf))
            names[1] = deep_gemm.get_last_config()
        names = ['', '']
        run.config = lambda: ' + '.join(names)
        return run

    def mk_c_fused():
        a2, b2 = _twin(co['a']), _twin(bf_c)
        o = out((m_pad,))
        return lambda: deep_gemm.m_grouped_fp8_gemm_nt_contiguous_swiglu(a2, b2, o, idx, rw_c)

    def mk_m_unfused():
        a2, b2 = _twin(mo['a']), _twin(mo['b'])
        h = torch.empty((g, max_m, n), dtype=torch.bfloat16, device=dev)
        q, sf = out((g * max_m,))

        def run():
            deep_gemm.m_grouped_fp8_gemm_nt_masked(a2, b2, h, mm, m['expected_m'])
            names[0] = deep_gemm.get_last_config()
            deep_gemm.moe_swiglu_apply_weight_to_fp8(h.view(g * max_m, n), rw_m.view(-1), out=(q, sf))
            names[1] = deep_gemm.get_last_config()
        names = ['', '']
        run.config = lambda: ' + '.join(names)
        return run

    def mk_m_fused():
        a2, b2 = _twin(mo['a']), _twin(bf_m)
        o = out((g, max_m))
        return lambda: deep_gemm.m_grouped_fp8_gemm_nt_masked_swiglu(a2, b2, o, mm, m['expected_m'], rw_m)

    sf_b = 4 * ((n + 127) // 128) * sfk
    c_bytes = m_pad * k + 8 * n * k + 4 * m_pad * sfk + 8 * sf_b + 4 * m_pad + m_pad * inter + \
        4 * m_pad * (inter // 128) + 4 * m_pad
    m_bytes = g * n * k + sum_m * k + 4 * sum_m * sfk + g * sf_b + sum_m * inter + 4 * sum_m * (inter // 128) + \
        4 * sum_m
    launches = [Launch('contiguous_unfused', mk_c_unfused, 2 * total * n * k, c_bytes),
                Launch('contiguous_fused', mk_c_fused, 2 * total * n * k, c_bytes),
                Launch('masked_unfused', mk_m_unfused, 2 * sum_m * n * k, m_bytes),
                Launch('masked_fused', mk_m_fused, 2 * sum_m * n * k, m_bytes)]
    cfg = {'workload': 'MoE L1 gate/up GEMM + SwiGLU x weight -> FP8, unfused vs fused (config 3 contiguous and '
                       'config 4 masked, N = 2 x 2048, K = 7168)',
           'tokens_per_expert': c['ms'], 'm_padded': m_pad, 'masked_m': m['masked_m'].tolist()}
    return launches, cfg


def make_moe_dispatch():
    """The MoE dispatch (token-major FP8 rows -> the contiguous expert layout):
    256 experts, top-8, at a decode-sized 4096 tokens (K = 7168) and at 65536
    tokens (K = 2048), close to the allocation-free entry point's bound. Bytes:
    each token row read once (codes and SF row) with its routing ids and weights;
    each routed row and each padding row (alignment 128) written once (codes, SF
    row, weight), m_indices over every row of the layout, and pos; no FLOPs."""
    import numpy as np
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    launches = []
    for t, kdim in [(4096, 7168), (65536, 2048)]:
        e, topk = 256, 8
        rng = np.random.default_rng(t)
        idx = torch.from_numpy(np.argsort(rng.random((t, e)), axis=1)[:, :topk].astype(np.int32)).to(dev)
        w = torch.rand((t, topk), generator=torch.Generator().manual_seed(t)).to(dev)
        x = deep_gemm.per_token_cast_to_fp8(torch.randn((t, kdim), device=dev, dtype=torch.bfloat16), False)

        def mk(x=x, idx=idx, w=w, e=e):
            x2 = _twin(x)
            return lambda: deep_gemm.moe_dispatch(x2, idx, e, layout='contiguous', topk_weights=w)
        sfk = (kdim + 127) // 128
        align = deep_gemm.get_mk_alignment_for_contiguous_layout()
        per_expert = np.bincount(idx.cpu().numpy().ravel(), minlength=e)
        seg_rows = int(((per_expert + align - 1) // align * align).sum())
        cap = int(deep_gemm._lib.dg_moe_dispatch_max_rows(t, topk, e, align))
        nbytes = (t * (kdim + 4 * sfk) + t * topk * 8                  # token rows, ids, weights
                  + seg_rows * (kdim + 4 * sfk + 4) + 4 * cap + 4 * t * topk)   # rows + padding, m_indices, pos
        launches.append(Launch(f't{t}_k{kdim}_e{e}_top{topk}', mk, 0, nbytes))
    cfg = {'workload': 'moe_dispatch contiguous layout, 256 experts, top-8', 'tk': [(4096, 7168), (65536, 2048)]}
    return launches, cfg


CAST_MK = [(4096, 7168), (4096, 16384), (4096, 1536), (32768, 7168)]


def make_cast():
    import torch
    import deep_gemm
    dev = torch.device('cuda:0')
    gen = torch.Generator().manual_seed(0)
    launches = []
    for m, k in CAST_MK:
        x = torch.randn((m, k), generator=gen).bfloat16().to(dev)
        def mk(x=x):
            x2 = _twin(x)
            return lambda: deep_gemm.per_token_cast_to_fp8_mn_major(x2, use_ue8m0=False)
        nbytes = 2 * m * k + m * k + 4 * m * ((k + 127) // 128)
        launches.append(Launch(f'm{m}_k{k}', mk, 0, nbytes))
    cfg = {'workload': 'per_token_cast_to_fp8 bf16 -> e4m3 + MN-major FP32 1x128 SFA', 'mk': CAST_MK}
    return launches, cfg


# ---------------------------------------------------------------- CPU baseline

def _cpu_model() -> str:
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or 'unknown'


def _median_time(fn, runs: int = 3) -> float:
    """One untimed warm-up call, then the median of `runs` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(workload: str, sample_m: int):
    """Time the oracle on the host on a bounded sample of the workload: the FP32
    dequantize-then-matmul the reference's tests use as their reference path
    (numpy dequantize, float32 BLAS matmul), or the numpy quantizer for the cast.
    One warm-up, then the median of 3 timed runs."""
    import numpy as np
    import torch
    from oracle import gemm as ogemm, quant as oquant
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, 'sched_getaffinity') else os.cpu_count()
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max((p.get('num_threads', 0) for p in threadpool_info() if p.get('user_api') == 'blas'),
                           default=0) or None
    except Exception:   # threadpoolctl absent: report what numpy's BLAS would take by default
        blas_threads = None
    host = {'cpu_model': _cpu_model(), 'os_cpu_count': os.cpu_count(), 'affinity_cpus': affinity,
            'torch_threads': torch.get_num_threads(), 'blas_threads': blas_threads, 'timing': 'median of 3 after 1 warm-up'}
    if workload == 'moe_dispatch':
        from oracle import moe as omoe
        t, kdim, e, topk = 8 * sample_m, 2048, 256, 8
        rng = np.random.default_rng(0)
        idx = np.argsort(rng.random((t, e)), axis=1)[:, :topk].astype(np.int32)
        w = rng.random((t, topk)).astype(np.float32)
        codes = rng.integers(0, 126, (t, kdim)).astype(np.uint8)
        sf = rng.random((t, kdim // 128)).astype(np.float32)
        secs = _median_time(lambda: omoe.dispatch(codes, sf, idx, e, 'contiguous', 128, topk_weights=w))
        nbytes = 2 * t * topk * (kdim + 4 * (kdim // 128) + 4) + t * topk * 8 + 4 * t * topk
        return dict({'value': round(nbytes / secs / 1e9, 3), 'unit': 'GB/s', 'cores': 1, 'kind': 'port',
                     'sample': f'T={t} tokens, K={kdim}, 256 experts, top-8: the oracle\'s dispatch (numpy, '
                               f'single-threaded), {secs:.2f} s per pass (median)'}, **host)
    if workload == 'cast':
        rows = 32 * sample_m   # the cast is far cheaper per row than a GEMM row
        nbytes, secs = 0, 0.0
        for _, k in CAST_MK:
            x = torch.randn((rows, k), generator=torch.Generator().manual_seed(1)).bfloat16().float().numpy()
            secs += _median_time(lambda: oquant.per_token_cast_to_fp8(x, use_ue8m0=False))
            nbytes += 3 * rows * k + 4 * rows * ((k + 127) // 128)
        return dict({'value': round(nbytes / secs / 1e9, 3), 'unit': 'GB/s', 'cores': 1, 'kind': 'port',
                     'sample': f'M={rows} rows of each (M,K) shape: the oracle\'s numpy per-token cast '
                               f'(single-threaded numpy), {secs:.2f} s per pass (median)'}, **host)
    nk = DENSE_NK if workload in ('dense', 'dense_acc') else [(4096, 7168), (7168, 2048)]
    if workload == 'moe_l1':   # the gate/up GEMM (the SwiGLU step is not timed on the host)
        nk = [(4096, 7168)]
    if workload == 'decode':   # config 1 itself: the whole 64-row workload
        nk, sample_m = [(2112, 7168)], 64
    flops, secs = 0, 0.0
    for n, k in nk:
        a = torch.randn((sample_m, k), generator=torch.Generator().manual_seed(1)).bfloat16().float().numpy()
        b = torch.randn((n, k), generator=torch.Generator().manual_seed(2)).bfloat16().float().numpy()
        qa, sfa = oquant.per_token_cast_to_fp8(a, use_ue8m0=False)
        qb, sfb = oquant.per_block_cast_to_fp8(b, use_ue8m0=False)
        secs += _median_time(lambda: ogemm.gemm_nt_f32(oquant.dequant_per_token(qa, sfa),
                                                       oquant.dequant_per_block(qb, sfb)))
        flops += 2 * sample_m * n * k
    threads = blas_threads or affinity
    return dict({'value': round(flops / secs / 1e12, 4), 'unit': 'TFLOPS', 'cores': threads, 'kind': 'port',
                 'sample': f'M={sample_m} rows of each (N,K) shape of the workload: FP32 dequantize (numpy) + '
                           f'FP32 matmul (numpy BLAS, {threads} host threads), {secs:.2f} s per pass (median)'},
                **host)


def load_traffic(workload, launches, configs):
    """Calibrated HBM bytes of one step from the committed counter summary,
    used only when every launch ran the kernel configuration it was measured on."""
    path = os.path.join(ROOT, 'profiles', PROFILE_NAMES[workload] + '.json')
    if not os.path.exists(path):
        return None, 'no counter summary for this workload'
    rec = json.load(open(path))
    per = rec.get('per_launch_bytes')
    if not per:
        return None, f'{os.path.basename(path)} holds no traffic figures'
    for l, c in zip(launches, configs):
        if rec.get('launch_config', {}).get(l.name) != c or l.name not in per:
            return None, f'{os.path.basename(path)} was measured on another kernel configuration'
    return sum(per[l.name]['total'] for l in launches), f'profiles/{os.path.basename(path)}'


# ---------------------------------------------------------------- timing

MAKERS = {'dense': lambda: make_dense(False), 'dense_acc': lambda: make_dense(True),
          'contiguous': make_contiguous, 'masked': make_masked, 'fp8fp4': make_fp8fp4, 'cast': make_cast,
          'kgrouped': make_kgrouped, 'decode': make_decode, 'moe_l1': make_moe_l1,
          'moe_dispatch': make_moe_dispatch}
# Configurations summarized next to the headline in the default run (per-launch
# kernel time and roofline fraction; the headline `value` stays config 2).
EXTRAS = ['dense_acc', 'contiguous', 'masked', 'fp8fp4', 'kgrouped', 'decode', 'moe_l1']


def t_min_us(flops, nbytes):
    """Roofline time of one launch: max(FLOPs / FP8 peak, bytes / HBM peak), in us."""
    return max(flops / (PEAK_FP8_TFLOPS * 1e6), nbytes / (PEAK_HBM_GBS * 1e3))


class Workload:
    """A workload's launches, each with `rot` rotating buffer sets, plus (unless
    eager) one HIP graph per launch over its sets and one per set over all
    launches."""

    def __init__(self, name, rot, eager):
        import torch
        import deep_gemm
        self.name, self.rot, self.eager = name, rot, eager
        self.launches, self.cfg = MAKERS[name]()
        # Rotating buffer sets: fns[i][r] runs launch i on its own copy r of the
        # inputs and outputs, so consecutive launches never find their operands in
        # L2 or the Infinity Cache (the sets of a step span well over 288 MB).
        self.fns = [[l.mk() for _ in range(rot)] for l in self.launches]
        torch.cuda.synchronize()
        # One eager pass over every set: library initialisation, and the kernel
        # configuration each launch resolves to.
        self.configs = []
        for i in range(len(self.launches)):
            for r in range(rot):
                self.fns[i][r]()
            # (a launch of several library calls describes them itself)
            describe = getattr(self.fns[i][rot - 1], 'config', None)
            self.configs.append(describe() if describe else deep_gemm.get_last_config())
        torch.cuda.synchronize()
        # HIP graphs (the library records into a capturing stream like any other);
        # replays take the Python launch overhead out of the timed regions.
        self.launch_graphs, self.step_graphs = [], []
        if not eager:
            for i in range(len(self.launches)):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for r in range(rot):
                        self.fns[i][r]()
                self.launch_graphs.append(g)
            for r in range(rot):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for i in range(len(self.launches)):
                        self.fns[i][r]()
                self.step_graphs.append(g)
            torch.cuda.synchronize()

    def run_launch(self, i):
        if self.eager:
            for r in range(self.rot):
                self.fns[i][r]()
        else:
            self.launch_graphs[i].replay()

    def run_step(self, sidx):
        if self.eager:
            for i in range(len(self.launches)):
                self.fns[i][sidx % self.rot]()
        else:
            self.step_graphs[sidx % self.rot].replay()

    def per_launch_us(self, reps):
        """Per-launch kernel durations: HIP events on the launch stream (torch's
        current stream, which the library and the graph replays launch on) around
        the launch run over all of its sets, / rot, with L2 and the 256 MB Infinity
        Cache flushed before each run, as the reference's bench_kineto flushes L2
        (deep_gemm/testing/bench.py:76-104), so operands come from HBM. The flush
        READS a 512 MiB buffer instead of zero-filling one: a fill leaves up to
        288 MB of dirty lines in L2 and the memory-side Infinity Cache whose
        write-back then lands inside the next timed kernel (up to 30% of an
        HBM-bound launch here); a read evicts the operands without that backlog."""
        import torch
        stream = torch.cuda.current_stream()
        flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.int32, device='cuda:0')
        per = []
        for i, l in enumerate(self.launches):
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            for e0, e1 in evs:
                torch.sum(flush, dtype=torch.int64)
                e0.record(stream)
                self.run_launch(i)
                e1.record(stream)
            torch.cuda.synchronize()
            us = sum(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3 / (reps * self.rot)
            per.append(us)
            log(f'  [{self.name}] {l.name}: {us:8.1f} us  {l.flops / us / 1e6:7.1f} TFLOPS  '
                f'{l.nbytes / us / 1e3:7.1f} GB/s  roofline {t_min_us(l.flops, l.nbytes) / us:.3f}  [{self.configs[i]}]')
        del flush
        return per

    def summary(self, per):
        """Per-launch and aggregate roofline scoring: each launch against its own
        bound t_min = max(FLOPs / P_fp8, bytes / BW); the aggregate fraction is
        sum(t_min) / sum(t_measured)."""
        t_mins = [t_min_us(l.flops, l.nbytes) for l in self.launches]
        bounds = ['mfma' if l.flops / (PEAK_FP8_TFLOPS * 1e6) >= l.nbytes / (PEAK_HBM_GBS * 1e3) else 'hbm'
                  for l in self.launches]
        return {
            'workload': self.cfg['workload'],
            'frac': round(sum(t_mins) / sum(per), 4),
            'kernel_us': round(sum(per), 2),
            'per_launch': {l.name: {'us': round(u, 2), 'tflops': round(l.flops / u / 1e6, 1),
                                    'gbs': round(l.nbytes / u / 1e3, 1), 'bound': b,
                                    'frac': round(tm / u, 4), 'config': c}
                           for l, u, tm, b, c in zip(self.launches, per, t_mins, bounds, self.configs)},
        }


# ---------------------------------------------------------------- main

def main():
    args = parse()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only: this build has no multi-GPU path '
              f'(requested --gpus {args.gpus}); run with --gpus 1', file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.calibrate_copy_mib > 0:
        x = torch.randn(args.calibrate_copy_mib * 1024 * 256, device='cuda:0')
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)
        torch.cuda.synchronize()
        del x, y
    global SFA_MAJOR
    SFA_MAJOR = args.sfa_major
    rot = args.rotate
    reps = max(5, args.steps)
    wl = Workload(args.workload, rot, args.eager)
    launches = wl.launches
    log(f'workload {args.workload}: {len(launches)} launches per step, {rot} rotating buffer sets')
    per = wl.per_launch_us(reps)

    for w in range(args.warmup):
        wl.run_step(w)
    # Whole-job timed region: K steps, synchronized on both sides.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for sidx in range(args.steps):
        wl.run_step(sidx)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    total_flops = sum(l.flops for l in launches) * args.steps
    total_bytes = sum(l.nbytes for l in launches)
    value = total_flops / elapsed / 1e12
    cast = args.workload in ('cast', 'moe_dispatch')
    if cast:   # a byte-moving workload: GB/s
        value = total_bytes * args.steps / elapsed / 1e9

    summ = wl.summary(per)
    kernel_us = sum(per)
    t_mins = [t_min_us(l.flops, l.nbytes) for l in launches]
    mfma_t = sum(l.flops / (PEAK_FP8_TFLOPS * 1e6) for l in launches)
    hbm_t = sum(l.nbytes / (PEAK_HBM_GBS * 1e3) for l in launches)
    bound = 'mfma' if mfma_t >= hbm_t else 'hbm'
    if all(b['bound'] == bound for b in summ['per_launch'].values()):
        # every launch has the same bound: the plain rate against that peak
        achieved = (sum(l.flops for l in launches) / kernel_us / 1e6 if bound == 'mfma'
                    else total_bytes / kernel_us / 1e3)
        how = (f'algorithmic {"FLOPs" if bound == "mfma" else "bytes"} of the step / sum of per-launch durations')
    else:
        # mixed bounds: each launch is scored against its own roofline time, and the
        # step's rate is that fraction of the dominant bound's peak
        achieved = sum(t_mins) / kernel_us * (PEAK_FP8_TFLOPS if bound == 'mfma' else PEAK_HBM_GBS)
        how = ('peak-equivalent rate: sum over launches of t_min = max(FLOPs/P_fp8, bytes/BW), / sum of '
               'per-launch durations, x the dominant bound\'s peak')
    peak = PEAK_FP8_TFLOPS if bound == 'mfma' else PEAK_HBM_GBS
    traffic, traffic_note = load_traffic(args.workload, launches, wl.configs)
    roofline = {'bound': bound, 'achieved': round(achieved, 2), 'peak': peak,
                'unit': 'TFLOP/s' if bound == 'mfma' else 'GB/s',
                'frac': round(achieved / peak, 4), 'traffic': traffic,
                'per': f'one step = {len(launches)} launch(es), one per shape; achieved = {how} (each the event '
                       f'time of {rot} back-to-back launches on rotating buffer sets after a cache flush, / {rot}); '
                       f'traffic = calibrated HBM bytes (FETCH_SIZE + WRITE_SIZE) of the step',
                'traffic_source': traffic_note,
                'kernel': sorted({c.split(' kind=')[0] for c in wl.configs}),
                'launch_config': {l.name: c for l, c in zip(launches, wl.configs)},
                'algorithmic_bytes': {l.name: l.nbytes for l in launches},
                'per_launch_us': {l.name: round(u, 2) for l, u in zip(launches, per)},
                'per_launch_tflops': {l.name: round(l.flops / u / 1e6, 1) for l, u in zip(launches, per)},
                'per_launch_gbs': {l.name: round(l.nbytes / u / 1e3, 1) for l, u in zip(launches, per)},
                'per_launch_frac': {k: v['frac'] for k, v in summ['per_launch'].items()},
                'per_launch_bound': {k: v['bound'] for k, v in summ['per_launch'].items()}}
    out = {
        'metric': ('MoE dispatch GB/s (routed FP8 rows into the contiguous expert layout)'
                   if args.workload == 'moe_dispatch' else
                   'FP8 per-token activation cast GB/s (bf16 -> e4m3 + 1x128 SFA)' if cast else
                   'FP8 block-scaled GEMM TFLOPS + % of MI355X FP8 MFMA peak, DSV3 shapes'),
        'value': round(value, 2),
        'unit': 'GB/s' if cast else 'TFLOPS',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(elapsed / args.steps * 1e3, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': ('e4m3 rows' if args.workload == 'moe_dispatch' else 'bf16 -> e4m3' if cast else
                  'e4m3 (fp32 accumulate)' if args.workload != 'fp8fp4' else 'e4m3 x e2m1 (fp32 accumulate)'),
        'data': 'synthetic (seeded randn, bf16 -> quantized)',
        'config': wl.cfg,
        'timing': {'launch': 'eager (Python)' if args.eager else 'hipGraph replay', 'rotating_sets': rot,
                   'per_launch_reps': reps},
        'roofline': roofline,
    }
    del wl
    torch.cuda.empty_cache()
    # The other configurations, kernel time and roofline fraction per launch
    # (not part of `value`, which is the headline configuration's whole-job rate).
    if args.workload == 'dense' and not args.no_extras:
        extras = {}
        for name in EXTRAS:
            log(f'extra workload {name} ...')
            w = Workload(name, rot, args.eager)
            extras[name] = w.summary(w.per_launch_us(reps))
            del w
            torch.cuda.empty_cache()
        out['other_configs'] = extras
    if args.workload == 'masked' and args.hbm_context:
        log('HBM context ...')
        out['hbm_context'] = hbm_context(reps)
    if args.workload == 'dense' and args.hipblaslt:
        log('hipBLASLt context ...')
        out['hipblaslt_fp8_context'] = hipblaslt_context(rot, reps)
    if not args.no_cpu_baseline:
        log('cpu baseline ...')
        out['cpu_baseline'] = cpu_baseline(args.workload, args.cpu_sample_m)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
