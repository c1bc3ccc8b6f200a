"""The allocation-free dispatch (dg_moe_dispatch_noalloc) against dg_moe_dispatch,
both called through the C-ABI.

Bar: bit-exact (dispatch is integer and copy work). Two calls in a row on one
device, the second with a smaller input, so the second reads the fixed device
scratch after the first left its contents there; a call whose workspace exceeds
the fixed scratch must fail with DG_ERR_INVALID before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from deep_gemm import _ffi
import generators as gen
from oracle import quant as oquant

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'
LAYOUTS = {'contiguous': 0, 'psum': 1, 'masked': 2}
SCRATCH_INTS = 262144
CHUNK_TOKENS = 64


def _inputs(t, k, e, kdim, seed):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, e, size=(t, k)).astype(np.int32)
    idx = np.where(rng.random((t, k)) < 0.1, -1, idx).astype(np.int32)
    w = rng.random((t, k)).astype(np.float32)
    q, sf = oquant.per_token_cast_to_fp8(gen.randn_bf16((t, kdim), seed), use_ue8m0=False)
    return (gen.to_dev(q, torch.float8_e4m3fn), gen.to_dev(sf), gen.to_dev(idx), gen.to_dev(w))


def _outputs(t, k, e, kdim, layout, max_m, alignment):
    """Output buffers filled with a sentinel, so untouched rows compare too."""
    sfk = (kdim + 127) // 128
    if layout == 'masked':
        rows = e * max_m
        a = torch.full((e, max_m, kdim), 0x7B, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
        sf = torch.full((e, max_m, sfk), -3.0, dtype=torch.float32, device=DEV)
        gl = torch.full((e,), -7, dtype=torch.int32, device=DEV)
    else:
        rows = int(_ffi.lib.dg_moe_dispatch_max_rows(t, k, e, alignment))
        assert rows >= 0
        a = torch.full((rows, kdim), 0x7B, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
        sf = torch.full((rows, sfk), -3.0, dtype=torch.float32, device=DEV)
        gl = torch.full((rows if layout == 'contiguous' else e,), -7, dtype=torch.int32, device=DEV)
    pos = torch.full((t, k), -7, dtype=torch.int32, device=DEV)
    rw = torch.full((rows,), -3.0, dtype=torch.float32, device=DEV)
    return [a, sf, gl, pos, rw]


def _call(fn_name, ins, outs, e, layout, alignment, workspace=None):
    x, x_sf, idx, w = ins
    d = [_ffi.describe(v) for v in (x, x_sf, idx, w)] + [_ffi.describe(v) for v in outs]
    args = [ctypes.byref(v) for v in d[:4]] + [e, LAYOUTS[layout], alignment] + \
        [ctypes.byref(v) for v in d[4:]]
    if workspace is not None:
        dws = _ffi.describe(workspace)
        args.append(ctypes.byref(dws))
    args.append(_ffi.stream_of(x))
    return getattr(_ffi.lib, fn_name)(*args)


def _dispatch_both(t, k, e, kdim, layout, seed, max_m=96, alignment=128):
    ins = _inputs(t, k, e, kdim, seed)
    print(f'noalloc dispatch layout={layout} t={t} k={k} e={e} kdim={kdim}', flush=True)
    ws_bytes = int(_ffi.lib.dg_moe_dispatch_workspace_size(t, e))
    ws = torch.empty((max(ws_bytes, 4) // 4,), dtype=torch.int32, device=DEV)
    ref = _outputs(t, k, e, kdim, layout, max_m, alignment)
    _ffi.check(_call('dg_moe_dispatch', ins, ref, e, layout, alignment, workspace=ws))
    got = _outputs(t, k, e, kdim, layout, max_m, alignment)
    _ffi.check(_call('dg_moe_dispatch_noalloc', ins, got, e, layout, alignment))
    torch.cuda.synchronize()
    for name, r, g in zip(('a', 'sf', 'grouped_layout', 'pos', 'row_weights'), ref, got):
        rb, gb = r.view(torch.uint8) if r.dtype == torch.float8_e4m3fn else r, \
            g.view(torch.uint8) if g.dtype == torch.float8_e4m3fn else g
        assert torch.equal(rb, gb), f'{name} differs ({layout}, t={t})'
    return got


@pytest.mark.parametrize('layout', ['contiguous', 'psum', 'masked'])
def test_noalloc_dispatch_equals_workspace_dispatch(layout):
    # a large call, then a smaller one: the second reuses the scratch the first filled
    big = _dispatch_both(4000, 8, 64, 512, layout, seed=1)
    small = _dispatch_both(37, 3, 16, 256, layout, seed=2)
    assert big[3].shape == (4000, 8) and small[3].shape == (37, 3)
    # the largest call the fixed scratch holds still runs
    e = 256
    t = ((SCRATCH_INTS - 2 * e - 1) // e) * CHUNK_TOKENS
    assert ((t + CHUNK_TOKENS - 1) // CHUNK_TOKENS) * e + 2 * e + 1 <= SCRATCH_INTS
    if layout == 'masked':
        _dispatch_both(t, 1, e, 128, layout, seed=3, max_m=512)


def test_noalloc_dispatch_rejects_oversize():
    e, kdim, max_m = 1024, 128, 4
    t = (SCRATCH_INTS // e + 1) * CHUNK_TOKENS          # needs more than the fixed scratch
    assert ((t + CHUNK_TOKENS - 1) // CHUNK_TOKENS) * e + 2 * e + 1 > SCRATCH_INTS
    x = torch.zeros((t, kdim), dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    x_sf = torch.ones((t, 1), dtype=torch.float32, device=DEV)
    idx = torch.zeros((t, 1), dtype=torch.int32, device=DEV)
    w = torch.ones((t, 1), dtype=torch.float32, device=DEV)
    outs = _outputs(t, 1, e, kdim, 'masked', max_m, 128)
    status = _call('dg_moe_dispatch_noalloc', (x, x_sf, idx, w), outs, e, 'masked', 128)
    assert status != 0
    msg = _ffi.lib.dg_last_error().decode()
    assert 'allocation-free' in msg and str(SCRATCH_INTS) in msg
    torch.cuda.synchronize()
    assert torch.all(outs[3] == -7)        # nothing ran
