"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects malformed arguments on the host (before any HIP
call) with the reference's error format."""
import ctypes
import os
import re

import pytest
import torch

import deep_gemm
from deep_gemm import _ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'deepgemm_mi355x.h')


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(dg_[a-z0-9_]+)\s*\(', text)))


def test_header_symbols_exported():
    syms = declared_symbols()
    assert len(syms) >= 15
    lib = ctypes.CDLL(_ffi.LIB_PATH)
    for s in syms:
        assert hasattr(lib, s), f'{s} declared in the header but not exported'
    assert set(syms) == set(_ffi.SIGNATURES), 'binding table out of sync with the header'


def test_version_and_init():
    assert b'gfx950' in _ffi.lib.dg_version()
    assert _ffi.lib.dg_init() == 0
    assert _ffi.lib.dg_last_error() == b''


def test_tma_aligned_size():
    assert deep_gemm.get_tma_aligned_size(4097, 4) == 4100
    assert deep_gemm.get_tma_aligned_size(4096, 4) == 4096
    assert deep_gemm.get_tma_aligned_size(5, 1) == 16
    with pytest.raises(RuntimeError, match='Assertion error'):
        deep_gemm.get_tma_aligned_size(5, 3)


def test_alignment_and_num_sms_knobs():
    assert deep_gemm.get_mk_alignment_for_contiguous_layout() == 128
    deep_gemm.set_mk_alignment_for_contiguous_layout(256)
    assert deep_gemm.get_m_alignment_for_contiguous_layout() == 256
    deep_gemm.set_mk_alignment_for_contiguous_layout(128)
    assert deep_gemm.get_theoretical_mk_alignment_for_contiguous_layout() == 128
    deep_gemm.set_num_sms(200)
    assert deep_gemm.get_num_sms() == 200
    deep_gemm.init()
    with pytest.raises(RuntimeError):
        deep_gemm.set_num_sms(0)
    with pytest.raises(RuntimeError, match='Unsupported'):
        deep_gemm.set_tile_override(96, 64, variant=1)
    with pytest.raises(RuntimeError, match='Unsupported'):
        deep_gemm.set_tile_override(64, 64, variant=2)


# ----------------------------------------------------------------- host validation
# dg_tensor structs with device = 0 and fake addresses: every call below must be
# rejected by a host check, before the library could touch device memory.

def fake(shape, dtype, strides=None, addr=0x10000000, device=0):
    t = _ffi.DgTensor()
    t.data = addr
    t.dtype = dtype
    t.ndim = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        t.sizes[i] = s
        t.strides[i] = st
    t.device = device
    return t


def call_nt(a, sfa, b, sfb, d, c=None, recipe=None, disable=0, ep=None):
    st = _ffi.lib.dg_fp8_fp4_gemm_nt(ctypes.byref(a), ctypes.byref(sfa), ctypes.byref(b), ctypes.byref(sfb),
                                    ctypes.byref(d), ctypes.byref(c) if c else None,
                                    ctypes.byref(recipe) if recipe else None, disable,
                                    ctypes.byref(ep) if ep else None, None)
    return st, _ffi.lib.dg_last_error().decode()


def good_dense(m=256, n=512, k=1024):
    return (fake((m, k), _ffi.DG_E4M3), fake((m, k // 128), _ffi.DG_F32), fake((n, k), _ffi.DG_E4M3),
            fake((n // 128, k // 128), _ffi.DG_F32), fake((m, n), _ffi.DG_BF16))


def test_rejects_host_tensors():
    a, sfa, b, sfb, d = good_dense()
    a.device = -1
    st, msg = call_nt(a, sfa, b, sfb, d)
    assert st == _ffi.DG_ERR_INVALID and 'on_device' in msg and msg.startswith('Assertion error (')


def test_rejects_shape_mismatch():
    a, sfa, b, sfb, _ = good_dense()
    st, msg = call_nt(a, sfa, b, sfb, fake((256, 500), _ffi.DG_BF16))
    assert st == _ffi.DG_ERR_INVALID and 'm == m_' in msg


def test_rejects_mn_major_a():
    m, k = 256, 1024
    _, sfa, b, sfb, d = good_dense()
    a = fake((m, k), _ffi.DG_E4M3, strides=(1, m))
    st, msg = call_nt(a, sfa, b, sfb, d)
    assert st == _ffi.DG_ERR_INVALID and 'is_k_major(a)' in msg


def test_rejects_bad_output_dtype():
    a, sfa, b, sfb, _ = good_dense()
    st, msg = call_nt(a, sfa, b, sfb, fake((256, 512), _ffi.DG_F16))
    assert st == _ffi.DG_ERR_INVALID and 'DG_BF16' in msg


def test_rejects_bad_sf_shapes():
    a, sfa, b, sfb, d = good_dense()
    st, msg = call_nt(a, fake((256, 7), _ffi.DG_F32), b, sfb, d)
    assert st == _ffi.DG_ERR_INVALID and 'sf.size(-1)' in msg
    st, msg = call_nt(a, sfa, b, fake((3, 8), _ffi.DG_F32), d)
    assert st == _ffi.DG_ERR_INVALID and 'sf.size(-2)' in msg


def test_rejects_recipe_and_pair_together():
    a, sfa, b, sfb, d = good_dense()
    r = _ffi.recipe_struct((1, 128, 128))
    r.has_recipe_ab = 1
    st, msg = call_nt(a, sfa, b, sfb, d, recipe=r)
    assert st == _ffi.DG_ERR_INVALID and 'has_recipe' in msg


def test_rejects_c_dtype_mismatch():
    a, sfa, b, sfb, _ = good_dense()
    d = fake((256, 512), _ffi.DG_F32)
    c = fake((256, 512), _ffi.DG_BF16, addr=0x20000000)
    st, msg = call_nt(a, sfa, b, sfb, d, c=c)
    assert st == _ffi.DG_ERR_INVALID and 'dtype' in msg


def test_rejects_unaligned_operand():
    a, sfa, b, sfb, d = good_dense()
    a.data = 0x10000008
    st, msg = call_nt(a, sfa, b, sfb, d)
    assert st == _ffi.DG_ERR_INVALID and '16-byte aligned' in msg


def test_1d1d_recipe_host_checks():
    """(1, 1, 128) with FP32 SFs is the 1D1D path: FP32 D and C required
    (sm90_fp8_gemm_1d1d.hpp:91), K % 128 == 0 here."""
    a, sfa, b, _, d = good_dense()
    sfb = fake((512, 8), _ffi.DG_F32)
    r = _ffi.recipe_struct(None, (1, 128), (1, 128))
    st, msg = call_nt(a, sfa, b, sfb, d, recipe=r)               # bf16 D, no C
    assert st == _ffi.DG_ERR_INVALID and 'o.c != nullptr' in msg
    d32 = fake((256, 512), _ffi.DG_F32)
    st, msg = call_nt(a, sfa, b, sfb, d32, recipe=r)             # FP32 D, no C
    assert st == _ffi.DG_ERR_INVALID and 'o.c != nullptr' in msg
    m, n, k = 256, 512, 1000
    st, msg = call_nt(fake((m, k), _ffi.DG_E4M3), fake((m, 8), _ffi.DG_F32), fake((n, k), _ffi.DG_E4M3),
                      fake((n, 8), _ffi.DG_F32), d32, c=d32, recipe=r)
    assert st == _ffi.DG_ERR_UNSUPPORTED and 'multiple of 128' in msg


def call_kg(a, sfa, b, sfb, d, ks, layout, c, recipe=(1, 1, 128), psum=0, tn=False):
    arr = (ctypes.c_int32 * max(1, len(ks)))(*ks)
    rec = (ctypes.c_int32 * 3)(*recipe)
    fn = _ffi.lib.dg_k_grouped_fp8_gemm_tn_contiguous if tn else _ffi.lib.dg_k_grouped_fp8_gemm_nt_contiguous
    st = fn(ctypes.byref(a), ctypes.byref(sfa), ctypes.byref(b), ctypes.byref(sfb), ctypes.byref(d), arr, len(ks),
            ctypes.byref(layout), ctypes.byref(c) if c else None, rec, psum, None)
    return st, _ffi.lib.dg_last_error().decode()


def test_k_grouped_host_checks():
    """The reference's argument checks of k_grouped_fp8_gemm_nt_contiguous
    (csrc/apis/gemm.hpp:369-404, check_k_grouped_args :55-76), all on the host."""
    g, m, n, ks = 2, 128, 256, [256, 128]
    sk = sum(ks)

    def ops(ks_=ks):
        s = sum(ks_)
        return (fake((s * m,), _ffi.DG_E4M3), fake((m, s // 128), _ffi.DG_F32), fake((s * n,), _ffi.DG_E4M3),
                fake((n, s // 128), _ffi.DG_F32), fake((g, m, n), _ffi.DG_F32))
    layout = fake((g,), _ffi.DG_I32)
    a, sfa, b, sfb, d = ops()
    st, msg = call_kg(a, sfa, b, sfb, d, ks, layout, d, recipe=(1, 1, 32))
    assert st == _ffi.DG_ERR_INVALID and 'r2 == 128' in msg
    st, msg = call_kg(a, sfa, b, sfb, d, ks, layout, d, psum=1)
    assert st == _ffi.DG_ERR_INVALID and 'use_psum_layout' in msg
    st, msg = call_kg(a, sfa, b, sfb, d, ks, layout, None)
    assert st == _ffi.DG_ERR_INVALID and 'c != nullptr' in msg
    st, msg = call_kg(a, sfa, b, sfb, d, [256, 100], layout, d)
    assert st == _ffi.DG_ERR_INVALID and '% 128' in msg
    st, msg = call_kg(a, sfa, b, sfb, d, [256], layout, d)
    assert st == _ffi.DG_ERR_INVALID and 'num_ks' in msg
    st, msg = call_kg(fake((sk * m + 16,), _ffi.DG_E4M3), sfa, b, sfb, d, ks, layout, d)
    assert st == _ffi.DG_ERR_INVALID and 'sum_k * m' in msg
    st, msg = call_kg(a, sfa, b, sfb, fake((g, m, n), _ffi.DG_BF16), ks, layout, d)
    assert st == _ffi.DG_ERR_INVALID and 'DG_F32' in msg
    st, msg = call_kg(a, fake((m, 2), _ffi.DG_F32), b, sfb, d, ks, layout, d)
    assert st == _ffi.DG_ERR_INVALID and 'sum_k / 128' in msg
    st, msg = call_kg(a, sfa, b, sfb, d, ks, layout, d, tn=True)
    assert st == _ffi.DG_ERR_UNSUPPORTED and 'Unsupported' in msg


def test_ue8m0_path_rejects_disable_cast():
    m, n, k = 128, 256, 512
    a = fake((m, k), _ffi.DG_E4M3)
    sfa = fake((m, k // 128), _ffi.DG_F32)
    b = fake((n, k // 2), _ffi.DG_I8)
    sfb = fake((n, k // 32), _ffi.DG_F32)
    d = fake((m, n), _ffi.DG_BF16)
    r = _ffi.recipe_struct(None, (1, 128), (1, 32))
    st, msg = call_nt(a, sfa, b, sfb, d, recipe=r, disable=1)
    assert st == _ffi.DG_ERR_INVALID and 'disable_ue8m0_cast' in msg


def test_grouped_validation():
    g, m, n, k = 4, 512, 256, 1024
    a = fake((m, k), _ffi.DG_E4M3)
    sfa = fake((m, k // 128), _ffi.DG_F32)
    b = fake((g, n, k), _ffi.DG_E4M3)
    sfb = fake((g, n // 128, k // 128), _ffi.DG_F32)
    d = fake((m, n), _ffi.DG_BF16)
    idx = fake((m - 1,), _ffi.DG_I32)
    st = _ffi.lib.dg_m_grouped_fp8_fp4_gemm_nt_contiguous(*(ctypes.byref(x) for x in (a, sfa, b, sfb, d, idx)),
                                                          None, 0, 0, 1, -1, None, None)
    assert st == _ffi.DG_ERR_INVALID and 'gl.size(0) == m' in _ffi.lib.dg_last_error().decode()
    # masked: masked_m length must equal G
    a3 = fake((g, 256, k), _ffi.DG_E4M3)
    sfa3 = fake((g, 256, k // 128), _ffi.DG_F32)
    d3 = fake((g, 256, n), _ffi.DG_BF16)
    mm = fake((g + 1,), _ffi.DG_I32)
    st = _ffi.lib.dg_m_grouped_fp8_fp4_gemm_nt_masked(*(ctypes.byref(x) for x in (a3, sfa3, b, sfb, d3, mm)),
                                                      128, None, 0, None, None)
    assert st == _ffi.DG_ERR_INVALID and 'g == g___' in _ffi.lib.dg_last_error().decode()
    # expected_m must be positive
    mm = fake((g,), _ffi.DG_I32)
    st = _ffi.lib.dg_m_grouped_fp8_fp4_gemm_nt_masked(*(ctypes.byref(x) for x in (a3, sfa3, b, sfb, d3, mm)),
                                                      0, None, 0, None, None)
    assert st == _ffi.DG_ERR_INVALID and 'expected_m > 0' in _ffi.lib.dg_last_error().decode()


def test_k_tail_rejects_256x256_override():
    """The 256 x 256 pipelined tile has no K-tail schedule (it would spill
    registers): a tile override that would launch it with K % 128 != 0 (plain
    or persistent) is refused on the host, before any launch."""
    a, sfa, b, sfb, d = good_dense(512, 512, 1040)
    sfa = fake((512, 9), _ffi.DG_F32)
    sfb = fake((4, 9), _ffi.DG_F32)
    for variant in (2, 4):
        deep_gemm.set_tile_override(256, 256, variant=variant)
        try:
            st, msg = call_nt(a, sfa, b, sfb, d)
        finally:
            deep_gemm.set_tile_override(0, 0)
        assert st == _ffi.DG_ERR_UNSUPPORTED and 'K % 128 == 0' in msg, (variant, msg)


def test_fused_swiglu_host_checks():
    """dg_m_grouped_fp8_gemm_nt_{contiguous,masked}_swiglu: shape, dtype and layout
    checks run on the host before any launch."""
    g, m, inter, k = 4, 512, 256, 1024
    n = 2 * inter
    a = fake((m, k), _ffi.DG_E4M3)
    sfa = fake((m, k // 128), _ffi.DG_F32)
    b = fake((g, n, k), _ffi.DG_E4M3)
    sfb = fake((g, n // 128, k // 128), _ffi.DG_F32)
    idx = fake((m,), _ffi.DG_I32)
    q = fake((m, inter), _ffi.DG_E4M3)
    sf = fake((m, inter // 128), _ffi.DG_F32)
    w = fake((m,), _ffi.DG_F32)

    def contiguous(a=a, b=b, sfb=sfb, q=q, sf=sf, w=w, psum=0):
        st = _ffi.lib.dg_m_grouped_fp8_gemm_nt_contiguous_swiglu(
            *(ctypes.byref(x) for x in (a, sfa, b, sfb, idx)), ctypes.byref(w) if w else None, 0.0,
            ctypes.byref(q), ctypes.byref(sf), psum, 1, None)
        return st, _ffi.lib.dg_last_error().decode()

    st, msg = contiguous(b=fake((g, 384, k), _ffi.DG_E4M3), sfb=fake((g, 3, k // 128), _ffi.DG_F32))
    assert st == _ffi.DG_ERR_UNSUPPORTED and 'multiple of 256' in msg
    st, msg = contiguous(q=fake((m, inter), _ffi.DG_BF16))
    assert st == _ffi.DG_ERR_INVALID and 'q.dtype() == DG_E4M3' in msg
    st, msg = contiguous(q=fake((m, n), _ffi.DG_E4M3))
    assert st == _ffi.DG_ERR_INVALID and 'q.size(-1) == inter' in msg
    st, msg = contiguous(q=fake((m, inter), _ffi.DG_E4M3, strides=(inter + 4, 1)))
    assert st == _ffi.DG_ERR_INVALID and 'ldq % 8 == 0' in msg
    st, msg = contiguous(sf=fake((m, inter // 64), _ffi.DG_F32))
    assert st == _ffi.DG_ERR_INVALID and 'sfq.size(-1) == inter / 128' in msg
    st, msg = contiguous(w=fake((m - 1,), _ffi.DG_F32))
    assert st == _ffi.DG_ERR_INVALID and 'wv.size(0) == m' in msg
    st, msg = contiguous(psum=1)   # psum: grouped_layout holds one end per group
    assert st == _ffi.DG_ERR_INVALID and 'gl.size(0) ==' in msg
    st, msg = contiguous(a=fake((m, k), _ffi.DG_E4M3, device=-1))
    assert st == _ffi.DG_ERR_INVALID and 'on_device' in msg
    # 256 x 256 tiles need K % 128 == 0 (the K-tail 256-row schedule is not built)
    a_t, sfa_t = fake((m, 1040), _ffi.DG_E4M3), fake((m, 9), _ffi.DG_F32)
    b_t, sfb_t = fake((g, n, 1040), _ffi.DG_E4M3), fake((g, n // 128, 9), _ffi.DG_F32)
    deep_gemm.set_tile_override(256, 256, variant=2)
    try:
        st = _ffi.lib.dg_m_grouped_fp8_gemm_nt_contiguous_swiglu(
            *(ctypes.byref(x) for x in (a_t, sfa_t, b_t, sfb_t, idx)), None, 0.0, ctypes.byref(q), ctypes.byref(sf),
            0, 1, None)
        msg = _ffi.lib.dg_last_error().decode()
    finally:
        deep_gemm.set_tile_override(0, 0)
    assert st == _ffi.DG_ERR_UNSUPPORTED and '128 x 256' in msg
    # masked: q is [G, max_m, I], masked_m has G entries, expected_m > 0
    max_m = 128
    a3 = fake((g, max_m, k), _ffi.DG_E4M3)
    sfa3 = fake((g, max_m, k // 128), _ffi.DG_F32)
    mm = fake((g,), _ffi.DG_I32)
    q3 = fake((g, max_m, inter), _ffi.DG_E4M3)
    sf3 = fake((g, max_m, inter // 128), _ffi.DG_F32)

    def masked(q=q3, expected_m=64, mm=mm):
        st = _ffi.lib.dg_m_grouped_fp8_gemm_nt_masked_swiglu(
            *(ctypes.byref(x) for x in (a3, sfa3, b, sfb, mm)), expected_m, None, 0.0, ctypes.byref(q),
            ctypes.byref(sf3), None)
        return st, _ffi.lib.dg_last_error().decode()

    st, msg = masked(q=fake((g * max_m, inter), _ffi.DG_E4M3))
    assert st == _ffi.DG_ERR_INVALID and 'dim() == n' in msg
    st, msg = masked(expected_m=0)
    assert st == _ffi.DG_ERR_INVALID and 'expected_m > 0' in msg
    st, msg = masked(mm=fake((g + 1,), _ffi.DG_I32))
    assert st == _ffi.DG_ERR_INVALID and 'gl.size(0) == g' in msg


def test_plan_sf_transform_kinds():
    def plan(sf, mn, k, recipe3=None, recipe2=None, groups=-1, is_sfa=-1, disable=0):
        kind = ctypes.c_int32(-1)
        r3 = (ctypes.c_int32 * 3)(*recipe3) if recipe3 else None
        r2 = (ctypes.c_int32 * 2)(*recipe2) if recipe2 else None
        st = _ffi.lib.dg_plan_sf_transform(ctypes.byref(sf), mn, k, r3, r2, groups, is_sfa, disable,
                                           ctypes.byref(kind))
        return st, kind.value
    assert plan(fake((4096, 56), _ffi.DG_F32), 4096, 7168, recipe3=(1, 128, 128), is_sfa=1) == (0, 1)
    assert plan(fake((17, 56), _ffi.DG_F32), 2112, 7168, recipe3=(1, 128, 128), is_sfa=0) == (0, 0)
    assert plan(fake((7168, 224), _ffi.DG_F32), 7168, 7168, recipe2=(1, 32)) == (0, 2)
    st, _ = plan(fake((7168, 224), _ffi.DG_F32), 7168, 7168, recipe2=(1, 32), disable=1)
    assert st == _ffi.DG_ERR_INVALID
    st, _ = plan(fake((4096, 55), _ffi.DG_F32), 4096, 7168, recipe3=(1, 128, 128), is_sfa=1)
    assert st == _ffi.DG_ERR_INVALID


def test_python_shim_errors():
    x = torch.zeros((128, 256), dtype=torch.float8_e4m3fn)
    s = torch.ones((128, 2))
    with pytest.raises(RuntimeError, match=r'Assertion error \(dg_api\.cpp:\d+\)'):
        deep_gemm.fp8_gemm_nt((x, s), (x, torch.ones((1, 2))), torch.empty((128, 128), dtype=torch.bfloat16))
    # (alpha reaches the library, whose device checks come first for host tensors)
    with pytest.raises(RuntimeError, match=r'Assertion error \(dg_api\.cpp:\d+\)'):
        deep_gemm.fp8_gemm_nt((x, s), (x, s), torch.empty((128, 128)), alpha=2.0)
    with pytest.raises(TypeError, match='epilogue'):
        deep_gemm.fp8_gemm_nt((x, s), (x, s), torch.empty((128, 128)), epilogue=object())


def test_epilogue_host_checks():
    """alpha / epilogue classes exist on the UE8M0 path only (reference
    csrc/apis/gemm.hpp:118-119 for the FP32-scale path); the FP8 stage is a BF16 D
    without C; unknown kinds are rejected. All checks run before any launch."""
    a, sfa, b, sfb, d = good_dense()
    st, msg = call_nt(a, sfa, b, sfb, d, ep=_ffi.DgEpilogue(_ffi.EPILOGUE_ALPHA, 2.0))
    assert st == _ffi.DG_ERR_INVALID and 'need UE8M0 scales' in msg, msg
    st, msg = call_nt(a, sfa, b, sfb, d, ep=_ffi.DgEpilogue(_ffi.EPILOGUE_IDENTITY, 1.0))
    assert st == _ffi.DG_ERR_INVALID and 'need UE8M0 scales' in msg, msg
    st, msg = call_nt(a, sfa, b, sfb, d, ep=_ffi.DgEpilogue(7, 1.0))
    assert st == _ffi.DG_ERR_INVALID and 'DG_EPILOGUE_IDENTITY' in msg, msg
    c = fake((256, 512), _ffi.DG_BF16)
    st, msg = call_nt(a, sfa, b, sfb, d, c=c, ep=_ffi.DgEpilogue(_ffi.EPILOGUE_FP8_STAGE, 1.0))
    assert st == _ffi.DG_ERR_INVALID and 'o.c == nullptr' in msg, msg


def test_epilogue_python_resolution():
    """The Python resolution mirrors resolve_epilogue_class
    (csrc/jit_kernels/impls/epilogue_class.hpp:111-124) before any device work."""
    import torch
    import deep_gemm
    ep = deep_gemm.epilogue
    a = (torch.zeros(4, 128, dtype=torch.float8_e4m3fn), torch.zeros(4, 1, dtype=torch.int32))
    b = (torch.zeros(4, 128, dtype=torch.float8_e4m3fn), torch.zeros(4, 1, dtype=torch.int32))
    d = torch.zeros(4, 4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='exclusive'):
        deep_gemm.fp8_fp4_gemm_nt(a, b, d, alpha=2.0, epilogue=ep.Identity())
    with pytest.raises(RuntimeError, match='StochasticRounding'):
        deep_gemm.fp8_fp4_gemm_nt(a, b, d, epilogue=ep.BF16StochasticRounding())
    with pytest.raises(RuntimeError, match='direct E4M3 output'):
        deep_gemm.fp8_fp4_gemm_nt(a, b, d, epilogue=ep.FP8Quantization(torch.zeros(4, 1, dtype=torch.int32)))
    with pytest.raises(RuntimeError, match='need UE8M0 scales'):
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous(a, b, d, [128], torch.zeros(1, dtype=torch.int32),
                                                   epilogue=ep.Identity())
    assert isinstance(ep.Alpha(0.5), ep.Epilogue) and ep.Alpha(0.5).alpha == 0.5
