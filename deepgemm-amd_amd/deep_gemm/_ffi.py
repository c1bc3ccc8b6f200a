"""ctypes binding of libdeepgemm_mi355x.so (the C ABI in include/deepgemm_mi355x.h).

Torch tensors are described to the library as `dg_tensor` structs (data
pointer, dtype code, sizes, element strides, device ordinal); the current HIP
stream of the output's device is passed as `void*`. A non-zero status raises
RuntimeError with the library's message, which mirrors the reference's
"Assertion error (file:line): condition" (csrc/utils/exception.hpp:17-19).

The library is required: importing this module without it raises ImportError.
There is no CPU or Python fallback.
"""
import ctypes
import os

import torch

_LIB_NAME = 'libdeepgemm_mi355x.so'
# DG_LIBRARY names another build of the same library (the sanitizer build of the
# host layer, tests/sanitize/build_asan.sh); by default the in-tree library.
_LIB_PATH = os.environ.get('DG_LIBRARY') or os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

DG_OK, DG_ERR_INVALID, DG_ERR_UNSUPPORTED, DG_ERR_HIP, DG_ERR_INTERNAL = 0, 1, 2, 3, 4
DG_F32, DG_BF16, DG_E4M3, DG_I32, DG_I8, DG_U8, DG_F16, DG_I64 = range(8)

_DTYPES = {
    torch.float32: DG_F32,
    torch.bfloat16: DG_BF16,
    torch.float8_e4m3fn: DG_E4M3,
    torch.int32: DG_I32,
    torch.int8: DG_I8,
    torch.uint8: DG_U8,
    torch.float16: DG_F16,
    torch.int64: DG_I64,
}
if hasattr(torch, 'float4_e2m1fn_x2'):
    _DTYPES[torch.float4_e2m1fn_x2] = DG_I8


class DgTensor(ctypes.Structure):
    _fields_ = [('data', ctypes.c_void_p),
                ('dtype', ctypes.c_int32),
                ('ndim', ctypes.c_int32),
                ('sizes', ctypes.c_int64 * 4),
                ('strides', ctypes.c_int64 * 4),
                ('device', ctypes.c_int32),
                ('reserved', ctypes.c_int32)]


class DgRecipe(ctypes.Structure):
    _fields_ = [('has_recipe', ctypes.c_int32),
                ('recipe', ctypes.c_int32 * 3),
                ('has_recipe_ab', ctypes.c_int32),
                ('recipe_a', ctypes.c_int32 * 2),
                ('recipe_b', ctypes.c_int32 * 2)]


class DgEpilogue(ctypes.Structure):
    _fields_ = [('kind', ctypes.c_int32),
                ('alpha', ctypes.c_float)]


EPILOGUE_IDENTITY, EPILOGUE_ALPHA, EPILOGUE_FP8_STAGE = 0, 1, 2

_P = ctypes.POINTER
_T = _P(DgTensor)
_R = _P(DgRecipe)
_E = _P(DgEpilogue)
_I = ctypes.c_int32
_V = ctypes.c_void_p

# name -> (restype, argtypes); every function the header declares.
SIGNATURES = {
    'dg_last_error': (ctypes.c_char_p, []),
    'dg_version': (ctypes.c_char_p, []),
    'dg_init': (_I, []),
    'dg_shutdown': (_I, []),
    'dg_fp8_fp4_gemm_nt': (_I, [_T, _T, _T, _T, _T, _T, _R, _I, _E, _V]),
    'dg_fp8_fp4_gemm_nt_ws': (_I, [_T, _T, _T, _T, _T, _T, _R, _I, _E, _T, _V]),
    'dg_fp8_gemm_nt_workspace_size': (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    'dg_m_grouped_fp8_fp4_gemm_nt_contiguous': (_I, [_T, _T, _T, _T, _T, _T, _R, _I, _I, _I, _I, _E, _V]),
    'dg_m_grouped_fp8_fp4_gemm_nt_masked': (_I, [_T, _T, _T, _T, _T, _T, _I, _R, _I, _E, _V]),
    'dg_get_tma_aligned_size': (_I, [_I, _I, _P(_I)]),
    'dg_get_mn_major_tma_aligned_tensor': (_I, [_T, _T, _V]),
    'dg_get_mn_major_tma_aligned_packed_ue8m0_tensor': (_I, [_T, _T, _V]),
    'dg_plan_sf_transform': (_I, [_T, _I, _I, _P(_I), _P(_I), _I, _I, _I, _P(_I)]),
    'dg_per_token_cast_to_fp8': (_I, [_T, _T, _T, _I, _I, _V]),
    'dg_moe_dispatch_workspace_size': (ctypes.c_int64, [ctypes.c_int64, _I]),
    'dg_moe_dispatch_max_rows': (ctypes.c_int64, [ctypes.c_int64, _I, _I, _I]),
    'dg_moe_dispatch': (_I, [_T, _T, _T, _T, _I, _I, _I, _T, _T, _T, _T, _T, _T, _V]),
    'dg_moe_dispatch_noalloc': (_I, [_T, _T, _T, _T, _I, _I, _I, _T, _T, _T, _T, _T, _V]),
    'dg_moe_swiglu_apply_weight_to_fp8': (_I, [_T, _T, _T, ctypes.c_float, _T, _T, _I, _V]),
    'dg_moe_combine': (_I, [_T, _T, _T, _T, _V]),
    'dg_m_grouped_fp8_gemm_nt_contiguous_swiglu': (_I, [_T, _T, _T, _T, _T, _T, ctypes.c_float, _T, _T, _I, _I, _V]),
    'dg_m_grouped_fp8_gemm_nt_masked_swiglu': (_I, [_T, _T, _T, _T, _T, _I, _T, ctypes.c_float, _T, _T, _V]),
    'dg_k_grouped_fp8_gemm_nt_contiguous': (_I, [_T, _T, _T, _T, _T, _P(_I), _I, _T, _T, _P(_I), _I, _V]),
    'dg_k_grouped_fp8_gemm_tn_contiguous': (_I, [_T, _T, _T, _T, _T, _P(_I), _I, _T, _T, _P(_I), _I, _V]),
    'dg_set_num_sms': (_I, [_I]),
    'dg_get_num_sms': (_I, [_P(_I)]),
    'dg_set_mk_alignment_for_contiguous_layout': (_I, [_I]),
    'dg_get_mk_alignment_for_contiguous_layout': (_I, []),
    'dg_get_theoretical_mk_alignment_for_contiguous_layout': (_I, [_I]),
    'dg_set_tile_override': (_I, [_I, _I, _I]),
    'dg_last_config': (_I, [ctypes.c_char_p, _I]),
}


def _load():
    if not os.path.exists(_LIB_PATH):
        raise ImportError(f'{_LIB_NAME} is not built (expected at {_LIB_PATH}); '
                          f'run `python -c "import __graft_entry__ as g; g.build()"` from the repository root')
    lib = ctypes.CDLL(_LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
LIB_PATH = _LIB_PATH


def check(status: int):
    if status != DG_OK:
        raise RuntimeError(lib.dg_last_error().decode())


def describe(t: torch.Tensor) -> DgTensor:
    """torch.Tensor -> dg_tensor (no copy; the tensor must outlive the call)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f'expected a torch.Tensor, got {type(t).__name__}')
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise RuntimeError(f'Assertion error (_ffi.py): unsupported dtype {t.dtype}')
    if t.dim() > 4:
        raise RuntimeError('Assertion error (_ffi.py): tensors of rank > 4 are not supported')
    d = DgTensor()
    d.data = t.data_ptr() if t.numel() > 0 else (t.data_ptr() or 0)
    d.dtype = code
    d.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.sizes[i] = s
        d.strides[i] = st
    d.device = t.device.index if t.device.type == 'cuda' and t.device.index is not None else \
        (torch.cuda.current_device() if t.device.type == 'cuda' else -1)
    return d


def ref(x):
    return ctypes.byref(x) if x is not None else None


def recipe_struct(recipe=None, recipe_a=None, recipe_b=None):
    """Build dg_recipe; None when no recipe is given (library default)."""
    if recipe is None and recipe_a is None and recipe_b is None:
        return None
    r = DgRecipe()
    if recipe is not None:
        if len(recipe) != 3:
            raise RuntimeError('Assertion error (_ffi.py): recipe must be (gran_m, gran_n, gran_k)')
        r.has_recipe = 1
        for i, v in enumerate(recipe):
            r.recipe[i] = int(v)
    if recipe_a is not None or recipe_b is not None:
        if recipe_a is None or recipe_b is None:
            raise RuntimeError('Assertion error (layout.hpp:76): recipe_a.has_value() == recipe_b.has_value()')
        r.has_recipe_ab = 1
        for i in range(2):
            r.recipe_a[i] = int(recipe_a[i])
            r.recipe_b[i] = int(recipe_b[i])
    return r


def stream_of(t: torch.Tensor):
    if t.device.type != 'cuda':
        return None
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def last_config() -> str:
    buf = ctypes.create_string_buffer(512)
    check(lib.dg_last_config(buf, 512))
    return buf.value.decode()
