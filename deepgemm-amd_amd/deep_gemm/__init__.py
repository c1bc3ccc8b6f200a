"""deep_gemm — MI355X (gfx950) FP8 block-scaled GEMMs with DeepGEMM's Python API.

Drop-in for the FP8/FP4 GEMM entry points of DeepGEMM 2.8.1
(reference: deep_gemm/__init__.py:15-127, signatures csrc/apis/gemm.hpp:835-930,
csrc/apis/layout.hpp:118-141, csrc/apis/config.hpp:8-47). Every GEMM runs
hand-written HIP kernels from libdeepgemm_mi355x.so through its C ABI; there is
no fallback path. Tensors must live on the GPU; D is written in place and the
functions return None. Launches are asynchronous on the current stream.

Scope: fp8_gemm_nt (and its fp8_fp4/fp4 aliases and nn/tn/tt transposing
wrappers), m_grouped_fp8_gemm_nt_contiguous (m_indices and psum layouts),
m_grouped_fp8_gemm_nt_masked, and the SF layout helpers. The reference's
BF16/einsum/attention/Mega-MoE/cuBLASLt kernels are not provided.
"""
from typing import Optional, Tuple

import ctypes

import torch

from . import _ffi
from ._ffi import check as _check, describe as _desc, ref as _ref

__version__ = '2.8.1+mi355x'

_lib = _ffi.lib
_check(_lib.dg_init())


# ------------------------------------------------------------------ config knobs

def init(library_root_path: Optional[str] = None, cuda_home: Optional[str] = None) -> None:
    """Reset the library knobs (reference `_C.init`; kernels are precompiled)."""
    _check(_lib.dg_init())


def shutdown() -> None:
    _check(_lib.dg_shutdown())


def set_num_sms(new_num_sms: int) -> None:
    """Number of compute units the kernels may assume (MI355X: 256)."""
    _check(_lib.dg_set_num_sms(int(new_num_sms)))


def get_num_sms() -> int:
    out = _ffi.ctypes.c_int32()
    _check(_lib.dg_get_num_sms(_ffi.ctypes.byref(out)))
    return out.value


_py_knobs = {'tc_util': 100, 'pdl': False, 'deterministic': True, 'ignore_compile_dims': False,
             'block_size_multiple_of': (1, 1)}


def set_tc_util(new_tc_util: int) -> None:
    """Accepted for compatibility; the gfx950 kernels have no tensor-core throttle."""
    _py_knobs['tc_util'] = int(new_tc_util)


def get_tc_util() -> int:
    return _py_knobs['tc_util']


def set_pdl(new_enable_pdl: bool) -> None:
    """Accepted for compatibility; programmatic dependent launch is an NVIDIA feature."""
    _py_knobs['pdl'] = bool(new_enable_pdl)


def get_pdl() -> bool:
    return _py_knobs['pdl']


def use_deterministic_algorithms(enabled: bool) -> None:
    """Accepted for compatibility; every kernel here is bitwise deterministic."""
    _py_knobs['deterministic'] = bool(enabled)


def set_ignore_compile_dims(new_value: bool) -> None:
    """Accepted for compatibility; kernels are not specialised on M/N/K."""
    _py_knobs['ignore_compile_dims'] = bool(new_value)


def set_block_size_multiple_of(new_value) -> None:
    _py_knobs['block_size_multiple_of'] = new_value if isinstance(new_value, tuple) else (new_value, new_value)


def set_mk_alignment_for_contiguous_layout(new_value: int) -> None:
    _check(_lib.dg_set_mk_alignment_for_contiguous_layout(int(new_value)))


def get_mk_alignment_for_contiguous_layout() -> int:
    return int(_lib.dg_get_mk_alignment_for_contiguous_layout())


def get_theoretical_mk_alignment_for_contiguous_layout(expected_m: Optional[int] = None) -> int:
    return int(_lib.dg_get_theoretical_mk_alignment_for_contiguous_layout(-1 if expected_m is None else int(expected_m)))


# ------------------------------------------------------------------ epilogues

class _EpilogueNamespace:
    """The reference's `deep_gemm.epilogue` classes (csrc/apis/epilogue_class.hpp:13-24;
    semantics csrc/jit_kernels/impls/epilogue_class.hpp:19-124). Identity, Alpha and
    FP8Quantization run on the UE8M0 (power-of-two scale) path, which is where the
    reference has them (its FP32-scale path takes none, csrc/apis/gemm.hpp:118-119).
    BF16StochasticRounding is not provided: its bits are those of NVIDIA's cvt.rs
    rounding."""

    class Epilogue:
        pass

    class Identity(Epilogue):
        def __init__(self):
            pass

    class Alpha(Epilogue):
        """D = C + alpha * (A @ B.T): alpha scales the product, before C is added."""
        def __init__(self, alpha: float):
            self.alpha = float(alpha)

    class FP8Quantization(Epilogue):
        """E4M3 D with per-row, per-32-column UE8M0 scales packed into the int32 words
        of `sfd` (MN-major, [M, ceil(N / 128)]): bitwise a BF16 D followed by
        per_token_cast_to_fp8(d, use_ue8m0=True, gran_k=32), which is how the reference
        defines it (deep_gemm/include/deep_gemm/epilogue/operators.cuh:65-69)."""
        def __init__(self, sfd: torch.Tensor):
            self.sfd = sfd

    class BF16StochasticRounding(Epilogue):
        def __init__(self):
            pass


epilogue = _EpilogueNamespace()


def _resolve_epilogue(ep, alpha=None):
    """(dg_epilogue or None, FP8Quantization or None): the reference's
    resolve_epilogue_class (csrc/jit_kernels/impls/epilogue_class.hpp:111-124)."""
    if (ep is not None) + (alpha is not None) > 1:
        raise RuntimeError('Assertion error (epilogue_class.hpp:116): (epilogue_class != nullptr) + '
                           'alpha.has_value() + sfd.has_value() <= 1 and "The epilogue class, `alpha` and the '
                           'FP8 output pair are exclusive"')
    if alpha is not None:
        ep = _EpilogueNamespace.Alpha(alpha)
    if ep is None:
        return None, None
    if isinstance(ep, _EpilogueNamespace.BF16StochasticRounding):
        raise RuntimeError('Unsupported error: the BF16StochasticRounding epilogue (NVIDIA cvt.rs) is not provided '
                           'on gfx950')
    if isinstance(ep, _EpilogueNamespace.Alpha):
        return _ffi.DgEpilogue(_ffi.EPILOGUE_ALPHA, ep.alpha), None
    if isinstance(ep, _EpilogueNamespace.FP8Quantization):
        return _ffi.DgEpilogue(_ffi.EPILOGUE_FP8_STAGE, 1.0), ep
    if isinstance(ep, _EpilogueNamespace.Identity):
        return _ffi.DgEpilogue(_ffi.EPILOGUE_IDENTITY, 1.0), None
    raise TypeError('epilogue must be one of deep_gemm.epilogue.Identity / Alpha / FP8Quantization')


def _check_epilogue(ep, alpha=None):
    """The FP32-scale K-grouped path takes no epilogue (reference csrc/apis/gemm.hpp:118-119)."""
    if ep is not None or alpha is not None:
        raise RuntimeError('Assertion error (gemm.hpp:118): not alpha.has_value() and epilogue_class == nullptr '
                           'and "alpha and epilogue classes need UE8M0 scales"')


def _fp8_quantized_output(d: torch.Tensor, c, k: int, fp8q, run_bf16) -> None:
    """FP8Quantization: run the GEMM into a BF16 stage, then cast it per 32 columns with
    UE8M0 scales into d and fp8q.sfd (the reference's definition of the fused form)."""
    if c is not None or d.dtype != torch.float8_e4m3fn:
        raise RuntimeError('Assertion error (epilogue_class.hpp:82): not c.has_value() and d.scalar_type() == '
                           'torch::kFloat8_e4m3fn and "FP8 quantization requires a direct E4M3 output"')
    if d.dim() != 2:
        raise RuntimeError('Unsupported error: the FP8Quantization epilogue takes a 2-D D here')
    m, n = d.shape
    sfd = fp8q.sfd
    words = (((n + 31) // 32) + 3) // 4
    if sfd.dtype != torch.int32 or tuple(sfd.shape) != (m, words):
        raise RuntimeError(f'Assertion error: sfd must be int32 [{m}, {words}] (packed UE8M0 words, MN-major)')
    if m == 0 or n == 0:
        return
    if k == 0:   # a zero D dequantizes to zero whatever the SF (reference csrc/apis/gemm.hpp:38-45)
        d.zero_()
        sfd.zero_()
        return
    stage = torch.empty((m, n), dtype=torch.bfloat16, device=d.device)
    run_bf16(stage)
    q, sf = per_token_cast_to_fp8(stage, use_ue8m0=True, gran_k=32)
    d.copy_(q)
    sfd.copy_(get_mn_major_tma_aligned_packed_ue8m0_tensor(sf))


def _pair(x, name):
    if not (isinstance(x, (tuple, list)) and len(x) == 2):
        raise TypeError(f'{name} must be a (tensor, scaling factor) pair')
    return x[0], x[1]


# ------------------------------------------------------------------ GEMMs

def fp8_fp4_gemm_nt(a: Tuple[torch.Tensor, torch.Tensor], b: Tuple[torch.Tensor, torch.Tensor], d: torch.Tensor,
                    c: Optional[torch.Tensor] = None, recipe: Optional[Tuple[int, int, int]] = None,
                    recipe_a: Optional[Tuple[int, int]] = None, recipe_b: Optional[Tuple[int, int]] = None,
                    compiled_dims: str = 'nk', disable_ue8m0_cast: bool = False, alpha: Optional[float] = None,
                    epilogue=None) -> None:
    """D = C + A @ B.T with block scales (reference csrc/apis/gemm.hpp:78-133); `alpha`
    and `epilogue` as the reference's UE8M0 path takes them (see `epilogue`)."""
    ep, fp8q = _resolve_epilogue(epilogue, alpha)
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    da, dsa, db, dsb = _desc(a_t), _desc(sfa), _desc(b_t), _desc(sfb)
    dc = _desc(c) if c is not None else None
    r = _ffi.recipe_struct(recipe, recipe_a, recipe_b)

    def run(out):
        dd = _desc(out)
        # Decode-sized calls (at most 64 rows) split K over workgroups when given a
        # workspace: it comes from torch's caching allocator on the output's stream.
        ws_bytes = 0
        if c is None and a_t.dim() == 2 and a_t.shape[0] <= 64 and out.dtype == torch.bfloat16:
            ws_bytes = int(_lib.dg_fp8_gemm_nt_workspace_size(a_t.shape[0], b_t.shape[0], a_t.shape[1]))
        if ws_bytes > 0:
            ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=out.device)
            _check(_lib.dg_fp8_fp4_gemm_nt_ws(_ref(da), _ref(dsa), _ref(db), _ref(dsb), _ref(dd), _ref(dc), _ref(r),
                                              int(bool(disable_ue8m0_cast)), _ref(ep), _ref(_desc(ws)),
                                              _ffi.stream_of(out)))
        else:
            _check(_lib.dg_fp8_fp4_gemm_nt(_ref(da), _ref(dsa), _ref(db), _ref(dsb), _ref(dd), _ref(dc), _ref(r),
                                           int(bool(disable_ue8m0_cast)), _ref(ep), _ffi.stream_of(out)))
    if fp8q is not None:
        _fp8_quantized_output(d, c, a_t.shape[-1], fp8q, run)
    else:
        run(d)


def fp8_fp4_gemm_nn(a, b, d, c=None, recipe=None, recipe_a=None, recipe_b=None, compiled_dims='nk',
                    disable_ue8m0_cast=False, alpha=None, epilogue=None) -> None:
    """Transposing wrapper (reference csrc/apis/gemm.hpp:135-148)."""
    fp8_fp4_gemm_nt(a, (b[0].transpose(0, 1), b[1].transpose(0, 1)), d, c, recipe, recipe_a, recipe_b,
                    compiled_dims, disable_ue8m0_cast, alpha, epilogue)


def fp8_fp4_gemm_tn(a, b, d, c=None, recipe=None, recipe_a=None, recipe_b=None, compiled_dims='mn',
                    disable_ue8m0_cast=False, alpha=None, epilogue=None) -> None:
    """Transposing wrapper (reference csrc/apis/gemm.hpp:150-164)."""
    fp8_fp4_gemm_nt((a[0].transpose(0, 1), a[1].transpose(0, 1)), (b[0].transpose(0, 1), b[1].transpose(0, 1)),
                    d, c, recipe, recipe_a, recipe_b, compiled_dims, disable_ue8m0_cast, alpha, epilogue)


def fp8_fp4_gemm_tt(a, b, d, c=None, recipe=None, recipe_a=None, recipe_b=None, compiled_dims='mn',
                    disable_ue8m0_cast=False, alpha=None, epilogue=None) -> None:
    """Transposing wrapper (reference csrc/apis/gemm.hpp:166-179)."""
    fp8_fp4_gemm_nt((a[0].transpose(0, 1), a[1].transpose(0, 1)), b, d, c, recipe, recipe_a, recipe_b,
                    compiled_dims, disable_ue8m0_cast, alpha, epilogue)


def m_grouped_fp8_fp4_gemm_nt_contiguous(a, b, d: torch.Tensor, grouped_layout: torch.Tensor,
                                         recipe=None, recipe_a=None, recipe_b=None, compiled_dims: str = 'nk',
                                         disable_ue8m0_cast: bool = False, use_psum_layout: bool = False,
                                         ensure_zero_padding: bool = True,
                                         expected_m_for_psum_layout: Optional[int] = None, epilogue=None) -> None:
    """D[r] = A[r] @ B[e(r)].T over 128-row-aligned expert segments
    (reference csrc/apis/gemm.hpp:181-250). Rows with grouped_layout == -1 are
    left untouched. `epilogue`: Identity or Alpha on the UE8M0 path."""
    ep, fp8q = _resolve_epilogue(epilogue)
    if fp8q is not None:
        raise RuntimeError('Unsupported error: the FP8Quantization epilogue takes the dense GEMM here')
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    da, dsa, db, dsb, dd, dl = _desc(a_t), _desc(sfa), _desc(b_t), _desc(sfb), _desc(d), _desc(grouped_layout)
    r = _ffi.recipe_struct(recipe, recipe_a, recipe_b)
    _check(_lib.dg_m_grouped_fp8_fp4_gemm_nt_contiguous(
        _ref(da), _ref(dsa), _ref(db), _ref(dsb), _ref(dd), _ref(dl), _ref(r), int(bool(disable_ue8m0_cast)),
        int(bool(use_psum_layout)), int(bool(ensure_zero_padding)),
        -1 if expected_m_for_psum_layout is None else int(expected_m_for_psum_layout), _ref(ep),
        _ffi.stream_of(d)))


def m_grouped_fp8_fp4_gemm_nn_contiguous(a, b, d, grouped_layout, recipe=None, recipe_a=None, recipe_b=None,
                                         compiled_dims='nk', disable_ue8m0_cast=False, use_psum_layout=False,
                                         ensure_zero_padding=True, epilogue=None) -> None:
    """Transposing wrapper (reference csrc/apis/gemm.hpp:252-267)."""
    m_grouped_fp8_fp4_gemm_nt_contiguous(a, (b[0].transpose(1, 2), b[1].transpose(1, 2)), d, grouped_layout,
                                         recipe, recipe_a, recipe_b, compiled_dims, disable_ue8m0_cast,
                                         use_psum_layout, ensure_zero_padding, None, epilogue)


def m_grouped_fp8_fp4_gemm_nt_masked(a, b, d: torch.Tensor, masked_m: torch.Tensor, expected_m: int,
                                     recipe=None, recipe_a=None, recipe_b=None, compiled_dims: str = 'nk',
                                     disable_ue8m0_cast: bool = False, epilogue=None) -> None:
    """D[g, r] = A[g, r] @ B[g].T for r < masked_m[g] (reference
    csrc/apis/gemm.hpp:269-318). Rows >= masked_m[g] are left untouched. `epilogue`:
    Identity or Alpha on the UE8M0 path."""
    ep, fp8q = _resolve_epilogue(epilogue)
    if fp8q is not None:
        raise RuntimeError('Unsupported error: the FP8Quantization epilogue takes the dense GEMM here')
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    da, dsa, db, dsb, dd, dm = _desc(a_t), _desc(sfa), _desc(b_t), _desc(sfb), _desc(d), _desc(masked_m)
    r = _ffi.recipe_struct(recipe, recipe_a, recipe_b)
    _check(_lib.dg_m_grouped_fp8_fp4_gemm_nt_masked(
        _ref(da), _ref(dsa), _ref(db), _ref(dsb), _ref(dd), _ref(dm), int(expected_m), _ref(r),
        int(bool(disable_ue8m0_cast)), _ref(ep), _ffi.stream_of(d)))


def _k_grouped(entry, a, b, d, ks_cpu, grouped_layout, c, recipe, use_psum_layout, epilogue):
    _check_epilogue(epilogue)
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    ks = [int(v) for v in (ks_cpu or [])]
    ks_arr = (ctypes.c_int32 * max(1, len(ks)))(*ks) if ks else None
    rec = (ctypes.c_int32 * 3)(*[int(v) for v in recipe]) if recipe is not None else None
    da, dsa, db, dsb, dd, dl = _desc(a_t), _desc(sfa), _desc(b_t), _desc(sfb), _desc(d), _desc(grouped_layout)
    dc = _desc(c) if c is not None else None
    _check(entry(_ref(da), _ref(dsa), _ref(db), _ref(dsb), _ref(dd), ks_arr, len(ks), _ref(dl), _ref(dc), rec,
                 int(bool(use_psum_layout)), _ffi.stream_of(d)))


def k_grouped_fp8_gemm_nt_contiguous(a, b, d: torch.Tensor, ks_cpu, grouped_layout: torch.Tensor,
                                     c: Optional[torch.Tensor] = None, recipe=(1, 1, 128),
                                     compiled_dims: str = 'mn', use_psum_layout: bool = False,
                                     epilogue=None) -> None:
    """D[g] = C[g] + A_g @ B_g.T over K-slices of A and B, FP32 out with per-row
    1x128 scales on both operands (reference csrc/apis/gemm.hpp:369-425)."""
    _k_grouped(_lib.dg_k_grouped_fp8_gemm_nt_contiguous, a, b, d, ks_cpu, grouped_layout, c, recipe,
               use_psum_layout, epilogue)


def k_grouped_fp8_gemm_tn_contiguous(a, b, d: torch.Tensor, ks_cpu, grouped_layout: torch.Tensor,
                                     c: Optional[torch.Tensor] = None, recipe=(1, 1, 128),
                                     compiled_dims: str = 'mn', use_psum_layout: bool = False,
                                     epilogue=None) -> None:
    """MN-major form (reference csrc/apis/gemm.hpp:320-367, SM100 only there): raises
    the reference's unsupported-architecture error, as its SM90 build does."""
    _k_grouped(_lib.dg_k_grouped_fp8_gemm_tn_contiguous, a, b, d, ks_cpu, grouped_layout, c, recipe,
               use_psum_layout, epilogue)


# Aliases (reference csrc/apis/gemm.hpp:920-930)
fp4_gemm_nt = fp8_fp4_gemm_nt
fp8_gemm_nt = fp8_fp4_gemm_nt
fp8_gemm_nn = fp8_fp4_gemm_nn
fp8_gemm_tn = fp8_fp4_gemm_tn
fp8_gemm_tt = fp8_fp4_gemm_tt
m_grouped_fp4_gemm_nt_contiguous = m_grouped_fp8_fp4_gemm_nt_contiguous
m_grouped_fp8_gemm_nt_contiguous = m_grouped_fp8_fp4_gemm_nt_contiguous
m_grouped_fp8_gemm_nn_contiguous = m_grouped_fp8_fp4_gemm_nn_contiguous
m_grouped_fp4_gemm_nt_masked = m_grouped_fp8_fp4_gemm_nt_masked
m_grouped_fp8_gemm_nt_masked = m_grouped_fp8_fp4_gemm_nt_masked


# ------------------------------------------------------------------ SF layouts

def get_tma_aligned_size(x: int, element_size: int) -> int:
    out = _ffi.ctypes.c_int32()
    _check(_lib.dg_get_tma_aligned_size(int(x), int(element_size), _ffi.ctypes.byref(out)))
    return out.value


def get_mn_major_tma_aligned_tensor(sf: torch.Tensor) -> torch.Tensor:
    """FP32 SF -> MN-major copy with row pitch align(mn, 4)
    (reference csrc/jit_kernels/impls/smxx_layout.hpp:60-106)."""
    if sf.dim() not in (2, 3) or sf.dtype != torch.float:
        raise RuntimeError('Assertion error (smxx_layout.hpp:50-51): dim == 2 or dim == 3; sf.scalar_type() == torch::kFloat')
    batched = sf.unsqueeze(0) if sf.dim() == 2 else sf
    g, mn, sfk = batched.shape
    amn = get_tma_aligned_size(mn, 4)
    if (batched.stride(0) == amn * sfk or sf.dim() == 2) and batched.stride(1) == 1 and batched.stride(2) == amn:
        return sf
    out = torch.empty_strided((g, mn, sfk), (amn * sfk, 1, amn), dtype=torch.float, device=sf.device)
    _check(_lib.dg_get_mn_major_tma_aligned_tensor(_ref(_desc(batched)), _ref(_desc(out)), _ffi.stream_of(out)))
    return out.squeeze(0) if sf.dim() == 2 else out


def get_mn_major_tma_aligned_packed_ue8m0_tensor(sf: torch.Tensor, psum_layout: Optional[torch.Tensor] = None):
    """FP32 power-of-two SF -> MN-major int32 words of 4 UE8M0 bytes along K
    (reference csrc/jit_kernels/impls/smxx_layout.hpp:133-216). `psum_layout`
    is accepted for compatibility; gap rows are packed like any other row."""
    if sf.dim() not in (2, 3) or sf.dtype != torch.float:
        raise RuntimeError('Assertion error (smxx_layout.hpp:50-51): dim == 2 or dim == 3; sf.scalar_type() == torch::kFloat')
    batched = sf.unsqueeze(0) if sf.dim() == 2 else sf
    g, mn, sfk = batched.shape
    amn = get_tma_aligned_size(mn, 4)
    pk = (sfk + 3) // 4
    out = torch.empty_strided((g, mn, pk), (amn * pk, 1, amn), dtype=torch.int32, device=sf.device)
    _check(_lib.dg_get_mn_major_tma_aligned_packed_ue8m0_tensor(_ref(_desc(batched)), _ref(_desc(out)),
                                                                _ffi.stream_of(out)))
    return out.squeeze(0) if sf.dim() == 2 else out


def transform_sf_into_required_layout(sf: torch.Tensor, mn: int, k: int, recipe, num_groups: Optional[int] = None,
                                      is_sfa: Optional[bool] = None, disable_ue8m0_cast: bool = False,
                                      psum_layout: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Reference csrc/apis/layout.hpp:11-58 for this device."""
    recipe = tuple(int(v) for v in recipe)
    r3 = r2 = None
    if len(recipe) == 3:
        r3 = (_ffi.ctypes.c_int32 * 3)(*recipe)
    elif len(recipe) == 2:
        r2 = (_ffi.ctypes.c_int32 * 2)(*recipe)
    else:
        raise RuntimeError('Assertion error (layout.hpp:31): Invalid recipe')
    kind = _ffi.ctypes.c_int32()
    _check(_lib.dg_plan_sf_transform(_ref(_desc(sf)), int(mn), int(k), r3, r2,
                                     -1 if num_groups is None else int(num_groups),
                                     -1 if is_sfa is None else int(bool(is_sfa)), int(bool(disable_ue8m0_cast)),
                                     _ffi.ctypes.byref(kind)))
    if kind.value == 0:
        return sf
    if kind.value == 1:
        return get_mn_major_tma_aligned_tensor(sf)
    gran_mn = recipe[0] if len(recipe) == 2 else (recipe[0] if is_sfa else recipe[1])
    if gran_mn != 1:
        rows = torch.arange(mn, device=sf.device) // gran_mn
        sf = sf.index_select(-2, rows)
    return get_mn_major_tma_aligned_packed_ue8m0_tensor(sf, psum_layout)


# ------------------------------------------------------------------ introspection

def set_tile_override(block_m: int = 0, block_n: int = 0, variant: int = 2) -> None:
    """Force the FP32-scale kernel variant and tile ((0, 0) = heuristic; variant 10,
    the split-K kernel, takes block_m 0 and block_n = K chunks, 0 = its own count).
    Testing/tuning aid."""
    if block_m == 0 and block_n == 0 and variant != 10:
        variant = 0
    _check(_lib.dg_set_tile_override(int(variant), int(block_m), int(block_n)))


def get_last_config() -> str:
    """Kernel configuration chosen by the last GEMM call on this thread."""
    return _ffi.last_config()


from . import testing  # noqa: E402
from . import utils  # noqa: E402
from .utils import *  # noqa: E402,F401,F403


# ------------------------------------------------------------------ activation cast

def _cast_on_device(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(-1) == 1 and x.size(1) < (1 << 27)


def per_token_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128,
                          use_packed_ue8m0: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """[m, n] -> (e4m3 [m, n], float32 SF [m, ceil(n / gran_k)] or packed int32 UE8M0 words)
    (reference deep_gemm/utils/math.py:26-49). BF16 device tensors take the fused HIP
    kernel (one HBM pass); anything else takes the torch ops of deep_gemm.utils.math."""
    if not _cast_on_device(x) or gran_k not in (32, 64, 128):
        return utils.math.per_token_cast_to_fp8(x, use_ue8m0, gran_k, use_packed_ue8m0)
    assert not use_packed_ue8m0 or use_ue8m0
    m, n = x.shape
    groups = (n + gran_k - 1) // gran_k
    q = torch.empty((m, n), dtype=torch.float8_e4m3fn, device=x.device)
    if use_packed_ue8m0:
        sf = torch.empty((m, (groups + 3) // 4), dtype=torch.int32, device=x.device)
    else:
        sf = torch.empty((m, groups), dtype=torch.float32, device=x.device)
    _check(_lib.dg_per_token_cast_to_fp8(_ref(_desc(x)), _ref(_desc(q)), _ref(_desc(sf)), int(gran_k),
                                         int(bool(use_ue8m0)), _ffi.stream_of(x)))
    return q, sf


# ------------------------------------------------------------------ MoE plumbing

_MOE_LAYOUTS = {'contiguous': 0, 'psum': 1, 'masked': 2}


def _opt(t):
    return _ref(_desc(t)) if t is not None else None


def moe_dispatch(x: Tuple[torch.Tensor, torch.Tensor], topk_idx: torch.Tensor, num_experts: int,
                 layout: str = 'contiguous', alignment: Optional[int] = None, max_m: Optional[int] = None,
                 topk_weights: Optional[torch.Tensor] = None):
    """Token-major FP8 rows -> the expert-grouped layout a grouped GEMM reads, the
    one-GPU form of DeepEP's expanded / low-latency receive buffers that the
    reference feeds its grouped GEMMs (tests/test_mega_moe.py:296-310, README.md:78,86).

    x = (e4m3 [T, K], f32 SF [T, ceil(K/128)]); topk_idx [T, topk] (negative ids are
    not routed). Returns (a, a_sf, grouped_layout, pos, row_weights):
      contiguous: a [R, K], m_indices [R] (-1 on padding), R = dg_moe_dispatch_max_rows;
      psum:       a [R, K], psum ends [E];
      masked:     a [E, max_m, K], masked_m [E] (entries past max_m dropped);
    pos [T, topk] int32 (row of each (token, slot), masked rows flattened as
    e * max_m + r, -1 if none); row_weights: the routing weight of each row (None
    without topk_weights). Deterministic: an expert's rows follow token order."""
    xq, xs = _pair(x, 'x')
    if layout not in _MOE_LAYOUTS:
        raise ValueError(f'layout must be one of {sorted(_MOE_LAYOUTS)}')
    t, kdim = xq.shape
    k = topk_idx.shape[1]
    dev = xq.device
    alignment = int(alignment or get_mk_alignment_for_contiguous_layout())
    sfk = (kdim + 127) // 128
    if layout == 'masked':
        if not max_m:
            raise ValueError('the masked layout needs max_m')
        a = torch.empty((num_experts, max_m, kdim), dtype=torch.float8_e4m3fn, device=dev)
        a_sf = torch.empty((num_experts, max_m, sfk), dtype=torch.float32, device=dev)
        gl = torch.empty((num_experts,), dtype=torch.int32, device=dev)
        rows = num_experts * max_m
    else:
        rows = int(_lib.dg_moe_dispatch_max_rows(int(t), int(k), int(num_experts), alignment))
        _check(0 if rows >= 0 else 1)
        a = torch.empty((rows, kdim), dtype=torch.float8_e4m3fn, device=dev)
        a_sf = torch.empty((rows, sfk), dtype=torch.float32, device=dev)
        gl = torch.empty((rows if layout == 'contiguous' else num_experts,), dtype=torch.int32, device=dev)
    pos = torch.empty((t, k), dtype=torch.int32, device=dev)
    w = torch.empty((rows,), dtype=torch.float32, device=dev) if topk_weights is not None else None
    ws_bytes = int(_lib.dg_moe_dispatch_workspace_size(int(t), int(num_experts)))
    ws = torch.empty((max(ws_bytes, 4) // 4,), dtype=torch.int32, device=dev)
    _check(_lib.dg_moe_dispatch(_ref(_desc(xq)), _ref(_desc(xs)), _ref(_desc(topk_idx)), _opt(topk_weights),
                                int(num_experts), _MOE_LAYOUTS[layout], alignment, _ref(_desc(a)), _ref(_desc(a_sf)),
                                _ref(_desc(gl)), _ref(_desc(pos)), _opt(w), _ref(_desc(ws)), _ffi.stream_of(xq)))
    if w is not None and layout == 'masked':
        w = w.view(num_experts, max_m)
    return a, a_sf, gl, pos, w


def moe_swiglu_apply_weight_to_fp8(x: torch.Tensor, row_weights: Optional[torch.Tensor] = None,
                                   row_layout: Optional[torch.Tensor] = None, clamp_value: Optional[float] = None,
                                   gran_k: int = 128, out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
                                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 [M, 2I] (gate | up, an L1 grouped GEMM's output) -> (e4m3 [M, I], f32 SF
    [M, I/gran_k]) of y = silu(gate) * up * w: the reference's
    swiglu_apply_weight_to_fp8 (third-party/tilelang_ops/swiglu_apply_weight_to_fp8.py)
    with per_token_cast_to_fp8's scale arithmetic, fused in one HBM pass.
    row_layout (m_indices): rows with a negative entry are written as zeros.
    out: optional preallocated (q, sf)."""
    m, i2 = x.shape
    if out is not None:
        q, sf = _pair(out, 'out')
    else:
        q = torch.empty((m, i2 // 2), dtype=torch.float8_e4m3fn, device=x.device)
        sf = torch.empty((m, i2 // 2 // gran_k), dtype=torch.float32, device=x.device)
    _check(_lib.dg_moe_swiglu_apply_weight_to_fp8(_ref(_desc(x)), _opt(row_weights), _opt(row_layout),
                                                  float(clamp_value or 0.0), _ref(_desc(q)), _ref(_desc(sf)),
                                                  int(gran_k), _ffi.stream_of(x)))
    return q, sf


def moe_combine(y: torch.Tensor, pos: torch.Tensor, topk_weights: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16 expert outputs ([R, N] or masked [E, max_m, N]) -> bf16 [T, N]:
    out[t] = sum over slots of w * y[pos[t, j]] in slot order (w = 1 without
    topk_weights), the one-GPU form of DeepEP's combine."""
    out = torch.empty((pos.shape[0], y.shape[-1]), dtype=torch.bfloat16, device=y.device)
    _check(_lib.dg_moe_combine(_ref(_desc(y)), _ref(_desc(pos)), _opt(topk_weights), _ref(_desc(out)),
                               _ffi.stream_of(y)))
    return out


def transform_l1_weights_for_swiglu(b: Tuple[torch.Tensor, torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """(e4m3 [(G,) 2I, K], f32 SF [(G,) 2I/128, K/128]) with the usual [gate | up]
    rows -> the same weights with gate and up interleaved in blocks of 128 rows
    (rows [256j, +128) = gate rows [128j, +128), rows [256j + 128, +128) = up rows
    [128j, +128)), the L1 weight layout of the fused SwiGLU grouped GEMMs. The
    reference's transform_weights_for_mega_moe interleaves at 8 rows
    (deep_gemm/mega/__init__.py:112-127) for its per-row FP4 scales; 128 x 128 FP32
    block scales keep whole 128-row blocks together. Run once per weight load."""
    w, sf = _pair(b, 'b')
    squeeze = w.dim() == 2
    if squeeze:
        w, sf = w.unsqueeze(0), sf.unsqueeze(0)
    g, n, k = w.shape
    if n % 256 != 0 or sf.shape[-2] * 128 != n:
        raise ValueError('the fused SwiGLU layout needs 2I % 256 == 0 and one SF row per 128 weight rows')
    nb = n // 256   # 128-row blocks per half
    wu = w.view(torch.uint8)
    wi = torch.stack([wu[:, :n // 2].reshape(g, nb, 128, k), wu[:, n // 2:].reshape(g, nb, 128, k)], dim=2)
    si = torch.stack([sf[:, :nb], sf[:, nb:]], dim=2)
    wi = wi.reshape(g, n, k).contiguous().view(w.dtype)
    si = si.reshape(g, 2 * nb, sf.shape[-1]).contiguous()
    return (wi[0], si[0]) if squeeze else (wi, si)


def m_grouped_fp8_gemm_nt_contiguous_swiglu(a, b, out: Tuple[torch.Tensor, torch.Tensor],
                                            grouped_layout: torch.Tensor, row_weights: Optional[torch.Tensor] = None,
                                            activation_clamp: Optional[float] = None, use_psum_layout: bool = False,
                                            ensure_zero_padding: bool = True) -> None:
    """The L1 grouped GEMM of an MoE layer with SwiGLU x routing weight -> FP8 in its
    epilogue: out = (e4m3 q [M, I], f32 sf [M, I/128]) receives
    moe_swiglu_apply_weight_to_fp8(D) of the contiguous grouped GEMM's BF16 D, bit for
    bit, without D going through HBM (the fusion of the reference's Mega-MoE L1
    epilogue, sm100_fp8_fp4_mega_moe.cuh:1066-1130). b: transform_l1_weights_for_swiglu
    output. Rows with grouped_layout == -1 are left untouched."""
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    q, sf = _pair(out, 'out')
    _check(_lib.dg_m_grouped_fp8_gemm_nt_contiguous_swiglu(
        _ref(_desc(a_t)), _ref(_desc(sfa)), _ref(_desc(b_t)), _ref(_desc(sfb)), _ref(_desc(grouped_layout)),
        _opt(row_weights), float(activation_clamp or 0.0), _ref(_desc(q)), _ref(_desc(sf)),
        int(bool(use_psum_layout)), int(bool(ensure_zero_padding)), _ffi.stream_of(q)))


def m_grouped_fp8_gemm_nt_masked_swiglu(a, b, out: Tuple[torch.Tensor, torch.Tensor], masked_m: torch.Tensor,
                                        expected_m: int, row_weights: Optional[torch.Tensor] = None,
                                        activation_clamp: Optional[float] = None) -> None:
    """The masked (decode) form of m_grouped_fp8_gemm_nt_contiguous_swiglu: out =
    (q [G, max_m, I], sf [G, max_m, I/128]); row_weights [G, max_m] or None. Rows
    >= masked_m[g] are left untouched."""
    a_t, sfa = _pair(a, 'a')
    b_t, sfb = _pair(b, 'b')
    q, sf = _pair(out, 'out')
    _check(_lib.dg_m_grouped_fp8_gemm_nt_masked_swiglu(
        _ref(_desc(a_t)), _ref(_desc(sfa)), _ref(_desc(b_t)), _ref(_desc(sfb)), _ref(_desc(masked_m)),
        int(expected_m), _opt(row_weights), float(activation_clamp or 0.0), _ref(_desc(q)), _ref(_desc(sf)),
        _ffi.stream_of(q)))


def per_token_cast_to_fp8_mn_major(x: torch.Tensor, use_ue8m0: bool,
                                   gran_k: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """per_token_cast_to_fp8 with the scales written straight into the MN-major
    TMA-aligned layout (strides (1, align(m, 4))), the fused form of
    per_token_cast_to_fp8 + get_mn_major_tma_aligned_tensor. No reference counterpart."""
    assert _cast_on_device(x), 'needs a 2-D bf16 device tensor with unit stride along K'
    m, n = x.shape
    groups = (n + gran_k - 1) // gran_k
    am = (m + 3) // 4 * 4
    q = torch.empty((m, n), dtype=torch.float8_e4m3fn, device=x.device)
    sf = torch.empty_strided((m, groups), (1, am), dtype=torch.float32, device=x.device)
    _check(_lib.dg_per_token_cast_to_fp8(_ref(_desc(x)), _ref(_desc(q)), _ref(_desc(sf)), int(gran_k),
                                         int(bool(use_ue8m0)), _ffi.stream_of(x)))
    return q, sf
