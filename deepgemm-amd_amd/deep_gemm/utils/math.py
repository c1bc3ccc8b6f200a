"""Quantizers of the GEMM's input contract, as torch ops on any device.

Same names, arguments and results as the reference's caller-side helpers
(deep_gemm/utils/math.py:5-176): per-group amax clamped at 1e-4, scale =
amax / 448 (FP8) or amax / 6 (FP4), optionally rounded up to a power of two
(UE8M0), values multiplied by the float32 reciprocal of the scale and cast
with round-to-nearest-even. The division by 448 / 6 is a multiplication by the
float32 reciprocal, as torch evaluates it on the GPU, on every device. They run wherever their input lives (on the GPU
for real workloads); they are not part of the GEMM kernels.
"""
from typing import Tuple

import torch

__all__ = ['ceil_div', 'align', 'ceil_to_ue8m0', 'pack_ue8m0_to_int', 'unpack_ue8m0_from_int',
           'per_token_cast_to_fp8', 'per_channel_cast_to_fp8', 'per_block_cast_to_fp8',
           'per_custom_dims_cast_to_fp8', 'per_token_cast_to_fp4', 'transpose_packed_fp4',
           'cast_back_from_fp8', 'cast_back_from_fp4']

_FP8_MAX = 448.0
_FP4_MAX = 6.0


def ceil_div(x: int, y: int) -> int:
    return (x + y - 1) // y


def align(x: int, y: int) -> int:
    return ceil_div(x, y) * y


def ceil_to_ue8m0(x: torch.Tensor) -> torch.Tensor:
    """Smallest power of two >= |x| (exponent clamped to [1, 254])."""
    bits = x.abs().float().view(torch.int32)
    exponent = (bits >> 23) & 0xFF
    exponent = exponent + ((bits & 0x7FFFFF) != 0).to(torch.int32)
    return (exponent.clamp(1, 254) << 23).view(torch.float32)


def pack_ue8m0_to_int(x: torch.Tensor) -> torch.Tensor:
    """Power-of-two float32 [..., 4j] -> int32 [..., j] of exponent bytes."""
    assert x.dtype == torch.float32 and x.size(-1) % 4 == 0
    bits = x.view(torch.int32)
    assert bool((bits >= 0).all()) and bool(((bits & 0x7FFFFF) == 0).all())
    return (bits >> 23).to(torch.uint8).view(torch.int32)


def unpack_ue8m0_from_int(packed: torch.Tensor) -> torch.Tensor:
    return (packed.view(torch.uint8).to(torch.int32) << 23).view(torch.float32)


def _group_scale(amax: torch.Tensor, max_code: float, use_ue8m0: bool) -> torch.Tensor:
    # amax times the float32 reciprocal of the largest code: what `amax / max_code`
    # evaluates to on the GPU, written so CPU tensors get the same bits.
    sf = amax * (1.0 / max_code)
    return ceil_to_ue8m0(sf) if use_ue8m0 else sf


def per_token_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128,
                          use_packed_ue8m0: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """[m, n] -> (e4m3 [m, n], float32 SF [m, ceil(n / gran_k)]); 1 x gran_k groups."""
    assert x.dim() == 2
    assert not use_packed_ue8m0 or use_ue8m0
    m, n = x.shape
    pn = align(n, gran_k)
    xp = torch.zeros((m, pn), dtype=x.dtype, device=x.device)
    xp[:, :n] = x
    groups = xp.view(m, pn // gran_k, gran_k)
    amax = groups.abs().float().amax(dim=2).clamp(1e-4)
    sf = _group_scale(amax, _FP8_MAX, use_ue8m0)
    q = (groups * (1.0 / sf.unsqueeze(2))).to(torch.float8_e4m3fn).view(m, pn)[:, :n].contiguous()
    if use_packed_ue8m0:
        if sf.size(-1) % 4:
            sf = torch.nn.functional.pad(sf, (0, align(sf.size(-1), 4) - sf.size(-1)), value=1.0)
        return q, pack_ue8m0_to_int(sf)
    return q, sf


def per_channel_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """[m, n] -> gran_k x 1 groups along m."""
    assert x.dim() == 2 and x.size(0) % gran_k == 0
    m, n = x.shape
    groups = x.view(-1, gran_k, n)
    amax = groups.abs().float().amax(dim=1).view(-1, n).clamp(1e-4)
    sf = _group_scale(amax, _FP8_MAX, use_ue8m0)
    return (groups * (1.0 / sf.unsqueeze(1))).to(torch.float8_e4m3fn).view(m, n), sf


def per_block_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """[m, n] -> (e4m3 [m, n], float32 SF [ceil(m/g), ceil(n/g)]); g x g blocks."""
    assert x.dim() == 2
    m, n = x.shape
    xp = torch.zeros((align(m, gran_k), align(n, gran_k)), dtype=x.dtype, device=x.device)
    xp[:m, :n] = x
    blocks = xp.view(-1, gran_k, xp.size(1) // gran_k, gran_k)
    amax = blocks.abs().float().amax(dim=(1, 3), keepdim=True).clamp(1e-4)
    sf = _group_scale(amax, _FP8_MAX, use_ue8m0)
    q = (blocks * (1.0 / sf)).to(torch.float8_e4m3fn)
    return q.view_as(xp)[:m, :n].contiguous(), sf.view(blocks.size(0), blocks.size(2))


def per_custom_dims_cast_to_fp8(x: torch.Tensor, dims: Tuple, use_ue8m0: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    reduce_dims = tuple(i for i in range(x.dim()) if i not in set(dims))
    amax = x.abs().float().amax(dim=reduce_dims, keepdim=True).clamp(1e-4)
    sf = _group_scale(amax, _FP8_MAX, use_ue8m0)
    return (x * (1.0 / sf)).to(torch.float8_e4m3fn), sf.squeeze()


# E2M1 rounding: magnitudes strictly above a "down" boundary, or at/above an
# "up" boundary, move to the next code (ties go to the even code).
_E2M1_DOWN = (0.25, 1.25, 2.5, 5.0)
_E2M1_UP = (0.75, 1.75, 3.5)


def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    ax = x.abs().float()
    down = torch.tensor(_E2M1_DOWN, dtype=torch.float32, device=x.device)
    up = torch.tensor(_E2M1_UP, dtype=torch.float32, device=x.device)
    code = torch.bucketize(ax, down, right=False) + torch.bucketize(ax, up, right=True)
    code = code.to(torch.uint8)
    neg = (x < 0) & (code != 0)
    return (code | (neg.to(torch.uint8) << 3)).view(torch.int8)


def per_token_cast_to_fp4(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128,
                          use_packed_ue8m0: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """[m, n] -> (packed e2m1 int8 [m, n/2], SF [m, ceil(n/gran_k)]); element 2i in the low nibble."""
    m, n = x.shape
    assert n % 2 == 0
    assert not use_packed_ue8m0 or use_ue8m0
    pn = align(n, gran_k)
    xp = torch.zeros((m, pn), dtype=x.dtype, device=x.device)
    xp[:, :n] = x
    groups = xp.view(m, -1, gran_k)
    amax = groups.abs().float().amax(dim=2).clamp_min(1e-4)
    sf = _group_scale(amax, _FP4_MAX, use_ue8m0)
    codes = _e2m1_codes(groups * (1.0 / sf.unsqueeze(2))).view(m, pn // 2, 2)
    packed = (codes[:, :, 0] & 0x0F) | ((codes[:, :, 1] & 0x0F) << 4)
    packed = packed[:, :n // 2].contiguous()
    if use_packed_ue8m0:
        if sf.size(-1) % 4:
            sf = torch.nn.functional.pad(sf, (0, align(sf.size(-1), 4) - sf.size(-1)), value=1.0)
        return packed, pack_ue8m0_to_int(sf)
    return packed, sf


def transpose_packed_fp4(a: torch.Tensor) -> torch.Tensor:
    """Packed e2m1 [m, n/2] -> packed e2m1 of the transpose, [n, m/2]."""
    assert a.dtype == torch.int8 and a.dim() == 2
    m, half_n = a.shape
    assert m % 2 == 0
    codes = torch.stack(((a & 0x0F), (a >> 4) & 0x0F), dim=-1).view(m, half_n * 2)
    t = codes.t().contiguous().view(half_n * 2, m // 2, 2)
    return ((t[:, :, 0] & 0x0F) | ((t[:, :, 1] & 0x0F) << 4)).contiguous()


_E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def cast_back_from_fp4(packed: torch.Tensor, sf: torch.Tensor, gran_k: int = 128,
                       use_packed_ue8m0: bool = False) -> torch.Tensor:
    m, half_n = packed.shape
    n = half_n * 2
    if use_packed_ue8m0:
        sf = unpack_ue8m0_from_int(sf)
    codes = torch.stack(((packed & 0x0F), (packed >> 4) & 0x0F), dim=-1).view(m, n).to(torch.int64)
    table = torch.tensor(_E2M1_VALUES, dtype=torch.float32, device=packed.device)
    mag = table[codes & 0x7]
    vals = torch.where((codes & 0x8) != 0, -mag, mag)
    return vals * sf[:, torch.arange(n, device=packed.device) // gran_k]


def cast_back_from_fp8(x_fp8: torch.Tensor, sf: torch.Tensor, gran_k: int = 128,
                       use_packed_ue8m0: bool = False) -> torch.Tensor:
    m, n = x_fp8.shape
    if use_packed_ue8m0:
        sf = unpack_ue8m0_from_int(sf)
    return x_fp8.float() * sf[:, torch.arange(n, device=x_fp8.device) // gran_k]
