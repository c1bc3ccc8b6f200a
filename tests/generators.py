"""Seeded inputs for the parity tests (test infrastructure).

Random values come from CPU generators only (torch.Generator for randn, numpy
default_rng for group sizes), so every box sees identical inputs. randn is
rounded to bf16 before quantization, as the reference's generators do
(tests/generators.py:357-358). Quantization uses the CPU oracle
(oracle/quant.py), so the GPU kernels are fed exactly the bytes the oracle
reasons about.
"""
import numpy as np
import torch

from oracle import quant


def randn_bf16(shape, seed: int) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).bfloat16().float().numpy()


def dense_inputs(m: int, n: int, k: int, seed: int = 0):
    """A per-token 1x128 e4m3, B per-block 128x128 e4m3 (configs 1-2 recipe)."""
    a = randn_bf16((m, k), seed)
    b = randn_bf16((n, k), seed + 1)
    qa, sfa = quant.per_token_cast_to_fp8(a, use_ue8m0=False)
    qb, sfb = quant.per_block_cast_to_fp8(b, use_ue8m0=False)
    return dict(a=a, b=b, qa=qa, sfa=sfa, qb=qb, sfb=sfb)


def contiguous_sizes(num_groups: int, total: int, seed: int, alignment: int = 128):
    """Tokens per expert ~ Multinomial(total, Dirichlet(1)), each padded to `alignment` (config 3)."""
    rng = np.random.default_rng(seed)
    w = rng.dirichlet(np.ones(num_groups))
    ms = rng.multinomial(total, w)
    aligned = [(int(x) + alignment - 1) // alignment * alignment for x in ms]
    return [int(x) for x in ms], aligned


def contiguous_inputs(ms, aligned, n: int, k: int, seed: int = 0):
    g = len(ms)
    m_pad = int(sum(aligned))
    a = randn_bf16((m_pad, k), seed)
    b = randn_bf16((g, n, k), seed + 1)
    m_indices = np.full(m_pad, -1, dtype=np.int32)
    start = 0
    for i, (mi, ai) in enumerate(zip(ms, aligned)):
        m_indices[start:start + mi] = i
        a[start + mi:start + ai] = 0.0       # padding rows of A are zero (reference generators.py:402-406)
        start += ai
    qa, sfa = quant.per_token_cast_to_fp8(a, use_ue8m0=False)
    qb = np.empty((g, n, k), dtype=np.uint8)
    sfb = np.empty((g, (n + 127) // 128, (k + 127) // 128), dtype=np.float32)
    for i in range(g):
        qb[i], sfb[i] = quant.per_block_cast_to_fp8(b[i], use_ue8m0=False)
    return dict(qa=qa, sfa=sfa, qb=qb, sfb=sfb, m_indices=m_indices, a=a, b=b)


def masked_inputs(num_groups: int, max_m: int, n: int, k: int, seed: int = 0, lo: int = 96, hi: int = 160):
    """masked_m ~ U{lo..hi} (config 4); SFA rows >= masked_m zeroed (reference generators.py:476-478)."""
    rng = np.random.default_rng(seed)
    masked_m = rng.integers(lo, hi + 1, size=num_groups).astype(np.int32)
    masked_m = np.minimum(masked_m, max_m)
    a = randn_bf16((num_groups, max_m, k), seed)
    b = randn_bf16((num_groups, n, k), seed + 1)
    qa = np.empty((num_groups, max_m, k), dtype=np.uint8)
    sfa = np.empty((num_groups, max_m, (k + 127) // 128), dtype=np.float32)
    qb = np.empty((num_groups, n, k), dtype=np.uint8)
    sfb = np.empty((num_groups, (n + 127) // 128, (k + 127) // 128), dtype=np.float32)
    for i in range(num_groups):
        qa[i], sfa[i] = quant.per_token_cast_to_fp8(a[i], use_ue8m0=False)
        qb[i], sfb[i] = quant.per_block_cast_to_fp8(b[i], use_ue8m0=False)
        sfa[i, masked_m[i]:] = 0.0
    return dict(qa=qa, sfa=sfa, qb=qb, sfb=sfb, masked_m=masked_m, a=a, b=b)


def fp8_fp4_inputs(m: int, n: int, k: int, seed: int = 0, gran_k_a: int = 128, gran_k_b: int = 32,
                   a_fp4: bool = False):
    """Config 5: A e4m3 with 1 x gran_k_a UE8M0 scales, B e2m1 with 1 x gran_k_b UE8M0 scales."""
    a = randn_bf16((m, k), seed)
    b = randn_bf16((n, k), seed + 1)
    if a_fp4:
        qa, sfa = quant.per_token_cast_to_fp4(a, use_ue8m0=True, gran_k=gran_k_a)
    else:
        qa, sfa = quant.per_token_cast_to_fp8(a, use_ue8m0=True, gran_k=gran_k_a)
    qb, sfb = quant.per_token_cast_to_fp4(b, use_ue8m0=True, gran_k=gran_k_b)
    return dict(a=a, b=b, qa=qa, sfa=sfa, qb=qb, sfb=sfb)


def to_dev(x: np.ndarray, dtype=None, device='cuda'):
    """numpy -> torch on `device`; uint8 codes reinterpret as `dtype` (e4m3 / int8)."""
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype is not None and t.dtype != dtype:
        t = t.view(dtype)
    return t.to(device)


def dense_call_same_order(deep_gemm, a, b, d):
    """fp8_gemm_nt on the pipelined 256 x 256 tile (256 x 192 when K % 128 != 0, which
    has no 256 x 256 schedule; every pipelined tile gives the same bits), whose MFMA
    pair and per-K-block promotion order every grouped kernel shares, so a
    contiguous segment or a masked expert must equal it bit for bit. (By default a
    dense call of at most 64 rows takes the tiny-M or split-K kernels, which group
    the K sum differently.)"""
    deep_gemm.set_tile_override(256, 256 if a[0].shape[-1] % 128 == 0 else 192, variant=2)
    try:
        deep_gemm.fp8_gemm_nt(a, b, d)
    finally:
        deep_gemm.set_tile_override(0, 0)
