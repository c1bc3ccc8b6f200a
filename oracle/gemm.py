"""Reference GEMMs, grouping rules, SF layout transforms and metrics (numpy).

TEST INFRASTRUCTURE: see ``oracle/__init__.py``.

All GEMM references dequantize in float32 exactly as the caller would
(``deep_gemm/utils/math.py:170-176`` ``cast_back_from_fp8``: fp8 value x SF as a
float32 product) and then multiply in float64, so the only rounding left on the
reference side is the final float64 -> output cast done by the test.

Functions and what they follow:

* ``calc_diff``            -- ``deep_gemm/testing/numeric.py:5-11``.
* ``gemm_nt``              -- D = C + A.B^T on dequantized operands
                              (``csrc/apis/gemm.hpp:78-133``; C semantics of
                              ``early_return`` ``:17-53``).
* ``contiguous_expert_of_block`` / ``gemm_contiguous``
                           -- expert of an M-block is ``max(0, layout[block*BM])``
                              (``scheduler/gemm.cuh:150-153``); rows with layout
                              < 0 are padding (``:299-300``) and stay untouched.
* ``psum_blocks`` / ``gemm_psum``
                           -- the psum-layout walk (``scheduler/gemm.cuh:92-94``
                              init, ``:205-225`` get_next_block, ``:306-307``
                              validity): group i owns the M blocks from
                              align(psum[i-1], BLOCK_M) up to psum[i]; rows
                              [psum[i], align(psum[i], alignment)) are padding,
                              zero-filled with ``ensure_zero_padding``
                              (``tests/utils.py:9-18``) and untouched otherwise.
* ``gemm_masked``          -- rows r < masked_m[g] of group g are computed
                              (``scheduler/gemm.cuh:188-204,301-302``); the rest
                              stay untouched.
* ``gemm_k_grouped``       -- ``csrc/apis/gemm.hpp:369-425`` with the data layout of
                              ``tests/generators.py:488-548`` (K-major branch): group
                              g multiplies the K-slice [sum_{j<g} K_j, +K_g) of A
                              and B, each stored [M, K_g] / [N, K_g] row-major one
                              after another; SF columns are the same K-slice in
                              128-blocks; D[g] = C[g] + A_g.B_g^T.
* ``mn_major_tma_aligned`` -- ``csrc/jit_kernels/impls/smxx_layout.hpp:60-106``:
                              values unchanged, strides (align(mn,4)*sf_k, 1, align(mn,4)).
* ``pack_ue8m0_mn_major``  -- ``tests/test_layout.py:20-42``: exponent bytes, four
                              per int32 along K (little end = lowest K), MN-major.

Pinned by ``tests/test_oracle.py``: pure-Python triple loops on tiny shapes,
all-ones / single-K-block closed forms, linearity in C, the grouped rules by
brute-force enumeration, and calc_diff closed forms.
"""
import numpy as np

from . import fp8, quant


def calc_diff(x, y) -> float:
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    den = float((x * x + y * y).sum())
    if den == 0.0:
        return 0.0
    return 1.0 - 2.0 * float((x * y).sum()) / den


def max_rel_err(x, ref, floor: float = 1e-2) -> float:
    """max |x - ref| / max(|ref|, floor * rms(ref)) — scale-aware relative error."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    rms = float(np.sqrt((ref * ref).mean())) or 1.0
    den = np.maximum(np.abs(ref), floor * rms)
    return float((np.abs(x - ref) / den).max())


def gemm_nt(a_deq: np.ndarray, b_deq: np.ndarray, c: np.ndarray = None) -> np.ndarray:
    """float64 D = C + A.B^T for A [M, K], B [N, K] (float32 dequantized)."""
    d = a_deq.astype(np.float64) @ b_deq.astype(np.float64).T
    if c is not None:
        d = d + np.asarray(c, dtype=np.float64)
    return d


def gemm_nt_f32(a_deq: np.ndarray, b_deq: np.ndarray) -> np.ndarray:
    """float32 D = A.B^T: the reference tests' FP32 dequantize-then-matmul, used as the
    timed CPU baseline (the float64 `gemm_nt` is the accuracy oracle)."""
    return np.asarray(a_deq, dtype=np.float32) @ np.asarray(b_deq, dtype=np.float32).T


def contiguous_expert_of_block(m_indices: np.ndarray, block_m: int) -> np.ndarray:
    """Expert id per M-block: max(0, m_indices[block * block_m])."""
    m = m_indices.shape[0]
    starts = np.arange(0, m, block_m)
    return np.maximum(m_indices[starts], 0)


def gemm_contiguous(a_deq: np.ndarray, b_deq: np.ndarray, m_indices: np.ndarray,
                    block_m: int = 128):
    """-> (D float64 [M, N] with NaN in padding rows, valid mask [M])."""
    m = a_deq.shape[0]
    n = b_deq.shape[1]
    d = np.full((m, n), np.nan, dtype=np.float64)
    experts = contiguous_expert_of_block(m_indices, block_m)
    valid = m_indices >= 0
    for blk, e in enumerate(experts):
        r0, r1 = blk * block_m, min(m, (blk + 1) * block_m)
        rows = np.arange(r0, r1)[valid[r0:r1]]
        if rows.size:
            d[rows] = a_deq[rows].astype(np.float64) @ b_deq[e].astype(np.float64).T
    return d, valid


def _align(x: int, y: int) -> int:
    return (x + y - 1) // y * y


def psum_blocks(psum, block_m: int):
    """The psum walk of ``scheduler/gemm.cuh:205-225`` over M blocks (the N blocks
    of a row of tiles repeat it): returns [(group, m_block_idx, row_end)] in walk
    order, where the block computes rows [m_block_idx * block_m, row_end) clipped
    to the block.

    Walk state as in the reference: group 0 starts at row 0 with
    ceil(psum[0] / block_m) blocks (``:92-94``); moving to group i sets
    last = align(psum[i-1], block_m) and gives it ceil((psum[i] - last) / block_m)
    blocks numbered from last / block_m (``:215-224``). The reference keeps these
    counts in uint32, which assumes psum[i] >= align(psum[i-1], block_m) (the
    layout its generator builds, ``tests/generators.py:459``); that is asserted."""
    psum = [int(v) for v in psum]
    out = []
    last, cur = 0, psum[0]
    for g in range(len(psum)):
        if g:
            last, cur = _align(cur, block_m), psum[g]
            assert cur >= last, 'psum layout: each group must start at or after the aligned end of the previous one'
        nmb = (cur - last + block_m - 1) // block_m
        for j in range(nmb):
            out.append((g, last // block_m + j, cur))
    return out


def gemm_psum(a_deq: np.ndarray, b_deq: np.ndarray, psum, block_m: int, alignment: int, zero_padding: bool):
    """Contiguous GEMM in the psum layout -> (D float64 [M, N], NaN where the
    call must leave D untouched; written mask [M]). Computed rows follow
    ``psum_blocks``; rows [psum[i], align(psum[i], alignment)) are 0 with
    ``zero_padding`` (``tests/utils.py:9-18``), untouched without."""
    m = a_deq.shape[0]
    n = b_deq.shape[1]
    d = np.full((m, n), np.nan, dtype=np.float64)
    written = np.zeros(m, dtype=bool)
    for g, mb, row_end in psum_blocks(psum, block_m):
        r0, r1 = mb * block_m, min((mb + 1) * block_m, row_end, m)
        if r1 > r0:
            d[r0:r1] = a_deq[r0:r1].astype(np.float64) @ b_deq[g].astype(np.float64).T
            written[r0:r1] = True
    if zero_padding:
        for end in psum:
            p0, p1 = int(end), min(_align(int(end), alignment), m)
            if p1 > p0:
                d[p0:p1] = 0.0
                written[p0:p1] = True
    return d, written


def gemm_masked(a_deq: np.ndarray, b_deq: np.ndarray, masked_m: np.ndarray):
    """A [G, max_m, K], B [G, N, K] -> (D [G, max_m, N] NaN outside, valid [G, max_m])."""
    g, max_m, _ = a_deq.shape
    n = b_deq.shape[1]
    d = np.full((g, max_m, n), np.nan, dtype=np.float64)
    valid = np.arange(max_m)[None, :] < np.asarray(masked_m)[:, None]
    for i in range(g):
        r = int(masked_m[i])
        if r > 0:
            d[i, :r] = a_deq[i, :r].astype(np.float64) @ b_deq[i].astype(np.float64).T
    return d, valid


def k_grouped_slices(flat: np.ndarray, ks, mn: int):
    """Flat K-grouped operand [sum(ks) * mn] -> list of [mn, K_g] row-major views."""
    out, off = [], 0
    for k in ks:
        out.append(flat[off * mn:(off + k) * mn].reshape(mn, k))
        off += k
    return out


def gemm_k_grouped(a_codes_flat, sfa, b_codes_flat, sfb, ks, c, dequant):
    """K-grouped D = C + A_g.B_g^T, float64. a_codes_flat [sum_k*M] codes, sfa [M,
    sum_k/128]; ``dequant(codes [mn, K_g], sf [mn, K_g/128])`` -> float32."""
    g, m, n = c.shape
    a_g = k_grouped_slices(a_codes_flat, ks, m)
    b_g = k_grouped_slices(b_codes_flat, ks, n)
    out = np.array(c, dtype=np.float64, copy=True)
    kb0 = 0
    for i, k in enumerate(ks):
        if k:
            kb = k // 128
            a_deq = dequant(a_g[i], sfa[:, kb0:kb0 + kb])
            b_deq = dequant(b_g[i], sfb[:, kb0:kb0 + kb])
            out[i] += a_deq.astype(np.float64) @ b_deq.astype(np.float64).T
            kb0 += kb
    return out


def tma_aligned_size(x: int, element_size: int) -> int:
    """``csrc/utils/math.hpp:23-27``: align x to 16 bytes worth of elements."""
    assert 16 % element_size == 0
    n = 16 // element_size
    return (x + n - 1) // n * n


def mn_major_tma_aligned(sf: np.ndarray):
    """Return (storage [G, sf_k, align(mn,4)] float32, view [G, mn, sf_k], strides).

    ``strides`` are in elements, (align(mn,4)*sf_k, 1, align(mn,4)); the view's
    values equal the input's.
    """
    s3 = sf[None] if sf.ndim == 2 else sf
    g, mn, sfk = s3.shape
    amn = tma_aligned_size(mn, 4)
    storage = np.zeros((g, sfk, amn), dtype=np.float32)
    storage[:, :, :mn] = np.swapaxes(s3, 1, 2)
    view = np.swapaxes(storage[:, :, :mn], 1, 2)
    return storage, view, (amn * sfk, 1, amn)


def pack_ue8m0_mn_major(sf: np.ndarray) -> np.ndarray:
    """Power-of-two float32 SF [.., mn, k] -> int32 storage [G, align(k,4)/4, align(mn,4)].

    Element (g, kk, r) packs the exponent bytes of sf[g, r, 4kk .. 4kk+3] with the
    lowest K in the least significant byte; padding bytes are zero.
    """
    s3 = sf[None] if sf.ndim == 2 else sf
    g, mn, k = s3.shape
    amn = tma_aligned_size(mn, 4)
    ak = (k + 3) // 4 * 4
    e = np.zeros((g, amn, ak), dtype=np.uint8)
    e[:, :mn, :k] = fp8.ue8m0_from_pow2_f32(s3)
    packed = e.reshape(g, amn, ak // 4, 4).astype(np.uint32)
    words = packed[..., 0] | (packed[..., 1] << 8) | (packed[..., 2] << 16) | (packed[..., 3] << 24)
    return np.ascontiguousarray(np.swapaxes(words.view(np.int32), 1, 2))


def fp8_fp4_gemm_nt(a_codes, sfa, b_packed, sfb, gran_k_a: int = 128, gran_k_b: int = 32,
                    c=None) -> np.ndarray:
    """A e4m3 [M, K] (1 x gran_k_a SF), B e2m1 packed [N, K/2] (1 x gran_k_b SF)."""
    a_deq = quant.dequant_per_token(a_codes, sfa, gran_k_a)
    b_deq = quant.dequant_fp4(b_packed, sfb, gran_k_b)
    return gemm_nt(a_deq, b_deq, c)
