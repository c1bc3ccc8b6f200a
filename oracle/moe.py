"""MoE plumbing around the grouped GEMMs, restated in numpy — TEST INFRASTRUCTURE.

See ``oracle/__init__.py``. The reference runs its MoE layer (one GPU's share) as
dispatch -> L1 grouped GEMM -> SwiGLU x routing weight -> FP8 cast -> L2 grouped
GEMM -> combine (``tests/test_mega_moe.py:296-330``, the non-overlapped
baseline). Dispatch and combine there are DeepEP (``deep_ep``, not vendored in
the reference; no version pinned); the grouped layouts they produce are fixed by
the reference's own generators and scheduler:

* ``dispatch``   -- token-major rows -> the expert-grouped layouts the GEMMs read:
  - contiguous: expert e's rows form one segment starting at an ``alignment``
    multiple, rows past its tokens are padding with m_indices = -1 and zero A
    (``tests/generators.py:383-407``, ``README.md:78``);
  - psum: the same rows, described by psum[e] = align(psum[e-1]) + count_e
    (``tests/generators.py:456-461``, ``scheduler/gemm.cuh:205-225``); A padding
    rows are zero (``tests/utils.py:9-18``);
  - masked: expert e's rows are rows [0, count_e) of slab e of [E, max_m, K],
    masked_m[e] = count_e (``tests/generators.py:447-478``; DeepEP's low-latency
    output is this layout, ``README.md:86``); entries past max_m are dropped.
  Inside an expert, entries keep token order, then top-k slot order (a stable
  expansion: each (token, slot) routed to e gets the next row of e's segment).
  ``pos[t, j]`` is the row of (t, j) in the flattened layout (-1 if not routed
  or dropped); routing ids < 0 (DeepEP's "no expert") are not routed.
* ``swiglu_apply_weight`` -- ``third-party/tilelang_ops/swiglu_apply_weight_to_fp8.py:86-94``:
  y = gate / (1 + exp(-gate)) * up * w, with gate = x[:, :I], up = x[:, I:],
  and the optional clamp (up to [-c, c], gate to <= c), in float32 as the
  reference's kernel computes it. Every step is one IEEE single operation
  rounded to nearest, exp included (``exp_f32``: Cody-Waite reduction and a
  degree-7 Taylor polynomial in Horner form), so the device kernels reproduce
  the bits. The FP8 cast of y is the reference's per-token quantizer
  (``oracle/quant.py``) applied to y.
* ``combine``    -- out[t] = sum over slots j in order of w[t, j] * y[pos[t, j]]
  (w = 1 when the weights were applied before L2), accumulated in float32,
  rounded once to bf16.

Pinned by ``tests/test_oracle.py``: dispatch against a per-entry loop over the
definitions above (each routed entry exactly once, segment alignment, stable
order, zero padding), psum ends against ``oracle.gemm.psum_blocks``; exp_f32
within 1.5 ulp of float64 exp over 6 million arguments and at its special
values, SwiGLU within a few ulp of the float64 closed form; combine against a
vectorized sum and against exactly representable sums and a case whose result
depends on the slot order.
"""
import numpy as np

from . import quant


def _align(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def expert_counts(topk_idx: np.ndarray, num_experts: int) -> np.ndarray:
    t = np.asarray(topk_idx).reshape(-1)
    t = t[(t >= 0) & (t < num_experts)]
    return np.bincount(t, minlength=num_experts).astype(np.int64)


def dispatch_rows(topk_idx: np.ndarray, num_experts: int, layout: str, alignment: int = 128,
                  max_m: int = 0):
    """Positions only: -> (pos int64 [T, k], layout metadata, total rows).

    contiguous: (m_indices [M], M = sum of aligned segment sizes);
    psum: (psum ends [E], M); masked: (masked_m [E], E * max_m)."""
    idx = np.asarray(topk_idx).astype(np.int64)
    t_n, k = idx.shape
    counts = expert_counts(idx, num_experts)
    pos = np.full((t_n, k), -1, dtype=np.int64)
    nxt = np.zeros(num_experts, dtype=np.int64)
    if layout == 'masked':
        for t in range(t_n):
            for j in range(k):
                e = idx[t, j]
                if 0 <= e < num_experts:
                    r = nxt[e]
                    nxt[e] += 1
                    if r < max_m:
                        pos[t, j] = e * max_m + r
        return pos, np.minimum(counts, max_m).astype(np.int32), num_experts * max_m
    starts = np.zeros(num_experts, dtype=np.int64)
    acc = 0
    for e in range(num_experts):
        starts[e] = acc
        acc += _align(int(counts[e]), alignment)
    for t in range(t_n):
        for j in range(k):
            e = idx[t, j]
            if 0 <= e < num_experts:
                pos[t, j] = starts[e] + nxt[e]
                nxt[e] += 1
    if layout == 'psum':
        return pos, (starts + counts).astype(np.int32), int(acc)
    m_indices = np.full(acc, -1, dtype=np.int32)
    for e in range(num_experts):
        m_indices[starts[e]:starts[e] + counts[e]] = e
    return pos, m_indices, int(acc)


def dispatch(x_codes: np.ndarray, x_sf: np.ndarray, topk_idx: np.ndarray, num_experts: int, layout: str,
             alignment: int = 128, max_m: int = 0, topk_weights: np.ndarray = None):
    """-> dict(a, sf, layout, pos, weights, rows): a [rows, K] uint8 codes (zero
    padding), sf [rows, K/128] float32 (zero padding), per-row routing weight
    (0 on padding). Masked: a/sf/weights are [E, max_m, ...] with untouched rows
    left at zero here (the GEMM never reads them)."""
    pos, meta, rows = dispatch_rows(topk_idx, num_experts, layout, alignment, max_m)
    t_n, k = pos.shape
    kk = x_codes.shape[1]
    a = np.zeros((rows, kk), dtype=np.uint8)
    sf = np.zeros((rows, x_sf.shape[1]), dtype=np.float32)
    w = np.zeros(rows, dtype=np.float32)
    for t in range(t_n):
        for j in range(k):
            p = pos[t, j]
            if p >= 0:
                a[p] = x_codes[t]
                sf[p] = x_sf[t]
                if topk_weights is not None:
                    w[p] = topk_weights[t, j]
    if layout == 'masked':
        a = a.reshape(num_experts, max_m, kk)
        sf = sf.reshape(num_experts, max_m, -1)
        w = w.reshape(num_experts, max_m)
    return dict(a=a, sf=sf, layout=meta, pos=pos, weights=w, rows=rows)


def _f32(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


# log2(e); ln2 in a 9-bit high part (n * hi is exact for |n| < 2^15) and the rest;
# the Taylor coefficients 1/7!, 1/6!, ..., 1/2, 1, 1 as float32 values
_LOG2E, _LN2_HI, _LN2_LO = _f32(0x3fb8aa3b), _f32(0x3f318000), _f32(0xb95e8083)
_EXP_POLY = (_f32(0x39500d01), _f32(0x3ab60b61), _f32(0x3c088889), _f32(0x3d2aaaab), _f32(0x3e2aaaab),
             np.float32(0.5), np.float32(1.0), np.float32(1.0))


def exp_f32(x: np.ndarray) -> np.ndarray:
    """exp of float32 x in [-87, 88]: n = rint(x log2 e), r = (x - n hi) - n lo,
    exp(r) by the degree-7 Taylor polynomial (Horner, |r| <= 0.35), times 2^n;
    each step one float32 operation rounded to nearest."""
    x = np.asarray(x, dtype=np.float32)
    n = np.rint(x * _LOG2E)
    r = (x - n * _LN2_HI) - n * _LN2_LO
    p = np.full_like(r, _EXP_POLY[0])
    for c in _EXP_POLY[1:]:
        p = p * r + c
    scale = ((n.astype(np.int32) + 127) << 23).astype(np.uint32).view(np.float32)
    return p * scale


def silu_f32(g: np.ndarray) -> np.ndarray:
    """g / (1 + exp(-g)) in float32: 1 + exp(-g) is 1 for g > 87, +inf for
    g < -88, NaN for NaN; one correctly rounded division."""
    g = np.asarray(g, dtype=np.float32)
    x = -g
    inner = np.clip(x, np.float32(-87.0), np.float32(88.0))
    with np.errstate(over='ignore', invalid='ignore'):
        den = np.float32(1.0) + exp_f32(inner)
        den = np.where(x > np.float32(88.0), np.float32(np.inf), den)
        den = np.where(x < np.float32(-87.0), np.float32(1.0), den)
        den = np.where(np.isnan(x), x, den).astype(np.float32)
        return (g / den).astype(np.float32)


def swiglu_apply_weight(x: np.ndarray, w: np.ndarray = None, clamp: float = None) -> np.ndarray:
    """x [M, 2I] (bf16 values) -> y [M, I] float32: silu(gate), times up, times w,
    each product rounded to float32 (w = 1 when absent)."""
    x = np.asarray(x, dtype=np.float32)
    i = x.shape[1] // 2
    gate, up = x[:, :i], x[:, i:]
    if clamp is not None:
        c = np.float32(clamp)
        up = np.fmin(c, np.fmax(-c, up))
        gate = np.fmin(c, gate)
    y = (silu_f32(gate) * up).astype(np.float32)
    wv = np.ones(x.shape[0], np.float32) if w is None else np.asarray(w, dtype=np.float32)
    return (y * wv[:, None]).astype(np.float32)


def swiglu_apply_weight_to_fp8(x: np.ndarray, w: np.ndarray = None, clamp: float = None, gran_k: int = 128):
    """The FP8 L2 input: the per-token quantizer applied to y."""
    y = swiglu_apply_weight(x, w, clamp)
    return quant.per_token_cast_to_fp8(y, use_ue8m0=False, gran_k=gran_k)


def combine(y_rows: np.ndarray, pos: np.ndarray, weights: np.ndarray = None) -> np.ndarray:
    """y_rows [rows, N] (bf16 values, flattened layout) -> out [T, N] bf16 values (float32)."""
    y = np.asarray(y_rows, dtype=np.float32)
    t_n, k = pos.shape
    out = np.zeros((t_n, y.shape[1]), dtype=np.float32)
    for t in range(t_n):
        acc = np.zeros(y.shape[1], dtype=np.float32)
        for j in range(k):
            p = pos[t, j]
            if p >= 0:
                term = y[p] if weights is None else (np.float32(weights[t, j]) * y[p]).astype(np.float32)
                acc = (acc + term).astype(np.float32)
        out[t] = acc
    return quant.bf16_round(out)
