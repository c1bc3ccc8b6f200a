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
  and the optional clamp (up to [-c, c], gate to <= c). The FP8 cast of y is the
  reference's per-token quantizer (``oracle/quant.py``) applied to y.
* ``combine``    -- out[t] = sum over slots j in order of w[t, j] * y[pos[t, j]]
  (w = 1 when the weights were applied before L2), accumulated in float32,
  rounded once to bf16.

Pinned by ``tests/test_oracle.py``: dispatch against a per-entry loop over the
definitions above (each routed entry exactly once, segment alignment, stable
order, zero padding), psum ends against ``oracle.gemm.psum_blocks``; SwiGLU
against float64 closed forms; combine against a triple loop.
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


def swiglu_apply_weight(x: np.ndarray, w: np.ndarray = None, clamp: float = None) -> np.ndarray:
    """x [M, 2I] (bf16 values) -> y [M, I] float64 (the exact value before rounding)."""
    x = np.asarray(x, dtype=np.float64)
    i = x.shape[1] // 2
    gate, up = x[:, :i], x[:, i:]
    if clamp is not None:
        up = np.minimum(clamp, np.maximum(-clamp, up))
        gate = np.minimum(clamp, gate)
    y = gate / (1.0 + np.exp(-gate)) * up
    if w is not None:
        y = y * np.asarray(w, dtype=np.float64)[:, None]
    return y


def swiglu_apply_weight_to_fp8(x: np.ndarray, w: np.ndarray = None, clamp: float = None, gran_k: int = 128):
    """The FP8 L2 input: the per-token quantizer applied to y rounded to float32."""
    y = swiglu_apply_weight(x, w, clamp).astype(np.float32)
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
