"""Accuracy metrics (reference deep_gemm/testing/numeric.py:5-44)."""
import torch

__all__ = ['calc_diff', 'count_bytes', 'assert_bitwise_equal']


def calc_diff(x: torch.Tensor, y: torch.Tensor) -> float:
    """1 - 2<x, y> / (|x|^2 + |y|^2) in float64; 0 when both are all zero."""
    x, y = x.double(), y.double()
    den = (x * x + y * y).sum()
    if den == 0:
        return 0.0
    return float(1 - 2 * (x * y).sum() / den)


def count_bytes(*tensors) -> int:
    total = 0
    for t in tensors:
        if isinstance(t, (tuple, list)):
            total += count_bytes(*t)
        elif t is not None:
            total += t.numel() * t.element_size()
    return total


def assert_bitwise_equal(x: torch.Tensor, y: torch.Tensor, label: str = '') -> None:
    assert x.shape == y.shape and x.dtype == y.dtype
    xb = x.contiguous().view(torch.uint8).flatten()
    yb = y.contiguous().view(torch.uint8).flatten()
    if torch.equal(xb, yb):
        return
    diff = (xb != yb).nonzero()
    first = int(diff[0])
    elem = first // x.element_size()
    coord = tuple(int(v) for v in torch.unravel_index(torch.tensor(elem), x.shape))
    raise AssertionError(f'bitwise mismatch{f" ({label})" if label else ""}: num_bytes={xb.numel()}, '
                         f'num_mismatch={diff.numel()}, first_byte={first}, elem={elem}, coord={coord}, '
                         f'x_val={x.flatten()[elem].item()}, y_val={y.flatten()[elem].item()}')
