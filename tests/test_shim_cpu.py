"""Host-side pieces of the deep_gemm shim on CPU tensors: the caller-side
quantizers agree bitwise with the oracle, and the metric helpers with theirs."""
import numpy as np
import torch

import deep_gemm
from deep_gemm.testing import calc_diff, count_bytes
from oracle import gemm as ogemm, quant as oquant


def bf16(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).bfloat16()


def test_per_token_cast_to_fp8_matches_oracle():
    x = bf16((64, 1000), 1)
    for ue8m0 in (False, True):
        q, s = deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=ue8m0)
        oq, os_ = oquant.per_token_cast_to_fp8(x.float().numpy(), use_ue8m0=ue8m0)
        assert np.array_equal(q.view(torch.uint8).numpy(), oq) and np.array_equal(s.numpy(), os_)


def test_per_block_cast_to_fp8_matches_oracle():
    x = bf16((300, 520), 2)
    q, s = deep_gemm.per_block_cast_to_fp8(x, use_ue8m0=False)
    oq, os_ = oquant.per_block_cast_to_fp8(x.float().numpy(), use_ue8m0=False)
    assert np.array_equal(q.view(torch.uint8).numpy(), oq) and np.array_equal(s.numpy(), os_)


def test_per_token_cast_to_fp4_matches_oracle():
    x = bf16((32, 512), 3)
    for gran in (32, 128):
        q, s = deep_gemm.per_token_cast_to_fp4(x, use_ue8m0=True, gran_k=gran)
        oq, os_ = oquant.per_token_cast_to_fp4(x.float().numpy(), use_ue8m0=True, gran_k=gran)
        assert np.array_equal(q.view(torch.uint8).numpy(), oq) and np.array_equal(s.numpy(), os_)
        back = deep_gemm.cast_back_from_fp4(q, s, gran)
        assert np.array_equal(back.numpy(), oquant.dequant_fp4(oq, os_, gran))


def test_packed_ue8m0_roundtrip_and_transpose_fp4():
    x = bf16((16, 256), 4)
    q, s = deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=True, gran_k=32, use_packed_ue8m0=True)
    assert s.dtype == torch.int32 and s.shape == (16, 2)
    _, s_f = deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=True, gran_k=32)
    assert torch.equal(deep_gemm.unpack_ue8m0_from_int(s), s_f)
    p, _ = deep_gemm.per_token_cast_to_fp4(x, use_ue8m0=True, gran_k=32)
    assert torch.equal(deep_gemm.transpose_packed_fp4(deep_gemm.transpose_packed_fp4(p)), p)


def test_cast_back_fp8_matches_oracle_dequant():
    x = bf16((8, 384), 5)
    q, s = deep_gemm.per_token_cast_to_fp8(x, use_ue8m0=False)
    back = deep_gemm.cast_back_from_fp8(q, s)
    assert np.array_equal(back.numpy(), oquant.dequant_per_token(q.view(torch.uint8).numpy(), s.numpy()))


def test_calc_diff_and_count_bytes():
    x = torch.randn(1000, dtype=torch.float64)
    y = torch.randn(1000, dtype=torch.float64)
    assert abs(calc_diff(x, y) - ogemm.calc_diff(x.numpy(), y.numpy())) < 1e-12
    assert count_bytes(torch.empty(10, dtype=torch.bfloat16), (torch.empty(3), None)) == 32


def test_transform_l1_weights_for_swiglu_cpu():
    """The fused SwiGLU weight layout on CPU tensors: rows [256j, +128) are gate rows
    [128j, +128), rows [256j + 128, +128) up rows [128j, +128) (up = rows [I, 2I)),
    and each SF row follows its 128-row block; 2-D weights keep their rank."""
    rng = np.random.default_rng(3)
    for g in (None, 2):
        inter, k = 384, 256
        shape = (2 * inter, k) if g is None else (g, 2 * inter, k)
        w = torch.from_numpy(rng.integers(0, 126, shape).astype(np.uint8)).view(torch.float8_e4m3fn)
        sf = torch.from_numpy(rng.random(shape[:-2] + (2 * inter // 128, k // 128)).astype(np.float32))
        wi, si = deep_gemm.transform_l1_weights_for_swiglu((w, sf))
        assert wi.shape == w.shape and si.shape == sf.shape and wi.dtype == w.dtype
        src, dst = w.view(torch.uint8).numpy(), wi.view(torch.uint8).numpy()
        for j in range(inter // 128):
            assert np.array_equal(dst[..., 256 * j:256 * j + 128, :], src[..., 128 * j:128 * j + 128, :])
            assert np.array_equal(dst[..., 256 * j + 128:256 * j + 256, :],
                                  src[..., inter + 128 * j:inter + 128 * j + 128, :])
            assert np.array_equal(si.numpy()[..., 2 * j, :], sf.numpy()[..., j, :])
            assert np.array_equal(si.numpy()[..., 2 * j + 1, :], sf.numpy()[..., inter // 128 + j, :])
