"""GPU parity of the fused per-token FP8 cast (dg_cast.hip) with the oracle's
restatement of the reference quantizer (oracle/quant.py, reference
deep_gemm/utils/math.py:26-49): codes and scales bit-exact."""
import numpy as np
import pytest
import torch

import deep_gemm
from oracle import fp8 as ofp8
from oracle import quant as oquant
import generators as gen

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def special_rows(m, n, seed):
    """randn rows plus rows that hit the edge cases: all zeros (amax clamp), huge
    and tiny magnitudes (subnormal codes), exact e4m3 ties."""
    x = gen.randn_bf16((m, n), seed)
    if m >= 4:
        x[0] = 0.0
        x[1] *= np.float32(3.0e4)
        x[2] *= np.float32(1.0e-3)
        x[3] = np.float32(1.0) + (np.arange(n) % 16).astype(np.float32) * np.float32(1.0 / 16.0)
    return torch.from_numpy(x).bfloat16().float().numpy()


def to_bf16_dev(x):
    return torch.from_numpy(x).bfloat16().to(DEV)


@pytest.mark.parametrize('m,n', [(4096, 7168), (33, 1000), (5, 100), (1, 8), (130, 4096)])
@pytest.mark.parametrize('gran,ue8m0', [(128, False), (128, True), (32, True), (64, False)])
def test_cast_matches_oracle(m, n, gran, ue8m0):
    print(f'cast m={m} n={n} gran={gran} ue8m0={ue8m0}', flush=True)
    x = special_rows(m, n, m + n + gran)
    oq, osf = oquant.per_token_cast_to_fp8(x, use_ue8m0=ue8m0, gran_k=gran)
    q, sf = deep_gemm.per_token_cast_to_fp8(to_bf16_dev(x), use_ue8m0=ue8m0, gran_k=gran)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(sf.cpu().numpy().view(np.int32), osf.view(np.int32))


def test_cast_mn_major_and_packed():
    m, n, gran = 300, 1536, 128
    x = special_rows(m, n, 5)
    xd = to_bf16_dev(x)
    oq, osf = oquant.per_token_cast_to_fp8(x, use_ue8m0=True, gran_k=gran)
    q, sf = deep_gemm.per_token_cast_to_fp8_mn_major(xd, use_ue8m0=True, gran_k=gran)
    torch.cuda.synchronize()
    am = (m + 3) // 4 * 4
    assert sf.shape == (m, n // gran) and sf.stride() == (1, am)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(sf.cpu().numpy().view(np.int32), osf.view(np.int32))
    # packed UE8M0 words (K-major), groups past the last padded with 1.0
    groups = osf.shape[1]
    padded = np.concatenate([osf, np.ones((m, (-groups) % 4), np.float32)], axis=1)
    exps = ofp8.ue8m0_from_pow2_f32(padded).astype(np.uint32).reshape(m, -1, 4)
    words = (exps[..., 0] | (exps[..., 1] << 8) | (exps[..., 2] << 16) | (exps[..., 3] << 24)).view(np.int32)
    q2, pk = deep_gemm.per_token_cast_to_fp8(xd, use_ue8m0=True, gran_k=gran, use_packed_ue8m0=True)
    assert np.array_equal(q2.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(pk.cpu().numpy(), words)
    # the fused cast feeds the GEMM directly: same bits as the separate transform
    b = gen.dense_inputs(64, 256, n, seed=9)
    bq, bsf = (gen.to_dev(b['qb'], torch.float8_e4m3fn), gen.to_dev(b['sfb']))
    d1 = torch.empty((m, 256), dtype=torch.bfloat16, device=DEV)
    d2 = torch.empty_like(d1)
    deep_gemm.fp8_gemm_nt((q, sf), (bq, bsf), d1)
    deep_gemm.fp8_gemm_nt((q, sf.contiguous()), (bq, bsf), d2)
    assert torch.equal(d1.view(torch.int16), d2.view(torch.int16))


def test_cast_strided_input():
    m, n = 64, 512
    x = special_rows(m, n + 64, 11)
    xd = to_bf16_dev(x)[:, :n]            # row stride n + 64
    oq, osf = oquant.per_token_cast_to_fp8(np.ascontiguousarray(x[:, :n]), use_ue8m0=False)
    q, sf = deep_gemm.per_token_cast_to_fp8(xd, use_ue8m0=False)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(sf.cpu().numpy().view(np.int32), osf.view(np.int32))


def test_cast_many_rows_and_empty():
    # more rows than one grid dimension of 65535 workgroups would hold
    m, n = 70001, 256
    x = special_rows(m, n, 13)
    oq, osf = oquant.per_token_cast_to_fp8(x, use_ue8m0=True)
    q, sf = deep_gemm.per_token_cast_to_fp8(to_bf16_dev(x), use_ue8m0=True)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(sf.cpu().numpy().view(np.int32), osf.view(np.int32))
    q0, sf0 = deep_gemm.per_token_cast_to_fp8(torch.empty((0, 512), dtype=torch.bfloat16, device=DEV),
                                              use_ue8m0=False)
    assert q0.shape == (0, 512) and sf0.shape == (0, 4)
