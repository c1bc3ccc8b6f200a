"""Write the small fixtures under tests/golden/ from the CPU oracle.

Fixtures hold seeded inputs, their quantized bytes and scales, and the oracle's
FP64 output (plus its BF16 bit pattern). They pin the oracle against drift
(tests/test_oracle.py) and give the GPU tests a stored expected output
(tests/test_golden_gpu.py). Run from the repository root:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import gemm as ogemm, quant as oquant  # noqa: E402


def bf16(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).bfloat16().float().numpy()


def dense():
    m, n, k = 40, 136, 640
    a, b = bf16((m, k), 100), bf16((n, k), 101)
    qa, sfa = oquant.per_token_cast_to_fp8(a, use_ue8m0=False)
    qb, sfb = oquant.per_block_cast_to_fp8(b, use_ue8m0=False)
    d = ogemm.gemm_nt(oquant.dequant_per_token(qa, sfa), oquant.dequant_per_block(qb, sfb))
    np.savez_compressed(os.path.join(HERE, 'dense_fp8_small.npz'), a=a, b=b, qa=qa, sfa=sfa, qb=qb, sfb=sfb, d=d,
                        d_bf16_bits=oquant.bf16_bits(d.astype(np.float32)))


def fp8_fp4():
    m, n, k = 32, 64, 256
    a, b = bf16((m, k), 200), bf16((n, k), 201)
    qa, sfa = oquant.per_token_cast_to_fp8(a, use_ue8m0=True, gran_k=128)
    qb, sfb = oquant.per_token_cast_to_fp4(b, use_ue8m0=True, gran_k=32)
    d = ogemm.fp8_fp4_gemm_nt(qa, sfa, qb, sfb, 128, 32)
    np.savez_compressed(os.path.join(HERE, 'fp8_fp4_small.npz'), a=a, b=b, qa=qa, sfa=sfa, qb=qb, sfb=sfb, d=d,
                        d_bf16_bits=oquant.bf16_bits(d.astype(np.float32)))


if __name__ == '__main__':
    dense()
    fp8_fp4()
    print('fixtures written to', HERE)
