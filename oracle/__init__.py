"""CPU oracle for the FP8 block-scaled GEMM path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
(``deep_gemm`` over ``libdeepgemm_mi355x.so``) never imports, links or calls it.

Modules
-------
``fp8``     OCP e4m3fn / e2m1 / UE8M0 codecs written from the format definitions
            (numpy, table based), independent of torch's casts.
``quant``   the caller-side quantizers of ``deep_gemm/utils/math.py`` restated in
            numpy on top of ``fp8``.
``gemm``    FP32-dequantize-then-FP64-matmul references for the dense, m-grouped
            contiguous, m-grouped masked and FP8xFP4 GEMMs, the contiguous-block
            expert rule and masked validity rule of ``scheduler/gemm.cuh``, the SF
            layout transforms, and ``calc_diff``.

Pinning status (what independently checks each function) is listed in the
module docstrings and exercised in ``tests/test_oracle.py``.
"""
