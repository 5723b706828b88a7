"""CPU oracle for the quantized preshuffle GEMM path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference computes on the host and in
its torch correctness oracles for this path:

* ``numerics``  fp8 e4m3fn encode/decode, bf16 round-to-nearest-even, rounding.
* ``quant``     per-row (per-token / per-channel) and block quantizers
                (``tests/utils.py:29-73`` of the reference, with the int8/int4
                rounding rule fixed to round-half-to-even).
* ``layout``    the B preshuffle permutation and the INT4 nibble packing
                (``tests/utils.py:76-96``, ``tests/kernels/test_preshuffle_gemm.py:165-174``).
* ``gemm``      dequantize-then-matmul oracles ``run_torch`` / ``run_torch_blockscale``
                (``tests/kernels/test_preshuffle_gemm.py:55-65``,
                ``tests/kernels/test_blockscale_preshuffle_gemm.py:86-109``),
                the exact int32 accumulator and the fused epilogue
                (``kernels/preshuffle_gemm.py:863-883``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this package, and only as the checker (or, in bench, as the timed CPU
baseline).  The product path (``flydsl_amd``) never imports it.

Pinning status of each function (what checks it other than its own formula) is
listed in each module's docstring; every function here is pinned by at least one
independent check in ``tests/test_oracle.py``.
"""
