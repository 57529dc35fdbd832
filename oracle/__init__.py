"""CPU oracle for the batch-1 INT8/BF16 decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path
the library accelerates, so that the HIP kernels can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker or as the timed CPU baseline; the
library itself never calls into it.

Modules and the reference code each one follows:

* ``quant``   — ``quantize_per_channel`` (bench_int8.py:19-24).
* ``rope``    — the theta=1e6 split-half table (verify_correctness_a10.py:23-33)
                and the legacy pair-duplicated table (bench_int8.py:270-279).
* ``ref_cpu`` — one decode step (a10_int8_decode_kernel.cu:21-815 and the
                bf16 twin a10_decode_kernel.cu:21-755), with the kernel's
                rounding points: bf16 hidden state between layers, bf16 K/V
                cache (the current token's K/V read back from it), fp32 for
                every stored intermediate.
* ``c/oracle.c`` — an independent C restatement of the quantizer, bf16
                rounding and the fp64 dequantized matvec, used to pin the
                Python restatement (built by ``oracle/Makefile``).

How each function is pinned (checked against something other than itself) is
listed in tests/test_oracle_pins.py; nothing here is "parity unpinned".
"""
