"""CPU oracle for the GEMM-family hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch-fp32 on the CPU, the oracles that
amd-shasriva/KORE's operator task suite uses to judge a candidate kernel.  It is
the checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.
The product path (``kore_amd``) never imports anything from here and fails loudly
when its HIP library is missing.

Modules
-------
gemm     dense / fused-epilogue / batched GEMM oracles and the activations
quant    OCP e4m3 fp8 codec, 1x128 / 128x128 quantisers, block-scaled GEMM oracle
moe      router (softmax -> top-k -> renorm), fused-MoE oracle, sort/align oracle
compare  the drivers' comparators (SNR, non-finite-aware allclose) and the
         four-prong per-pair verdict (rel-err + SNR + strict non-finite)

The seeded input generators live in ``kore_amd/workloads.py`` (product side: the
bench and the tests draw the same inputs from them).

Parity status of each function (how it is pinned) is listed in its docstring;
every function here is pinned by at least one check in ``tests/test_oracle_*.py``
(closed form, fp64 brute force, an independent second path, or a known-answer
vector restated from the reference's own tests).
"""
