"""CPU oracle for the AKV warm-tier hot path (test infrastructure only).

This package restates, on the host in numpy, the arithmetic of the reference
implementation (Arvind679715/adaptive-kv-memory) for the three pieces of the
warm-tier hot path: bit-packing, block-affine quantization, and the
dequant-attention plus importance update.  Every function cites the
reference file:line it follows.

It is the CHECKER, never the product: only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` import it.  The product path
(``akv`` under ``adaptive-kv-memory_amd/``) never calls into this package and
fails loudly when its HIP library is missing.

Pinning status (what checks each function against something other than a
retyped formula) is listed in each module's header; tests live in
``tests/test_oracle_*.py``.
"""
