"""CPU oracle for the fused projections — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference's unfused torch path
computes for the two fused projections. It is the checker the HIP kernels are
measured against; it is never part of the product path:

- only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
- ``llms_amd`` never imports it, and the product path has no CPU fallback.

Modules:

- :mod:`oracle.ref` — numpy restatement (bf16 inputs held as uint16 bit
  patterns, exact fp64 contractions, the bf16 rounding points of the torch
  path) plus the admissible-rounding parity check.
- :mod:`oracle.torch_path` — the reference's eager torch path itself
  (``F.linear`` + split, ``F.silu(F.linear) * F.linear``), run on the CPU; used
  to pin :mod:`oracle.ref` and as the timed CPU baseline.

Parity status per function (each is pinned by tests/test_oracle.py):

- ``ref_qkv``, ``ref_gate_up_silu``: pinned by the reference's math-contract
  test shapes (exact in fp64), by torch CPU bf16 ``F.linear`` (the literal
  reference call), by exact rational brute force on tiny inputs, by closed
  forms (one-hot inputs), and by committed golden vectors.
- ``quantize_w8_per_row``, ``dequant_w8``, ``ref_*_w8``: the reference has no
  int8 path (reference DESIGN.md:120 names quantisation as future work), so the
  definition comes from the task's stated formula; pinned by closed forms
  (symmetry, the row maximum maps to +-127, all-zero rows), by a torch
  restatement, and by golden vectors.
"""
