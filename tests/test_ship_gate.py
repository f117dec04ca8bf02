"""The reference's microbench ship gate on the GPU.

Reference: tests/test_kernels_fused_qkv.py:286-311 (fused QKV median <=
eager_3_linears median) and tests/test_kernels_fused_ffn.py:238-265 (fused
gate-up-SiLU median <= eager median), Qwen3-4B shapes, M in {1, 5, 8}, the
median of 200 per-call HIP-event timings after 50 warm-up calls
(src/bench/microbench_fused_*.py). ``bench.py --ship-gate`` prints the same
table as JSON.
"""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_ship_gate():
    import torch

    import bench
    from llms_amd import kernels

    res = bench.ship_gate_run(torch, kernels)
    print(res)
    for op in ("qkv", "gate_up"):
        for m, row in res[op].items():
            assert row["pass"], f"{op} {m}: {row}"
