"""Per-output-channel symmetric int8 weight packing (the swap-time step of the
int8 weight-only projections).

The reference has no int8 path (reference DESIGN.md:120 lists quantisation as future
work); the format is this build's: for each output row r of an ``[N, K]``
weight, ``s[r] = max_k |W[r, k]| / 127`` in fp32 and
``q[r, k] = clamp(rint(W[r, k] / s[r]), -127, 127)`` as int8 (ties to even;
rows that are all zero get ``s = 0, q = 0``). The kernels compute with the
dequantised weight ``bf16(fp32(q * s))``.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._checks import inner_contiguous, require_bf16_hip


def quantize_w8_per_row(W: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise a bf16 ``[N, K]`` weight on its HIP device.

    Returns ``(q, s)``: int8 ``[N, K]`` (contiguous) and fp32 ``[N]``.
    """
    if W.dim() != 2:
        raise ValueError(f"W must be 2D (N, K), got shape {tuple(W.shape)}")
    require_bf16_hip("quantize_w8_per_row", W=W)
    q, s = _lib.ops().quantize_w8(inner_contiguous(W))
    return q, s


def dequantize_w8(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``bf16(q.float() * s[:, None])``: the weight the int8 kernels compute
    with (a torch expression, for inspection; not used by the kernels)."""
    return (q.float() * s[:, None]).to(torch.bfloat16)
