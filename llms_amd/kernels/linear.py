"""Plain projection ``x @ W.T`` on the fused-projection kernels: the
``down`` and ``o`` Linears of a Qwen3 block (reference
``src/engine/model.py:37`` and ``src/engine/attention.py:98, :183``), which
stay ``nn.Linear`` (hipBLASLt) in the reference's fused engine.

Path: wrapper -> ``torch.ops.llms_amd.linear`` -> C ABI ``fp_linear_bf16`` ->
the same row-streaming / split-K / LDS-tiled kernels as the QKV projection,
with every output column a plain dot product (no epilogue). The int8 variant
dequantises per-row int8 weights in registers as the fused int8 projections
do (no bf16 copy of the weights), with k split across workgroups where the
plan says so. The result equals matmul on ``bf16(q * s)``.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ._checks import inner_contiguous, require_bf16_hip, require_device


def fused_linear(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """``x @ W.T`` (``F.linear(x, W)`` without bias) in one HIP launch.

    Args:
        x: ``(..., K)``, bfloat16, on a HIP device.
        W: ``(N, K)`` bfloat16 (``nn.Linear.weight`` layout).

    Returns:
        ``(..., N)`` bfloat16 on x's device.
    """
    if W.dim() != 2:
        raise ValueError(f"W must be 2D (N, K), got shape {tuple(W.shape)}")
    if x.shape[-1] != W.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != W.shape[1] {W.shape[1]}")
    if x.device != W.device:
        raise ValueError(f"x ({x.device}) and W ({W.device}) must be on the same device")
    require_bf16_hip("fused_linear", x=x, W=W)

    N, K = W.shape
    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().linear(x2, inner_contiguous(W))
    return y.reshape(*leading_shape, N)


def fused_linear_w8(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """int8 weight-only ``x @ bf16(q * s[:, None]).T``, the weights
    dequantised in registers (see the module docstring)."""
    if q.dim() != 2:
        raise ValueError(f"q must be 2D (N, K), got shape {tuple(q.shape)}")
    if x.shape[-1] != q.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != q.shape[1] {q.shape[1]}")
    N, K = q.shape
    if s.shape != (N,):
        raise ValueError(f"s shape {tuple(s.shape)} != ({N},)")
    if q.dtype != torch.int8 or s.dtype != torch.float32:
        raise TypeError("fused_linear_w8: q must be int8 and s float32")
    if not (x.device == q.device == s.device):
        raise ValueError(
            f"x ({x.device}), q ({q.device}), s ({s.device}) must be on the same device"
        )
    require_bf16_hip("fused_linear_w8", x=x)
    require_device("fused_linear_w8", q, "q")

    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().linear_w8(x2, inner_contiguous(q), s.contiguous())
    return y.reshape(*leading_shape, N)


class FusedLinear(nn.Module):
    """A bias-free ``nn.Linear`` replacement on the HIP projection kernels.

    bf16: keeps the wrapped Linear's ``weight`` Parameter (same state-dict
    key, no copy). int8: keeps ``q`` (int8) and ``s`` (float32 row scales)
    buffers instead.
    """

    def __init__(self, in_features: int, out_features: int) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features), requires_grad=False)
        self.int8 = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.int8:
            return fused_linear_w8(x, self.q, self.s)
        return fused_linear(x, self.weight)

    @classmethod
    def from_linear(cls, lin: nn.Linear, *, int8: bool = False) -> "FusedLinear":
        """Wrap a bias-free ``nn.Linear`` (its weight is shared, not copied);
        ``int8=True`` quantises it per output row on its device instead."""
        if getattr(lin, "bias", None) is not None:
            raise ValueError("FusedLinear wraps bias-free Linears only")
        out = cls.__new__(cls)
        nn.Module.__init__(out)
        out.in_features = lin.in_features
        out.out_features = lin.out_features
        out.int8 = bool(int8)
        if out.int8:
            from .quant import quantize_w8_per_row

            q, s = quantize_w8_per_row(lin.weight.detach())
            out.register_buffer("q", q)
            out.register_buffer("s", s)
            out.weight = None
        else:
            out.weight = lin.weight
        return out

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, int8={self.int8}"
