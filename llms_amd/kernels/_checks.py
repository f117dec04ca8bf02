"""Argument checks shared by the fused-projection wrappers."""

from __future__ import annotations

import torch


def require_bf16_hip(fn: str, **tensors: torch.Tensor) -> None:
    """The HIP kernels take bfloat16 activations/weights on a HIP device.

    Raises ``TypeError`` for another dtype and ``ValueError`` for a tensor that
    is not on a HIP device (there is no CPU or fp32 path).
    """
    for name, t in tensors.items():
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{fn}: {name} must be torch.bfloat16, got {t.dtype}")
        if t.device.type != "cuda":
            raise ValueError(
                f"{fn}: {name} is on {t.device}; the fused projections run only on a "
                "HIP (ROCm) device"
            )


def require_device(fn: str, t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(
            f"{fn}: {name} is on {t.device}; the fused projections run only on a "
            "HIP (ROCm) device"
        )


def inner_contiguous(t: torch.Tensor) -> torch.Tensor:
    """t with unit stride along the last dim (the C ABI takes row strides)."""
    if t.dim() >= 1 and t.shape[-1] > 1 and t.stride(-1) != 1:
        return t.contiguous()
    return t
