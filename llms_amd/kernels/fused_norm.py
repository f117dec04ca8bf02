"""RMSNorm prologue fused with the QKV and gate-up-SiLU projections.

The reference's decoder block normalises before each projection
(``self.attn(self.norm1(x), ...)``, ``self.ffn(self.norm2(h))``,
``src/engine/model.py:57-66``; RMSNorm ``src/engine/attention.py:28-33``).
Here the norm runs inside the projection call: for decode-sized calls (the
row-streaming regime) in the same launch, with x normalised on its way into
LDS; for larger M as a prologue kernel writing the normalised rows to a torch
workspace, then the usual kernels. Rounding follows the reference: fp32
statistics, ``bf16(x * rsqrt(mean(x^2) + eps))``, then the bf16 product with
the norm weight.

Path: wrapper -> ``torch.ops.llms_amd.rmsnorm_*`` -> C ABI ``fp_rmsnorm_*``.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._checks import inner_contiguous, require_bf16_hip, require_device


def _check_norm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, fn: str) -> None:
    if norm_weight.dim() != 1 or norm_weight.shape[0] != x.shape[-1]:
        raise ValueError(
            f"{fn}: norm weight shape {tuple(norm_weight.shape)} != ({x.shape[-1]},)"
        )
    if not (eps >= 0.0) or eps == float("inf"):
        raise ValueError(f"{fn}: eps must be finite and >= 0, got {eps}")
    require_bf16_hip(fn, x=x, norm_weight=norm_weight)
    if norm_weight.device != x.device:
        raise ValueError(f"{fn}: x ({x.device}) and norm weight ({norm_weight.device}) "
                         "must be on the same device")


def fused_rmsnorm_qkv(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      W_qkv: torch.Tensor, *, n_q: int, n_k: int):
    """``triton_fused_qkv(RMSNorm(x), W_qkv, n_q=n_q, n_k=n_k)`` in one call:
    returns ``(q, k, v)`` views of one output buffer."""
    if W_qkv.dim() != 2:
        raise ValueError(f"W_qkv must be 2D (n_q+2*n_k, K), got shape {tuple(W_qkv.shape)}")
    n_total = W_qkv.shape[0]
    if n_q + 2 * n_k != n_total:
        raise ValueError(
            f"n_q + 2*n_k ({n_q} + 2*{n_k} = {n_q + 2 * n_k}) != W_qkv.shape[0] ({n_total})"
        )
    if x.shape[-1] != W_qkv.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != W_qkv.shape[1] {W_qkv.shape[1]}")
    _check_norm(x, norm_weight, eps, "fused_rmsnorm_qkv")
    require_bf16_hip("fused_rmsnorm_qkv", W_qkv=W_qkv)
    K = W_qkv.shape[1]
    lead = x.shape[:-1]
    y = _lib.ops().rmsnorm_qkv(inner_contiguous(x.reshape(-1, K)), norm_weight.contiguous(),
                               float(eps), inner_contiguous(W_qkv), n_q, n_k)
    return y.reshape(*lead, n_total).split([n_q, n_k, n_k], dim=-1)


def fused_rmsnorm_gate_up_silu(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                               Wg: torch.Tensor, Wu: torch.Tensor) -> torch.Tensor:
    """``triton_fused_gate_up_silu(RMSNorm(x), Wg, Wu)`` in one call."""
    if Wg.shape != Wu.shape:
        raise ValueError(f"Wg shape {tuple(Wg.shape)} != Wu shape {tuple(Wu.shape)}")
    if Wg.dim() != 2:
        raise ValueError(f"Wg must be 2D (N, K), got shape {tuple(Wg.shape)}")
    if x.shape[-1] != Wg.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != Wg.shape[1] {Wg.shape[1]}")
    _check_norm(x, norm_weight, eps, "fused_rmsnorm_gate_up_silu")
    require_bf16_hip("fused_rmsnorm_gate_up_silu", Wg=Wg, Wu=Wu)
    N, K = Wg.shape
    lead = x.shape[:-1]
    y = _lib.ops().rmsnorm_gate_up_silu(inner_contiguous(x.reshape(-1, K)),
                                        norm_weight.contiguous(), float(eps),
                                        inner_contiguous(Wg), inner_contiguous(Wu))
    return y.reshape(*lead, N)


def fused_rmsnorm_qkv_w8(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                         q_qkv: torch.Tensor, s_qkv: torch.Tensor, *, n_q: int, n_k: int):
    """int8 weight-only form of :func:`fused_rmsnorm_qkv`."""
    n_total = q_qkv.shape[0]
    if q_qkv.dim() != 2 or n_q + 2 * n_k != n_total:
        raise ValueError(f"q_qkv shape {tuple(q_qkv.shape)} does not hold n_q={n_q}, n_k={n_k}")
    if x.shape[-1] != q_qkv.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != q_qkv.shape[1] {q_qkv.shape[1]}")
    if q_qkv.dtype != torch.int8 or s_qkv.dtype != torch.float32 or s_qkv.shape != (n_total,):
        raise TypeError("fused_rmsnorm_qkv_w8: q_qkv must be int8 and s_qkv float32 [N]")
    _check_norm(x, norm_weight, eps, "fused_rmsnorm_qkv_w8")
    require_device("fused_rmsnorm_qkv_w8", q_qkv, "q_qkv")
    K = q_qkv.shape[1]
    lead = x.shape[:-1]
    y = _lib.ops().rmsnorm_qkv_w8(inner_contiguous(x.reshape(-1, K)), norm_weight.contiguous(),
                                  float(eps), inner_contiguous(q_qkv), s_qkv.contiguous(),
                                  n_q, n_k)
    return y.reshape(*lead, n_total).split([n_q, n_k, n_k], dim=-1)


def fused_rmsnorm_gate_up_silu_w8(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                                  qg: torch.Tensor, sg: torch.Tensor,
                                  qu: torch.Tensor, su: torch.Tensor) -> torch.Tensor:
    """int8 weight-only form of :func:`fused_rmsnorm_gate_up_silu`."""
    if qg.shape != qu.shape or qg.dim() != 2:
        raise ValueError(f"qg shape {tuple(qg.shape)} != qu shape {tuple(qu.shape)}")
    if x.shape[-1] != qg.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != qg.shape[1] {qg.shape[1]}")
    N, K = qg.shape
    if qg.dtype != torch.int8 or qu.dtype != torch.int8:
        raise TypeError("fused_rmsnorm_gate_up_silu_w8: qg and qu must be int8")
    for name, s in (("sg", sg), ("su", su)):
        if s.shape != (N,) or s.dtype != torch.float32:
            raise TypeError(f"fused_rmsnorm_gate_up_silu_w8: {name} must be float32 [{N}]")
    _check_norm(x, norm_weight, eps, "fused_rmsnorm_gate_up_silu_w8")
    require_device("fused_rmsnorm_gate_up_silu_w8", qg, "qg")
    lead = x.shape[:-1]
    y = _lib.ops().rmsnorm_gate_up_silu_w8(inner_contiguous(x.reshape(-1, K)),
                                           norm_weight.contiguous(), float(eps),
                                           inner_contiguous(qg), sg.contiguous(),
                                           inner_contiguous(qu), su.contiguous())
    return y.reshape(*lead, N)
