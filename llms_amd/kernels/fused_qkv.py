"""Fused QKV projection on MI355X: one contraction over the row-stacked
``[Wq; Wk; Wv]`` in a hand-written gfx950 HIP kernel, then a zero-copy split.

Drop-in for ``src/kernels/fused_qkv.py`` of the reference: the same public
names (``triton_fused_qkv``, ``TritonAttention``), signatures, return views and
``ValueError`` messages. The name prefix ``triton_`` is kept only so callers
need no change; there is no Triton here. The computation goes
Python wrapper -> ``torch.ops.llms_amd.qkv`` -> C ABI ``fp_qkv_bf16``
(``include/llms_amd_fp.h``) -> HIP kernel on torch's current stream.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ._checks import inner_contiguous, require_bf16_hip, require_device
from ._eager import RMSNorm, apply_rope, attend, write_kv


def triton_fused_qkv(
    x: torch.Tensor,
    W_qkv: torch.Tensor,
    *,
    n_q: int,
    n_k: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(q, k, v) = split(x @ W_qkv.T, [n_q, n_k, n_k])`` in one HIP launch.

    Mirrors ``triton_fused_qkv`` (reference ``src/kernels/fused_qkv.py:88-149``).

    Args:
        x: ``(..., K)``, bfloat16, on a HIP device.
        W_qkv: ``(n_q + 2*n_k, K)``, bfloat16, the row-stacked Q/K/V weights.
        n_q: rows of W_qkv that belong to Q.
        n_k: rows that belong to K (and to V).

    Returns:
        ``(q, k, v)`` of shapes ``(..., n_q)``, ``(..., n_k)``, ``(..., n_k)``:
        views of one ``(..., n_q + 2*n_k)`` buffer (zero-copy split).

    Raises:
        ValueError: shape or device problems (the reference's messages).
        TypeError: a dtype other than bfloat16.
        RuntimeError: the C ABI reported an error.
    """
    if W_qkv.dim() != 2:
        raise ValueError(
            f"W_qkv must be 2D (n_q+2*n_k, K), got shape {tuple(W_qkv.shape)}"
        )
    n_total, K = W_qkv.shape
    if n_q + 2 * n_k != n_total:
        raise ValueError(
            f"n_q + 2*n_k ({n_q} + 2*{n_k} = {n_q + 2 * n_k}) "
            f"!= W_qkv.shape[0] ({n_total})"
        )
    if x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} != W_qkv.shape[1] {K}")
    if x.device != W_qkv.device:
        raise ValueError(
            f"x ({x.device}) and W_qkv ({W_qkv.device}) must be on the same device"
        )
    require_bf16_hip("triton_fused_qkv", x=x, W_qkv=W_qkv)

    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().qkv(x2, inner_contiguous(W_qkv), n_q, n_k)
    y = y.reshape(*leading_shape, n_total)
    q, k, v = y.split([n_q, n_k, n_k], dim=-1)
    return q, k, v


fused_qkv = triton_fused_qkv


def fused_qkv_w8(
    x: torch.Tensor,
    q_qkv: torch.Tensor,
    s_qkv: torch.Tensor,
    *,
    n_q: int,
    n_k: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """int8 weight-only fused QKV: ``split(x @ bf16(q * s).T)``.

    ``q_qkv`` is the ``(n_q + 2*n_k, K)`` int8 weight and ``s_qkv`` its
    per-row fp32 scale (see :func:`llms_amd.kernels.quant.quantize_w8_per_row`).
    The weights are dequantised in registers at every row count (in the
    prefill tiles once per workgroup, into on-chip LDS): no bf16 copy of the
    weights exists. Every plan computes matmul on ``bf16(q * s)``, up to the
    fp32 summation order of the plan that runs.
    """
    if q_qkv.dim() != 2:
        raise ValueError(
            f"q_qkv must be 2D (n_q+2*n_k, K), got shape {tuple(q_qkv.shape)}"
        )
    n_total, K = q_qkv.shape
    if n_q + 2 * n_k != n_total:
        raise ValueError(
            f"n_q + 2*n_k ({n_q} + 2*{n_k} = {n_q + 2 * n_k}) "
            f"!= q_qkv.shape[0] ({n_total})"
        )
    if x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} != q_qkv.shape[1] {K}")
    if s_qkv.shape != (n_total,):
        raise ValueError(f"s_qkv shape {tuple(s_qkv.shape)} != ({n_total},)")
    if q_qkv.dtype != torch.int8 or s_qkv.dtype != torch.float32:
        raise TypeError("fused_qkv_w8: q_qkv must be int8 and s_qkv float32")
    if not (x.device == q_qkv.device == s_qkv.device):
        raise ValueError(
            f"x ({x.device}), q_qkv ({q_qkv.device}), s_qkv ({s_qkv.device}) "
            "must be on the same device"
        )
    require_bf16_hip("fused_qkv_w8", x=x)
    require_device("fused_qkv_w8", q_qkv, "q_qkv")

    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().qkv_w8(x2, inner_contiguous(q_qkv), s_qkv.contiguous(), n_q, n_k)
    y = y.reshape(*leading_shape, n_total)
    q, k, v = y.split([n_q, n_k, n_k], dim=-1)
    return q, k, v


class TritonAttention(nn.Module):
    """Drop-in for the reference's ``TritonAttention``
    (``src/kernels/fused_qkv.py:152-282``): stores one stacked ``W_qkv``
    instead of ``q``/``k``/``v`` Linears and runs the fused HIP projection;
    QK-norm, RoPE, the KV-cache write, attention and ``o`` stay eager (the
    attention core is :func:`attend`, fp32 softmax attention with the
    reference's causal semantics).

    With ``from_eager(..., int8=True)`` the stacked weight is kept as
    per-row int8 (``q_qkv``, ``s_qkv`` buffers) and the int8 kernel runs.
    ``prenorm`` (set by ``apply_triton_kernels(..., fuse_norm=True)``) is the
    block's pre-attention RMSNorm, run inside the projection call.
    """

    def __init__(
        self,
        *,
        hidden_size: int,
        num_heads: int,
        num_kv_heads: int,
        head_dim: int,
        rms_eps: float,
    ) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.n_q = num_heads * head_dim
        self.n_k = num_kv_heads * head_dim
        n_total = self.n_q + 2 * self.n_k
        self.W_qkv = nn.Parameter(torch.empty(n_total, hidden_size), requires_grad=False)
        self.o = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        self.q_norm = RMSNorm(head_dim, eps=rms_eps)
        self.k_norm = RMSNorm(head_dim, eps=rms_eps)
        self.int8 = False
        self.prenorm = None

    @classmethod
    def from_eager(cls, eager: nn.Module, *, int8: bool = False) -> "TritonAttention":
        """Build from an eager ``Attention`` with loaded weights: row-stack
        ``[Wq; Wk; Wv]`` once, reuse ``o``, ``q_norm`` and ``k_norm`` (no copy).

        int8=True quantises the stacked weight per output row on the device
        and keeps only the int8 weight and its scales.
        """
        out = cls.__new__(cls)
        nn.Module.__init__(out)
        out.hidden_size = eager.q.in_features
        out.num_heads = eager.num_heads
        out.num_kv_heads = eager.num_kv_heads
        out.head_dim = eager.head_dim
        out.n_q = eager.num_heads * eager.head_dim
        out.n_k = eager.num_kv_heads * eager.head_dim
        W_qkv = torch.cat([eager.q.weight, eager.k.weight, eager.v.weight], dim=0)
        out.int8 = bool(int8)
        if out.int8:
            from .quant import quantize_w8_per_row

            q, s = quantize_w8_per_row(W_qkv.detach())
            out.register_buffer("q_qkv", q)
            out.register_buffer("s_qkv", s)
            out.W_qkv = None
        else:
            out.W_qkv = nn.Parameter(W_qkv, requires_grad=False)
        out.o = eager.o
        out.q_norm = eager.q_norm
        out.k_norm = eager.k_norm
        out.prenorm = None
        return out

    def project(self, x: torch.Tensor):
        """The fused projection alone: ``(q, k, v)`` flat views (of the
        RMS-normalised x when a ``prenorm`` was fused in)."""
        pn = getattr(self, "prenorm", None)
        if pn is not None:
            from .fused_norm import fused_rmsnorm_qkv, fused_rmsnorm_qkv_w8

            if self.int8:
                return fused_rmsnorm_qkv_w8(x, pn.weight, pn.eps, self.q_qkv, self.s_qkv,
                                            n_q=self.n_q, n_k=self.n_k)
            return fused_rmsnorm_qkv(x, pn.weight, pn.eps, self.W_qkv, n_q=self.n_q, n_k=self.n_k)
        if self.int8:
            return fused_qkv_w8(x, self.q_qkv, self.s_qkv, n_q=self.n_q, n_k=self.n_k)
        return triton_fused_qkv(x, self.W_qkv, n_q=self.n_q, n_k=self.n_k)

    def forward(
        self,
        x: torch.Tensor,
        *,
        kv_cache,
        layer_idx: int,
        cos: torch.Tensor,
        sin: torch.Tensor,
        start_pos: int,
    ) -> torch.Tensor:
        # The reference forward (src/kernels/fused_qkv.py:242-282) with the
        # fused HIP projection in place of the Triton call and attend() in
        # place of its three SDPA branches. start_pos may be a 0-dim device
        # tensor (a step captured in a HIP graph, replayed at any position).
        B, T, _ = x.shape
        q_flat, k_flat, v_flat = self.project(x)
        q = q_flat.view(B, T, self.num_heads, self.head_dim)
        k = k_flat.view(B, T, self.num_kv_heads, self.head_dim)
        v = v_flat.view(B, T, self.num_kv_heads, self.head_dim)

        q = self.q_norm(q).transpose(1, 2)
        k = self.k_norm(k).transpose(1, 2)
        v = v.transpose(1, 2)
        q, k = apply_rope(q, k, cos, sin)

        full_k, full_v = write_kv(kv_cache.k[layer_idx], kv_cache.v[layer_idx], k, v, start_pos)

        n_rep = self.num_heads // self.num_kv_heads
        if n_rep > 1:
            full_k = full_k.repeat_interleave(n_rep, dim=1)
            full_v = full_v.repeat_interleave(n_rep, dim=1)

        attn = attend(q, full_k, full_v, start_pos)
        attn = attn.transpose(1, 2).reshape(B, T, self.num_heads * self.head_dim)
        return self.o(attn)
