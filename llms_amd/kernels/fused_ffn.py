"""Fused gate-up-SiLU on MI355X: ``silu(x @ Wg.T) * (x @ Wu.T)`` as one
gfx950 HIP contraction over Wg and Wu with the epilogue in registers.

Drop-in for ``src/kernels/fused_ffn.py`` of the reference: the same public
names (``triton_fused_gate_up_silu``, ``TritonFFN``), signatures and
``ValueError`` messages (the ``triton_`` prefix is kept only for the callers;
there is no Triton here). Path: wrapper -> ``torch.ops.llms_amd.gate_up_silu``
-> C ABI ``fp_gate_up_silu_bf16`` -> HIP kernel on torch's current stream.

Rounding: the epilogue rounds g, u, silu(g) and the product to bf16 at the
same points as the unfused torch path ``F.silu(F.linear(x, Wg)) *
F.linear(x, Wu)``, so the fused result tracks that path to within fp32
summation-order effects.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ._checks import inner_contiguous, require_bf16_hip, require_device


def triton_fused_gate_up_silu(
    x: torch.Tensor, Wg: torch.Tensor, Wu: torch.Tensor
) -> torch.Tensor:
    """``silu(x @ Wg.T) * (x @ Wu.T)`` in one HIP launch.

    Mirrors ``triton_fused_gate_up_silu`` (reference
    ``src/kernels/fused_ffn.py:98-152``).

    Args:
        x: ``(..., K)``, bfloat16, on a HIP device.
        Wg, Wu: ``(N, K)`` bfloat16 (``nn.Linear.weight`` layout).

    Returns:
        ``(..., N)`` bfloat16 on x's device.
    """
    if Wg.shape != Wu.shape:
        raise ValueError(f"Wg shape {tuple(Wg.shape)} != Wu shape {tuple(Wu.shape)}")
    if Wg.dim() != 2:
        raise ValueError(f"Wg must be 2D (N, K), got shape {tuple(Wg.shape)}")
    if x.shape[-1] != Wg.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != Wg.shape[1] {Wg.shape[1]}")
    if x.device != Wg.device or x.device != Wu.device:
        raise ValueError(
            f"x ({x.device}), Wg ({Wg.device}), Wu ({Wu.device}) "
            "must be on the same device"
        )
    require_bf16_hip("triton_fused_gate_up_silu", x=x, Wg=Wg, Wu=Wu)

    N, K = Wg.shape
    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().gate_up_silu(x2, inner_contiguous(Wg), inner_contiguous(Wu))
    return y.reshape(*leading_shape, N)


fused_gate_up_silu = triton_fused_gate_up_silu


def fused_gate_up_silu_w8(
    x: torch.Tensor,
    qg: torch.Tensor,
    sg: torch.Tensor,
    qu: torch.Tensor,
    su: torch.Tensor,
) -> torch.Tensor:
    """int8 weight-only gate-up-SiLU: the bf16 contract on the dequantised
    weights ``bf16(q * s)``, dequantised in registers at every row count (in
    the prefill tiles once per workgroup, into on-chip LDS): no bf16 copy of
    the weights exists. The result is the dequantise-then-matmul result up
    to the fp32 summation order of the plan that runs."""
    if qg.shape != qu.shape:
        raise ValueError(f"qg shape {tuple(qg.shape)} != qu shape {tuple(qu.shape)}")
    if qg.dim() != 2:
        raise ValueError(f"qg must be 2D (N, K), got shape {tuple(qg.shape)}")
    if x.shape[-1] != qg.shape[1]:
        raise ValueError(f"x last dim {x.shape[-1]} != qg.shape[1] {qg.shape[1]}")
    N, K = qg.shape
    for name, s in (("sg", sg), ("su", su)):
        if s.shape != (N,):
            raise ValueError(f"{name} shape {tuple(s.shape)} != ({N},)")
        if s.dtype != torch.float32:
            raise TypeError(f"fused_gate_up_silu_w8: {name} must be float32, got {s.dtype}")
    if qg.dtype != torch.int8 or qu.dtype != torch.int8:
        raise TypeError("fused_gate_up_silu_w8: qg and qu must be int8")
    if not all(t.device == x.device for t in (qg, sg, qu, su)):
        raise ValueError("x, qg, sg, qu, su must be on the same device")
    require_bf16_hip("fused_gate_up_silu_w8", x=x)
    require_device("fused_gate_up_silu_w8", qg, "qg")

    leading_shape = x.shape[:-1]
    x2 = inner_contiguous(x.reshape(-1, K))
    y = _lib.ops().gate_up_silu_w8(x2, inner_contiguous(qg), sg.contiguous(),
                                   inner_contiguous(qu), su.contiguous())
    return y.reshape(*leading_shape, N)


class TritonFFN(nn.Module):
    """Drop-in for the reference's ``TritonFFN`` (``src/kernels/fused_ffn.py:155-185``):
    ``down(fused_gate_up_silu(x, gate.weight, up.weight))``; parameter names
    ``gate``/``up``/``down`` match the eager ``FFN``.

    ``from_eager(..., int8=True)`` keeps per-row int8 gate/up weights
    (``qg``, ``sg``, ``qu``, ``su`` buffers) and runs the int8 kernel.
    ``prenorm`` (set by ``apply_triton_kernels(..., fuse_norm=True)``) is the
    block's pre-FFN RMSNorm, run inside the projection call.
    """

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.gate = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down = nn.Linear(intermediate_size, hidden_size, bias=False)
        self.int8 = False
        self.prenorm = None

    def gate_up(self, x: torch.Tensor) -> torch.Tensor:
        """The fused projection alone: ``silu(x Wg^T) * (x Wu^T)`` (of the
        RMS-normalised x when a ``prenorm`` was fused in)."""
        pn = getattr(self, "prenorm", None)
        if pn is not None:
            from .fused_norm import fused_rmsnorm_gate_up_silu, fused_rmsnorm_gate_up_silu_w8

            if self.int8:
                return fused_rmsnorm_gate_up_silu_w8(x, pn.weight, pn.eps, self.qg, self.sg,
                                                     self.qu, self.su)
            return fused_rmsnorm_gate_up_silu(x, pn.weight, pn.eps, self.gate.weight,
                                              self.up.weight)
        if self.int8:
            return fused_gate_up_silu_w8(x, self.qg, self.sg, self.qu, self.su)
        return triton_fused_gate_up_silu(x, self.gate.weight, self.up.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down(self.gate_up(x))

    @classmethod
    def from_eager(cls, eager: nn.Module, *, int8: bool = False) -> "TritonFFN":
        """Wrap a module with ``gate``/``up``/``down`` Linears, sharing their
        parameters (no copy). int8=True quantises gate and up per output row
        and drops the bf16 gate/up modules."""
        out = cls.__new__(cls)
        nn.Module.__init__(out)
        out.down = eager.down
        out.int8 = bool(int8)
        out.prenorm = None
        if out.int8:
            from .quant import quantize_w8_per_row

            qg, sg = quantize_w8_per_row(eager.gate.weight.detach())
            qu, su = quantize_w8_per_row(eager.up.weight.detach())
            for name, t in (("qg", qg), ("sg", sg), ("qu", qu), ("su", su)):
                out.register_buffer(name, t)
            out.gate = None
            out.up = None
        else:
            out.gate = eager.gate
            out.up = eager.up
        return out
