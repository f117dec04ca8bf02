"""In-place swap of engine modules for their fused-HIP counterparts.

Drop-in for ``src/kernels/swap.py`` of the reference (same function names,
keyword arguments and semantics):

    model = Qwen3Model.from_loaded(loaded).to(device).eval()
    apply_triton_kernels(model)       # in place; also returned
    prewarm_triton_kernels(model)     # load code objects before timed regions
"""

from __future__ import annotations

import itertools

import torch
from torch import nn

from .fused_ffn import TritonFFN
from .fused_qkv import TritonAttention
from .linear import FusedLinear


def apply_triton_kernels(
    model: nn.Module,
    *,
    fused_ffn: bool = True,
    fused_qkv: bool = True,
    int8: bool = False,
    linear_down_o: bool = False,
    fuse_norm: bool = False,
) -> nn.Module:
    """Replace ``block.ffn`` / ``block.attn`` of every ``model.layers`` block
    with ``TritonFFN`` / ``TritonAttention`` (reference ``swap.py:22-46``).

    Idempotent: blocks already swapped are left as they are. ``int8=True``
    (not in the reference) builds the int8 weight-only modules instead.
    ``linear_down_o=True`` (not in the reference) also replaces each block's
    ``ffn.down`` and ``attn.o`` Linears with :class:`FusedLinear`, int8 when
    ``int8`` is set. ``fuse_norm=True`` (not in the reference) moves each
    block's ``norm1`` / ``norm2`` RMSNorm into the fused QKV / gate-up module
    (``prenorm``) and leaves ``nn.Identity`` in its place, so the norm runs
    inside the projection call; the block's forward is unchanged.
    """
    for block in model.layers:
        if fused_ffn and not isinstance(block.ffn, TritonFFN):
            block.ffn = TritonFFN.from_eager(block.ffn, int8=int8)
        if fused_qkv and not isinstance(block.attn, TritonAttention):
            block.attn = TritonAttention.from_eager(block.attn, int8=int8)
        if fuse_norm:
            if isinstance(block.attn, TritonAttention) and not isinstance(block.norm1, nn.Identity):
                block.attn.prenorm = block.norm1
                block.norm1 = nn.Identity()
            if isinstance(block.ffn, TritonFFN) and not isinstance(block.norm2, nn.Identity):
                block.ffn.prenorm = block.norm2
                block.norm2 = nn.Identity()
        if linear_down_o:
            if not isinstance(block.ffn.down, FusedLinear):
                block.ffn.down = FusedLinear.from_linear(block.ffn.down, int8=int8)
            if not isinstance(block.attn.o, FusedLinear):
                block.attn.o = FusedLinear.from_linear(block.attn.o, int8=int8)
    return model


def _device(module: nn.Module) -> torch.device:
    """The device of a module's first parameter or buffer (int8 modules keep
    their weights as buffers)."""
    for t in itertools.chain(module.parameters(), module.buffers()):
        return t.device
    raise ValueError(f"{type(module).__name__} holds no tensors")


def prewarm_triton_kernels(
    model: nn.Module,
    *,
    m_values: tuple[int, ...] = (1, 2, 3, 4, 5, 6, 7, 8),
) -> None:
    """Fire every distinct fused projection shape once per M in ``m_values``
    (reference ``swap.py:49-111``).

    There is no autotuner here (tile choice is a static function of M, N, K),
    so this only loads the HIP code objects and touches every kernel variant
    outside any timed region. It does not change later outputs: the kernels
    are deterministic. No-op on a model without fused modules.
    """
    ffn_by_shape: dict[tuple, TritonFFN] = {}
    for m in model.modules():
        if isinstance(m, TritonFFN):
            w = m.qg if m.int8 else m.gate.weight
            ffn_by_shape.setdefault((m.int8, *w.shape), m)
    attn_by_shape: dict[tuple, TritonAttention] = {}
    for m in model.modules():
        if isinstance(m, TritonAttention):
            w = m.q_qkv if m.int8 else m.W_qkv
            attn_by_shape.setdefault((m.int8, *w.shape), m)
    lin_by_shape: dict[tuple, FusedLinear] = {}
    for m in model.modules():
        if isinstance(m, FusedLinear):
            w = m.q if m.int8 else m.weight
            lin_by_shape.setdefault((m.int8, *w.shape), m)
    if not ffn_by_shape and not attn_by_shape and not lin_by_shape:
        return

    with torch.inference_mode():
        for (_, _, K), ffn in ffn_by_shape.items():
            dev = _device(ffn)
            for M in m_values:
                ffn.gate_up(torch.zeros((1, M, K), dtype=torch.bfloat16, device=dev))
        for (_, _, K), attn in attn_by_shape.items():
            dev = _device(attn)
            for M in m_values:
                attn.project(torch.zeros((1, M, K), dtype=torch.bfloat16, device=dev))
        for (_, _, K), lin in lin_by_shape.items():
            dev = _device(lin)
            for M in m_values:
                lin(torch.zeros((1, M, K), dtype=torch.bfloat16, device=dev))

    if torch.cuda.is_available():
        torch.cuda.synchronize()
