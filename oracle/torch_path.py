"""The reference's unfused eager path, in torch, on the CPU (test oracle).

These are the exact torch calls the reference engine makes when the fused
kernels are not swapped in, restated as pure functions:

- QKV: ``self.q(x), self.k(x), self.v(x)`` (``src/engine/attention.py:119-121``),
  equivalently one ``F.linear`` on the row-stacked weight then ``split``
  (``src/bench/microbench_fused_qkv.py:101-103``, ``src/kernels/fused_qkv.py:148``).
- gate-up-SiLU: ``F.silu(self.gate(x)) * self.up(x)`` (``src/engine/model.py:37``).
- RMSNorm: ``RMSNorm.forward`` (``src/engine/attention.py:28-33``), applied
  before QKV and gate-up (``src/engine/model.py:57-66``).
- down / o: ``self.down(...)`` (``src/engine/model.py:37``) and ``self.o(attn)``
  (``src/engine/attention.py:183``), bias-free ``F.linear``.
- int8 weight-only: dequantise to bf16, then the calls above (the task's
  definition; the reference has no int8 path).

Used (a) to pin :mod:`oracle.ref` against the library routine the reference
actually calls, and (b) as the timed CPU baseline in ``bench.py``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def torch_qkv(x: torch.Tensor, w_qkv: torch.Tensor, n_q: int, n_k: int):
    """``F.linear(x, W_qkv).split([n_q, n_k, n_k], -1)``."""
    return F.linear(x, w_qkv).split([n_q, n_k, n_k], dim=-1)


def torch_qkv_3(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor):
    """The three separate projections of ``Attention.forward``."""
    return F.linear(x, wq), F.linear(x, wk), F.linear(x, wv)


def torch_gate_up_silu(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor) -> torch.Tensor:
    """``F.silu(F.linear(x, Wg)) * F.linear(x, Wu)``."""
    return F.silu(F.linear(x, wg)) * F.linear(x, wu)


def torch_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    orig_dtype = x.dtype
    x32 = x.float()
    var = x32.pow(2).mean(-1, keepdim=True)
    x32 = x32 * torch.rsqrt(var + eps)
    return weight * x32.to(orig_dtype)


def torch_linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return F.linear(x, w)


def torch_linear_w8(x, q, s):
    return F.linear(x, torch_dequant(q, s))


def torch_quantize_w8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8 (s = amax/127; zero rows -> s = 0, q = 0)."""
    wf = w.float()
    s = wf.abs().amax(dim=1) / 127.0
    safe = torch.where(s > 0, s, torch.ones_like(s))
    q = torch.clamp(torch.round(wf / safe[:, None]), -127, 127)
    q = torch.where(s[:, None] > 0, q, torch.zeros_like(q))
    return q.to(torch.int8), s


def torch_dequant(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``(q.float() * s[:, None]).to(bfloat16)``."""
    return (q.float() * s[:, None]).to(torch.bfloat16)


def torch_qkv_w8(x, q, s, n_q: int, n_k: int):
    return torch_qkv(x, torch_dequant(q, s), n_q, n_k)


def torch_gate_up_silu_w8(x, qg, sg, qu, su):
    return torch_gate_up_silu(x, torch_dequant(qg, sg), torch_dequant(qu, su))
