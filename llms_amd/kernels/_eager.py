"""The eager (non-projection) pieces the attention forward needs.

Plain torch restatements of the Qwen3 attention neighbours of the fused QKV
projection — RMSNorm with fp32 statistics (``src/engine/attention.py:20-33``)
and rotate-half RoPE (``src/engine/attention.py:36-76``). They are not on the
fused path; ``TritonAttention`` applies them after the projection exactly as
the reference's forward does.
"""

from __future__ import annotations

import torch
from torch import nn


class RMSNorm(nn.Module):
    """y = weight * (x / sqrt(mean(x^2) + eps)), statistics in fp32, the
    normalised value cast back to x.dtype before the weight multiply."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + self.eps)
        return self.weight * (xf * inv).to(x.dtype)


def build_rope_tables(head_dim: int, max_pos: int, base: float, *,
                      device: torch.device | str = "cpu",
                      dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [max_pos, head_dim]; the two halves of head_dim share
    frequencies base^(-2i/head_dim) (rotate-half convention)."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    inv_freq = base ** (-exps)
    pos = torch.arange(max_pos, dtype=torch.float32, device=device)
    ang = pos[:, None] * inv_freq[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def rotate_half(t: torch.Tensor) -> torch.Tensor:
    h = t.shape[-1] // 2
    return torch.cat((-t[..., h:], t[..., :h]), dim=-1)


def write_kv(cache_k: torch.Tensor, cache_v: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             start_pos):
    """Store k, v [B, H, T, D] at positions start_pos .. start_pos+T-1 of the
    layer's cache [max_batch, H, max_seq, D] and return the keys/values the
    queries attend over: positions 0 .. start_pos+T-1 for an int start_pos
    (the reference's slicing, ``src/engine/attention.py:132-136``), the whole
    cache for a device-tensor start_pos (masked by ``attend``)."""
    B, T = k.shape[0], k.shape[2]
    if torch.is_tensor(start_pos):
        idx = start_pos + torch.arange(T, device=k.device)
        cache_k[:B].index_copy_(2, idx, k)
        cache_v[:B].index_copy_(2, idx, v)
        return cache_k[:B], cache_v[:B]
    end = start_pos + T
    cache_k[:B, :, start_pos:end, :] = k
    cache_v[:B, :, start_pos:end, :] = v
    return cache_k[:B, :, :end, :], cache_v[:B, :, :end, :]


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """q, k [B, H, T, D]; cos, sin [T, D]."""
    c = cos[None, None]
    s = sin[None, None]
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, start_pos) -> torch.Tensor:
    """Causal softmax attention of queries at positions start_pos .. start_pos+T-1
    over keys/values at positions 0 .. S-1. ``start_pos`` may also be a 0-dim
    device tensor (a step captured in a HIP graph and replayed at any
    position): the mask is then built on the device and always applied, so S
    may be the whole cache.

    q [B, H, T, D]; k, v [B, H, S, D] (GQA heads already expanded). Same
    result as the reference's three ``scaled_dot_product_attention`` branches
    (``src/engine/attention.py:152-160``: no mask for T == 1, ``is_causal`` at
    start_pos 0, an explicit ``q_pos >= k_pos`` mask otherwise), which all
    reduce to "key position <= query position" with scale D^-0.5.

    The core runs in fp32 on contiguous operands and casts back to q.dtype:
    the result then does not depend on which SDPA backend torch would pick,
    and no bf16 batched product sees a transposed operand.

    With a device-tensor ``start_pos`` the cache slots past the last query
    position are never attended, and they may hold anything (a cache
    allocated with ``torch.empty``, as the reference's ``KVCache.alloc`` does):
    their scores are masked to -inf and their values are zeroed before
    ``p @ v``, so NaN or Inf there cannot reach the output (0 * NaN is NaN).
    """
    T, S = q.shape[2], k.shape[2]
    vf = v.float()
    scores = torch.matmul(q.float().contiguous(), k.float().transpose(-2, -1).contiguous())
    scores = scores * (q.shape[-1] ** -0.5)
    if torch.is_tensor(start_pos):
        q_pos = (start_pos + torch.arange(T, device=q.device))[:, None]
        k_pos = torch.arange(S, device=q.device)[None, :]
        scores = scores.masked_fill(k_pos > q_pos, float("-inf"))
        vf = vf.masked_fill((k_pos > q_pos[-1]).reshape(S, 1), 0.0)
    elif T > 1:
        q_pos = torch.arange(start_pos, start_pos + T, device=q.device)[:, None]
        k_pos = torch.arange(S, device=q.device)[None, :]
        scores = scores.masked_fill(k_pos > q_pos, float("-inf"))
    p = torch.softmax(scores, dim=-1)
    return torch.matmul(p, vf.contiguous()).to(q.dtype)
