"""Shared test helpers: bf16 <-> numpy bit views and seeded inputs."""

from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    assert t.dtype == torch.bfloat16
    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    """numpy uint16 bit patterns -> CPU bf16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn_bf16(g: torch.Generator, *shape: int, std: float = 1.0) -> torch.Tensor:
    """N(0, std^2) sampled in fp32 on the CPU, rounded to bf16."""
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def qkv_inputs(seed: int, M: int, K: int, n_q: int, n_k: int, w_std: float = 0.02):
    """x ~ N(0,1) [M,K], W_qkv ~ N(0,w_std) [n_q+2n_k, K] (bf16, CPU)."""
    g = gen(seed)
    x = randn_bf16(g, M, K)
    w = randn_bf16(g, n_q + 2 * n_k, K, std=w_std)
    return x, w


def ffn_inputs(seed: int, M: int, K: int, N: int, w_std: float = 0.02):
    """x ~ N(0,1) [M,K], Wg, Wu ~ N(0,w_std) [N,K] (bf16, CPU)."""
    g = gen(seed)
    x = randn_bf16(g, M, K)
    wg = randn_bf16(g, N, K, std=w_std)
    wu = randn_bf16(g, N, K, std=w_std)
    return x, wg, wu
