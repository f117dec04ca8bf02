"""The RMSNorm prologue fused into QKV and gate-up-SiLU (one launch in the
row-streaming regime, a prologue kernel plus the usual kernels above it)
against the oracle: reference RMSNorm (``src/engine/attention.py:28-33``)
followed by the reference's unfused projection, with the projection hull
widened by the norm's admissible rounding spread."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import ref
from tests._util import bits, ffn_inputs, gen, qkv_inputs, randn_bf16

DEV = "cuda"
EPS = 1e-6


def _norm_weight(seed: int, K: int) -> torch.Tensor:
    return (1.0 + 0.3 * torch.randn(K, generator=gen(seed))).to(torch.bfloat16)


def _x(seed: int, M: int, K: int, std: float = 3.0) -> torch.Tensor:
    return randn_bf16(gen(seed), M, K, std=std)


def _rows(M: int, limit: int = 96) -> np.ndarray:
    if M <= limit:
        return np.arange(M)
    return np.unique(np.concatenate([np.linspace(0, M - 1, limit).astype(int), [M - 1]]))


def _check(y: torch.Tensor, out: ref.OracleOut, label: str) -> None:
    p = ref.check_parity(bits(y), out)
    print(f"{label}: {p}")
    assert p.ok, f"{label}: {p}"


def _kern():
    from llms_amd import kernels

    return kernels


def check_norm_qkv(M, K, n_q, n_k, seed=0, std=3.0, eps=EPS, gamma=None):
    x = _x(seed + 1, M, K, std)
    _, w = qkv_inputs(seed + 2, 1, K, n_q, n_k)
    g = _norm_weight(seed + 3, K) if gamma is None else gamma
    q, k, v = _kern().fused_rmsnorm_qkv(x.to(DEV), g.to(DEV), eps, w.to(DEV), n_q=n_q, n_k=n_k)
    y = torch.cat([q, k, v], dim=-1).cpu()
    rows = _rows(M)
    out = ref.ref_rmsnorm_qkv_full(bits(x)[rows], bits(g), eps, bits(w), n_q, n_k)
    _check(y[rows], out, f"norm+qkv M={M} K={K}")


def check_norm_gate_up(M, K, N, seed=0, std=3.0, eps=EPS):
    x = _x(seed + 1, M, K, std)
    _, wg, wu = ffn_inputs(seed + 2, 1, K, N)
    g = _norm_weight(seed + 3, K)
    y = _kern().fused_rmsnorm_gate_up_silu(x.to(DEV), g.to(DEV), eps, wg.to(DEV), wu.to(DEV)).cpu()
    rows = _rows(M)
    out = ref.ref_rmsnorm_gate_up_silu_full(bits(x)[rows], bits(g), eps, bits(wg), bits(wu))
    _check(y[rows], out, f"norm+gate-up M={M} K={K} N={N}")


# ------------------------------------------------------------------ CPU


def test_workspace_bytes_and_errors():
    """The workspace query always leaves room for the normalised rows:
    decode-sized calls usually run as one launch and leave it unused, but
    fall back to the two-launch path when a pointer or stride is not 16-byte
    aligned; larger calls add split partials. Argument errors come back
    before any launch."""
    from llms_amd import _lib

    lib = _lib.capi()
    wb = lib.fp_rmsnorm_workspace_bytes
    rows = lambda M, K: (M * K * 2 + 255) // 256 * 256  # noqa: E731
    assert wb(1, 6144, 2560, 0, 0) == rows(1, 2560) and wb(2, 9728, 2560, 1, 0) == rows(2, 2560)
    assert wb(4, 9728, 2560, 1, 1) == rows(4, 2560)   # int8 rows kernel to 4 rows
    assert wb(3, 6144, 2560, 0, 0) == rows(3, 2560)   # bf16 from 3 rows
    assert wb(1, 6144, 2541, 0, 0) == (2541 * 2 + 255) // 256 * 256  # K % 8 != 0
    assert wb(512, 2560, 9728, 0, 0) > 512 * 9728 * 2  # rows + split partials
    P = ctypes.c_void_p(16)
    # fp_rmsnorm_qkv_bf16(x, ldx, gamma, eps, w, ldw, y, ldy, M, n_q, n_k, K, ws, ws_bytes, stream)
    assert lib.fp_rmsnorm_qkv_bf16(P, 64, None, 1e-6, P, 64, P, 96, 2, 64, 16, 64, None, 0, None) == 1
    assert lib.fp_rmsnorm_qkv_bf16(P, 64, P, -1.0, P, 64, P, 96, 2, 64, 16, 64, None, 0, None) == 2
    assert lib.fp_rmsnorm_qkv_bf16(P, 64, P, float("nan"), P, 64, P, 96, 2, 64, 16, 64, None, 0,
                                   None) == 2
    assert lib.fp_rmsnorm_qkv_bf16(P, 64, P, 1e-6, P, 64, P, 96, 2, 64, 16, 64, ctypes.c_void_p(8),
                                   64, None) == 6
    assert lib.fp_rmsnorm_gate_up_silu_bf16(P, 64, P, 1e-6, P, 64, P, 60, P, 32, 2, 32, 64, None, 0,
                                            None) == 3
    assert lib.fp_rmsnorm_qkv_w8(P, 64, P, 1e-6, P, 64, None, P, 96, 2, 64, 16, 64, None, 0,
                                 None) == 1
    assert lib.fp_rmsnorm_gate_up_silu_w8(None, 64, None, 1e-6, None, 64, None, None, 64, None, None,
                                          32, 0, 32, 64, None, 0, None) == 0  # M == 0


def test_python_argument_errors():
    kern = _kern()
    x = torch.randn(2, 64).bfloat16()
    w = torch.randn(96, 64).bfloat16()
    with pytest.raises(ValueError, match="norm weight shape"):
        kern.fused_rmsnorm_qkv(x, torch.ones(63).bfloat16(), EPS, w, n_q=64, n_k=16)
    with pytest.raises(ValueError, match="eps"):
        kern.fused_rmsnorm_qkv(x, torch.ones(64).bfloat16(), -1.0, w, n_q=64, n_k=16)
    with pytest.raises(ValueError, match="HIP"):
        kern.fused_rmsnorm_qkv(x, torch.ones(64).bfloat16(), EPS, w, n_q=64, n_k=16)
    with pytest.raises(ValueError, match="Wg shape"):
        kern.fused_rmsnorm_gate_up_silu(x, torch.ones(64).bfloat16(), EPS, w, w[:10])


# ------------------------------------------------------------------ GPU


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 64, 300])
def test_norm_qkv_qwen3_4b(M):
    check_norm_qkv(M, 2560, 4096, 1024, seed=M)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 5, 64, 300])
def test_norm_gate_up_qwen3_4b(M):
    check_norm_gate_up(M, 2560, 9728, seed=10 + M)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K", [(1, 1024), (2, 16384), (1, 2541), (3, 2541), (1, 32768),
                                 (2, 8), (70, 1032)])
def test_norm_shapes_and_paths(M, K):
    """Small and large K, K % 8 != 0 (the element-wise prologue), the rows
    kernel's LDS limit, tiny K."""
    check_norm_qkv(M, K, 96, 16, seed=20 + K + M)
    check_norm_gate_up(M, K, 100, seed=21 + K + M)


@pytest.mark.gpu
def test_norm_edge_values():
    """An all-zero row (r = 1/sqrt(eps), output 0), a large eps, tiny and
    large row scales, and a norm weight that is not 16-byte aligned (a view at
    offset 1: the one-launch path is refused, the prologue runs)."""
    K, n_q, n_k = 2560, 256, 64
    for std in (1e-3, 40.0):
        check_norm_qkv(2, K, n_q, n_k, seed=31, std=std)
    check_norm_qkv(2, K, n_q, n_k, seed=32, eps=0.5)
    x = _x(33, 2, K)
    x[0] = 0
    _, w = qkv_inputs(34, 1, K, n_q, n_k)
    g = _norm_weight(35, K)
    q, k, v = _kern().fused_rmsnorm_qkv(x.to(DEV), g.to(DEV), EPS, w.to(DEV), n_q=n_q, n_k=n_k)
    y = torch.cat([q, k, v], dim=-1).cpu()
    assert torch.all(y[0] == 0)
    _check(y, ref.ref_rmsnorm_qkv_full(bits(x), bits(g), EPS, bits(w), n_q, n_k), "zero row")
    gbig = torch.empty(K + 1, dtype=torch.bfloat16, device=DEV)
    gbig[1:] = g.to(DEV)
    q, k, v = _kern().fused_rmsnorm_qkv(x.to(DEV), gbig[1:], EPS, w.to(DEV), n_q=n_q, n_k=n_k)
    _check(torch.cat([q, k, v], dim=-1).cpu(),
           ref.ref_rmsnorm_qkv_full(bits(x), bits(g), EPS, bits(w), n_q, n_k), "misaligned gamma")


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 100])
def test_norm_int8(M):
    kern = _kern()
    K, n_q, n_k, I = 2560, 4096, 1024, 9728
    x = _x(40 + M, M, K)
    g = _norm_weight(41, K)
    _, w = qkv_inputs(42, 1, K, n_q, n_k)
    q8, s8 = kern.quantize_w8_per_row(w.to(DEV))
    q, k, v = kern.fused_rmsnorm_qkv_w8(x.to(DEV), g.to(DEV), EPS, q8, s8, n_q=n_q, n_k=n_k)
    rows = _rows(M)
    wd = ref.dequant_w8(q8.cpu().numpy(), s8.cpu().numpy())
    _check(torch.cat([q, k, v], dim=-1).cpu()[rows],
           ref.ref_rmsnorm_qkv_full(bits(x)[rows], bits(g), EPS, wd, n_q, n_k), f"int8 norm+qkv M={M}")
    _, wg, wu = ffn_inputs(43, 1, K, I)
    qg, sg = kern.quantize_w8_per_row(wg.to(DEV))
    qu, su = kern.quantize_w8_per_row(wu.to(DEV))
    y = kern.fused_rmsnorm_gate_up_silu_w8(x.to(DEV), g.to(DEV), EPS, qg, sg, qu, su).cpu()
    _check(y[rows], ref.ref_rmsnorm_gate_up_silu_full(
        bits(x)[rows], bits(g), EPS, ref.dequant_w8(qg.cpu().numpy(), sg.cpu().numpy()),
        ref.dequant_w8(qu.cpu().numpy(), su.cpu().numpy())), f"int8 norm+gate-up M={M}")


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 64])
def test_norm_deterministic_and_raw_abi(M):
    """Repeated calls are bit-identical; through the raw C ABI a call that
    needs the prologue and gets no workspace returns FP_ERR_WORKSPACE and
    launches nothing (y keeps its sentinel)."""
    from llms_amd import _lib

    kern = _kern()
    K, n_q, n_k = 2560, 4096, 1024
    x = _x(50 + M, M, K).to(DEV)
    g = _norm_weight(51, K).to(DEV)
    _, w = qkv_inputs(52, 1, K, n_q, n_k)
    w = w.to(DEV)
    a = torch.cat(kern.fused_rmsnorm_qkv(x, g, EPS, w, n_q=n_q, n_k=n_k), dim=-1)
    b = torch.cat(kern.fused_rmsnorm_qkv(x, g, EPS, w, n_q=n_q, n_k=n_k), dim=-1)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    lib = _lib.capi()
    N = n_q + 2 * n_k
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    need = lib.fp_rmsnorm_workspace_bytes(M, N, K, 0, 0)
    assert need >= (M * K * 2 + 255) // 256 * 256
    st = lib.fp_rmsnorm_qkv_bf16(P(x), K, P(g), EPS, P(w), K, P(y), N, M, n_q, n_k, K, None, 0, stream)
    if M > 2:  # past the one-launch decode path: the normalised rows need room
        assert st == 6
        torch.cuda.synchronize()
        assert torch.all(y == 7.0)
    else:
        assert st == 0
    if M <= 2:
        # an odd row stride keeps x off the one-launch path: the queried
        # workspace is enough for the two-launch path
        xs = torch.zeros(M, K + 1, dtype=torch.bfloat16, device=DEV)
        xs[:, :K] = x
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        y2 = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
        assert lib.fp_rmsnorm_qkv_bf16(P(xs), K + 1, P(g), EPS, P(w), K, P(y2), N, M, n_q, n_k, K,
                                       None, 0, stream) == 6
        assert lib.fp_rmsnorm_qkv_bf16(P(xs), K + 1, P(g), EPS, P(w), K, P(y2), N, M, n_q, n_k, K,
                                       P(ws), need, stream) == 0
        torch.cuda.synchronize()
        _check(y2.cpu(), ref.ref_rmsnorm_qkv_full(bits(x), bits(g), EPS, bits(w), n_q, n_k),
               f"norm+qkv strided x M={M}")
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
    assert lib.fp_rmsnorm_qkv_bf16(P(x), K, P(g), EPS, P(w), K, P(y), N, M, n_q, n_k, K, P(ws),
                                   need, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), a.view(torch.int16))
