"""Seeded random shapes across every dispatch regime, against the oracle.

The targeted GPU tests pin each kernel family at the shapes that select it.
This file draws shapes at random (fixed seed) so that the planner's
boundaries are crossed at places nobody picked: row counts from 1 to a few
thousand (the row-streaming, streaming, split-K, staged, tiled and
persistent-tile regimes, with and without the k split across workgroups),
K aligned to 64 or 128, aligned to 8 only, or ragged, and output widths that
leave partial tiles; every third case passes x as a row-strided view. Each
shape runs the bf16 QKV, gate-up-SiLU and plain projections and their int8
weight-only forms through the Python surface (which passes the split
workspace the torch ops allocate), and is checked against the oracle on up
to 48 rows (``oracle.ref.check_parity``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref
from tests._util import bits, ffn_inputs, qkv_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
SPECIAL_M = (1, 2, 3, 5, 8, 9, 16, 17, 48, 63, 64, 65, 96, 128, 129, 255, 256, 257, 511, 512,
             513, 1023, 1536, 2048, 2049)


def _shapes(n: int, seed: int = 2024):
    """(M, K, n_q, n_k, I): M log-uniform in [1, 3000] or a regime edge; K a
    multiple of 64 (60%), of 8 only (25%) or anything (15%), at most 5120;
    output widths with partial tiles, N x K at most 1.6e7 (oracle time)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        if i % 2 == 0:
            M = int(rng.choice(SPECIAL_M))
        else:
            M = int(np.exp(rng.uniform(0, np.log(3000))))
        u = rng.uniform()
        if u < 0.6:
            K = 64 * int(rng.integers(1, 81))
        elif u < 0.85:
            K = 8 * int(rng.integers(1, 641))
        else:
            K = int(rng.integers(1, 5121))
        nmax = max(16, int(1.6e7 // K))
        n_k = int(rng.integers(1, max(2, min(1024, nmax // 6)) + 1))
        n_q = int(rng.integers(1, max(2, min(4096, nmax - 2 * n_k)) + 1))
        inter = int(rng.integers(1, max(2, min(12288, nmax // 2)) + 1))
        out.append((M, K, n_q, n_k, inter))
    return out


SHAPES = _shapes(64)


def _kernels():
    from llms_amd import kernels

    return kernels


def _rows(M: int, seed: int) -> np.ndarray:
    if M <= 48:
        return np.arange(M)
    r = np.random.default_rng(seed).choice(M, size=46, replace=False)
    return np.sort(np.concatenate([r, [0, M - 1]]))


def _check(y: torch.Tensor, out: ref.OracleOut, label: str) -> None:
    p = ref.check_parity(bits(y), out)
    print(f"{label}: {p}")
    assert p.ok, f"{label}: {p}"


def _on_device(x: torch.Tensor, i: int) -> torch.Tensor:
    """x on the device; every third case as a row-strided view (row stride K
    plus 1-24 elements, unit inner stride), as a slice of a wider buffer."""
    if i % 3 != 1:
        return x.to(DEV)
    pad = 1 + (i * 7) % 24
    full = torch.zeros(x.shape[0], x.shape[1] + pad, dtype=x.dtype)
    full[:, : x.shape[1]] = x
    return full.to(DEV)[:, : x.shape[1]]


def _quant(w: torch.Tensor):
    q, s = _kernels().quantize_w8_per_row(w.to(DEV))
    qo, so = ref.quantize_w8_per_row(bits(w))
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    return q, s


@pytest.mark.parametrize("i", range(len(SHAPES)))
def test_random_shape(i):
    M, K, n_q, n_k, inter = SHAPES[i]
    kern = _kernels()
    tag = f"case {i}: M={M} K={K} n_q={n_q} n_k={n_k} I={inter}"
    rows = _rows(M, i)

    x, w = qkv_inputs(5000 + i, M, K, n_q, n_k)
    xd = _on_device(x, i)
    q, k, v = kern.triton_fused_qkv(xd, w.to(DEV), n_q=n_q, n_k=n_k)
    y = torch.cat([q, k, v], -1).cpu()
    _check(y[rows], ref.ref_qkv_full(bits(x)[rows], bits(w), n_q, n_k), f"{tag} qkv")

    # the plain projection on the same operands (one column block)
    y = kern.fused_linear(xd, w.to(DEV)).cpu()
    _check(y[rows], ref.ref_linear(bits(x)[rows], bits(w)), f"{tag} linear")

    qw, sw = _quant(w)
    q, k, v = kern.fused_qkv_w8(xd, qw, sw, n_q=n_q, n_k=n_k)
    y = torch.cat([q, k, v], -1).cpu()
    out = ref.ref_qkv_w8_full(bits(x)[rows], qw.cpu().numpy(), sw.cpu().numpy(), n_q, n_k)
    _check(y[rows], out, f"{tag} int8 qkv")

    y = kern.fused_linear_w8(xd, qw, sw).cpu()
    out = ref.ref_linear_w8(bits(x)[rows], qw.cpu().numpy(), sw.cpu().numpy())
    _check(y[rows], out, f"{tag} int8 linear")

    x, wg, wu = ffn_inputs(6000 + i, M, K, inter)
    xd = _on_device(x, i)
    y = kern.triton_fused_gate_up_silu(xd, wg.to(DEV), wu.to(DEV)).cpu()
    _check(y[rows], ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu)), f"{tag} gate-up")

    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su).cpu()
    out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                       qu.cpu().numpy(), su.cpu().numpy())
    _check(y[rows], out, f"{tag} int8 gate-up")


def test_shapes_cover_the_regimes():
    """No GPU needed for the draw itself, but it lives with the GPU cases:
    the seeded shapes must reach every regime the test claims."""
    Ms = [s[0] for s in SHAPES]
    Ks = [s[1] for s in SHAPES]
    assert min(Ms) <= 2 and any(3 <= m <= 8 for m in Ms) and any(9 <= m <= 64 for m in Ms)
    assert any(65 <= m <= 256 for m in Ms) and any(m >= 512 for m in Ms)
    assert any(k % 64 == 0 for k in Ks) and any(k % 64 != 0 and k % 8 == 0 for k in Ks)
    assert any(k % 8 != 0 for k in Ks)


def _verify8_shapes(n: int, seed: int = 77):
    """(M, K, N, I): int8 shapes inside the x-staging verify kernel's domain
    (2-16 rows, K a multiple of 64 from 2048 to 2560, at least 4096 outputs),
    output widths with partial blocks of 16."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(2, 17)), 64 * int(rng.integers(32, 41)),
             int(rng.integers(4096, 9001)), int(rng.integers(4096, 12001))) for _ in range(n)]


VERIFY8_SHAPES = _verify8_shapes(8)


@pytest.mark.parametrize("i", range(len(VERIFY8_SHAPES)))
def test_random_int8_verify_shape(i):
    """Seeded int8 shapes at spec-verify row counts with K from 2048 to 2560:
    QKV-like, plain and gate-up calls against the oracle, every other case
    with x as a row-strided view."""
    M, K, N, inter = VERIFY8_SHAPES[i]
    kern = _kernels()
    tag = f"verify8 case {i}: M={M} K={K} N={N} I={inter}"
    n_k = 512
    x, w = qkv_inputs(7000 + i, M, K, N - 2 * n_k, n_k)
    xd = _on_device(x, 3 * i + 1) if i % 2 else x.to(DEV)
    qw, sw = _quant(w)
    q, k, v = kern.fused_qkv_w8(xd, qw, sw, n_q=N - 2 * n_k, n_k=n_k)
    y = torch.cat([q, k, v], -1).cpu()
    out = ref.ref_qkv_w8_full(bits(x), qw.cpu().numpy(), sw.cpu().numpy(), N - 2 * n_k, n_k)
    _check(y, out, f"{tag} int8 qkv")
    y = kern.fused_linear_w8(xd, qw, sw).cpu()
    _check(y, ref.ref_linear_w8(bits(x), qw.cpu().numpy(), sw.cpu().numpy()), f"{tag} int8 linear")

    x, wg, wu = ffn_inputs(8000 + i, M, K, inter)
    xd = _on_device(x, 3 * i + 1) if i % 2 else x.to(DEV)
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su).cpu()
    out = ref.ref_gate_up_silu_w8_full(bits(x), qg.cpu().numpy(), sg.cpu().numpy(),
                                       qu.cpu().numpy(), su.cpu().numpy())
    _check(y, out, f"{tag} int8 gate-up")


def test_verify8_shapes_in_domain():
    """The seeded draw stays inside the domain it claims, and reaches both
    of the kernel's x stagings (up to 8 rows, and 9-16)."""
    assert all(2 <= m <= 16 and 2048 <= k <= 2560 and k % 64 == 0 and n >= 4096 and i >= 4096
               for m, k, n, i in VERIFY8_SHAPES)
    assert any(m <= 8 for m, *_ in VERIFY8_SHAPES) and any(m > 8 for m, *_ in VERIFY8_SHAPES)
    assert any(n % 16 for _, _, n, _ in VERIFY8_SHAPES)
