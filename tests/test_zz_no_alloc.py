"""The allocation-free entry point fp_rmsnorm_qkv_bf16_noalloc.

It has no counterpart in the reference: it is fp_rmsnorm_qkv_bf16 with the
workspace taken from the library's static device scratch (FP_SCRATCH_BYTES
per GPU) for callers that cannot allocate. Through the raw C ABI it must
give the bits of the workspace entry point on two calls in a row (the second
with fewer rows, which leaves the first call's contents in the scratch), match
the oracle, and refuse a call that needs more scratch than the maximum before
launching anything.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import ref
from tests._util import bits, gen, qkv_inputs, randn_bf16

DEV = "cuda"
EPS = 1e-6


def _lib():
    from llms_amd import _lib

    return _lib


def test_noalloc_cpu_contract():
    """Host side, no GPU: the scratch limit is exported as declared, sizes
    beyond it are refused with FP_ERR_SCRATCH, argument errors and M == 0
    come back like the workspace entry point's."""
    L = _lib()
    lib = L.capi()
    assert L.FP_SCRATCH_BYTES == 32 << 20
    assert L.status_string(7).startswith("the call needs more than the library's static scratch")
    P = ctypes.c_void_p(256)
    # 8B-shaped QKV: 4096 rows (BASELINE's largest) need exactly the maximum
    # (32 MiB of normalised rows), one more row is refused; so is 8192
    wb = lib.fp_rmsnorm_workspace_bytes
    assert wb(4096, 6144, 4096, 0, 0) == L.FP_SCRATCH_BYTES
    assert wb(4097, 6144, 4096, 0, 0) > L.FP_SCRATCH_BYTES
    f = lib.fp_rmsnorm_qkv_bf16_noalloc
    # (only calls that are refused before any launch: these pointers are fake)
    assert f(P, 4096, P, EPS, P, 4096, P, 6144, 4097, 4096, 1024, 4096, None) == 7
    assert f(P, 4096, P, EPS, P, 4096, P, 6144, 8192, 4096, 1024, 4096, None) == 7
    assert f(P, 64, P, EPS, P, 64, P, 96, 0, 64, 16, 64, None) == 0      # M == 0
    assert f(P, 64, None, EPS, P, 64, P, 96, 2, 64, 16, 64, None) == 1   # NULL gamma
    assert f(P, 64, P, -1.0, P, 64, P, 96, 2, 64, 16, 64, None) == 2     # bad eps
    assert f(P, 64, P, EPS, P, 64, P, 95, 2, 64, 16, 64, None) == 3      # ldy < N
    assert f(P, 64, P, EPS, P, 64, P, 96, 2, 0, 16, 64, None) == 2       # n_q < 1


def _call(fn_ws: bool, x, g, w, n_q, n_k, y, stream):
    L = _lib()
    lib = L.capi()
    M, K = x.shape
    N = n_q + 2 * n_k
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    if fn_ws:
        need = lib.fp_rmsnorm_workspace_bytes(M, N, K, 0, 0)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=DEV)
        st = lib.fp_rmsnorm_qkv_bf16(P(x), x.stride(0), P(g), EPS, P(w), w.stride(0), P(y),
                                     y.stride(0), M, n_q, n_k, K, P(ws), need, stream)
        torch.cuda.synchronize()
        del ws
    else:
        st = lib.fp_rmsnorm_qkv_bf16_noalloc(P(x), x.stride(0), P(g), EPS, P(w), w.stride(0),
                                             P(y), y.stride(0), M, n_q, n_k, K, stream)
    assert st == 0, L.status_string(st)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["4b", "8b"])
def test_noalloc_matches_workspace_entry(shape):
    """Calls in a row on one GPU, each with fewer rows than the last: each
    equals the workspace entry point bit for bit and passes the oracle. The
    shapes cover the normalised-rows scratch (4B at 300 rows: the norm
    kernel, then the MFMA grid), the whole scratch (8B at 4096 rows: 32 MiB
    of normalised rows), the k split across workgroups with its fp32 partials
    in the scratch after the rows (4B and 8B at 128 rows: 0.6 or 1 MiB of
    rows + 6 MiB of partials; asserted to split) and a small last call (3 or
    5 rows: the streaming kernel) over what the earlier calls left in the
    scratch."""
    K, n_q, n_k, Ms = {"4b": (2560, 4096, 1024, (300, 128, 3)),
                       "8b": (4096, 4096, 1024, (4096, 128, 5))}[shape]
    N = n_q + 2 * n_k
    lib = _lib().capi()
    # 128 rows split k across workgroups: the scratch holds partials beyond
    # the normalised rows (so the case cannot silently stop splitting)
    assert lib.fp_rmsnorm_workspace_bytes(128, N, K, 0, 0) > 128 * K * 2
    _, w = qkv_inputs(900 + K, 1, K, n_q, n_k)
    g = randn_bf16(gen(901 + K), K, std=0.5) + 1.0
    wd, gd = w.to(DEV), g.to(torch.bfloat16).to(DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, M in enumerate(Ms):
        x = (torch.randn(M, K, generator=gen(910 + i + K)) * 2.0).to(torch.bfloat16)
        xd = x.to(DEV)
        ya = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
        yb = torch.full((M, N), -7.0, dtype=torch.bfloat16, device=DEV)
        _call(False, xd, gd, wd, n_q, n_k, ya, stream)
        torch.cuda.synchronize()
        _call(True, xd, gd, wd, n_q, n_k, yb, stream)
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), f"{shape} call {i} M={M}"
        rows = np.arange(M) if M <= 64 else np.sort(np.random.default_rng(i).choice(M, 64, False))
        out = ref.ref_rmsnorm_qkv_full(bits(x)[rows], bits(gd.cpu()), EPS, bits(w), n_q, n_k)
        p = ref.check_parity(bits(ya.cpu())[rows], out)
        print(f"noalloc {shape} M={M}: {p}")
        assert p.ok, p


@pytest.mark.gpu
def test_noalloc_in_graph_capture():
    """The advertised use: the allocation-free call captured in a HIP graph
    (torch.cuda.graph) and replayed. Every replay, with eager work and
    synchronisations between replays, equals the eager workspace entry point
    bit for bit; replays of the same graph after the scratch was overwritten
    by an eager call of another size still give the captured call's result.
    4B QKV at 128 rows: the norm kernel, then k split across workgroups with
    its partials in the scratch."""
    K, n_q, n_k, M = 2560, 4096, 1024, 128
    N = n_q + 2 * n_k
    x, w = qkv_inputs(950, M, K, n_q, n_k)
    g = randn_bf16(gen(951), K, std=0.5) + 1.0
    xd, wd, gd = x.to(DEV), w.to(DEV), g.to(torch.bfloat16).to(DEV)
    ref_y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _call(True, xd, gd, wd, n_q, n_k, ref_y,
          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    y = torch.zeros(M, N, dtype=torch.bfloat16, device=DEV)
    # the first call on this device (symbol lookup) happens before capture
    _call(False, xd, gd, wd, n_q, n_k, y, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        _call(False, xd, gd, wd, n_q, n_k, y, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    x2, _ = qkv_inputs(952, 300, K, n_q, n_k)
    x2d = x2.to(DEV)
    y2 = torch.empty(300, N, dtype=torch.bfloat16, device=DEV)
    for r in range(4):
        y.fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref_y.view(torch.int16)), f"replay {r}"
        # eager work on the same scratch between replays (another size)
        _call(False, x2d, gd, wd, n_q, n_k, y2,
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
    del graph
