"""The C ABI: every declared symbol is exported, argument errors are caught
before any launch (CPU), and raw-pointer calls match the oracle (GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ref
from tests._util import bits, ffn_inputs, qkv_inputs

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared_functions() -> list[str]:
    names = []
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(fp_\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared_functions()
    for expected in ("fp_qkv_bf16", "fp_gate_up_silu_bf16", "fp_qkv_w8",
                     "fp_gate_up_silu_w8", "fp_quantize_w8_per_row",
                     "fp_linear_bf16", "fp_linear_w8", "fp_workspace_bytes",
                     "fp_qkv_bf16_ws", "fp_gate_up_silu_bf16_ws", "fp_linear_bf16_ws",
                     "fp_status_string", "fp_abi_version"):
        assert expected in names


def test_library_exports_every_declared_symbol():
    from llms_amd import _lib

    lib = _lib.capi()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _lib.CAPI_SIGNATURES, f"{name} has no ctypes signature"
    assert lib.fp_abi_version() >> 16 == 1
    # minor 5: the allocation-free entry point, FP_ERR_SCRATCH and the
    # fused-norm workspace sizing that covers the normalised rows
    if hasattr(lib, "fp_rmsnorm_qkv_bf16_noalloc"):
        assert lib.fp_abi_version() & 0xFFFF >= 5


def test_int8_workspace_is_split_partials_only():
    """int8 calls never expand their weights to bf16: at every BASELINE int8
    configuration (Qwen3-4B M = 1, 4, 2048; Qwen3-8B M = 1 ... 4096) and at
    other row counts, fp_workspace_bytes_w8 is 0, or exactly the fp32
    partials of k split over 4-16 workgroups (S planes of M x W floats, W =
    N, gate-up 2N) where the split plan takes the call. No GPU needed."""
    from llms_amd import _lib

    lib = _lib.capi()
    shapes = {"4b": (2560, 6144, 9728), "8b": (4096, 6144, 12288)}
    for model, (K, n_qkv, inter) in shapes.items():
        for M in (1, 3, 4, 8, 16, 64, 128, 129, 256, 512, 1024, 2048, 4096, 8192):
            for N, gu in ((n_qkv, 0), (inter, 1)):
                ws = lib.fp_workspace_bytes_w8(M, N, K, gu)
                plane = 4 * M * N * (2 if gu else 1)
                assert ws == 0 or (ws % plane == 0 and 4 <= ws // plane <= 16), (model, M, N, ws)
                if gu or M in (1, 4, 2048, 4096) or model == "4b":
                    assert ws == 0, (model, M, N, gu, ws)


def test_workspace_bytes_plan():
    """The split-k plan (a host function: no GPU needed). Splits only where
    the unsplit grid leaves the chip idle and k is long: Qwen3 down from 32
    rows, o at 256 rows, 8B QKV at 128, 8B gate-up at 40, 8B TP=8 QKV shards
    (768 columns) at 512; never for short K, few rows, K % 64 != 0, a
    chip-filling grid, where one round of tiles with 128-wide k-steps runs
    instead with at most 6 splits (4B QKV at 256 rows, 4B o at 640) or 3 (8B
    o at 1024), or where a round of small three-stage tiles with enough tiles
    per k-step runs instead (8B QKV at 256 rows, 8B gate-up at 64, 4B TP=4
    QKV shards at 512). The workspace holds one fp32 plane per k range,
    2..16 ranges, of M x N (gate-up: M x 2N)."""
    from llms_amd import _lib

    wb = _lib.capi().fp_workspace_bytes

    def planes(M, N, K, gu=0):
        b = wb(M, N, K, gu)
        plane = 4 * M * N * (2 if gu else 1)
        assert b % plane == 0
        return b // plane

    for M in (32, 64, 128, 256, 512, 1024):
        assert 2 <= planes(M, 2560, 9728) <= 16, M          # 4B down
        assert 2 <= planes(M, 4096, 12288) <= 16, M         # 8B down
    assert 2 <= planes(128, 6144, 4096) <= 16               # 8B QKV, 128 rows
    assert 2 <= planes(128, 2560, 4096) <= 16               # 4B o, 128 rows
    assert 2 <= planes(256, 2560, 4096) <= 16               # 4B o, 256 rows: 108 small tiles
    assert 2 <= planes(512, 768, 4096) <= 16                # 8B TP=8 QKV: 64 tiles, 32 k-steps
    assert 2 <= planes(128, 1024, 3072) <= 16               # 0.6B down, few tiles
    assert 2 <= planes(300, 1001, 8192) <= 16                # narrow, ragged N
    assert 2 <= planes(40, 12288, 4096, 1) <= 16             # 8B gate-up, 40 rows
    assert 2 <= planes(200, 1001, 8192, 1) <= 16             # gate-up, ragged N
    for args in [(16, 2560, 9728, 0), (31, 2560, 9728, 0), (512, 6144, 2560, 0),
                 (2048, 9728, 2560, 1), (256, 4096, 1024, 0), (64, 2560, 4096, 0),
                 (512, 2560, 9736, 0), (8192, 2560, 9728, 0), (0, 2560, 9728, 0),
                 (512, 0, 9728, 0), (64, 9728, 2560, 1), (32, 12288, 4096, 1),
                 (128, 9728, 2560, 1), (32, 6144, 4096, 0), (256, 6144, 2560, 0),
                 (640, 2560, 4096, 0), (1024, 4096, 4096, 0), (256, 6144, 4096, 0),
                 (512, 1536, 2560, 0), (64, 12288, 4096, 1)]:
        assert wb(*args) == 0, args
    # ranges hold at least 8 k-steps of 64
    assert planes(32, 2560, 2048) <= 4


def test_status_strings():
    from llms_amd import _lib

    for code, name in _lib.FP_STATUS.items():
        assert _lib.status_string(code)
    assert "unknown" in _lib.status_string(99)


def test_argument_errors_return_before_launch():
    """Invalid arguments come back as status codes; nothing touches a GPU."""
    from llms_amd import _lib

    lib = _lib.capi()
    P = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # fp_qkv_bf16(x, ldx, w, ldw, y, ldy, M, n_q, n_k, K, stream)
    assert lib.fp_qkv_bf16(P, 64, P, 64, P, 96, 2, 0, 16, 64, None) == 2      # n_q < 1
    assert lib.fp_qkv_bf16(P, 64, P, 64, P, 96, 2, 64, -1, 64, None) == 2    # n_k < 0
    assert lib.fp_qkv_bf16(P, 64, P, 64, P, 96, -1, 64, 16, 64, None) == 2   # M < 0
    assert lib.fp_qkv_bf16(P, 64, P, 64, P, 96, 2, 64, 16, 0, None) == 2     # K < 1
    assert lib.fp_qkv_bf16(P, 32, P, 64, P, 96, 2, 64, 16, 64, None) == 3    # ldx < K
    assert lib.fp_qkv_bf16(P, 64, P, 63, P, 96, 2, 64, 16, 64, None) == 3    # ldw < K
    assert lib.fp_qkv_bf16(P, 64, P, 64, P, 95, 2, 64, 16, 64, None) == 3    # ldy < N
    assert lib.fp_qkv_bf16(None, 64, P, 64, P, 96, 2, 64, 16, 64, None) == 1  # NULL x
    assert lib.fp_qkv_bf16(None, 64, None, 64, None, 96, 0, 64, 16, 64, None) == 0  # M == 0
    # fp_gate_up_silu_bf16(x, ldx, wg, ldwg, wu, ldwu, y, ldy, M, N, K, stream)
    assert lib.fp_gate_up_silu_bf16(P, 64, P, 64, P, 60, P, 32, 2, 32, 64, None) == 3
    assert lib.fp_gate_up_silu_bf16(P, 64, P, 64, None, 64, P, 32, 2, 32, 64, None) == 1
    assert lib.fp_gate_up_silu_bf16(P, 64, P, 64, P, 64, P, 32, 2, 0, 64, None) == 2
    # int8 variants
    assert lib.fp_qkv_w8(P, 64, P, 64, None, P, 96, 2, 64, 16, 64, None) == 1   # NULL scale
    assert lib.fp_gate_up_silu_w8(P, 64, P, 64, P, P, 64, None, P, 32, 2, 32, 64, None) == 1
    assert lib.fp_gate_up_silu_w8(P, 64, P, 10, P, P, 64, P, P, 32, 2, 32, 64, None) == 3
    # fp_linear_bf16(x, ldx, w, ldw, y, ldy, M, N, K, stream)
    assert lib.fp_linear_bf16(P, 64, P, 64, P, 32, 2, 0, 64, None) == 2      # N < 1
    assert lib.fp_linear_bf16(P, 64, P, 64, P, 31, 2, 32, 64, None) == 3     # ldy < N
    assert lib.fp_linear_bf16(P, 64, None, 64, P, 32, 2, 32, 64, None) == 1  # NULL w
    assert lib.fp_linear_w8(P, 64, P, 64, None, P, 32, 2, 32, 64, None) == 1  # NULL scale
    assert lib.fp_linear_w8(P, 64, P, 63, P, P, 32, 2, 32, 64, None) == 3    # ldq < K
    # workspace variants: negative size or a misaligned workspace
    assert lib.fp_linear_bf16_ws(P, 64, P, 64, P, 32, 2, 32, 64, P, -4, None) == 6
    assert lib.fp_linear_bf16_ws(P, 64, P, 64, P, 32, 2, 32, 64, ctypes.c_void_p(20), 64, None) == 6
    assert lib.fp_qkv_bf16_ws(P, 64, P, 64, P, 96, 2, 64, 16, 64, ctypes.c_void_p(8), 64, None) == 6
    assert lib.fp_gate_up_silu_bf16_ws(P, 64, P, 64, P, 64, P, 32, 2, 32, 64, P, -1, None) == 6
    assert lib.fp_qkv_bf16_ws(P, 64, P, 64, P, 96, 2, 0, 16, 64, None, 0, None) == 2
    assert lib.fp_linear_bf16_ws(None, 64, None, 64, None, 32, 0, 32, 64, None, 0, None) == 0
    assert lib.fp_quantize_w8_per_row(P, 64, P, 63, P, 8, 64, None) == 3
    assert lib.fp_quantize_w8_per_row(P, 64, P, 64, P, -1, 64, None) == 2
    assert lib.fp_quantize_w8_per_row(None, 64, None, 64, None, 0, 64, None) == 0


def test_python_wrappers_raise_reference_errors():
    """The wrappers' shape checks run before anything else, with the
    reference's messages (tests/test_kernels_fused_ffn.py:203-229,
    tests/test_kernels_fused_qkv.py:253-277); CPU tensors are then refused."""
    from llms_amd.kernels import triton_fused_gate_up_silu, triton_fused_qkv

    x = torch.randn(2, 64)
    Wg = torch.randn(128, 64)
    with pytest.raises(ValueError, match="Wg shape.*Wu shape"):
        triton_fused_gate_up_silu(x, Wg, torch.randn(127, 64))
    with pytest.raises(ValueError, match="Wg shape.*Wu shape"):
        triton_fused_gate_up_silu(x, Wg, torch.randn(128, 63))
    W3 = torch.randn(2, 128, 64)
    with pytest.raises(ValueError, match="Wg must be 2D"):
        triton_fused_gate_up_silu(x, W3, W3)
    with pytest.raises(ValueError, match="x last dim.*Wg.shape"):
        triton_fused_gate_up_silu(torch.randn(2, 63), Wg, Wg)

    W_qkv = torch.randn(96, 64)
    with pytest.raises(ValueError, match="n_q .* 2.n_k"):
        triton_fused_qkv(x, W_qkv, n_q=64, n_k=15)
    with pytest.raises(ValueError, match="x last dim .* W_qkv"):
        triton_fused_qkv(torch.randn(2, 63), W_qkv, n_q=64, n_k=16)
    with pytest.raises(ValueError, match="W_qkv must be 2D"):
        triton_fused_qkv(x, torch.randn(2, 96, 64), n_q=64, n_k=16)

    with pytest.raises(TypeError, match="bfloat16"):
        triton_fused_qkv(x, W_qkv, n_q=64, n_k=16)
    with pytest.raises(ValueError, match="HIP"):
        triton_fused_qkv(x.bfloat16(), W_qkv.bfloat16(), n_q=64, n_k=16)


def test_prewarm_no_op_without_fused_modules():
    """Reference test_prewarm_no_op_without_triton_modules: a model with no
    fused modules (and no .layers) is left alone."""
    from llms_amd.kernels import prewarm_triton_kernels

    prewarm_triton_kernels(torch.nn.Sequential(torch.nn.Linear(4, 4)))


# ----------------------------------------------------------------- GPU


def _p(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.gpu
def test_capi_raw_pointers_match_oracle():
    """Call the C ABI directly (as a non-Python host would) on device buffers
    and torch's current stream."""
    from llms_amd import _lib

    lib = _lib.capi()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    M, K, n_q, n_k = 4, 2560, 4096, 1024
    x, w = qkv_inputs(90, M, K, n_q, n_k)
    xd, wd = x.cuda(), w.cuda()
    N = n_q + 2 * n_k
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    st = lib.fp_qkv_bf16(_p(xd), K, _p(wd), K, _p(y), N, M, n_q, n_k, K, stream)
    assert st == 0, _lib.status_string(st)
    torch.cuda.synchronize()
    p = ref.check_parity(bits(y), ref.ref_qkv_full(bits(x), bits(w), n_q, n_k))
    assert p.ok, p

    I = 9728
    x, wg, wu = ffn_inputs(91, M, K, I)
    xd, gd, ud = x.cuda(), wg.cuda(), wu.cuda()
    y = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    st = lib.fp_gate_up_silu_bf16(_p(xd), K, _p(gd), K, _p(ud), K, _p(y), I, M, I, K, stream)
    assert st == 0, _lib.status_string(st)
    torch.cuda.synchronize()
    p = ref.check_parity(bits(y), ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu)))
    assert p.ok, p

    # the workspace variant: split k (planned for this shape) and unsplit
    # (workspace one float short) both match the oracle; the unsplit call is
    # bit-identical to the plain entry point
    Mw, Kw, Nw = 512, 9728, 2560
    xw, ww = qkv_inputs(92, Mw, Kw, Nw, 0)
    xwd, wwd = xw.cuda(), ww.cuda()
    need = lib.fp_workspace_bytes(Mw, Nw, Kw, 0)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y_split = torch.empty(Mw, Nw, dtype=torch.bfloat16, device="cuda")
    y_short = torch.empty_like(y_split)
    y_plain = torch.empty_like(y_split)
    assert lib.fp_linear_bf16_ws(_p(xwd), Kw, _p(wwd), Kw, _p(y_split), Nw, Mw, Nw, Kw, _p(ws),
                                 need, stream) == 0
    assert lib.fp_linear_bf16_ws(_p(xwd), Kw, _p(wwd), Kw, _p(y_short), Nw, Mw, Nw, Kw, _p(ws),
                                 need - 4, stream) == 0
    assert lib.fp_linear_bf16(_p(xwd), Kw, _p(wwd), Kw, _p(y_plain), Nw, Mw, Nw, Kw, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(y_short.view(torch.int16), y_plain.view(torch.int16))
    rows = np.arange(0, Mw, 5)
    for y_ in (y_split, y_plain):
        p = ref.check_parity(bits(y_)[rows], ref.ref_linear(bits(xw)[rows], bits(ww)))
        assert p.ok, p

    # the other workspace variants with the planned workspace (QKV at 128
    # rows with K = 4096 splits; gate-up here does not, so its workspace is
    # unused)
    Mq, nq, nk, Kq = 128, 4096, 1024, 4096
    xq, wq = qkv_inputs(93, Mq, Kq, nq, nk)
    xqd, wqd = xq.cuda(), wq.cuda()
    Nq = nq + 2 * nk
    need = lib.fp_workspace_bytes(Mq, Nq, Kq, 0)
    assert need > 0
    wsq = torch.empty(need, dtype=torch.uint8, device="cuda")
    yq = torch.empty(Mq, Nq, dtype=torch.bfloat16, device="cuda")
    assert lib.fp_qkv_bf16_ws(_p(xqd), Kq, _p(wqd), Kq, _p(yq), Nq, Mq, nq, nk, Kq, _p(wsq), need,
                              stream) == 0
    torch.cuda.synchronize()
    rows = np.arange(0, Mq, 3)
    p = ref.check_parity(bits(yq)[rows], ref.ref_qkv_full(bits(xq)[rows], bits(wq), nq, nk))
    assert p.ok, p
    yg = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    assert lib.fp_gate_up_silu_bf16_ws(_p(xd), K, _p(gd), K, _p(ud), K, _p(yg), I, M, I, K,
                                       _p(wsq), need, stream) == 0
    torch.cuda.synchronize()
    p = ref.check_parity(bits(yg), ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu)))
    assert p.ok, p

    # int8 through the raw ABI: quantise on device, then the fused call
    q = torch.empty(I, K, dtype=torch.int8, device="cuda")
    s = torch.empty(I, dtype=torch.float32, device="cuda")
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    assert lib.fp_quantize_w8_per_row(_p(gd), K, _p(q), K, _p(s), I, K, stream) == 0
    assert lib.fp_quantize_w8_per_row(_p(ud), K, _p(q2), K, _p(s2), I, K, stream) == 0
    st = lib.fp_gate_up_silu_w8(_p(xd), K, _p(q), K, _p(s), _p(q2), K, _p(s2), _p(y), I,
                                M, I, K, stream)
    assert st == 0, _lib.status_string(st)
    torch.cuda.synchronize()
    out = ref.ref_gate_up_silu_w8_full(bits(x), q.cpu().numpy(), s.cpu().numpy(),
                                       q2.cpu().numpy(), s2.cpu().numpy())
    p = ref.check_parity(bits(y), out)
    assert p.ok, p

    # int8 QKV-shaped and plain projections on the same quantised Wg (I rows)
    y8 = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    assert lib.fp_qkv_w8(_p(xd), K, _p(q), K, _p(s), _p(y8), I, M, I - 2 * 1024, 1024, K,
                         stream) == 0
    y9 = torch.empty_like(y8)
    assert lib.fp_linear_w8(_p(xd), K, _p(q), K, _p(s), _p(y9), I, M, I, K, stream) == 0
    torch.cuda.synchronize()
    out = ref.ref_linear_w8(bits(x), q.cpu().numpy(), s.cpu().numpy())
    for yy in (y8, y9):
        p = ref.check_parity(bits(yy), out)
        assert p.ok, p


@pytest.mark.gpu
def test_int8_entry_points_without_workspace_prefill():
    """The plain int8 entry points (no workspace to dequantise into) at
    prefill sizes: gate-up, QKV and the long-K plain projection run the gemm
    with in-register dequantisation."""
    from llms_amd import _lib

    lib = _lib.capi()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = np.sort(np.random.default_rng(3).choice(2048, 64, replace=False))
    for M, K, N, kind in [(2048, 2560, 1000, "gate-up"), (700, 2560, 4352, "qkv"), (512, 9728, 520, "linear")]:
        x, w = qkv_inputs(700 + M, M, K, N, 0)
        xd = x.cuda()
        q = torch.empty(N, K, dtype=torch.int8, device="cuda")
        s = torch.empty(N, dtype=torch.float32, device="cuda")
        assert lib.fp_quantize_w8_per_row(_p(w.cuda()), K, _p(q), K, _p(s), N, K, stream) == 0
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        r = rows[rows < M]
        if kind == "gate-up":
            st = lib.fp_gate_up_silu_w8(_p(xd), K, _p(q), K, _p(s), _p(q), K, _p(s), _p(y), N, M, N, K, stream)
            out = lambda: ref.ref_gate_up_silu_w8_full(bits(x)[r], q.cpu().numpy(), s.cpu().numpy(),  # noqa: E731
                                                       q.cpu().numpy(), s.cpu().numpy())
        elif kind == "qkv":
            st = lib.fp_qkv_w8(_p(xd), K, _p(q), K, _p(s), _p(y), N, M, N - 256, 128, K, stream)
            out = lambda: ref.ref_qkv_w8_full(bits(x)[r], q.cpu().numpy(), s.cpu().numpy(), N - 256, 128)  # noqa: E731
        else:
            st = lib.fp_linear_w8(_p(xd), K, _p(q), K, _p(s), _p(y), N, M, N, K, stream)
            out = lambda: ref.ref_linear_w8(bits(x)[r], q.cpu().numpy(), s.cpu().numpy())  # noqa: E731
        assert st == 0, _lib.status_string(st)
        torch.cuda.synchronize()
        p = ref.check_parity(bits(y.cpu())[r], out())
        assert p.ok, (kind, M, p)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,M,K,N", [("qkv", 384, 1024, 6144),      # 96 x 128, 128-wide k-steps
                                        ("linear", 200, 1024, 1001),   # 64 x 64, 128-wide k-steps
                                        ("gate-up", 500, 1024, 3000),  # 128 x 128, 128-wide k-steps
                                        ("qkv", 3000, 1024, 6144)])    # 320 x 256
def test_padded_strides_on_prefill_tiles(kind, M, K, N):
    """Row strides larger than the rows (ldx = K + 64, ldw = K + 128, ldy =
    N + 8) through the C ABI on the prefill tiles: operands are addressed by
    stride, padding is never read or written."""
    from llms_amd import _lib

    lib = _lib.capi()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ldx, ldw, ldy = K + 64, K + 128, N + 8
    if kind == "gate-up":
        x, wg, wu = ffn_inputs(800 + M, M, K, N)
        mats = [wg, wu]
    else:
        x, w = qkv_inputs(800 + M, M, K, N, 0)
        mats = [w]
    xs = torch.full((M, ldx), 7.0, dtype=torch.bfloat16, device="cuda")
    xs[:, :K] = x.cuda()
    ws = []
    for m in mats:
        t = torch.full((N, ldw), 7.0, dtype=torch.bfloat16, device="cuda")
        t[:, :K] = m.cuda()
        ws.append(t)
    y = torch.full((M, ldy), 3.0, dtype=torch.bfloat16, device="cuda")
    if kind == "gate-up":
        st = lib.fp_gate_up_silu_bf16(_p(xs), ldx, _p(ws[0]), ldw, _p(ws[1]), ldw, _p(y), ldy,
                                      M, N, K, stream)
    elif kind == "qkv":
        n_k = N // 6
        st = lib.fp_qkv_bf16(_p(xs), ldx, _p(ws[0]), ldw, _p(y), ldy, M, N - 2 * n_k, n_k, K, stream)
    else:
        st = lib.fp_linear_bf16(_p(xs), ldx, _p(ws[0]), ldw, _p(y), ldy, M, N, K, stream)
    assert st == 0, _lib.status_string(st)
    torch.cuda.synchronize()
    yc = y.cpu()
    assert torch.all(yc[:, N:] == 3.0), "output padding written"
    r = np.sort(np.random.default_rng(5).choice(M, min(M, 96), replace=False))
    if kind == "gate-up":
        out = ref.ref_gate_up_silu_full(bits(x)[r], bits(wg), bits(wu))
    elif kind == "qkv":
        out = ref.ref_qkv_full(bits(x)[r], bits(w), N - 2 * (N // 6), N // 6)
    else:
        out = ref.ref_linear(bits(x)[r], bits(w))
    p = ref.check_parity(bits(yc[:, :N].contiguous())[r], out)
    assert p.ok, (kind, M, p)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,M,K", [("qkv", 2048, 2560), ("gate-up", 2048, 2560),
                                      ("gate-up", 1300, 2560), ("gate-up", 2048, 64),
                                      ("gate-up", 2048, 192), ("qkv", 2048, 128)])
def test_int8_tiles_dequantise_once(kind, M, K):
    """The one-tile-per-CU kernel with int8 weights (each weight dequantised
    once per workgroup into LDS) on Qwen3-4B shapes, through the plain entry
    points (no workspace): QKV at 2048 rows is one round of 192 x 256 tiles,
    gate-up runs whole rounds of 256 x 256 tiles plus a 256 x 128 tail. The
    same k order as the bf16 kernels, so the outputs equal the bf16 call on
    the dequantised weights bit for bit; a row subset is checked against the
    oracle as well. K of 64, 128 and 192 gives tiles of 1, 2 and 3 k-steps
    (the dequantisation one step ahead reads stale staging on the last)."""
    from llms_amd import _lib
    from llms_amd import kernels as kern

    n_q, n_k, inter = 4096, 1024, 9728
    lib = _lib.capi()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = np.sort(np.random.default_rng(5).choice(M, 48, replace=False))
    if kind == "qkv":
        N = n_q + 2 * n_k
        x, w = qkv_inputs(900 + M, M, K, n_q, n_k)
        xd = x.cuda()
        q, s = kern.quantize_w8_per_row(w.cuda())
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        st = lib.fp_qkv_w8(_p(xd), K, _p(q), K, _p(s), _p(y), N, M, n_q, n_k, K, stream)
        assert st == 0, _lib.status_string(st)
        wd = kern.dequantize_w8(q, s)
        yb = torch.cat(kern.triton_fused_qkv(xd, wd, n_q=n_q, n_k=n_k), dim=-1)
        out = ref.ref_qkv_w8_full(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy(), n_q, n_k)
    else:
        x, wg, wu = ffn_inputs(900 + M, M, K, inter)
        xd = x.cuda()
        qg, sg = kern.quantize_w8_per_row(wg.cuda())
        qu, su = kern.quantize_w8_per_row(wu.cuda())
        y = torch.empty(M, inter, dtype=torch.bfloat16, device="cuda")
        st = lib.fp_gate_up_silu_w8(_p(xd), K, _p(qg), K, _p(sg), _p(qu), K, _p(su), _p(y), inter,
                                    M, inter, K, stream)
        assert st == 0, _lib.status_string(st)
        yb = kern.triton_fused_gate_up_silu(xd, kern.dequantize_w8(qg, sg), kern.dequantize_w8(qu, su))
        out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                           qu.cpu().numpy(), su.cpu().numpy())
    torch.cuda.synchronize()
    assert torch.equal(y, yb.reshape(M, -1)), f"{kind} M={M}: int8 tiles differ from bf16 on bf16(q*s)"
    p = ref.check_parity(bits(y.cpu())[rows], out)
    assert p.ok, (kind, M, p)
