"""GPU parity of the fused projections against the CPU oracle.

Mirrors the reference's kernel test ladder (tests/test_kernels_fused_ffn.py
and tests/test_kernels_fused_qkv.py: small bf16 shapes, Qwen3-4B shapes, N and
K tails, leading dims, head views, error messages) and adds the task's
configurations: Qwen3-0.6B decode, Qwen3-4B decode/spec-verify and prefill,
int8 weight-only, and the Qwen3-8B M sweep.

The bar (``oracle.ref.check_parity``): every output element within 2e-2 of
the oracle's admissible-rounding hull, rel-L2 <= 5e-3 against the oracle's
exact-rounding value. For large M a seeded subset of rows is checked (each
output row depends only on its own x row); size-independent properties
(determinism, row-permutation equivariance) run at full size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref
from tests._util import bits, ffn_inputs, gen, qkv_inputs, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda"

# Qwen3 layer shapes: (K, n_q, n_k, I)
QWEN3_0_6B = (1024, 2048, 1024, 3072)
QWEN3_4B = (2560, 4096, 1024, 9728)
QWEN3_8B = (4096, 4096, 1024, 12288)


def _kernels():
    from llms_amd import kernels

    return kernels


def _rows(M: int, limit: int = 192, seed: int = 0) -> np.ndarray:
    if M <= limit:
        return np.arange(M)
    r = np.random.default_rng(seed).choice(M, size=limit, replace=False)
    return np.sort(np.concatenate([r, [0, M - 1]]))


def _check(kernel_out: torch.Tensor, oracle_out: ref.OracleOut, label: str) -> ref.Parity:
    p = ref.check_parity(bits(kernel_out), oracle_out)
    print(f"{label}: {p}")
    assert p.ok, f"{label}: {p}"
    return p


def run_qkv(x, w, n_q, n_k):
    q, k, v = _kernels().triton_fused_qkv(x.to(DEV), w.to(DEV), n_q=n_q, n_k=n_k)
    return torch.cat([q, k, v], dim=-1).cpu()


def check_qkv(seed, M, K, n_q, n_k, w_std=0.02, label=""):
    x, w = qkv_inputs(seed, M, K, n_q, n_k, w_std=w_std)
    y = run_qkv(x, w, n_q, n_k)
    rows = _rows(M)
    out = ref.ref_qkv_full(bits(x)[rows], bits(w), n_q, n_k)
    return _check(y[rows], out, label or f"qkv M={M} K={K} n_q={n_q} n_k={n_k}")


def check_ffn(seed, M, K, N, w_std=0.02, label=""):
    x, wg, wu = ffn_inputs(seed, M, K, N, w_std=w_std)
    y = _kernels().triton_fused_gate_up_silu(x.to(DEV), wg.to(DEV), wu.to(DEV)).cpu()
    rows = _rows(M)
    out = ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu))
    return _check(y[rows], out, label or f"gate-up M={M} K={K} N={N}")


# ----- reference step 2: small bf16 shapes (weights N(0,1), as there) --------


@pytest.mark.parametrize("M,n_q,n_k,K", [(1, 128, 64, 192), (2, 128, 64, 192), (3, 160, 32, 192)])
def test_qkv_small(M, n_q, n_k, K):
    x, w = qkv_inputs(0, M, K, n_q, n_k, w_std=1.0)
    y = run_qkv(x, w, n_q, n_k)
    _check(y, ref.ref_qkv_full(bits(x), bits(w), n_q, n_k), f"qkv small {M},{n_q},{n_k},{K}")
    # the reference's own envelope: max|a-e| < 1e-2 * max|e| + 1e-2
    e = ref.ref_qkv_full(bits(x), bits(w), n_q, n_k).central
    assert np.abs(y.float().numpy() - e).max() < 1e-2 * np.abs(e).max() + 1e-2


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (2, 128, 128), (3, 160, 192)])
def test_gate_up_small(M, N, K):
    x, wg, wu = ffn_inputs(0, M, K, N, w_std=1.0)
    y = _kernels().triton_fused_gate_up_silu(x.to(DEV), wg.to(DEV), wu.to(DEV)).cpu()
    out = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))
    _check(y, out, f"gate-up small {M},{N},{K}")
    e = out.central
    assert np.abs(y.float().numpy() - e).max() < 1e-2 * np.abs(e).max() + 1e-2


# ----- committed golden vectors (tests/golden/fixtures.npz) -------------------


def test_golden_fixtures():
    """The HIP kernels reproduce the committed vectors of the reference's
    eager path: within the bar against the oracle hull, and max-abs <= 2e-2
    against the stored torch outputs themselves."""
    from pathlib import Path

    from tests._util import from_bits

    kern = _kernels()
    with np.load(Path(__file__).parent / "golden" / "fixtures.npz", allow_pickle=False) as z:
        fx = {k: z[k] for k in z.files}
    dev = lambda b: from_bits(b).to(DEV)  # noqa: E731
    n_q, n_k = int(fx["qkv_nq"]), int(fx["qkv_nk"])

    def both(y, stored, out, label):
        _check(y.cpu(), out, label)
        d = np.abs(ref.bf16_to_f32(bits(y)).astype(np.float64) - ref.bf16_to_f32(stored))
        assert d.max() <= ref.MAX_ABS_TOL, (label, d.max())

    for xk, yk in (("qkv_x", "qkv_y"), ("qkv3_x", "qkv3_y")):
        q, k, v = kern.triton_fused_qkv(dev(fx[xk]), dev(fx["qkv_w"]), n_q=n_q, n_k=n_k)
        both(torch.cat([q, k, v], -1), fx[yk], ref.ref_qkv_full(fx[xk], fx["qkv_w"], n_q, n_k), yk)
    for p in ("ffn", "ffn37"):
        y = kern.triton_fused_gate_up_silu(dev(fx[p + "_x"]), dev(fx[p + "_wg"]), dev(fx[p + "_wu"]))
        out = ref.ref_gate_up_silu_full(fx[p + "_x"], fx[p + "_wg"], fx[p + "_wu"])
        both(y, fx[p + "_y"], out, p)
    q, s = kern.quantize_w8_per_row(dev(fx["q8_w"]))
    np.testing.assert_array_equal(q.cpu().numpy(), fx["q8_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), fx["q8_s"])
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    y = kern.fused_gate_up_silu_w8(dev(fx["w8_x"]), t(fx["w8_qg"]), t(fx["w8_sg"]), t(fx["w8_qu"]), t(fx["w8_su"]))
    out = ref.ref_gate_up_silu_w8_full(fx["w8_x"], fx["w8_qg"], fx["w8_sg"], fx["w8_qu"], fx["w8_su"])
    both(y, fx["w8_y"], out, "w8 gate-up")
    q, k, v = kern.fused_qkv_w8(dev(fx["w8q_x"]), t(fx["w8q_q"]), t(fx["w8q_s"]), n_q=n_q, n_k=n_k)
    out = ref.ref_qkv_w8_full(fx["w8q_x"], fx["w8q_q"], fx["w8q_s"], n_q, n_k)
    both(torch.cat([q, k, v], -1), fx["w8q_y"], out, "w8 qkv")


# ----- Qwen3-0.6B decode (the CPU-runnable configuration) --------------------


def test_qwen3_0_6b_decode():
    K, n_q, n_k, I = QWEN3_0_6B
    check_qkv(0, 1, K, n_q, n_k, label="0.6B qkv M=1")
    check_ffn(0, 1, K, I, label="0.6B gate-up M=1")


# ----- reference step 3 + Qwen3-4B decode / spec-verify ----------------------


@pytest.mark.parametrize("M", [1, 3, 4, 5, 8])
def test_qwen3_4b_qkv_decode(M):
    K, n_q, n_k, _ = QWEN3_4B
    check_qkv(M, M, K, n_q, n_k)


@pytest.mark.parametrize("M", [1, 3, 4, 5, 8, 12, 16])
def test_qwen3_4b_gate_up_decode(M):
    K, _, _, I = QWEN3_4B
    check_ffn(M, M, K, I)


@pytest.mark.parametrize("M", [8, 16, 17, 32, 33, 47])
def test_gate_up_verify_tiles_ragged(M):
    """The 96-row split-K tiles of wide short-K gate-up at 8-47 rows (16, 32
    and 64 x rows) with a partial last tile (9700 outputs: 48 per tile) and
    partial x tiles, against the oracle."""
    check_ffn(90 + M, M, 2560, 9700, label=f"gate-up verify tiles M={M} N=9700")


def _bf16_from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b.astype(np.uint16)).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("M", [1, 512], ids=["row-kernel", "mfma-grid"])
def test_gate_up_epilogue_every_bf16_g(M):
    """Every finite bf16 value of g goes through the silu epilogue: x rows are
    one-hot and Wu is all ones, so output (m, n) is bf16(silu(g)) with g one
    chosen weight. M = 1 runs the decode row kernel over 65024 outputs; M = 512
    with K = 64 runs the MFMA prefill grid, g[m, n] = Wg[n, m % 64]. Checked
    against the oracle (silu in float64, hull of one fp32 silu rounding)."""
    b = np.arange(65536, dtype=np.uint32)
    vals = b[((b >> 7) & 0xFF) != 0xFF].astype(np.uint16)  # the 65024 finite bf16
    one = np.uint16(0x3F80)
    K = 64
    if M == 1:
        N = vals.size
        wg = np.zeros((N, K), np.uint16)
        wg[:, 0] = vals
        wu = np.zeros((N, K), np.uint16)
        wu[:, 0] = one
        x = np.zeros((1, K), np.uint16)
        x[0, 0] = one
    else:
        N = -(-vals.size // K)
        flat = np.zeros(N * K, np.uint16)
        flat[: vals.size] = vals
        wg = flat.reshape(N, K)
        wu = np.full((N, K), one, np.uint16)
        x = np.zeros((M, K), np.uint16)
        x[np.arange(M), np.arange(M) % K] = one
    xt, wgt, wut = _bf16_from_bits(x), _bf16_from_bits(wg), _bf16_from_bits(wu)
    y = _kernels().triton_fused_gate_up_silu(xt.to(DEV), wgt.to(DEV), wut.to(DEV)).cpu()
    _check(y, ref.ref_gate_up_silu_full(x, wg, wu), f"silu epilogue, all bf16 g, M={M}")


def test_gate_up_non_pow2_N():
    """N-tail: N=9700 (reference test_triton_bf16_non_pow2_N), and a tile-tail
    N for the prefill kernel."""
    check_ffn(1, 1, 2560, 9700, label="gate-up N=9700 M=1")
    check_ffn(1, 300, 2560, 9700, label="gate-up N=9700 M=300")
    check_ffn(2, 65, 256, 37, label="gate-up N=37 M=65")


def test_qkv_non_pow2_K():
    """K-tail: K=2541 (reference test_triton_qkv_bf16_non_pow2_K): rows are
    only 2-byte aligned, so the unaligned load path runs."""
    check_qkv(1, 1, 2541, 4096, 1024, label="qkv K=2541 M=1")
    check_qkv(1, 7, 2541, 4096, 1024, label="qkv K=2541 M=7")
    check_qkv(1, 130, 2541, 512, 128, label="qkv K=2541 M=130")
    check_ffn(3, 3, 2536, 512, label="gate-up K=2536 (K % 32 != 0) M=3")
    check_ffn(3, 100, 2536, 512, label="gate-up K=2536 M=100")


def test_preserves_leading_dims_and_head_views():
    K = _kernels()
    g = gen(2)
    x = randn_bf16(g, 2, 3, 64).to(DEV)
    wg = randn_bf16(g, 128, 64, std=0.1).to(DEV)
    wu = randn_bf16(g, 128, 64, std=0.1).to(DEV)
    y = K.triton_fused_gate_up_silu(x, wg, wu)
    assert y.shape == (2, 3, 128)
    out = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))
    _check(y.cpu(), out, "gate-up (2,3,64)")

    B, T, H, Hkv, D, Kd = 1, 5, 32, 8, 128, 2560
    x = randn_bf16(gen(3), B, T, Kd).to(DEV)
    w = randn_bf16(gen(4), (H + 2 * Hkv) * D, Kd, std=0.02).to(DEV)
    q, k, v = K.triton_fused_qkv(x, w, n_q=H * D, n_k=Hkv * D)
    assert q.shape == (B, T, H * D) and k.shape == (B, T, Hkv * D) and v.shape == (B, T, Hkv * D)
    assert q.view(B, T, H, D).shape == (B, T, H, D)
    assert k.view(B, T, Hkv, D).shape == (B, T, Hkv, D)
    assert v.view(B, T, Hkv, D).shape == (B, T, Hkv, D)
    # zero-copy split: the three are views of one buffer
    assert q.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()


def test_strided_x_and_empty_input():
    K = _kernels()
    g = gen(5)
    base = randn_bf16(g, 6, 2 * 256).to(DEV)
    x = base[:, :256]  # row stride 512, inner stride 1
    wg = randn_bf16(g, 96, 256, std=0.05).to(DEV)
    wu = randn_bf16(g, 96, 256, std=0.05).to(DEV)
    y = K.triton_fused_gate_up_silu(x, wg, wu).cpu()
    _check(y, ref.ref_gate_up_silu_full(bits(x.contiguous()), bits(wg), bits(wu)), "strided x")
    xt = randn_bf16(g, 256, 6).to(DEV).t()  # inner stride != 1 -> copied
    y = K.triton_fused_gate_up_silu(xt, wg, wu).cpu()
    _check(y, ref.ref_gate_up_silu_full(bits(xt.contiguous()), bits(wg), bits(wu)), "transposed x")
    e = torch.zeros(0, 256, dtype=torch.bfloat16, device=DEV)
    assert K.triton_fused_gate_up_silu(e, wg, wu).shape == (0, 96)
    w = torch.cat([wg, wu])
    q, k, v = K.triton_fused_qkv(e, w, n_q=128, n_k=32)
    assert q.shape == (0, 128) and k.shape == (0, 32)


def test_dtype_and_device_errors():
    K = _kernels()
    x = torch.randn(2, 64, device=DEV)
    w = torch.randn(96, 64, device=DEV)
    with pytest.raises(TypeError, match="bfloat16"):
        K.triton_fused_qkv(x, w, n_q=64, n_k=16)
    xb = x.to(torch.bfloat16)
    with pytest.raises(ValueError, match="same device"):
        K.triton_fused_qkv(xb, w.to(torch.bfloat16).cpu(), n_q=64, n_k=16)


# ----- Qwen3-4B prefill (MFMA regime) ------------------------------------------


@pytest.mark.parametrize("M", [512, 2048])
def test_qwen3_4b_prefill(M):
    K, n_q, n_k, I = QWEN3_4B
    check_qkv(10 + M, M, K, n_q, n_k, label=f"4B qkv M={M}")
    check_ffn(10 + M, M, K, I, label=f"4B gate-up M={M}")


def test_qwen3_4b_prefill_8192_rows():
    K, n_q, n_k, I = QWEN3_4B
    check_qkv(8192, 8192, K, n_q, n_k, label="4B qkv M=8192 (row subset)")
    check_ffn(8192, 8192, K, I, label="4B gate-up M=8192 (row subset)")


# Row counts whose prefill grids differ. Qwen3-4B: 64 x 64 tiles with
# 128-wide k-steps (QKV 160 and 256 rows), 96 x 128 (QKV 384) and 128 x 128
# (QKV 640) with 128-wide k-steps, 64 x 128 (gate-up 128 rows), 128 x 128
# (gate-up 384, QKV 768), 192 x 256 (gate-up 512, QKV 1536 and 2048),
# 256 x 256 (gate-up 1536) and 320 x 256 tiles (gate-up 1024 and 2048, QKV
# 3072), and whole 256 x 256 rounds followed by a 128 x 128 tail launch (QKV
# 3800; at 4096 rows two rounds of 192 x 256 run instead). Qwen3-0.6B: 64 x 64 (gate-up 96 and 320, QKV 128) and 128 x 128
# (gate-up 512, QKV 640) with 128-wide k-steps, 128 x 128 (gate-up 1024, QKV
# 1536 and 3072) and 192 x 256 (gate-up 2048).
PLAN_ROWS = {"gate_up": (QWEN3_4B, 2048, [128, 384, 512, 1024, 1536]),
             "qkv": (QWEN3_4B, 3800, [160, 256, 384, 640, 768, 1536, 2048, 3072]),
             "gate_up_0.6b": (QWEN3_0_6B, 2048, [96, 320, 512, 1024]),
             "qkv_0.6b": (QWEN3_0_6B, 3072, [128, 640, 1536])}


@pytest.mark.parametrize("kind", list(PLAN_ROWS))
def test_prefill_rows_independent_of_grid_plan(kind):
    """Every unsplit prefill grid plan (64- or 128-wide k-steps, one launch or
    two) contracts each output over k in the same order, so a row's bits do
    not depend on how many rows the call has (and with it which tiles, or
    which of two launches, computed it). The largest call is checked against
    the oracle on a row subset; the smaller calls must reproduce its rows bit
    for bit."""
    (K, n_q, n_k, I), M_full, Ms = PLAN_ROWS[kind]
    if kind.startswith("qkv"):
        x, w = qkv_inputs(77, M_full, K, n_q, n_k)
        xd, wd = x.to(DEV), w.to(DEV)

        def run(xx):
            q, k, v = _kernels().triton_fused_qkv(xx, wd, n_q=n_q, n_k=n_k)
            return torch.cat([q, k, v], dim=-1).cpu()
        y = run(xd)
        rows = _rows(M_full)
        _check(y[rows], ref.ref_qkv_full(bits(x)[rows], bits(w), n_q, n_k), f"{kind} M={M_full}")
    else:
        x, wg, wu = ffn_inputs(77, M_full, K, I)
        xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)

        def run(xx):
            return _kernels().triton_fused_gate_up_silu(xx, wgd, wud).cpu()
        y = run(xd)
        rows = _rows(M_full)
        _check(y[rows], ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu)),
               f"{kind} M={M_full}")
    for M in Ms:
        ym = run(xd[:M].contiguous())
        assert torch.equal(ym.view(torch.int16), y[:M].view(torch.int16)), f"{kind} M={M}"


@pytest.mark.parametrize("M,K,N", [
    (512, 2560, 9728),    # Qwen3-4B: one round of 160 x 256 four-wave tiles
    (500, 2560, 9700),    # the same, partial tiles in M and N
    (512, 4096, 12288),   # Qwen3-8B: 192 x 256 tiles with four waves, 64 k-steps
    (500, 4096, 12200),   # the same, partial tiles in M and N
    (2048, 1024, 3072),   # Qwen3-0.6B, 16 k-steps: eight waves
    (512, 2496, 9728)])   # 39 k-steps (odd): 192 x 256 with eight waves
def test_gate_up_four_wave_tiles(M, K, N):
    """bf16 gate-up calls planned on 192 x 256 tiles run four waves per
    workgroup (accumulators in AGPRs) when the k-step count is even and at
    least 32, else eight, and a round of 160 x 256 tiles four: all against
    the oracle, and repeated calls bit-identical (the tile order and the k
    order do not depend on timing)."""
    x, wg, wu = ffn_inputs(230 + M, M, K, N)
    xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)
    y = _kernels().triton_fused_gate_up_silu(xd, wgd, wud).cpu()
    rows = _rows(M)
    _check(y[rows], ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu)),
           f"gate-up 192 x 256 M={M} K={K} N={N}")
    y2 = _kernels().triton_fused_gate_up_silu(xd, wgd, wud).cpu()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("case", ["gate-up 8b", "gate-up ragged", "qkv"])
def test_192x128_four_wave_tiles(case):
    """Calls planned as one round of 192 x 128 tiles with four waves (240-256
    tiles): against the oracle on a row subset, and bit-identical to the
    same rows computed by a larger call on another plan (192 x 256 or 128 x
    128 tiles: the same k-steps in the same order)."""
    if case == "qkv":
        K, n_q, n_k, M, M2 = 2560, 2048, 512, 2048, 1536
        x, w = qkv_inputs(260, M, K, n_q, n_k)
        xd, wd = x.to(DEV), w.to(DEV)

        def run(xx):
            q, k, v = _kernels().triton_fused_qkv(xx, wd, n_q=n_q, n_k=n_k)
            return torch.cat([q, k, v], dim=-1).cpu()
        y = run(xd)
        rows = _rows(M)
        _check(y[rows], ref.ref_qkv_full(bits(x)[rows], bits(w), n_q, n_k), f"192x128 {case}")
        y2 = run(xd[:M2].contiguous())
        assert torch.equal(y2.view(torch.int16), y[:M2].view(torch.int16))
        return
    K, N, M, M2 = (4096, 12288, 256, 512) if case == "gate-up 8b" else (4096, 12200, 250, 500)
    x, wg, wu = ffn_inputs(270 + M, M2, K, N)
    xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)
    y2 = _kernels().triton_fused_gate_up_silu(xd, wgd, wud).cpu()
    y = _kernels().triton_fused_gate_up_silu(xd[:M].contiguous(), wgd, wud).cpu()
    rows = _rows(M, limit=96)
    _check(y[rows], ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu)), f"192x128 {case}")
    assert torch.equal(y.view(torch.int16), y2[:M].view(torch.int16))


@pytest.mark.parametrize("op,M,M2,K,N", [
    ("gate-up", 2048, 1500, 2560, 1216),  # 128 x 160 tiles; 1500 rows: 128 x 128
    ("gate-up", 2000, 1500, 2560, 1216),  # 128 x 160, partial last m-tile
    ("gate-up", 512, 1024, 2560, 4864),   # 160 x 128 (one wave column); 1024 rows: 192 x 256
    ("gate-up", 512, 1024, 2560, 9728),   # 160 x 256, 64-wide steps; 1024 rows: 320 x 256
    ("qkv", 1024, 768, 2560, 5000),       # 160 x 128; 768 rows: 128 x 128
    ("qkv", 2048, 1024, 2560, 2432)])     # 128 x 160; 1024 rows: 128 x 128
def test_four_wave_128_wide_steps(op, M, M2, K, N):
    """One round of four-wave tiles with 128-wide k-steps (128 x 160 and
    160 x 128 planned on 240-256 tiles; 128 x 128 one-round grids): against
    the oracle on a row subset, and bit-identical to the same rows computed
    on the other plan of a call with M2 rows."""
    Mx = max(M, M2)
    if op == "qkv":
        n_k = N // 6
        n_q = N - 2 * n_k
        x, w = qkv_inputs(280 + M, Mx, K, n_q, n_k)
        xd, wd = x.to(DEV), w.to(DEV)

        def run(rows):
            q, k, v = _kernels().triton_fused_qkv(xd[:rows].contiguous(), wd, n_q=n_q, n_k=n_k)
            return torch.cat([q, k, v], dim=-1).cpu()
        y = run(M)
        sub = _rows(M)
        _check(y[sub], ref.ref_qkv_full(bits(x)[sub], bits(w), n_q, n_k), f"{op} M={M} N={N}")
    else:
        x, wg, wu = ffn_inputs(290 + M, Mx, K, N)
        xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)

        def run(rows):
            return _kernels().triton_fused_gate_up_silu(xd[:rows].contiguous(), wgd, wud).cpu()
        y = run(M)
        sub = _rows(M)
        _check(y[sub], ref.ref_gate_up_silu_full(bits(x)[sub], bits(wg), bits(wu)),
               f"{op} M={M} N={N}")
    y2 = run(M2)
    r = min(M, M2)
    assert torch.equal(y[:r].view(torch.int16), y2[:r].view(torch.int16)), f"{op} M={M} vs {M2}"


@pytest.mark.parametrize("op,M,M2,K,N", [
    ("qkv", 512, 1024, 2560, 3072),      # 96 x 64, three stages (256 tiles); 1024 rows: 96 x 128
    ("qkv", 500, 1024, 2560, 3000),      # 96 x 64, partial last tiles in M and N
    ("qkv", 256, 1024, 4096, 6144),      # 96 x 64 over 32 k-steps
    ("qkv", 512, 1024, 1280, 3072),      # 96 x 64, 10 k-steps (10 % 3 = 1)
    ("qkv", 512, 1024, 1408, 3072),      # 96 x 64, 11 k-steps (11 % 3 = 2)
    ("qkv", 512, 2048, 4096, 4096),      # 64 x 128, three stages
    ("gate-up", 512, 2048, 4096, 1536),  # 96 x 64, one wave column
    ("gate-up", 500, 2048, 2560, 1200),  # 96 x 64, ragged
    ("gate-up", 512, 2048, 2560, 2000),  # 64 x 128, one wave column
    ("gate-up", 512, 2048, 4096, 3072),  # 96 x 128, one wave column, two stages
    ("gate-up", 500, 2048, 2560, 2400)])  # 96 x 128, ragged
def test_small_round_tiles(op, M, M2, K, N):
    """One round of small four-wave tiles (96 x 64 and 64 x 128 with three
    LDS stages, gate-up 96 x 128): against the oracle on a row subset, and
    bit-identical to the same rows computed on the other plan of a call with
    M2 rows."""
    test_four_wave_128_wide_steps(op, M, M2, K, N)


@pytest.mark.parametrize("model", ["4b", "8b"])
@pytest.mark.parametrize("M", [1, 4, 8, 64, 512, 2048])
def test_tp8_shards(model, M):
    """The per-GPU shard of TP = 8 (QKV: 4 q heads + 1 k + 1 v head, 768
    columns; gate-up: I / 8 columns of Wg and of Wu), the shapes one GPU runs
    in a tensor-parallel layer, against the oracle."""
    K, n_q, n_k, I = QWEN3_4B if model == "4b" else QWEN3_8B
    check_qkv(240 + M, M, K, n_q // 8, n_k // 8, label=f"{model} tp8 qkv M={M}")
    check_ffn(250 + M, M, K, I // 8, label=f"{model} tp8 gate-up M={M}")


@pytest.mark.parametrize("M", [17, 64, 65, 100, 256])
def test_regime_boundaries(M):
    """Around the streaming / tiled switch and partial M tiles."""
    check_qkv(20 + M, M, 1024, 512, 128)
    check_ffn(20 + M, M, 1024, 640)


@pytest.mark.parametrize("M,K", [(9, 1024), (16, 64), (23, 320), (33, 2560), (48, 128),
                                 (64, 4096), (65, 1024), (130, 2560), (256, 320)])
def test_split_k_regime(M, K):
    """9 <= M <= 64 (and QKV-sized N up to 256 rows) run the split-K tiles,
    each wave of a workgroup with its own k-steps (64 k each, interleaved)
    and a fixed-order reduction: a single k-step (waves without work), k-step
    counts that do not divide evenly over the waves, x tiles of 16..64 rows
    with ragged M, and N not a multiple of the 16/32-output tiles."""
    check_qkv(80 + M, M, K, 256 + 48, 40, label=f"qkv M={M} K={K} N=384")
    check_ffn(81 + M, M, K, 100, label=f"gate-up M={M} K={K} N=100")
    if M <= 64:
        check_ffn(82 + M, M, K, 1000, label=f"gate-up M={M} K={K} N=1000")


@pytest.mark.parametrize("M,K,N", [(1, 8, 5), (1, 520, 33), (1, 2536, 9701), (1, 16384, 64),
                                   (1, 16392, 24), (1, 32768, 24), (1, 32776, 16), (1, 4096, 1),
                                   (2, 8, 7), (2, 2536, 1001), (2, 8192, 40), (2, 9728, 24),
                                   (2, 16384, 24), (2, 16392, 16)])
def test_row_streaming_edges(M, K, N):
    """M <= 2 bf16 runs the row-streaming kernel (one wave per weight row, K
    in 512-element chunks, M x rows in LDS up to 64 KiB, i.e. M * K <=
    32768): tiny and ragged K (the last chunk partly past the row), N not a
    multiple of the rows per workgroup, the largest K it takes and the first
    K it hands to the streaming kernel."""
    n_q = max(N - 2 * (N // 4), 1)
    n_k = (N - n_q) // 2
    check_qkv(40 + K + M, M, K, n_q, n_k, label=f"qkv M={M} K={K} N={n_q + 2 * n_k}")
    check_ffn(41 + K + M, M, K, N, label=f"gate-up M={M} K={K} N={N}")


# ----- int8 weight-only --------------------------------------------------------


def _quant(w):
    q, s = _kernels().quantize_w8_per_row(w.to(DEV))
    qo, so = ref.quantize_w8_per_row(bits(w))
    np.testing.assert_array_equal(q.cpu().numpy(), qo)   # device packing == oracle, bit-exact
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    return q, s


@pytest.mark.parametrize("M", [1, 4, 2048])
def test_qwen3_4b_int8(M):
    K, n_q, n_k, I = QWEN3_4B
    kern = _kernels()
    x, w = qkv_inputs(30 + M, M, K, n_q, n_k)
    q, s = _quant(w)
    yq, yk, yv = kern.fused_qkv_w8(x.to(DEV), q, s, n_q=n_q, n_k=n_k)
    y = torch.cat([yq, yk, yv], -1).cpu()
    rows = _rows(M)
    out = ref.ref_qkv_w8_full(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy(), n_q, n_k)
    _check(y[rows], out, f"4B int8 qkv M={M}")

    x, wg, wu = ffn_inputs(40 + M, M, K, I)
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                       qu.cpu().numpy(), su.cpu().numpy())
    _check(y[rows], out, f"4B int8 gate-up M={M}")


@pytest.mark.parametrize("M", [1, 4, 16, 100])
def test_int8_dequant_bit_exact(M):
    """In-register dequantisation is bit-exact: with one-hot x rows the QKV
    output is a single dequantised weight, y[m, n] = bf16(q[n, k_m] * s[n])
    (a one-term sum is exact, then rounded to bf16, which it already is), so it
    must equal the oracle's dequant_w8 column bit for bit — through the row
    kernel (M = 1 and 4 on this 384-output shape) and the split-K tiles (M = 16
    from the streaming dispatch, M = 100 from the tiled one)."""
    K, N = 2560, 384
    _, w = qkv_inputs(70 + M, 1, K, N - 128, 64, w_std=0.05)
    q, s = _quant(w)
    deq = ref.dequant_w8(q.cpu().numpy(), s.cpu().numpy())            # [N, K] bf16 bits
    ks = np.random.default_rng(M).choice(K, size=M, replace=False)
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    x[np.arange(M), ks] = 1.0
    yq, yk, yv = _kernels().fused_qkv_w8(x.to(DEV), q, s, n_q=N - 128, n_k=64)
    y = bits(torch.cat([yq, yk, yv], -1).cpu())
    np.testing.assert_array_equal(y, deq[:, ks].T)


@pytest.mark.parametrize("K", [1040, 2560, 4096, 4112])
def test_int8_gate_up_one_row_bit_exact(K):
    """int8 gate-up at one x row runs the 8-byte-chunk row kernel (x from L2
    up to K = 2560, staged in LDS above; 1040 and 4112 leave a partial last
    512-k chunk). With one-hot x each output is silu(g) * u of single
    dequantised weights, so the kernel must equal the oracle's exact rounding
    bit for bit; with random x it must pass the parity bar."""
    kern = _kernels()
    N = 100
    x, wg, wu = ffn_inputs(880 + K, 1, K, N, w_std=0.05)
    wg[7] = 0  # an all-zero row: s = 0, q = 0
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    args = (qg.cpu().numpy(), sg.cpu().numpy(), qu.cpu().numpy(), su.cpu().numpy())
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    _check(y, ref.ref_gate_up_silu_w8_full(bits(x), *args), f"int8 gate-up M=1 K={K}")
    k = int(np.random.default_rng(K).integers(K))
    x1 = torch.zeros(1, K, dtype=torch.bfloat16)
    x1[0, k] = 1.0
    y = kern.fused_gate_up_silu_w8(x1.to(DEV), qg, sg, qu, su).cpu()
    p = _check(y, ref.ref_gate_up_silu_w8_full(bits(x1), *args), f"int8 gate-up one-hot K={K}")
    assert p.n_differ == 0, p


@pytest.mark.parametrize("M,K,N", [(3, 2560, 6144), (8, 2560, 6150), (16, 4096, 6144),
                                   (5, 4096, 5000), (11, 2048, 6136), (24, 4096, 6144),
                                   (33, 2560, 6150), (64, 4096, 5000), (50, 2048, 6144)])
def test_qkv_verify_24_row_tiles(M, K, N):
    """bf16 QKV at 3-64 rows with 4096 < N <= 6144 runs split-K tiles of 24
    weight rows (at most 256 of them; 16, 32 or 64 x rows); their second MFMA
    block reaches 8 rows past the tile, which must never be stored. Whole
    tiles (6144), a partial last tile (6150, 5000, 6136), partial x tiles
    (33, 50) and K = 2048, 2560, 4096, against the oracle."""
    n_k = 512
    x, w = qkv_inputs(1500 + M, M, K, N - 2 * n_k, n_k)
    q, k, v = _kernels().triton_fused_qkv(x.to(DEV), w.to(DEV), n_q=N - 2 * n_k, n_k=n_k)
    y = torch.cat([q, k, v], -1).cpu()
    _check(y, ref.ref_qkv_full(bits(x), bits(w), N - 2 * n_k, n_k), f"qkv M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [2, 3, 5, 8, 13, 16])
def test_int8_verify_rows_qwen3_4b(M):
    """int8 at 2-16 rows with K = 2560 (x staged once per workgroup, every
    weight load in flight): Qwen3-4B-sized QKV and gate-up against the oracle,
    with output widths that leave a partial last block of 16 rows (6150 and
    9732) and x as a row-strided view; then one-hot x rows, whose QKV outputs
    are single dequantised weights, y[m, n] = bf16(q[n, k_m] * s[n]), equal to
    the oracle's dequant_w8 bit for bit."""
    K, n_q, n_k, I = QWEN3_4B
    kern = _kernels()
    x, w = qkv_inputs(1300 + M, M, K, n_q + 6, n_k, w_std=0.05)
    q, s = _quant(w)
    full = torch.zeros(M, K + 24, dtype=torch.bfloat16)
    full[:, :K] = x
    xd = full.to(DEV)[:, :K]
    yq, yk, yv = kern.fused_qkv_w8(xd, q, s, n_q=n_q + 6, n_k=n_k)
    y = torch.cat([yq, yk, yv], -1).cpu()
    qn, sn = q.cpu().numpy(), s.cpu().numpy()
    _check(y, ref.ref_qkv_w8_full(bits(x), qn, sn, n_q + 6, n_k), f"int8 qkv M={M} N=6150")

    ks = np.random.default_rng(M).choice(K, size=M, replace=False)
    x1 = torch.zeros(M, K, dtype=torch.bfloat16)
    x1[np.arange(M), ks] = 1.0
    yq, yk, yv = kern.fused_qkv_w8(x1.to(DEV), q, s, n_q=n_q + 6, n_k=n_k)
    np.testing.assert_array_equal(bits(torch.cat([yq, yk, yv], -1).cpu()),
                                  ref.dequant_w8(qn, sn)[:, ks].T)

    x, wg, wu = ffn_inputs(1400 + M, M, K, I + 4)
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    full[:, :K] = x
    xd = full.to(DEV)[:, :K]
    y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su).cpu()
    out = ref.ref_gate_up_silu_w8_full(bits(x), qg.cpu().numpy(), sg.cpu().numpy(),
                                       qu.cpu().numpy(), su.cpu().numpy())
    _check(y, out, f"int8 gate-up M={M} N=9732")


@pytest.mark.parametrize("M", [2, 3, 16, 33, 64, 100, 128])
def test_int8_split_k_tiles(M):
    """The int8 split-K tiles (weights land in LDS as int8, each lane
    dequantises its MFMA fragment): gate-up, QKV and the plain projection with
    output counts that leave partial tiles, an all-zero weight row, and for the
    projection both a short K (split-K from 5 rows) and a long K (split-K up to
    64 rows, then the split across workgroups or the prefill tiles)."""
    kern = _kernels()
    K = 2048
    x, wg, wu = ffn_inputs(500 + M, M, K, 1000)
    wg[7] = 0
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    _check(y, ref.ref_gate_up_silu_w8_full(bits(x), qg.cpu().numpy(), sg.cpu().numpy(),
                                           qu.cpu().numpy(), su.cpu().numpy()),
           f"int8 split-K gate-up M={M} N=1000")
    n_q, n_k = 256, 72
    x, w = qkv_inputs(510 + M, M, K, n_q, n_k)
    w[5] = 0
    q, s = _quant(w)
    yq, yk, yv = kern.fused_qkv_w8(x.to(DEV), q, s, n_q=n_q, n_k=n_k)
    _check(torch.cat([yq, yk, yv], -1).cpu(),
           ref.ref_qkv_w8_full(bits(x), q.cpu().numpy(), s.cpu().numpy(), n_q, n_k),
           f"int8 split-K qkv M={M} N={n_q + 2 * n_k}")
    for Kl, N in ((4096, 300), (9728, 264)):
        x, w = qkv_inputs(520 + M + Kl, M, Kl, N, 0)
        q, s = _quant(w)
        y = kern.fused_linear_w8(x.to(DEV), q, s).cpu()
        _check(y, ref.ref_linear_w8(bits(x), q.cpu().numpy(), s.cpu().numpy()),
               f"int8 linear M={M} K={Kl} N={N}")


@pytest.mark.parametrize("M", [17, 32, 40, 64, 65, 96, 100, 112, 113, 128])
def test_int8_split_k_wide_gate_up_tiles(M):
    """The int8 split-K tiles of 96 weight rows (48 outputs) that wide
    gate-up outputs take from 17 rows: x tiles of 32, 48, 64, 96 and 112 rows
    with 4 waves and 128 rows with 3, ragged outputs (9700 columns: a partial
    last tile), an all-zero weight row, the cross-wave sum in passes (the
    partials of the larger tiles exceed one LDS stage). Checked against the
    oracle on a row subset and for repeatability."""
    kern = _kernels()
    K, N = 2560, 9700
    x, wg, wu = ffn_inputs(540 + M, M, K, N)
    wu[17] = 0
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    xd = x.to(DEV)
    y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su)
    assert torch.equal(y.view(torch.int16), kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su).view(torch.int16))
    rows = _rows(M, limit=40)
    _check(y.cpu()[rows], ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                                       qu.cpu().numpy(), su.cpu().numpy()),
           f"int8 wide split-K gate-up M={M} N={N}")


@pytest.mark.parametrize("M,K,N", [(129, 2560, 9728), (200, 2560, 9700), (256, 4096, 12288)])
def test_int8_gate_up_192x128_tiles(M, K, N):
    """int8 gate-up at 129-256 rows on one round of 192 x 128 dequantise-once
    tiles (Qwen3-4B: 204 tiles, ragged outputs; Qwen3-8B: 256): bit-identical
    to the bf16 call on the dequantised weights (the same k order), and a row
    subset against the oracle."""
    kern = _kernels()
    x, wg, wu = ffn_inputs(560 + M, M, K, N)
    xd = x.to(DEV)
    qg, sg = kern.quantize_w8_per_row(wg.to(DEV))
    qu, su = kern.quantize_w8_per_row(wu.to(DEV))
    y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su)
    yb = kern.triton_fused_gate_up_silu(xd, kern.dequantize_w8(qg, sg), kern.dequantize_w8(qu, su))
    assert torch.equal(y.view(torch.int16), yb.view(torch.int16)), f"int8 192 x 128 M={M} N={N}"
    rows = _rows(M, limit=32)
    _check(y.cpu()[rows], ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                                       qu.cpu().numpy(), su.cpu().numpy()),
           f"int8 gate-up 192 x 128 M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [129, 300, 1024])
def test_int8_gemm_in_register(M):
    """The prefill gemm with int8 weight tiles dequantised in registers:
    gate-up with a partial last tile and an all-zero weight row, QKV with more
    than 4096 outputs, and the dequantisation bit for bit (one-hot x rows give
    single dequantised weights)."""
    kern = _kernels()
    K = 2560
    x, wg, wu = ffn_inputs(600 + M, M, K, 1000)
    wg[11] = 0
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    rows = _rows(M, limit=96)
    _check(y[rows], ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                                 qu.cpu().numpy(), su.cpu().numpy()),
           f"int8 gemm gate-up M={M} N=1000")
    if M > 512:
        return
    n_q, n_k = 4096, 128
    _, w = qkv_inputs(610 + M, 1, K, n_q, n_k, w_std=0.05)
    q, s = _quant(w)
    deq = ref.dequant_w8(q.cpu().numpy(), s.cpu().numpy())
    ks = np.random.default_rng(M).choice(K, size=M, replace=False)
    xo = torch.zeros(M, K, dtype=torch.bfloat16)
    xo[np.arange(M), ks] = 1.0
    yq, yk, yv = kern.fused_qkv_w8(xo.to(DEV), q, s, n_q=n_q, n_k=n_k)
    np.testing.assert_array_equal(bits(torch.cat([yq, yk, yv], -1).cpu()), deq[:, ks].T)


def test_int8_tails_and_zero_rows():
    kern = _kernels()
    for M, K, N in [(3, 2541, 100), (70, 2541, 100), (5, 1040, 48), (90, 1040, 48),
                    (1, 16, 5), (1, 1040, 33), (1, 2541, 9), (1, 16384, 20), (1, 16400, 7),
                    (2, 1040, 33), (3, 2560, 17), (4, 4096, 9), (4, 4112, 5),
                    (1, 32768, 9), (1, 32784, 5), (2, 16384, 7), (2, 16400, 5),
                    (3, 8192, 5), (4, 8192, 9), (4, 8208, 5)]:
        x, wg, wu = ffn_inputs(M + K, M, K, N)
        wg[3] = 0  # an all-zero row: s = 0, q = 0
        qg, sg = _quant(wg)
        qu, su = _quant(wu)
        y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
        out = ref.ref_gate_up_silu_w8_full(bits(x), qg.cpu().numpy(), sg.cpu().numpy(),
                                           qu.cpu().numpy(), su.cpu().numpy())
        _check(y, out, f"int8 gate-up M={M} K={K} N={N}")


# ----- Qwen3-8B M sweep, bf16 and int8 -----------------------------------------


@pytest.mark.parametrize("M", [1, 4, 16, 64, 256, 4096])
def test_qwen3_8b_sweep(M):
    K, n_q, n_k, I = QWEN3_8B
    check_qkv(50 + M, M, K, n_q, n_k, label=f"8B qkv M={M}")
    check_ffn(50 + M, M, K, I, label=f"8B gate-up M={M}")


@pytest.mark.parametrize("M", [1, 4, 16, 64, 256, 4096])
def test_qwen3_8b_int8(M):
    """BASELINE's Qwen3-8B sweep with int8 weights, both projections, against
    the dequantise-then-matmul oracle (a seeded subset of rows at large M)."""
    K, n_q, n_k, I = QWEN3_8B
    kern = _kernels()
    rows = _rows(M)
    x, w = qkv_inputs(80 + M, M, K, n_q, n_k)
    q, s = _quant(w)
    y = torch.cat(kern.fused_qkv_w8(x.to(DEV), q, s, n_q=n_q, n_k=n_k), dim=-1).cpu()
    out = ref.ref_qkv_w8_full(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy(), n_q, n_k)
    _check(y[rows], out, f"8B int8 qkv M={M}")
    del q, s, y
    x, wg, wu = ffn_inputs(60 + M, M, K, I)
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                       qu.cpu().numpy(), su.cpu().numpy())
    _check(y[rows], out, f"8B int8 gate-up M={M}")


# ----- plain projections: down and o (bias-free Linear) ----------------------


def check_linear(seed, M, K, N, label=""):
    x, w = qkv_inputs(seed, M, K, N, 0)
    y = _kernels().fused_linear(x.to(DEV), w.to(DEV)).cpu()
    rows = _rows(M)
    return _check(y[rows], ref.ref_linear(bits(x)[rows], bits(w)), label or f"linear M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16, 64, 256, 512, 2048])
@pytest.mark.parametrize("K,N", [(9728, 2560), (4096, 2560)], ids=["4b-down", "4b-o"])
def test_linear_down_o(M, K, N):
    """The Qwen3-4B down (K = intermediate) and o (K = heads * head_dim)
    projections across the regimes: row streaming, split-K, LDS tiles."""
    check_linear(100 + M, M, K, N, label=f"linear K={K} N={N} M={M}")


@pytest.mark.parametrize("M", [1, 16, 4096])
def test_linear_8b_down(M):
    check_linear(110 + M, M, 12288, 4096, label=f"8B down M={M}")


@pytest.mark.parametrize("M,K,N", [(1, 8, 3), (1, 203, 33), (3, 200, 33), (9, 1040, 100),
                                   (70, 2536, 130), (300, 1001, 77)])
def test_linear_tails(M, K, N):
    """Ragged K and N in every regime, including K not a multiple of 8 (the
    unaligned streaming path)."""
    check_linear(120 + M, M, K, N)


@pytest.mark.parametrize("op,M,K,N", [
    ("linear", 200, 1024, 1001),    # 64 x 64, 128-wide k-steps; odd N: scalar stores
    ("gate-up", 150, 1024, 1000),   # 64 x 64 gate-up, ragged M and N
    ("gate-up", 500, 1024, 3000),   # 128 x 128, 128-wide k-steps, ragged
    ("qkv", 384, 1024, 6144),       # 96 x 128, 128-wide k-steps
    ("qkv", 250, 2560, 4800),       # 64 x 64, ragged M
    ("gate-up", 1000, 1024, 9728),  # 320 x 256 gate-up, partial last tiles
    ("qkv", 3000, 1024, 6144)])     # 320 x 256, partial last tiles
def test_wide_k_and_320_tiles_ragged(op, M, K, N):
    """Ragged calls on the tiles with 128-wide k-steps and on 320 x 256 tiles
    (which tile runs is the planner's choice for these shapes): partial tiles
    in M and N, odd output widths, against the oracle."""
    if op == "linear":
        check_linear(200 + M, M, K, N)
    elif op == "gate-up":
        check_ffn(210 + M, M, K, N)
    else:
        n_k = N // 6
        check_qkv(220 + M, M, K, N - 2 * n_k, n_k)


@pytest.mark.parametrize("M,N,K,op", [
    (32, 2560, 9728, "linear"), (100, 4096, 12288, "linear"), (300, 1001, 8192, "linear"),
    (1024, 2560, 9728, "linear"), (2048, 2560, 9728, "linear"), (128, 6144, 4096, "qkv"),
    (40, 12288, 4096, "gate-up"), (200, 1001, 8192, "gate-up"), (77, 4096, 4096, "linear"),
    (512, 768, 4096, "qkv"), (136, 3072, 4096, "qkv"), (150, 1000, 8192, "gate-up"),
    (150, 1002, 8192, "gate-up"), (40, 1002, 12288, "gate-up")])
def test_split_k_across_workgroups(M, N, K, op):
    """Calls the planner splits across workgroups (fp32 partials in a torch
    workspace, fixed-order reduce): narrow and ragged N (scalar partial
    stores), ragged M, every split tile (with 128-wide steps mostly the
    staged 96 x 64 four-wave tiles); repeated calls are bit-identical."""
    from llms_amd import _lib

    assert _lib.capi().fp_workspace_bytes(M, N, K, int(op == "gate-up")) > 0
    kern = _kernels()
    if op == "gate-up":
        x, wg, wu = ffn_inputs(150 + M, M, K, N)
        xd, gd, ud = x.to(DEV), wg.to(DEV), wu.to(DEV)
        y = kern.triton_fused_gate_up_silu(xd, gd, ud)
        assert torch.equal(y.view(torch.int16), kern.triton_fused_gate_up_silu(xd, gd, ud).view(torch.int16))
        rows = _rows(M, limit=96)
        _check(y.cpu()[rows], ref.ref_gate_up_silu_full(bits(x)[rows], bits(wg), bits(wu)), f"split gate-up M={M} N={N} K={K}")
        return
    x, w = qkv_inputs(160 + M, M, K, N, 0)
    xd, wd = x.to(DEV), w.to(DEV)
    if op == "qkv":
        n_k = N // 6
        run = lambda: torch.cat(kern.triton_fused_qkv(xd, wd, n_q=N - 2 * n_k, n_k=n_k), dim=-1)  # noqa: E731
    else:
        run = lambda: kern.fused_linear(xd, wd)  # noqa: E731
    y = run()
    assert torch.equal(y.view(torch.int16), run().view(torch.int16))
    rows = _rows(M, limit=96)
    _check(y.cpu()[rows], ref.ref_linear(bits(x)[rows], bits(w)), f"split {op} M={M} N={N} K={K}")


@pytest.mark.parametrize("M,K,N,op,split", [(47, 2576, 6144, "qkv", False),
                                            (48, 2576, 6144, "qkv", False),
                                            (48, 2560, 6144, "qkv", False),
                                            (64, 1040, 1001, "gate-up", False),
                                            (200, 1040, 1001, "gate-up", False),
                                            (256, 1040, 1001, "gate-up", False),
                                            (128, 9728, 2560, "linear", True),
                                            (128, 4096, 2560, "linear", False),
                                            (512, 9728, 2560, "linear", True),
                                            (1024, 9728, 2560, "linear", False),
                                            (300, 2560, 9728, "gate-up", False),
                                            (1100, 2560, 1000, "gate-up", False),
                                            (200, 2560, 4352, "qkv", False),
                                            (600, 2560, 4352, "qkv", False)])
def test_int8_routes_in_register(M, K, N, op, split):
    """Every int8 route dequantises in registers (once per workgroup into
    LDS in the prefill tiles): the only int8 workspace is the fp32 partials
    where k is split across at least 4 workgroups (down projections here),
    and no call writes a bf16 copy of its weights. Across the routes (the
    streaming kernel for K % 64 != 0, the split-K tiles, the split across
    workgroups, the prefill tiles and gemm_kernel, ragged shapes) the result
    matches the dequantise-then-matmul oracle, and where nothing splits the
    call through the C ABI without a workspace gives the same bits."""
    import ctypes

    from llms_amd import _lib

    gu = op == "gate-up"
    lib = _lib.capi()
    assert (lib.fp_workspace_bytes_w8(M, N, K, int(gu)) > 0) == split
    kern = _kernels()
    rows = _rows(M, limit=64)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if gu:
        x, wg, wu = ffn_inputs(170 + M, M, K, N)
        qg, sg = _quant(wg)
        qu, su = _quant(wu)
        xd = x.to(DEV)
        yd = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su)
        out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                           qu.cpu().numpy(), su.cpu().numpy())
        yr = torch.empty_like(yd)
        assert lib.fp_gate_up_silu_w8(xd.data_ptr(), K, qg.data_ptr(), K, sg.data_ptr(),
                                      qu.data_ptr(), K, su.data_ptr(), yr.data_ptr(), N, M, N, K,
                                      st) == 0
    else:
        x, w = qkv_inputs(180 + M, M, K, N, 0)
        q, s = _quant(w)
        xd = x.to(DEV)
        n_k = N // 6 if op == "qkv" else 0
        if op == "qkv":
            yd = torch.cat(kern.fused_qkv_w8(xd, q, s, n_q=N - 2 * n_k, n_k=n_k), dim=-1)
        else:
            yd = kern.fused_linear_w8(xd, q, s)
        out = ref.ref_linear_w8(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy())
        yr = torch.empty_like(yd)
        assert lib.fp_qkv_w8(xd.data_ptr(), K, q.data_ptr(), K, s.data_ptr(), yr.data_ptr(), N, M,
                             N - 2 * n_k, n_k, K, st) == 0
    torch.cuda.synchronize()
    _check(yd.cpu()[rows], out, f"int8 {op} M={M} K={K} N={N}")
    if not split:
        assert torch.equal(yd.view(torch.int16), yr.view(torch.int16)), f"int8 {op} M={M} no-ws bits"
    else:
        _check(yr.cpu()[rows], out, f"int8 {op} M={M} K={K} N={N} unsplit")


@pytest.mark.parametrize("cell", ["4b-gate-up-2048", "8b-qkv-4096", "8b-gate-up-4096"])
def test_int8_prefill_cells_equal_bf16_on_dequantised(cell):
    """BASELINE's int8 prefill cells run in registers (no workspace) and
    contract every output over the same k-steps in the same order as the
    bf16 call, so the whole output equals the bf16 call on bf16(q * s) bit
    for bit; a row subset also against the oracle."""
    from llms_amd import _lib

    kern = _kernels()
    if cell == "8b-qkv-4096":
        K, n_q, n_k, _ = QWEN3_8B
        M, N = 4096, n_q + 2 * n_k
        x, w = qkv_inputs(230, M, K, n_q, n_k)
        q, s = kern.quantize_w8_per_row(w.to(DEV))
        assert _lib.capi().fp_workspace_bytes_w8(M, N, K, 0) == 0
        xd = x.to(DEV)
        y = torch.cat(kern.fused_qkv_w8(xd, q, s, n_q=n_q, n_k=n_k), dim=-1)
        yb = torch.cat(kern.triton_fused_qkv(xd, kern.dequantize_w8(q, s), n_q=n_q, n_k=n_k), dim=-1)
        rows = _rows(M, limit=24)
        out = ref.ref_qkv_w8_full(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy(), n_q, n_k)
    else:
        K, _, _, N = QWEN3_8B if cell.startswith("8b") else QWEN3_4B
        M = 4096 if cell.startswith("8b") else 2048
        x, wg, wu = ffn_inputs(240, M, K, N)
        qg, sg = kern.quantize_w8_per_row(wg.to(DEV))
        qu, su = kern.quantize_w8_per_row(wu.to(DEV))
        del wg, wu
        assert _lib.capi().fp_workspace_bytes_w8(M, N, K, 1) == 0
        xd = x.to(DEV)
        y = kern.fused_gate_up_silu_w8(xd, qg, sg, qu, su)
        yb = kern.triton_fused_gate_up_silu(xd, kern.dequantize_w8(qg, sg), kern.dequantize_w8(qu, su))
        rows = _rows(M, limit=24)
        out = ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                           qu.cpu().numpy(), su.cpu().numpy())
    assert torch.equal(y.view(torch.int16), yb.view(torch.int16)), cell
    _check(y.cpu()[rows], out, f"int8 {cell}")


@pytest.mark.parametrize("M,K,N,op", [(128, 9728, 2560, "linear"), (256, 4096, 6144, "qkv"),
                                      (256, 4096, 2560, "linear"), (200, 12288, 1001, "linear")])
def test_int8_split_across_workgroups(M, K, N, op):
    """int8 calls whose split plan splits k across at least 4 workgroups run
    that split on the int8 weights, dequantising in registers: the workspace
    is just the partials, repeated calls are bit-identical, and the result
    matches the oracle. Covers Qwen3 down at 128 rows, 8B QKV and 4B o at 256
    and a ragged narrow output. (The bf16 calls of these shapes split over
    128-wide k-steps on other tiles, or run a round of small tiles, so their
    results are not bit-identical to these.)"""
    from llms_amd import _lib

    lib = _lib.capi()
    assert lib.fp_workspace_bytes_w8(M, N, K, 0) > 0
    kern = _kernels()
    x, w = qkv_inputs(190 + M, M, K, N, 0)
    q, s = _quant(w)
    xd = x.to(DEV)
    if op == "qkv":
        n_k = N // 6
        run = lambda: torch.cat(kern.fused_qkv_w8(xd, q, s, n_q=N - 2 * n_k, n_k=n_k), dim=-1)  # noqa: E731
    else:
        run = lambda: kern.fused_linear_w8(xd, q, s)  # noqa: E731
    y = run()
    assert torch.equal(y.view(torch.int16), run().view(torch.int16)), f"int8 split {op} M={M}"
    rows = _rows(M, limit=64)
    _check(y.cpu()[rows], ref.ref_linear_w8(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy()),
           f"int8 split {op} M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [1, 4, 64, 2048])
def test_linear_int8(M):
    K, N = 9728, 2560
    x, w = qkv_inputs(130 + M, M, K, N, 0)
    q, s = _quant(w)
    y = _kernels().fused_linear_w8(x.to(DEV), q, s).cpu()
    rows = _rows(M)
    out = ref.ref_linear_w8(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy())
    _check(y[rows], out, f"int8 down M={M}")


def test_linear_errors_and_leading_dims():
    kern = _kernels()
    x, w = qkv_inputs(140, 6, 256, 96, 0)
    y = kern.fused_linear(x.view(2, 3, 256).to(DEV), w.to(DEV))
    assert y.shape == (2, 3, 96)
    _check(y.reshape(6, 96).cpu(), ref.ref_linear(bits(x), bits(w)), "linear leading dims")
    assert kern.fused_linear(x[:0].to(DEV), w.to(DEV)).shape == (0, 96)
    with pytest.raises(ValueError, match="x last dim"):
        kern.fused_linear(x[:, :-8].to(DEV), w.to(DEV))
    with pytest.raises(TypeError, match="bfloat16"):
        kern.fused_linear(x.float().to(DEV), w.to(DEV))
    q, s = _quant(w)
    with pytest.raises(ValueError, match="s shape"):
        kern.fused_linear_w8(x.to(DEV), q, s[:-1])


# ----- size-independent properties at full size ------------------------------


@pytest.mark.parametrize("M", [1, 8, 2048])
def test_deterministic_and_row_permutation_equivariant(M):
    """Repeated calls are bit-identical (the reference's prewarm test demands
    diff == 0.0), and permuting weight rows permutes output columns exactly."""
    K, _, _, I = QWEN3_4B
    kern = _kernels()
    x, wg, wu = ffn_inputs(70 + M, M, K, I)
    x, wg, wu = x.to(DEV), wg.to(DEV), wu.to(DEV)
    y1 = kern.triton_fused_gate_up_silu(x, wg, wu)
    y2 = kern.triton_fused_gate_up_silu(x, wg, wu)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    perm = torch.randperm(I, generator=gen(M)).to(DEV)
    yp = kern.triton_fused_gate_up_silu(x, wg[perm].contiguous(), wu[perm].contiguous())
    assert torch.equal(yp.view(torch.int16), y1[:, perm].view(torch.int16))


def test_against_torch_gpu_path():
    """Report-only comparison with the reference's unfused path on the same
    device (hipBLASLt F.linear + F.silu): both must sit inside the oracle hull
    with the same tolerance."""
    import torch.nn.functional as F

    K, n_q, n_k, I = QWEN3_4B
    for M in (1, 8, 512):
        x, wg, wu = ffn_inputs(80 + M, M, K, I)
        xd, gd, ud = x.to(DEV), wg.to(DEV), wu.to(DEV)
        ours = _kernels().triton_fused_gate_up_silu(xd, gd, ud).cpu()
        theirs = (F.silu(F.linear(xd, gd)) * F.linear(xd, ud)).cpu()
        out = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))
        p_ours = ref.check_parity(bits(ours), out)
        p_theirs = ref.check_parity(bits(theirs), out)
        print(f"M={M} ours: {p_ours}\nM={M} torch-gpu: {p_theirs}")
        assert p_ours.ok


# ----- persistent tile loops with few k-steps ---------------------------------



@pytest.mark.parametrize("M,K,n_q,n_k", [
    (2048, 2560, 4096, 1024),   # Qwen3-4B: one round of 192 x 256 tiles, four waves
    (4096, 4096, 4096, 1024),   # Qwen3-8B: two rounds (not 256 x 256 + tail), 64 k-steps
    (2000, 2560, 4000, 1000),   # partial tiles in M and N
    (2048, 2496, 4096, 1024)])  # 39 k-steps (odd): eight waves
def test_qkv_four_wave_tiles(M, K, n_q, n_k):
    """bf16 QKV calls planned on 192 x 256 tiles run four waves per
    workgroup (96 x 128 per wave, accumulators in AGPRs) with an even count
    of at least 32 k-steps, else eight: against the oracle, and repeated
    calls bit-identical."""
    x, w = qkv_inputs(240 + M + K, M, K, n_q, n_k)
    y = run_qkv(x, w, n_q, n_k)
    assert torch.equal(y.view(torch.int16), run_qkv(x, w, n_q, n_k).view(torch.int16))
    rows = _rows(M)
    _check(y[rows], ref.ref_qkv_full(bits(x)[rows], bits(w), n_q, n_k), f"qkv 192 x 256 M={M} K={K}")

@pytest.mark.parametrize("K", [64, 128, 192, 320])
def test_tile_loops_few_ksteps(K):
    """The one-tile-per-CU kernels at 2048 rows with 1, 2, 3 and 5 k-steps of
    64: the pipelined loop (gate-up, 320 x 256 and int8 256 x 256 tiles: the
    last step's reads of the next stage are stale and unused, odd step counts
    end inside the unrolled pair) and the plain loop (QKV, 192 x 256; int8
    QKV pipelined with its dequantisation one step ahead)."""
    M, N, n_q, n_k = 2048, 9728, 4096, 1024
    check_qkv(1700 + K, M, K, n_q, n_k, label=f"qkv M={M} K={K}")
    check_ffn(1800 + K, M, K, N, label=f"gate-up M={M} K={K}")
    kern = _kernels()
    rows = _rows(M, limit=64)
    x, w = qkv_inputs(1900 + K, M, K, n_q, n_k)
    q, s = _quant(w)
    y = torch.cat(kern.fused_qkv_w8(x.to(DEV), q, s, n_q=n_q, n_k=n_k), dim=-1).cpu()
    _check(y[rows], ref.ref_qkv_w8_full(bits(x)[rows], q.cpu().numpy(), s.cpu().numpy(), n_q, n_k),
           f"int8 qkv M={M} K={K}")
    x, wg, wu = ffn_inputs(2000 + K, M, K, N)
    qg, sg = _quant(wg)
    qu, su = _quant(wu)
    y = kern.fused_gate_up_silu_w8(x.to(DEV), qg, sg, qu, su).cpu()
    _check(y[rows], ref.ref_gate_up_silu_w8_full(bits(x)[rows], qg.cpu().numpy(), sg.cpu().numpy(),
                                                 qu.cpu().numpy(), su.cpu().numpy()),
           f"int8 gate-up M={M} K={K}")
