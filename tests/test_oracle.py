"""Pin the CPU oracle (oracle/ref.py) before trusting it as the parity checker.

Each oracle function is checked against something that does not share its
code: torch's own bf16 conversion and ``F.linear``/``F.silu`` on the CPU (the
calls the reference makes), exact rational arithmetic on tiny inputs, closed
forms (one-hot inputs, known silu values, quantisation identities), and the
reference's own math-contract test shapes. Mutants of the oracle (a transposed
weight, swapped gate/up, a dropped rounding point, a shifted split, a wrong
quantisation rounding) are shown to fail those same checks.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ref
from oracle import torch_path as tp
from tests._util import bits, ffn_inputs, from_bits, gen, qkv_inputs, randn_bf16

# --------------------------------------------------------------- bf16 rounding


def exact_round_bf16(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest bf16 value, ties to even."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (max(e, -126) - 7)
    t = a / ulp
    fl = t.numerator // t.denominator
    rem = t - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


@pytest.mark.parametrize(
    "f32_bits, bf16_bits",
    [
        (0x3F800000, 0x3F80),  # 1.0
        (0x3F808000, 0x3F80),  # 1 + 2^-8: tie, stays even
        (0x3F818000, 0x3F82),  # 1 + 3*2^-8: tie, rounds up to even
        (0x3F808001, 0x3F81),  # just above the tie
        (0x3EAAAAAB, 0x3EAB),  # 1/3
        (0xC0200000, 0xC020),  # -2.5
        (0x7F800000, 0x7F80),  # +inf
        (0x7F7FFFFF, 0x7F80),  # FLT_MAX rounds to inf
        (0x7FC00001, 0x7FC0),  # NaN -> canonical
        (0x00000001, 0x0000),  # smallest denormal rounds to +0
        (0x80000000, 0x8000),  # -0
    ],
)
def test_f32_to_bf16_known_values(f32_bits, bf16_bits):
    f = np.array([f32_bits], dtype=np.uint32).view(np.float32)
    assert int(ref.f32_to_bf16(f)[0]) == bf16_bits


def test_f32_to_bf16_matches_torch():
    g = gen(0)
    f = torch.randn(200_000, generator=g) * torch.exp(torch.randn(200_000, generator=g) * 8)
    expect = bits(f.to(torch.bfloat16))
    got = ref.f32_to_bf16(f.numpy())
    np.testing.assert_array_equal(got, expect)
    back = ref.bf16_to_f32(expect)
    np.testing.assert_array_equal(back, f.to(torch.bfloat16).float().numpy())


def test_round_bf16_f64_matches_exact_rational():
    rng = np.random.default_rng(1)
    vals = list(rng.standard_normal(300) * np.exp(rng.standard_normal(300) * 5))
    # exact ties and near-ties around 1.0 and 3.0
    for base in (1.0, 3.0, -5.0):
        ulp = 2.0 ** (math.floor(math.log2(abs(base))) - 7)
        vals += [base + ulp / 2, base + ulp * 1.5, base + ulp / 2 + 1e-12, base + ulp / 2 - 1e-12]
    got = ref.round_bf16_f64(np.array(vals))
    for v, r in zip(vals, got):
        assert Fraction(float(r)) == exact_round_bf16(Fraction(v)), v


# ----------------------------------------------------- contraction contract


@pytest.mark.parametrize(
    "shape",
    # the reference's math-contract shapes, tests/test_kernels_fused_qkv.py:40-48
    [(1, 1, 64, 32, 8), (1, 8, 96, 48, 12), (2, 4, 80, 40, 10), (3, 5, 72, 36, 9)],
)
def test_exact_linear_is_nn_linear(shape):
    """The oracle's contraction is nn.Linear (weight [out, in]) on the same
    values, and the split order is q | k | v (fp64: exact to rounding noise)."""
    B, T, K, n_q, n_k = shape
    g = gen(0)
    x = randn_bf16(g, B, T, K)
    wq, wk, wv = (randn_bf16(g, n, K, std=0.1) for n in (n_q, n_k, n_k))
    w = torch.cat([wq, wk, wv])
    acc = ref.exact_linear(bits(x).reshape(-1, K), bits(w)).reshape(B, T, -1)
    parts = ref.split_qkv(acc, n_q, n_k)
    for part, wpart in zip(parts, (wq, wk, wv)):
        lin = torch.nn.Linear(K, wpart.shape[0], bias=False).double()
        with torch.no_grad():
            lin.weight.copy_(wpart.double())
        expect = lin(x.double()).detach().numpy()
        np.testing.assert_allclose(part, expect, rtol=1e-12, atol=1e-12)


def _hull_contains(kernel_bits, out: ref.OracleOut) -> ref.Parity:
    return ref.check_parity(kernel_bits, out, max_abs_tol=0.0)


@pytest.mark.parametrize("M,K,n_q,n_k", [(1, 1024, 256, 64), (5, 2560, 128, 32), (8, 96, 48, 12)])
def test_qkv_matches_torch_bf16_linear(M, K, n_q, n_k):
    """torch's CPU bf16 F.linear + split (the reference's unfused call) lands
    inside the oracle's admissible hull at every element, and on the oracle's
    central value almost everywhere."""
    x, w = qkv_inputs(3, M, K, n_q, n_k)
    out = ref.ref_qkv_full(bits(x), bits(w), n_q, n_k)
    q, k, v = tp.torch_qkv(x, w, n_q, n_k)
    tb = np.concatenate([bits(q), bits(k), bits(v)], axis=-1)
    p = _hull_contains(tb, out)
    assert p.n_outside == 0, p
    assert p.n_differ <= max(2, p.n // 200), p
    for got, exp in zip(ref.ref_qkv(bits(x), bits(w), n_q, n_k), (q, k, v)):
        assert got.shape == tuple(exp.shape)


@pytest.mark.parametrize(
    "M,K,N", [(1, 128, 32), (8, 256, 32), (4, 64, 32), (5, 96, 32), (3, 2560, 512), (1, 1024, 3072)]
)
def test_gate_up_matches_torch_bf16_path(M, K, N):
    """F.silu(F.linear(x, Wg)) * F.linear(x, Wu) in bf16 on the CPU lands
    inside the oracle's hull everywhere (reference FFN.forward, model.py:37)."""
    x, wg, wu = ffn_inputs(4, M, K, N, w_std=0.05)
    out = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))
    y = tp.torch_gate_up_silu(x, wg, wu)
    p = _hull_contains(bits(y), out)
    assert p.n_outside == 0, p
    assert p.n_differ <= max(2, p.n // 100), p


def test_gate_up_fp32_contract_matches_nn_modules():
    """The reference's step-1 contract: silu(x Wg^T) * (x Wu^T) equals
    F.silu(gate(x)) * up(x); the oracle's rounding-free composition (fp64)
    agrees with it."""
    g = gen(0)
    x = randn_bf16(g, 2, 4, 64)
    gate = torch.nn.Linear(64, 32, bias=False)
    up = torch.nn.Linear(64, 32, bias=False)
    with torch.no_grad():
        gate.weight.copy_(gate.weight.to(torch.bfloat16).float())
        up.weight.copy_(up.weight.to(torch.bfloat16).float())
    expect = (F.silu(gate(x.double().float())) * up(x.float())).detach().double().numpy()
    wg_b = bits(gate.weight.to(torch.bfloat16))
    wu_b = bits(up.weight.to(torch.bfloat16))
    gx = ref.exact_linear(bits(x).reshape(-1, 64), wg_b)
    ux = ref.exact_linear(bits(x).reshape(-1, 64), wu_b)
    got = (ref.silu_f64(gx) * ux).reshape(2, 4, 32)
    np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M,K,N", [(1, 9728, 64), (4, 4096, 96), (7, 200, 33)])
def test_linear_matches_torch_bf16_linear(M, K, N):
    """The down/o contract: torch's CPU bf16 F.linear (reference model.py:37,
    attention.py:183) lands inside the oracle's hull everywhere."""
    x, w = qkv_inputs(16, M, K, N, 0)
    out = ref.ref_linear(bits(x), bits(w))
    p = _hull_contains(bits(tp.torch_linear(x, w)), out)
    assert p.n_outside == 0, p
    assert p.n_differ <= max(2, p.n // 200), p
    qw, sw = tp.torch_quantize_w8(w)
    out = ref.ref_linear_w8(bits(x), qw.numpy(), sw.numpy())
    p = _hull_contains(bits(tp.torch_linear_w8(x, qw, sw)), out)
    assert p.n_outside == 0, p


# ------------------------------------------------------------- RMSNorm prologue


def _norm_inputs(seed, M, K, std, w_spread=0.3):
    g = gen(seed)
    x = randn_bf16(g, M, K, std=std)
    w = (1.0 + w_spread * torch.randn(K, generator=g)).to(torch.bfloat16)
    return x, w


@pytest.mark.parametrize("M,K,std,eps", [(8, 2560, 3.0, 1e-6), (5, 1024, 0.5, 1.0),
                                         (4, 4096, 0.01, 1e-6), (3, 200, 1.0, 1e-2)])
def test_rmsnorm_matches_torch_reference(M, K, std, eps):
    """The reference's RMSNorm.forward restated in torch on the CPU gives the
    oracle's central value everywhere except at elements the oracle flags as
    ambiguous, and there it stays within the flagged spread."""
    x, w = _norm_inputs(20 + K, M, K, std)
    out = ref.ref_rmsnorm(bits(x), bits(w), eps)
    t = tp.torch_rmsnorm(x, w, eps)
    amb = out.spread > 0
    assert amb.mean() < 0.01
    assert np.array_equal(out.bits[~amb], bits(t)[~amb])
    dv = np.abs(ref.bf16_to_f32(out.bits).astype(np.float64) - ref.bf16_to_f32(bits(t)))
    assert np.all(dv <= out.spread)


def test_rmsnorm_closed_forms():
    """Rows of a constant c with eps = 0: r = 1/|c| exactly for powers of two,
    so x * r = sign(c) and the output is sign(c) * w. A one-hot row a e_j:
    mean(x^2) = a^2 / K, so x_j * r = sign(a) sqrt(K) (exactly 16 for K = 256)."""
    K = 256
    w = (1.0 + 0.3 * torch.randn(K, generator=gen(3))).to(torch.bfloat16)
    x = torch.full((2, K), 4.0, dtype=torch.bfloat16)
    x[1] = -0.5
    out = ref.ref_rmsnorm(bits(x), bits(w), 0.0)
    wf = ref.bf16_to_f32(bits(w))
    np.testing.assert_array_equal(ref.bf16_to_f32(out.bits[0]), wf)
    np.testing.assert_array_equal(ref.bf16_to_f32(out.bits[1]), -wf)
    x = torch.zeros(1, K, dtype=torch.bfloat16)
    x[0, 7] = -3.0
    out = ref.ref_rmsnorm(bits(x), bits(w), 0.0)
    y = ref.bf16_to_f32(out.bits[0])
    assert y[7] == ref.bf16_to_f32(ref.f32_to_bf16(np.float32(-16.0) * wf[7:8]))[0]
    assert np.count_nonzero(y) == 1


def _mutant_norm_single_rounding(xb, wb, eps):
    x = ref.bf16_to_f32(xb).astype(np.float64)
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return ref.f32_to_bf16((ref.bf16_to_f32(wb) * x * r).astype(np.float32))


def _mutant_norm_unbiased(xb, wb, eps):
    x = ref.bf16_to_f32(xb)
    K = x.shape[-1]
    var = ((x.astype(np.float64) ** 2).sum(-1, keepdims=True) / (K - 1)).astype(np.float32)
    t = x * (np.float32(1) / np.sqrt(var + np.float32(eps)))
    return ref.f32_to_bf16(ref.bf16_to_f32(wb) * ref.bf16_to_f32(ref.f32_to_bf16(t)))


def test_rmsnorm_mutants_fail_the_pins():
    x, w = _norm_inputs(30, 16, 1024, 2.0)
    t = bits(tp.torch_rmsnorm(x, w, 1e-6))
    out = ref.ref_rmsnorm(bits(x), bits(w), 1e-6)
    ok = out.spread == 0
    for mutant in (_mutant_norm_single_rounding, _mutant_norm_unbiased):
        mb = mutant(bits(x), bits(w), 1e-6)
        assert np.count_nonzero(mb[ok] != t[ok]) > 50, mutant
    # eps matters when it is not negligible against mean(x^2)
    x, w = _norm_inputs(31, 4, 512, 0.5)
    assert not np.array_equal(ref.ref_rmsnorm(bits(x), bits(w), 0.0).bits,
                              bits(tp.torch_rmsnorm(x, w, 1.0)))


@pytest.mark.parametrize("M,K,N", [(4, 2560, 96), (3, 1024, 64)])
def test_fused_norm_oracles_hold_the_torch_path(M, K, N):
    """RMSNorm then F.linear / silu-gate-up in bf16 on the CPU (the reference's
    norm1 -> q/k/v and norm2 -> gate/up) lands inside the fused oracles'
    hulls everywhere."""
    x, w = _norm_inputs(40 + K, M, K, 2.0)
    _, wq = qkv_inputs(41, M, K, N - 32, 16)
    xn = tp.torch_rmsnorm(x, w, 1e-6)
    q, k, v = tp.torch_qkv(xn, wq, N - 32, 16)
    out = ref.ref_rmsnorm_qkv_full(bits(x), bits(w), 1e-6, bits(wq), N - 32, 16)
    p = _hull_contains(np.concatenate([bits(q), bits(k), bits(v)], axis=-1), out)
    assert p.n_outside == 0, p
    _, wg, wu = ffn_inputs(42, M, K, N, w_std=0.05)
    y = tp.torch_gate_up_silu(xn, wg, wu)
    out = ref.ref_rmsnorm_gate_up_silu_full(bits(x), bits(w), 1e-6, bits(wg), bits(wu))
    p = _hull_contains(bits(y), out)
    assert p.n_outside == 0, p


# ------------------------------------------------------------- brute force


def _frac(bits_arr):
    return [[Fraction(float(v)) for v in row] for row in ref.bf16_to_f32(bits_arr)]


def test_qkv_exact_rational_bruteforce():
    x, w = qkv_inputs(11, 3, 40, 8, 4, w_std=0.3)
    xb, wb = bits(x), bits(w)
    xf, wf = _frac(xb), _frac(wb)
    out = ref.ref_qkv_full(xb, wb, 8, 4)
    for m in range(3):
        for n in range(16):
            s = sum(a * b for a, b in zip(xf[m], wf[n]))
            assert Fraction(float(out.central[m, n])) == exact_round_bf16(s)


def test_linear_exact_rational_bruteforce():
    x, w = qkv_inputs(17, 2, 24, 10, 0, w_std=0.3)
    xb, wb = bits(x), bits(w)
    xf, wf = _frac(xb), _frac(wb)
    out = ref.ref_linear(xb, wb)
    for m in range(2):
        for n in range(10):
            s = sum(a * b for a, b in zip(xf[m], wf[n]))
            assert Fraction(float(out.central[m, n])) == exact_round_bf16(s)
    with pytest.raises(ValueError, match="x last dim"):
        ref.ref_linear(xb[:, :-1], wb)


def test_gate_up_exact_rational_bruteforce():
    x, wg, wu = ffn_inputs(12, 2, 48, 12, w_std=0.3)
    xb, gb, ub = bits(x), bits(wg), bits(wu)
    xf, gf, uf = _frac(xb), _frac(gb), _frac(ub)
    out = ref.ref_gate_up_silu_full(xb, gb, ub)
    for m in range(2):
        for n in range(12):
            gr = exact_round_bf16(sum(a * b for a, b in zip(xf[m], gf[n])))
            ur = exact_round_bf16(sum(a * b for a, b in zip(xf[m], uf[n])))
            sg = float(gr) / (1.0 + math.exp(-float(gr)))
            sr = exact_round_bf16(Fraction(sg))
            y = exact_round_bf16(sr * ur)
            assert Fraction(float(out.central[m, n])) == y


# ------------------------------------------------------------- closed forms


def test_qkv_one_hot_selects_weight_column_and_row():
    K, n_q, n_k = 64, 16, 8
    _, w = qkv_inputs(5, 1, K, n_q, n_k, w_std=0.5)
    x = torch.zeros(K, K, dtype=torch.bfloat16)
    x[torch.arange(K), torch.arange(K)] = 1.0
    y = ref.ref_qkv_full(bits(x), bits(w), n_q, n_k).central
    np.testing.assert_array_equal(y, ref.bf16_to_f32(bits(w)).T.astype(np.float64))
    # one-hot weight rows pick x columns
    xr, _ = qkv_inputs(6, 3, K, n_q, n_k)
    wsel = torch.zeros(n_q + 2 * n_k, K, dtype=torch.bfloat16)
    cols = torch.arange(n_q + 2 * n_k) % K
    wsel[torch.arange(n_q + 2 * n_k), cols] = 1.0
    y = ref.ref_qkv_full(bits(xr), bits(wsel), n_q, n_k).central
    np.testing.assert_array_equal(y, ref.bf16_to_f32(bits(xr))[:, cols.numpy()].astype(np.float64))


def test_gate_up_one_hot_and_silu_values():
    K, N = 32, 8
    _, wg, wu = ffn_inputs(7, 1, K, N, w_std=1.0)
    x = torch.zeros(1, K, dtype=torch.bfloat16)
    x[0, 5] = 1.0
    y = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu)).central[0]
    g = ref.bf16_to_f32(bits(wg))[:, 5].astype(np.float64)
    u = ref.bf16_to_f32(bits(wu))[:, 5].astype(np.float64)
    s = np.array([float(exact_round_bf16(Fraction(v / (1 + math.exp(-v))))) for v in g])
    np.testing.assert_array_equal(y, [float(exact_round_bf16(Fraction(a) * Fraction(b))) for a, b in zip(s, u)])
    # silu(0) = 0; silu(20) rounds to 20; silu(1) = 0.7310585786... -> bf16 0.73046875
    np.testing.assert_array_equal(ref.round_bf16_f64(ref.silu_f64(np.array([0.0, 20.0, 1.0]))),
                                  [0.0, 20.0, 0.73046875])


def test_empty_and_leading_dims():
    x = torch.zeros(0, 16, dtype=torch.bfloat16)
    _, w = qkv_inputs(1, 1, 16, 8, 4)
    q, k, v = ref.ref_qkv(bits(x), bits(w), 8, 4)
    assert q.shape == (0, 8) and k.shape == (0, 4) and v.shape == (0, 4)
    x3 = randn_bf16(gen(2), 2, 3, 16)
    q, k, v = ref.ref_qkv(bits(x3), bits(w), 8, 4)
    assert q.shape == (2, 3, 8) and v.shape == (2, 3, 4)


def test_oracle_error_messages_match_reference():
    xb = np.zeros((2, 64), np.uint16)
    wb = np.zeros((96, 64), np.uint16)
    with pytest.raises(ValueError, match="n_q .* 2.n_k"):
        ref.ref_qkv(xb, wb, 64, 15)
    with pytest.raises(ValueError, match="x last dim .* W_qkv"):
        ref.ref_qkv(np.zeros((2, 63), np.uint16), wb, 64, 16)
    with pytest.raises(ValueError, match="W_qkv must be 2D"):
        ref.ref_qkv(xb, np.zeros((2, 96, 64), np.uint16), 64, 16)
    wg = np.zeros((128, 64), np.uint16)
    with pytest.raises(ValueError, match="Wg shape.*Wu shape"):
        ref.ref_gate_up_silu(xb, wg, np.zeros((127, 64), np.uint16))
    with pytest.raises(ValueError, match="Wg must be 2D"):
        ref.ref_gate_up_silu(xb, np.zeros((2, 128, 64), np.uint16), np.zeros((2, 128, 64), np.uint16))
    with pytest.raises(ValueError, match="x last dim.*Wg.shape"):
        ref.ref_gate_up_silu(np.zeros((2, 63), np.uint16), wg, wg)


# ------------------------------------------------------------- int8


def test_quantize_closed_forms():
    w = torch.tensor(
        [[0.5, -0.25, 0.0, 0.125],
         [0.0, 0.0, 0.0, 0.0],
         [-1.0, 0.5, 0.25, 1.0],
         [3.0, 1.0, -1.5, 0.0]], dtype=torch.bfloat16)
    q, s = ref.quantize_w8_per_row(bits(w))
    np.testing.assert_array_equal(s, np.array([0.5, 0.0, 1.0, 3.0], np.float32) / np.float32(127))
    assert q[0, 0] == 127 and q[0, 1] == -64 and q[0, 2] == 0   # -63.5 ties to even
    assert np.all(q[1] == 0)
    assert q[2, 0] == -127 and q[2, 3] == 127
    assert q[3, 0] == 127 and q[3, 2] == -64                      # -63.5 -> -64


def test_quantize_identities_and_torch_restatement():
    _, w = qkv_inputs(8, 1, 256, 96, 16)
    wb = bits(w)
    q, s = ref.quantize_w8_per_row(wb)
    qn, sn = ref.quantize_w8_per_row(bits(-w))
    np.testing.assert_array_equal(qn, -q)             # symmetric
    np.testing.assert_array_equal(sn, s)
    assert np.abs(q).max() <= 127
    assert np.all(np.abs(q).max(axis=1) == 127)       # the row max maps to +-127
    # reconstruction error <= half a quantisation step, plus half an fp32 ulp
    # of the quotient w/s (< 128, so ulp <= 2^-17) from the fp32 divide
    wf = ref.bf16_to_f32(wb).astype(np.float64)
    err = np.abs(wf - q.astype(np.float64) * s.astype(np.float64)[:, None])
    assert np.all(err <= s.astype(np.float64)[:, None] * (0.5 + 2.0 ** -17))
    qt, st = tp.torch_quantize_w8(w)
    np.testing.assert_array_equal(q, qt.numpy())
    np.testing.assert_array_equal(s, st.numpy())
    np.testing.assert_array_equal(ref.dequant_w8(q, s), bits(tp.torch_dequant(qt, st)))


def test_w8_paths_match_torch_dequant_then_matmul():
    x, wg, wu = ffn_inputs(9, 4, 512, 64)
    qg, sg = tp.torch_quantize_w8(wg)
    qu, su = tp.torch_quantize_w8(wu)
    out = ref.ref_gate_up_silu_w8_full(bits(x), qg.numpy(), sg.numpy(), qu.numpy(), su.numpy())
    p = _hull_contains(bits(tp.torch_gate_up_silu_w8(x, qg, sg, qu, su)), out)
    assert p.n_outside == 0, p
    xq, w = qkv_inputs(10, 4, 512, 64, 16)
    qw, sw = tp.torch_quantize_w8(w)
    out = ref.ref_qkv_w8_full(bits(xq), qw.numpy(), sw.numpy(), 64, 16)
    tq = torch.cat(tp.torch_qkv_w8(xq, qw, sw, 64, 16), dim=-1)
    p = _hull_contains(bits(tq), out)
    assert p.n_outside == 0, p


# ------------------------------------------------------------- mutants


def _mutant_qkv_transposed(xb, wb, n_q, n_k):
    acc = ref._as_f64(xb) @ ref._as_f64(wb)  # W used as [K, N]: wrong operand orientation
    d = ref.TAU_SUM * np.sqrt((ref._as_f64(xb) ** 2) @ (ref._as_f64(wb) ** 2))
    return ref.OracleOut(ref.round_bf16_f64(acc), *ref._candidates(acc, d))


def _mutant_qkv_shifted_split(xb, wb, n_q, n_k):
    out = ref.ref_qkv_full(xb, wb, n_q, n_k)
    roll = lambda a: np.roll(a, 1, axis=-1)  # noqa: E731  (off-by-one column)
    return ref.OracleOut(roll(out.central), roll(out.lo), roll(out.hi))


def _mutant_gate_up_swapped(xb, gb, ub):
    return ref.ref_gate_up_silu_full(xb, ub, gb)


def _mutant_gate_up_no_g_rounding(xb, gb, ub):
    g = ref.exact_linear(xb, gb)
    u_c = ref.round_bf16_f64(ref.exact_linear(xb, ub))
    y = ref.round_bf16_f64(ref.round_bf16_f64(ref.silu_f64(g)) * u_c)
    return ref.OracleOut(y, y, y)


def _mutant_gate_up_dropped_term(xb, gb, ub):
    xb2 = xb.copy()
    xb2[:, -1] = 0  # one k term missing from every dot product
    return ref.ref_gate_up_silu_full(xb2, gb, ub)


def test_mutants_fail_the_pins():
    K, n_q, n_k = 64, 48, 8
    x, w = qkv_inputs(13, 6, K, n_q, n_k, w_std=0.2)  # n_q + 2 n_k == K: square W
    tq = np.concatenate([bits(t) for t in tp.torch_qkv(x, w, n_q, n_k)], axis=-1)
    assert _hull_contains(tq, ref.ref_qkv_full(bits(x), bits(w), n_q, n_k)).n_outside == 0
    for mutant in (_mutant_qkv_transposed, _mutant_qkv_shifted_split):
        assert _hull_contains(tq, mutant(bits(x), bits(w), n_q, n_k)).n_outside > 0, mutant

    x, wg, wu = ffn_inputs(14, 8, 512, 96, w_std=0.1)
    ty = bits(tp.torch_gate_up_silu(x, wg, wu))
    assert _hull_contains(ty, ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))).n_outside == 0
    for mutant in (_mutant_gate_up_swapped, _mutant_gate_up_no_g_rounding, _mutant_gate_up_dropped_term):
        assert _hull_contains(ty, mutant(bits(x), bits(wg), bits(wu))).n_outside > 0, mutant


def test_mutant_quantizer_fails_the_pins():
    _, w = qkv_inputs(15, 1, 128, 32, 8)
    qt, _ = tp.torch_quantize_w8(w)
    wf = ref.bf16_to_f32(bits(w))
    s = np.max(np.abs(wf), axis=1) / np.float32(127)
    q_trunc = np.clip(np.trunc(wf / s[:, None]), -127, 127).astype(np.int8)  # truncation, not RNE
    assert np.any(q_trunc != qt.numpy())


def test_parity_check_flags_real_errors():
    """check_parity itself: a 1-ulp flip at a non-ambiguous element of
    magnitude >= 4 fails the 2e-2 bar; a large-scale error fails rel-L2."""
    x, wg, wu = ffn_inputs(16, 64, 256, 256, w_std=0.15)
    out = ref.ref_gate_up_silu_full(bits(x), bits(wg), bits(wu))
    good = out.bits
    assert ref.check_parity(good, out).ok
    flat = out.central.ravel()
    idx = np.flatnonzero((np.abs(flat) >= 4) & (out.lo.ravel() == out.hi.ravel()))
    assert idx.size > 0
    bad = good.copy().ravel()
    bad[idx[0]] += 1  # one ulp away
    assert not ref.check_parity(bad.reshape(good.shape), out).ok
    scaled = ref.f32_to_bf16((ref.bf16_to_f32(good) * 1.02).astype(np.float32))
    assert ref.check_parity(scaled, out).rel_l2 > ref.REL_L2_TOL
