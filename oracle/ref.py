"""numpy restatement of the reference's unfused projection path (test oracle).

bf16 tensors are carried as ``uint16`` bit patterns (numpy has no bfloat16).
Every contraction is evaluated exactly: a product of two bf16 values is exact
in fp64 and a fp64 sum of K <= 2^16 such products carries a relative error
below 2^-37, far under any bf16 rounding decision. The rounding points are
those of the torch path the reference runs when the fused kernels are off:

- QKV (``src/engine/attention.py:119-121``; fused form
  ``src/kernels/fused_qkv.py:28-85`` + split ``:147-149``; test reference
  ``tests/test_kernels_fused_qkv.py:22-34``): ``y = bf16(x . W^T)``, then
  ``split([n_q, n_k, n_k], -1)``.
- gate-up-SiLU (``src/engine/model.py:36-37``; fused form
  ``src/kernels/fused_ffn.py:20-95``; test reference
  ``tests/test_kernels_fused_ffn.py:21-30``): ``g = bf16(x.Wg^T)``,
  ``u = bf16(x.Wu^T)``, ``s = bf16(silu(g))`` with silu evaluated on the
  rounded g, ``y = bf16(s * u)``.
- plain projections ``down`` / ``o`` (``src/engine/model.py:37``,
  ``src/engine/attention.py:183``): ``y = bf16(x . W^T)``.
- RMSNorm prologue (``src/engine/attention.py:28-33``, applied before QKV and
  gate-up in ``src/engine/model.py:57-66``): fp32 statistics, then
  ``bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))``.
- int8 weight-only (no reference counterpart; the reference names weight
  quantisation as future work only, reference ``DESIGN.md:120``): per output row
  ``s_r = max|w_r| / 127`` (fp32), ``q = clamp(rint(w / s_r), -127, 127)``;
  the dequantised weight is ``bf16(fp32(q * s_r))`` and the bf16 path above
  runs on it ("dequantise then matmul").

Parity check. Any fp32-accumulating GEMM (the reference's own Triton kernel,
cuBLAS, hipBLASLt, oneDNN, these HIP kernels) differs from the exact sum by an
amount that scales with the size of the summed terms, not of the result:
about 2^-24 * ||(x_k w_k)_k||_2 times a small factor set by the summation
order (cancellation makes small results fragile). Where the exact
pre-rounding value lies within that distance of a bf16 rounding midpoint,
more than one bf16 value is a correct rounding. The oracle therefore returns,
per output element, the exact-rounding value ("central") and the hull
[lo, hi] of the outputs reachable when each rounding point may round any
value within its window: ``TAU_SUM * ||(x_k w_k)_k||_2`` for a contraction,
``TAU_SILU * |silu(g)|`` for the fp32 silu. Elements away from every
midpoint have lo == hi == central. :func:`check_parity` applies the task's
bar — max-abs error <= 2e-2 against that hull, rel-L2 <= 5e-3 against
central.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# Half-width of the rounding-ambiguity window of a contraction output, in
# units of ||(x_k w_k)_k||_2. Measured fp32 GEMM deviations from the exact sum
# are ~2^-25 of that norm (oneDNN) and are expected to stay below ~2^-21 for
# blocked MFMA accumulation; 2^-16 leaves a wide margin while keeping the
# window far below one bf16 ulp of a typical output (2^-7 at |y| ~ 1).
TAU_SUM = 2.0 ** -16
# Relative half-width for silu(g) evaluated in fp32 (a few fp32 ulps from exp
# and the divide).
TAU_SILU = 2.0 ** -20

MAX_ABS_TOL = 2e-2
REL_L2_TOL = 5e-3


# ----------------------------------------------------------------- bf16 bits


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7fc0."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def _ulp_bf16(v: np.ndarray) -> np.ndarray:
    """Spacing of the bf16 grid in the binade of |v| (denormal range fixed)."""
    _, ex = np.frexp(np.abs(v))          # |v| = m * 2^ex, m in [0.5, 1)
    e = np.maximum(ex - 1, -126)         # |v| in [2^e, 2^(e+1))
    return np.ldexp(1.0, e - 7)


def round_bf16_f64(v: np.ndarray) -> np.ndarray:
    """fp64 -> nearest bf16 value (ties to even), as fp64; one rounding."""
    v = np.asarray(v, dtype=np.float64)
    ulp = _ulp_bf16(v)
    return np.round(v / ulp) * ulp       # np.round: half to even


def _candidates(v: np.ndarray, delta: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Hull [lo, hi] of the bf16 roundings of every value within +-delta of
    the exact v (lo == hi == round(v) unless a rounding midpoint is that
    close)."""
    v = np.asarray(v, dtype=np.float64)
    return round_bf16_f64(v - delta), round_bf16_f64(v + delta)


# ------------------------------------------------------------ contractions


def _as_f64(bits: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bits).astype(np.float64)


def exact_linear(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """Exact x . W^T for bf16 x [M,K] and W [N,K] (fp64 result)."""
    return _as_f64(x_bits) @ _as_f64(w_bits).T


def term_norm(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """||(x_k w_k)_k||_2 for every output element: sqrt(x^2 . (W^2)^T)."""
    x = _as_f64(x_bits)
    w = _as_f64(w_bits)
    return np.sqrt((x * x) @ (w * w).T)


def silu_f64(g: np.ndarray) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)), the form torch evaluates (fp64 here)."""
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


@dataclass
class OracleOut:
    """Oracle output for one projection: central value and admissible hull,
    all as fp64 arrays of the output shape, plus the bf16 bits of central."""

    central: np.ndarray
    lo: np.ndarray
    hi: np.ndarray

    @property
    def bits(self) -> np.ndarray:
        return f32_to_bf16(self.central.astype(np.float32))


def _check_qkv_args(x_shape, w_shape, n_q: int, n_k: int) -> None:
    # Same checks, order and wording as src/kernels/fused_qkv.py:108-121.
    if len(w_shape) != 2:
        raise ValueError(f"W_qkv must be 2D (n_q+2*n_k, K), got shape {tuple(w_shape)}")
    n_total, K = w_shape
    if n_q + 2 * n_k != n_total:
        raise ValueError(
            f"n_q + 2*n_k ({n_q} + 2*{n_k} = {n_q + 2 * n_k}) != W_qkv.shape[0] ({n_total})"
        )
    if x_shape[-1] != K:
        raise ValueError(f"x last dim {x_shape[-1]} != W_qkv.shape[1] {K}")


def _check_gate_up_args(x_shape, wg_shape, wu_shape) -> None:
    # Same checks, order and wording as src/kernels/fused_ffn.py:110-119.
    if tuple(wg_shape) != tuple(wu_shape):
        raise ValueError(f"Wg shape {tuple(wg_shape)} != Wu shape {tuple(wu_shape)}")
    if len(wg_shape) != 2:
        raise ValueError(f"Wg must be 2D (N, K), got shape {tuple(wg_shape)}")
    if x_shape[-1] != wg_shape[1]:
        raise ValueError(f"x last dim {x_shape[-1]} != Wg.shape[1] {wg_shape[1]}")


def ref_qkv_full(x_bits: np.ndarray, w_bits: np.ndarray, n_q: int, n_k: int,
                 tau: float = TAU_SUM, extra: np.ndarray | None = None) -> OracleOut:
    """The fused QKV output y [..., n_q+2n_k] (before the split).

    Follows src/kernels/fused_qkv.py:108-148: validate, flatten the leading
    dims, one contraction against the row-stacked weight, restore the leading
    dims.
    """
    _check_qkv_args(x_bits.shape, w_bits.shape, n_q, n_k)
    lead = x_bits.shape[:-1]
    K = w_bits.shape[1]
    x2 = x_bits.reshape(-1, K)
    acc = exact_linear(x2, w_bits)
    delta = tau * term_norm(x2, w_bits)
    if extra is not None:  # admissible spread of the inputs (a prologue's rounding)
        delta = delta + extra.reshape(delta.shape)
    lo, hi = _candidates(acc, delta)
    central = round_bf16_f64(acc)
    shp = (*lead, w_bits.shape[0])
    return OracleOut(central.reshape(shp), lo.reshape(shp), hi.reshape(shp))


def ref_linear(x_bits: np.ndarray, w_bits: np.ndarray, tau: float = TAU_SUM) -> OracleOut:
    """``bf16(x . W^T)`` for a bias-free Linear: the ``down`` and ``o``
    projections (src/engine/model.py:37, src/engine/attention.py:183, both
    ``nn.Linear(..., bias=False)`` applied in bf16). The same contraction and
    single rounding as the QKV output before its split."""
    if w_bits.ndim != 2:
        raise ValueError(f"W must be 2D (N, K), got shape {tuple(w_bits.shape)}")
    if x_bits.shape[-1] != w_bits.shape[1]:
        raise ValueError(f"x last dim {x_bits.shape[-1]} != W.shape[1] {w_bits.shape[1]}")
    return ref_qkv_full(x_bits, w_bits, w_bits.shape[0], 0, tau)


def split_qkv(y: np.ndarray, n_q: int, n_k: int):
    """(q, k, v) column blocks of y, as views (fused_qkv.py:148)."""
    return y[..., :n_q], y[..., n_q:n_q + n_k], y[..., n_q + n_k:n_q + 2 * n_k]


def ref_qkv(x_bits, w_bits, n_q: int, n_k: int):
    """(q, k, v) bf16 bits of split(bf16(x . W_qkv^T)) — the reference's
    QKV contract (tests/test_kernels_fused_qkv.py:22-34)."""
    return split_qkv(ref_qkv_full(x_bits, w_bits, n_q, n_k).bits, n_q, n_k)


def _silu_candidates(g_vals: np.ndarray, tau_s: float):
    s = silu_f64(g_vals)
    return _candidates(s, tau_s * np.abs(s))


def ref_gate_up_silu_full(x_bits: np.ndarray, wg_bits: np.ndarray, wu_bits: np.ndarray,
                          tau: float = TAU_SUM, tau_s: float = TAU_SILU,
                          extra_g: np.ndarray | None = None,
                          extra_u: np.ndarray | None = None) -> OracleOut:
    """silu(x.Wg^T) * (x.Wu^T) with the torch bf16 rounding points.

    Follows src/engine/model.py:37 (F.silu(self.gate(x)) * self.up(x)) and the
    wrapper's validation/flattening in src/kernels/fused_ffn.py:110-152.
    """
    _check_gate_up_args(x_bits.shape, wg_bits.shape, wu_bits.shape)
    lead = x_bits.shape[:-1]
    K = wg_bits.shape[1]
    x2 = x_bits.reshape(-1, K)
    g = exact_linear(x2, wg_bits)
    u = exact_linear(x2, wu_bits)
    # central: every rounding point rounds the exact value once
    g_c = round_bf16_f64(g)
    u_c = round_bf16_f64(u)
    s_c = round_bf16_f64(silu_f64(g_c))
    central = round_bf16_f64(s_c * u_c)  # product of two bf16 is exact in fp64
    # hull over admissible roundings of g, u and silu(g)
    dg = tau * term_norm(x2, wg_bits)
    du = tau * term_norm(x2, wu_bits)
    if extra_g is not None:
        dg = dg + extra_g.reshape(dg.shape)
    if extra_u is not None:
        du = du + extra_u.reshape(du.shape)
    g_lo, g_hi = _candidates(g, dg)
    u_lo, u_hi = _candidates(u, du)
    lo = np.full(g.shape, np.inf)
    hi = np.full(g.shape, -np.inf)
    for gv in (g_lo, g_hi):
        s_lo, s_hi = _silu_candidates(gv, tau_s)
        for sv in (s_lo, s_hi):
            for uv in (u_lo, u_hi):
                y = round_bf16_f64(sv * uv)
                np.minimum(lo, y, out=lo)
                np.maximum(hi, y, out=hi)
    shp = (*lead, wg_bits.shape[0])
    return OracleOut(central.reshape(shp), lo.reshape(shp), hi.reshape(shp))


def ref_gate_up_silu(x_bits, wg_bits, wu_bits) -> np.ndarray:
    """bf16 bits of F.silu(F.linear(x, Wg)) * F.linear(x, Wu)."""
    return ref_gate_up_silu_full(x_bits, wg_bits, wu_bits).bits


# ------------------------------------------------------------ RMSNorm prologue

# Relative half-width of the window of x * r in which its bf16 rounding is
# implementation-defined: the fp32 mean of squares depends on the summation
# order (a few ulps for K <= 2^16), r = 1 / sqrt(var + eps) halves that, and
# rsqrt implementations differ by about an ulp.
TAU_NORM = 2.0 ** -18


@dataclass
class NormOut:
    """Normalised rows: bf16 bits of the central value, and per element the
    spread |hi - lo| of the admissible values (0 where the rounding of x * r is
    unambiguous)."""

    bits: np.ndarray
    spread: np.ndarray


def ref_rmsnorm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float,
                tau: float = TAU_NORM) -> NormOut:
    """RMSNorm of bf16 rows with a bf16 weight, src/engine/attention.py:28-33:
    ``x32 = x.float(); var = x32.pow(2).mean(-1); x32 = x32 * rsqrt(var + eps);
    return weight * x32.to(bf16)``. The statistics are evaluated exactly and
    rounded once to fp32; every later step is the fp32 / bf16 operation torch
    performs."""
    x = bf16_to_f32(x_bits)
    K = x.shape[-1]
    x64 = x.astype(np.float64)
    var = ((x64 * x64).sum(axis=-1, keepdims=True) / K).astype(np.float32)
    r = np.float32(1.0) / np.sqrt(var + np.float32(eps))
    t = (x * r).astype(np.float32)
    w = bf16_to_f32(w_bits)
    bits = f32_to_bf16(w * bf16_to_f32(f32_to_bf16(t)))
    t_lo, t_hi = _candidates(t.astype(np.float64), tau * np.abs(t.astype(np.float64)))
    y_lo = bf16_to_f32(f32_to_bf16(w * t_lo.astype(np.float32))).astype(np.float64)
    y_hi = bf16_to_f32(f32_to_bf16(w * t_hi.astype(np.float32))).astype(np.float64)
    return NormOut(bits, np.abs(y_hi - y_lo))


def ref_rmsnorm_qkv_full(x_bits, g_bits, eps: float, w_bits, n_q: int, n_k: int) -> OracleOut:
    """The fused norm + QKV call: the QKV contract on the normalised rows, its
    hull widened by the norm's admissible spread times |W|."""
    nrm = ref_rmsnorm(x_bits, g_bits, eps)
    K = w_bits.shape[1]
    extra = nrm.spread.reshape(-1, K) @ np.abs(_as_f64(w_bits)).T
    return ref_qkv_full(nrm.bits, w_bits, n_q, n_k, extra=extra)


def ref_rmsnorm_gate_up_silu_full(x_bits, g_bits, eps: float, wg_bits, wu_bits) -> OracleOut:
    """The fused norm + gate-up-SiLU call (see :func:`ref_rmsnorm_qkv_full`)."""
    nrm = ref_rmsnorm(x_bits, g_bits, eps)
    K = wg_bits.shape[1]
    sp = nrm.spread.reshape(-1, K)
    return ref_gate_up_silu_full(nrm.bits, wg_bits, wu_bits,
                                 extra_g=sp @ np.abs(_as_f64(wg_bits)).T,
                                 extra_u=sp @ np.abs(_as_f64(wu_bits)).T)


# ---------------------------------------------------------- int8 weights


def quantize_w8_per_row(w_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8: s = max|w_row| / 127 (fp32),
    q = clamp(rint(w / s), -127, 127) (ties to even); all-zero rows give
    s = 0 and q = 0."""
    wf = bf16_to_f32(w_bits)
    amax = np.max(np.abs(wf), axis=1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(wf / safe[:, None]), -127, 127)
    q = np.where(s[:, None] > 0, q, 0).astype(np.int8)
    return q, s


def dequant_w8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """bf16 bits of (q.float() * s[:, None]).to(bfloat16): one fp32 rounding
    of q*s, then round-to-nearest-even to bf16."""
    w32 = q.astype(np.float32) * np.asarray(s, dtype=np.float32)[:, None]
    return f32_to_bf16(w32)


def ref_qkv_w8_full(x_bits, q, s, n_q: int, n_k: int) -> OracleOut:
    """int8 QKV: dequantise then the bf16 QKV contract."""
    return ref_qkv_full(x_bits, dequant_w8(q, s), n_q, n_k)


def ref_linear_w8(x_bits, q, s) -> OracleOut:
    """int8 Linear: dequantise then the bf16 Linear contract."""
    return ref_linear(x_bits, dequant_w8(q, s))


def ref_gate_up_silu_w8_full(x_bits, qg, sg, qu, su) -> OracleOut:
    """int8 gate-up-SiLU: dequantise both weights then the bf16 contract."""
    return ref_gate_up_silu_full(x_bits, dequant_w8(qg, sg), dequant_w8(qu, su))


# ---------------------------------------------------------------- parity


@dataclass
class Parity:
    n: int
    max_abs: float          # max |kernel - central|
    rel_l2: float           # ||kernel - central|| / ||central||
    max_excess: float       # max distance outside the admissible hull
    n_outside: int          # elements farther than MAX_ABS_TOL from the hull
    n_differ: int           # elements not bit-equal to central
    n_ambiguous: int        # elements whose hull is wider than one point

    @property
    def ok(self) -> bool:
        return self.n_outside == 0 and self.rel_l2 <= REL_L2_TOL

    def __str__(self) -> str:
        return (f"n={self.n} max_abs={self.max_abs:.4g} rel_l2={self.rel_l2:.3g} "
                f"max_excess={self.max_excess:.4g} outside={self.n_outside} "
                f"differ={self.n_differ} ambiguous={self.n_ambiguous}")


def check_parity(kernel_bits: np.ndarray, ref: OracleOut,
                 max_abs_tol: float = MAX_ABS_TOL) -> Parity:
    """Compare kernel output bits against an oracle output (see module doc)."""
    y = bf16_to_f32(kernel_bits).astype(np.float64).ravel()
    c = ref.central.ravel()
    lo = ref.lo.ravel()
    hi = ref.hi.ravel()
    diff = np.abs(y - c)
    excess = np.maximum(lo - y, y - hi)
    excess = np.maximum(excess, 0.0)
    finite = np.isfinite(y)
    n = y.size
    denom = float(np.sqrt(np.sum(c * c))) if n else 0.0
    rel = float(np.sqrt(np.sum(np.where(finite, diff, np.inf) ** 2)) / denom) if denom > 0 else (
        0.0 if not n or np.all(diff == 0) else float("inf"))
    return Parity(
        n=n,
        max_abs=float(diff.max()) if n else 0.0,
        rel_l2=rel,
        max_excess=float(excess.max()) if n else 0.0,
        n_outside=int(np.count_nonzero((excess > max_abs_tol) | ~finite)),
        n_differ=int(np.count_nonzero(y != c)),
        n_ambiguous=int(np.count_nonzero(lo != hi)),
    )
