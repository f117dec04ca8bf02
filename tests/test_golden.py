"""The oracle reproduces the committed golden vectors (tests/golden/)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import ref

FIX = Path(__file__).resolve().parent / "golden" / "fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _in_hull(expect_bits, out: ref.OracleOut):
    p = ref.check_parity(expect_bits, out, max_abs_tol=0.0)
    assert p.n_outside == 0, p
    return p


def test_golden_qkv(fx):
    n_q, n_k = int(fx["qkv_nq"]), int(fx["qkv_nk"])
    _in_hull(fx["qkv_y"], ref.ref_qkv_full(fx["qkv_x"], fx["qkv_w"], n_q, n_k))
    out3 = ref.ref_qkv_full(fx["qkv3_x"], fx["qkv_w"], n_q, n_k)
    assert out3.central.shape == fx["qkv3_y"].shape == (2, 3, n_q + 2 * n_k)
    _in_hull(fx["qkv3_y"], out3)


def test_golden_gate_up(fx):
    _in_hull(fx["ffn_y"], ref.ref_gate_up_silu_full(fx["ffn_x"], fx["ffn_wg"], fx["ffn_wu"]))
    _in_hull(fx["ffn37_y"], ref.ref_gate_up_silu_full(fx["ffn37_x"], fx["ffn37_wg"], fx["ffn37_wu"]))


def test_golden_quantize(fx):
    q, s = ref.quantize_w8_per_row(fx["q8_w"])
    np.testing.assert_array_equal(q, fx["q8_q"])
    np.testing.assert_array_equal(s, fx["q8_s"])
    assert np.all(fx["q8_q"][5] == 0) and fx["q8_s"][5] == 0


def test_golden_int8(fx):
    out = ref.ref_gate_up_silu_w8_full(fx["w8_x"], fx["w8_qg"], fx["w8_sg"], fx["w8_qu"], fx["w8_su"])
    _in_hull(fx["w8_y"], out)
    n_q, n_k = int(fx["qkv_nq"]), int(fx["qkv_nk"])
    _in_hull(fx["w8q_y"], ref.ref_qkv_w8_full(fx["w8q_x"], fx["w8q_q"], fx["w8q_s"], n_q, n_k))
