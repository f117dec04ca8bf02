"""The attention core of ``TritonAttention.forward`` against the reference's.

The reference's forward ends in one of three ``F.scaled_dot_product_attention``
calls (``src/kernels/fused_qkv.py:271-279``, the same as
``src/engine/attention.py:152-160``): no mask for a single query (T == 1),
``is_causal=True`` for a prefill from position 0, and an explicit boolean mask
``q_pos >= k_pos`` otherwise. ``llms_amd.kernels._eager.attend`` replaces the
three with one fp32 softmax attention. These CPU tests run the reference's
exact calls with torch's CPU SDPA on the same operands (GQA heads expanded
with ``repeat_interleave`` as the reference does) and bound the difference:

- fp32 operands: max-abs <= 2e-6 (both are fp32 evaluations of the same
  softmax; only the summation order differs).
- bf16 operands: torch's CPU SDPA rounds its intermediates (scores,
  probabilities) to bf16, ``attend`` rounds once at the end. Against the
  fp64 evaluation of the same branch, ``attend`` is within half a bf16 ulp
  (|a - t| <= 2^-8 |t| + 1e-5, the second term for the fp32 evaluation
  error of outputs that cancel towards zero) and its rel-L2 error is no larger than SDPA's; the
  two differ by at most two bf16 ulps of the largest output (max-abs <=
  2^-6 max|b|; SDPA's rounded scores shift small outputs by an absolute
  amount) with rel-L2 <= 5e-3 (measured on these cases: max-abs
  7.8e-3, one ulp at |y| in [1, 2); rel-L2 1.3e-3 .. 2.3e-3; attend's own
  rel-L2 error 1.4e-3 .. 1.7e-3 against SDPA's 1.6e-3 .. 2.1e-3).

The device-tensor ``start_pos`` form (a step captured in a HIP graph) attends
over the whole cache with a mask; it must stay finite and equal the int form
to fp32 rounding (one bf16 ulp for bf16 operands) even when the unwritten
cache slots hold NaN and Inf, as the reference's ``torch.empty`` cache may.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from llms_amd.kernels._eager import attend

H, HKV, D = 8, 2, 64


def _ops(seed: int, B: int, T: int, start_pos: int, dtype: torch.dtype):
    g = torch.Generator().manual_seed(seed)
    end = start_pos + T
    q = torch.randn(B, H, T, D, generator=g).to(dtype)
    k = torch.randn(B, HKV, end, D, generator=g).to(dtype)
    v = torch.randn(B, HKV, end, D, generator=g).to(dtype)
    n_rep = H // HKV
    return q, k.repeat_interleave(n_rep, dim=1), v.repeat_interleave(n_rep, dim=1)


def _reference_sdpa(q, full_k, full_v, start_pos: int) -> torch.Tensor:
    """The reference's three branches, verbatim in meaning."""
    T = q.shape[2]
    end_pos = start_pos + T
    if T == 1:
        return F.scaled_dot_product_attention(q, full_k, full_v, is_causal=False)
    if start_pos == 0:
        return F.scaled_dot_product_attention(q, full_k, full_v, is_causal=True)
    q_pos = torch.arange(start_pos, end_pos, device=q.device).unsqueeze(1)
    k_pos = torch.arange(0, end_pos, device=q.device).unsqueeze(0)
    return F.scaled_dot_product_attention(q, full_k, full_v, attn_mask=q_pos >= k_pos)


CASES = [  # (B, T, start_pos): the three branches
    (1, 1, 0), (2, 1, 37),           # T == 1: no mask
    (1, 9, 0), (2, 128, 0),          # start_pos == 0: is_causal
    (1, 4, 20), (2, 8, 100),         # explicit mask (spec-verify shapes)
]


@pytest.mark.parametrize("B,T,start_pos", CASES)
def test_attend_matches_sdpa_fp32(B, T, start_pos):
    q, k, v = _ops(B * 1000 + T * 10 + start_pos, B, T, start_pos, torch.float32)
    a = attend(q, k, v, start_pos)
    b = _reference_sdpa(q, k, v, start_pos)
    assert a.dtype == b.dtype == torch.float32
    assert (a - b).abs().max().item() <= 2e-6


@pytest.mark.parametrize("B,T,start_pos", CASES)
def test_attend_matches_sdpa_bf16(B, T, start_pos):
    q, k, v = _ops(B * 1000 + T * 10 + start_pos + 1, B, T, start_pos, torch.bfloat16)
    a = attend(q, k, v, start_pos).double()
    b = _reference_sdpa(q, k, v, start_pos).double()
    t = _reference_sdpa(q.double(), k.double(), v.double(), start_pos)
    # half an ulp, plus the fp32 evaluation error (relative to the terms of
    # p @ v, not to a result that cancels towards zero)
    assert bool(((a - t).abs() <= 2.0 ** -8 * t.abs() + 1e-5).all())
    rel = lambda e: (e.norm() / t.norm()).item()  # noqa: E731
    assert rel(a - t) <= rel(b - t) * 1.01 + 1e-12
    d = (a - b).abs()
    assert d.max().item() <= 2.0 ** -6 * b.abs().max().item()
    assert (d.norm() / b.norm()).item() <= 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,start_pos", [(1, 0), (1, 17), (4, 0), (4, 30), (8, 55)])
def test_attend_device_position_form(dtype, T, start_pos):
    """Whole-cache attention with a tensor start_pos equals the int form on
    the sliced cache, with NaN/Inf in every slot past the last query."""
    B, S = 2, 64
    q, k, v = _ops(7 + T + start_pos, B, T, start_pos, dtype)
    end = start_pos + T
    ck = torch.empty(B, H, S, D, dtype=dtype)
    cv = torch.empty(B, H, S, D, dtype=dtype)
    ck[:, :, :end] = k
    cv[:, :, :end] = v
    ck[:, :, end:] = float("nan")
    cv[:, :, end:] = float("nan")
    cv[:, :, end::3] = float("inf")
    a = attend(q, ck, cv, torch.tensor(start_pos))
    b = attend(q, k, v, start_pos)
    assert torch.isfinite(a).all()
    # the same fp32 attention over S = 64 instead of start_pos + T keys: the
    # matmul blocking (hence the fp32 summation order) may differ
    d = (a.double() - b.double()).abs().max().item()
    if dtype == torch.float32:
        assert d <= 1e-6
    else:
        assert d <= 2.0 ** -7 * b.double().abs().max().item()
