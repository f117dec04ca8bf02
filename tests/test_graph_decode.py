"""Decode and speculative-verify steps captured in HIP graphs (``StepGraph``,
``llms_amd/harness.py``) replay at any position and give the eager step's
logits: the whole step — fused projections (with the norms fused in), RoPE
gather, cache write, masked attention, tied head — runs from one graph, with
the program's eager work between replays."""

from __future__ import annotations

import pytest
import torch

from llms_amd.harness import Cfg, StepGraph, greedy_generate, graph_greedy_generate, tiny_model, tiny_state
from llms_amd.kernels import apply_triton_kernels

DEV = "cuda"
TINY = Cfg()
WIDE = Cfg(vocab_size=64, hidden_size=256, num_hidden_layers=2, num_attention_heads=8,
           num_key_value_heads=2, head_dim=32, intermediate_size=384,
           max_position_embeddings=512)
VARIANTS = {
    "eager": {},
    "fused": dict(fused_ffn=True, fused_qkv=True),
    "all": dict(fused_ffn=True, fused_qkv=True, fuse_norm=True, linear_down_o=True),
}


def _model(c: Cfg, variant: str):
    st = tiny_state(c, seed=1, embed_scale=0.05)
    m = tiny_model(c, state=st, device=DEV)
    return apply_triton_kernels(m, **VARIANTS[variant]) if VARIANTS[variant] else m


def _tol(ref: torch.Tensor) -> float:
    # a few bf16 ulps of the largest logit (the graph attends over the whole
    # masked cache, the eager step over the filled prefix: fp32 sums differ)
    return 4.0 * 2.0 ** (torch.floor(torch.log2(ref.abs().max())).item() - 7)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", list(VARIANTS))
@pytest.mark.parametrize("c", [TINY, WIDE], ids=["tiny", "wide"])
def test_decode_graph_replays_match_eager_steps(c, variant):
    """Along the eager greedy trajectory, replaying the captured T = 1 step at
    each position gives the eager step's logits (within a few bf16 ulps) and
    the same argmax wherever the top-2 margin is not a near-tie."""
    m = _model(c, variant)
    prompt = torch.randint(0, c.vocab_size, (1, 12), generator=torch.Generator().manual_seed(3))
    n_new = 24
    S = prompt.shape[1] + n_new + 4
    ce, cg = m.alloc_cache(S), m.alloc_cache(S)
    with torch.inference_mode():
        le = m(prompt.to(DEV), ce, start_pos=0)
        m(prompt.to(DEV), cg, start_pos=0)
    step = StepGraph(m, cg, T=1)
    nt = le[:, -1:].argmax(-1)
    pos = prompt.shape[1]
    worst = 0.0
    for i in range(n_new):
        with torch.inference_mode():
            le = m(nt, ce, start_pos=pos).float()
        lg = step(nt, pos).float()
        d = (le - lg).abs().max().item()
        worst = max(worst, d)
        assert d <= _tol(le), f"step {i}: max |logit diff| {d}"
        top2 = le[0, -1].topk(2).values
        if (top2[0] - top2[1]).item() > 2 * d + 1e-6:
            assert le[0, -1].argmax().item() == lg[0, -1].argmax().item(), f"step {i}"
        nt = le[:, -1:].argmax(-1)
        pos += 1
    print(f"\n{variant} {c.hidden_size}: worst |logit diff| {worst:.4f}")


@pytest.mark.gpu
@pytest.mark.parametrize("T", [2, 4, 9])
def test_verify_graph_matches_eager(T):
    """A T-token verify step (speculative decoding's target pass) captured
    once and replayed at two positions with different drafts."""
    c = WIDE
    m = _model(c, "all")
    g = torch.Generator().manual_seed(T)
    prompt = torch.randint(0, c.vocab_size, (1, 20), generator=g)
    S = 64
    ce, cg = m.alloc_cache(S), m.alloc_cache(S)
    with torch.inference_mode():
        m(prompt.to(DEV), ce, start_pos=0)
        m(prompt.to(DEV), cg, start_pos=0)
    step = StepGraph(m, cg, T=T)
    pos = prompt.shape[1]
    for _ in range(2):
        draft = torch.randint(0, c.vocab_size, (1, T), generator=g).to(DEV)
        with torch.inference_mode():
            le = m(draft, ce, start_pos=pos).float()
        lg = step(draft, pos).float()
        assert (le - lg).abs().max().item() <= _tol(le)
        pos += T


@pytest.mark.gpu
def test_graph_greedy_generate_tokens():
    """``graph_greedy_generate`` (prefill eager, every decode step a replay)
    produces the eager greedy tokens up to the first near-tie."""
    c = WIDE
    m = _model(c, "all")
    prompt = torch.randint(0, c.vocab_size, (30,), generator=torch.Generator().manual_seed(4)).tolist()
    te = greedy_generate(m, prompt, 20, DEV)
    tg = graph_greedy_generate(m, prompt, 20, DEV)
    same = next((i for i, (a, b) in enumerate(zip(te, tg)) if a != b), len(te))
    print(f"\neager {te}\ngraph {tg}")
    assert same >= 8, (te, tg)


@pytest.mark.gpu
def test_prefill_calls_replay_in_graph():
    """Prefill-sized calls captured in one HIP graph — QKV on 96 x 128 tiles
    with 128-wide k-steps (384 rows), gate-up on 320 x 256 tiles (2048 rows),
    a down projection split across workgroups (fp32 partials in a workspace
    from the graph's pool, then the reduce) and an int8 down projection split
    the same way, int8 QKV at 2048 rows (one round of tiles that dequantise
    in LDS) and int8 gate-up at 2048 rows (two launches of tiles that
    dequantise once per workgroup in LDS, no workspace) — replay
    bit-identically to the eager calls, several times, with eager work
    between the replays."""
    from llms_amd import kernels as K
    from tests._util import ffn_inputs, qkv_inputs

    xq, wq = qkv_inputs(31, 384, 2560, 4096, 1024)
    xg, wg, wu = ffn_inputs(32, 2048, 2560, 9728)
    xd, wdn = qkv_inputs(33, 512, 9728, 2560, 0)
    xq2, _ = qkv_inputs(34, 2048, 2560, 0, 0)
    xq, wq, xg, wg, wu, xd, wdn, xq2 = (t.to(DEV) for t in (xq, wq, xg, wg, wu, xd, wdn, xq2))
    q8, s8 = K.quantize_w8_per_row(wdn)
    qq, sq = K.quantize_w8_per_row(wq)
    qg, sg = K.quantize_w8_per_row(wg)
    qu, su = K.quantize_w8_per_row(wu)

    def calls():
        q, k, v = K.triton_fused_qkv(xq, wq, n_q=4096, n_k=1024)
        q2, k2, v2 = K.fused_qkv_w8(xq2, qq, sq, n_q=4096, n_k=1024)
        return [q, k, v, K.triton_fused_gate_up_silu(xg, wg, wu),
                K.fused_linear(xd, wdn), K.fused_linear_w8(xd, q8, s8), q2, k2, v2,
                K.fused_gate_up_silu_w8(xg, qg, sg, qu, su)]

    eager = [t.clone() for t in calls()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()                      # warm the allocator outside the capture
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = calls()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (rep, i)
        _ = (xq.float() @ wq[:64].float().t()).sum().item()   # eager work between replays


@pytest.mark.gpu
def test_int8_verify_calls_replay_in_graph():
    """Verify-sized int8 calls on Qwen3-4B shapes (4 and 12 rows: x staged
    once per workgroup in LDS, 8 and 16 staged rows) and the decode-sized
    ones (1 row: the row kernels) captured in one HIP graph replay
    bit-identically to the eager calls, several times, with eager work
    between the replays."""
    from llms_amd import kernels as K
    from tests._util import ffn_inputs, qkv_inputs

    _, wq = qkv_inputs(41, 1, 2560, 4096, 1024)
    _, wg, wu = ffn_inputs(42, 1, 2560, 9728)
    qq, sq = K.quantize_w8_per_row(wq.to(DEV))
    qg, sg = K.quantize_w8_per_row(wg.to(DEV))
    qu, su = K.quantize_w8_per_row(wu.to(DEV))
    xs = [qkv_inputs(43 + M, M, 2560, 0, 0)[0].to(DEV) for M in (1, 4, 12)]

    def calls():
        out = []
        for x in xs:
            out += list(K.fused_qkv_w8(x, qq, sq, n_q=4096, n_k=1024))
            out.append(K.fused_gate_up_silu_w8(x, qg, sg, qu, su))
        return out

    eager = [t.clone() for t in calls()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()                      # warm the allocator outside the capture
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = calls()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (rep, i)
        _ = (xs[2].float() @ wq[:64].to(DEV).float().t()).sum().item()   # eager work between replays
