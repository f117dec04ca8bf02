"""An engine-shaped Qwen3 decoder for swapping in the fused modules, capturing
decode steps in HIP graphs, and measuring end-to-end decode.

It restates the reference's eager engine so that ``apply_triton_kernels`` /
``prewarm_triton_kernels`` run against the module structure the reference's
callers have, without network weights:

- ``KVCache``: per-layer ``k``/``v`` tensors ``(max_batch, n_kv, max_seq, D)``
  and ``cur_len`` (reference ``src/engine/kv_cache.py:19-47``).
- ``Attention``: separate ``q``/``k``/``v``/``o`` Linears, QK-norm, RoPE, cache
  write, GQA expansion (reference ``src/engine/attention.py:79-163``). The
  attention core is the same ``attend`` the fused module uses, so eager and
  fused models differ only in the projections (and, with ``fuse_norm``, in
  where the block norms run).
- ``FFN``: ``down(silu(gate(x)) * up(x))`` (reference ``src/engine/model.py:27-37``).
- ``Qwen3Model``: embed, pre-norm blocks, final norm, tied head, rope tables,
  ``alloc_cache``; ``forward(ids, cache, start_pos=None)`` continues at
  ``cache.cur_len`` (reference ``src/engine/model.py:40-186``).
- ``Cfg`` / ``tiny_model``: the reference's tiny Qwen3-shaped fixture
  (``tests/_tiny.py:20-74``): random projections ``randn * 0.1``, unit norms;
  ``QWEN3_4B`` / ``random_model``: the real Qwen3-4B shapes with random
  weights initialised on the device.

Graph mode (not in the reference, whose decode is launch-bound): ``start_pos``
may be a 0-dim device tensor. RoPE rows are then gathered, the cache written
with ``index_copy_`` and attention masked on the device over the whole cache,
so one decode (T = 1) or verify (T = 2..9) step captured by ``StepGraph`` in a
HIP graph replays at any position.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .kernels._eager import RMSNorm, apply_rope, attend, build_rope_tables, write_kv


@dataclass(frozen=True)
class Cfg:
    vocab_size: int = 32
    hidden_size: int = 64
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 16
    intermediate_size: int = 128
    max_position_embeddings: int = 64
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0


# Qwen3-4B (hidden 2560, 36 layers, 32 q / 8 kv heads of 128, FFN 9728, tied
# 151936-token embedding); max_position_embeddings trimmed to what the decode
# measurements need.
QWEN3_4B = Cfg(vocab_size=151936, hidden_size=2560, num_hidden_layers=36,
               num_attention_heads=32, num_key_value_heads=8, head_dim=128,
               intermediate_size=9728, max_position_embeddings=4096, rope_theta=1000000.0)


@dataclass
class KVCache:
    k: list
    v: list
    cur_len: int = 0


class Attention(nn.Module):
    def __init__(self, c: Cfg) -> None:
        super().__init__()
        self.num_heads = c.num_attention_heads
        self.num_kv_heads = c.num_key_value_heads
        self.head_dim = c.head_dim
        H, KV = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
        self.q = nn.Linear(c.hidden_size, H, bias=False)
        self.k = nn.Linear(c.hidden_size, KV, bias=False)
        self.v = nn.Linear(c.hidden_size, KV, bias=False)
        self.o = nn.Linear(H, c.hidden_size, bias=False)
        self.q_norm = RMSNorm(c.head_dim, eps=c.rms_norm_eps)
        self.k_norm = RMSNorm(c.head_dim, eps=c.rms_norm_eps)

    def forward(self, x, *, kv_cache, layer_idx, cos, sin, start_pos):
        B, T, _ = x.shape
        q = self.q(x).view(B, T, self.num_heads, self.head_dim)
        k = self.k(x).view(B, T, self.num_kv_heads, self.head_dim)
        v = self.v(x).view(B, T, self.num_kv_heads, self.head_dim)
        q = self.q_norm(q).transpose(1, 2)
        k = self.k_norm(k).transpose(1, 2)
        v = v.transpose(1, 2)
        q, k = apply_rope(q, k, cos, sin)
        full_k, full_v = write_kv(kv_cache.k[layer_idx], kv_cache.v[layer_idx], k, v, start_pos)
        rep = self.num_heads // self.num_kv_heads
        if rep > 1:
            full_k = full_k.repeat_interleave(rep, dim=1)
            full_v = full_v.repeat_interleave(rep, dim=1)
        a = attend(q, full_k, full_v, start_pos)
        return self.o(a.transpose(1, 2).reshape(B, T, self.num_heads * self.head_dim))


class FFN(nn.Module):
    def __init__(self, c: Cfg) -> None:
        super().__init__()
        self.gate = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.up = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.down = nn.Linear(c.intermediate_size, c.hidden_size, bias=False)

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class DecoderBlock(nn.Module):
    def __init__(self, c: Cfg) -> None:
        super().__init__()
        self.norm1 = RMSNorm(c.hidden_size, eps=c.rms_norm_eps)
        self.attn = Attention(c)
        self.norm2 = RMSNorm(c.hidden_size, eps=c.rms_norm_eps)
        self.ffn = FFN(c)

    def forward(self, x, *, kv_cache, layer_idx, cos, sin, start_pos):
        h = x + self.attn(self.norm1(x), kv_cache=kv_cache, layer_idx=layer_idx,
                          cos=cos, sin=sin, start_pos=start_pos)
        return h + self.ffn(self.norm2(h))


class Qwen3Model(nn.Module):
    def __init__(self, c: Cfg) -> None:
        super().__init__()
        self.cfg = c
        self.embed = nn.Embedding(c.vocab_size, c.hidden_size)
        self.layers = nn.ModuleList([DecoderBlock(c) for _ in range(c.num_hidden_layers)])
        self.final_norm = RMSNorm(c.hidden_size, eps=c.rms_norm_eps)
        cos, sin = build_rope_tables(c.head_dim, c.max_position_embeddings, c.rope_theta)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def alloc_cache(self, max_seq_len: int, *, max_batch: int = 1) -> KVCache:
        c = self.cfg
        w = self.embed.weight
        shape = (max_batch, c.num_key_value_heads, max_seq_len, c.head_dim)
        mk = lambda: [torch.zeros(shape, dtype=w.dtype, device=w.device)  # noqa: E731
                      for _ in range(c.num_hidden_layers)]
        return KVCache(k=mk(), v=mk())

    def forward(self, input_ids, kv_cache, start_pos=None):
        """Logits for ``input_ids`` [B, T] at positions start_pos ..; an int
        start_pos (default ``kv_cache.cur_len``) advances ``cur_len``, a 0-dim
        device tensor (graph mode) leaves it to the caller."""
        if start_pos is None:
            start_pos = kv_cache.cur_len
        T = input_ids.shape[1]
        h = self.embed(input_ids)
        if torch.is_tensor(start_pos):
            rows = start_pos + torch.arange(T, device=input_ids.device)
            cos = self.rope_cos.index_select(0, rows)
            sin = self.rope_sin.index_select(0, rows)
        else:
            cos = self.rope_cos[start_pos:start_pos + T]
            sin = self.rope_sin[start_pos:start_pos + T]
        for i, layer in enumerate(self.layers):
            h = layer(h, kv_cache=kv_cache, layer_idx=i, cos=cos, sin=sin, start_pos=start_pos)
        h = self.final_norm(h)
        if not torch.is_tensor(start_pos):
            kv_cache.cur_len = start_pos + T
        return F.linear(h, self.embed.weight)  # tied head: h @ embed.weight.T


def tiny_state(c: Cfg, *, seed: int = 0, embed_scale: float = 1.0) -> dict[str, torch.Tensor]:
    """Random fp32 weights in the reference fixture's recipe. ``embed_scale``
    shrinks the (tied) embedding so the blocks, not the token's own embedding,
    decide the next token (the recipe's unit embedding makes greedy decoding
    repeat the last token)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    H, KV = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
    st = {"embed.weight": r(c.vocab_size, c.hidden_size) * embed_scale,
          "final_norm.weight": torch.ones(c.hidden_size)}
    for i in range(c.num_hidden_layers):
        p = f"layers.{i}."
        st[p + "norm1.weight"] = torch.ones(c.hidden_size)
        st[p + "norm2.weight"] = torch.ones(c.hidden_size)
        st[p + "attn.q.weight"] = r(H, c.hidden_size) * 0.1
        st[p + "attn.k.weight"] = r(KV, c.hidden_size) * 0.1
        st[p + "attn.v.weight"] = r(KV, c.hidden_size) * 0.1
        st[p + "attn.o.weight"] = r(c.hidden_size, H) * 0.1
        st[p + "attn.q_norm.weight"] = torch.ones(c.head_dim)
        st[p + "attn.k_norm.weight"] = torch.ones(c.head_dim)
        st[p + "ffn.gate.weight"] = r(c.intermediate_size, c.hidden_size) * 0.1
        st[p + "ffn.up.weight"] = r(c.intermediate_size, c.hidden_size) * 0.1
        st[p + "ffn.down.weight"] = r(c.hidden_size, c.intermediate_size) * 0.1
    return st


def tiny_model(c: Cfg, *, seed: int = 0, dtype=torch.bfloat16, device="cpu",
               state: dict | None = None) -> Qwen3Model:
    m = Qwen3Model(c)
    missing, unexpected = m.load_state_dict(state if state is not None else tiny_state(c, seed=seed),
                                            strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return m.to(dtype=dtype, device=device).eval()


@torch.no_grad()
def random_model(c: Cfg, *, device="cuda", seed: int = 0, dtype=torch.bfloat16) -> Qwen3Model:
    """A model of config c with random weights drawn on the device (the 4B
    shapes would take minutes and 16 GB of host memory through tiny_state):
    projections N(0, 0.02), embedding N(0, 0.02), norm weights 1 + N(0, 0.05)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    with torch.device(device):
        m = Qwen3Model(c)
    for name, p in m.named_parameters():
        if name.endswith("norm.weight") or ".norm" in name or "_norm" in name:
            p.copy_(1.0 + 0.05 * torch.randn(p.shape, generator=g, device=device))
        else:
            p.copy_(0.02 * torch.randn(p.shape, generator=g, device=device))
    return m.to(device=device, dtype=dtype).eval()


def greedy_generate(model: Qwen3Model, prompt: list[int], n_new: int, device) -> list[int]:
    """Prefill the prompt, then decode n_new tokens one at a time (argmax)."""
    ids = torch.tensor([prompt], dtype=torch.long, device=device)
    cache = model.alloc_cache(len(prompt) + n_new + 4)
    out: list[int] = []
    with torch.inference_mode():
        logits = model(ids, cache, start_pos=0)
        nt = logits[:, -1, :].argmax(-1, keepdim=True)
        out.append(int(nt.item()))
        for _ in range(n_new - 1):
            logits = model(nt, cache)
            nt = logits[:, -1, :].argmax(-1, keepdim=True)
            out.append(int(nt.item()))
    return out


def teacher_forced_logits(model: Qwen3Model, tokens: list[int], device) -> torch.Tensor:
    """Logits at every position of ``tokens`` fed as one prefill."""
    ids = torch.tensor([tokens], dtype=torch.long, device=device)
    with torch.inference_mode():
        return model(ids, model.alloc_cache(len(tokens) + 4), start_pos=0)[0].float()


class StepGraph:
    """One forward step of T tokens (T = 1: decode; T = 2..9: speculative
    verify) captured in a HIP graph against a fixed cache, replayable at any
    position: ``step(ids, pos)`` copies the tokens and the position into the
    graph's static buffers, replays, and returns the static logits tensor
    (overwritten by the next replay). The warm-up runs before capture write
    the last T positions of the cache, so callers keep those free."""

    def __init__(self, model: Qwen3Model, cache: KVCache, T: int = 1, batch: int = 1):
        dev = model.embed.weight.device
        self.model, self.cache, self.T = model, cache, T
        self.ids = torch.zeros((batch, T), dtype=torch.long, device=dev)
        self.pos = torch.full((), cache.k[0].shape[2] - T, dtype=torch.long, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.inference_mode(), torch.cuda.stream(side):
            for _ in range(2):  # load code objects, settle the caching allocator
                model(self.ids, cache, start_pos=self.pos)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.graph):
            self.logits = model(self.ids, cache, start_pos=self.pos)
        torch.cuda.synchronize(dev)

    def __call__(self, ids: torch.Tensor, pos: int) -> torch.Tensor:
        self.ids.copy_(ids)
        self.pos.fill_(pos)
        self.graph.replay()
        return self.logits


def graph_greedy_generate(model: Qwen3Model, prompt: list[int], n_new: int, device) -> list[int]:
    """``greedy_generate`` with every decode step replayed from one captured
    ``StepGraph`` (the prefill runs eagerly)."""
    ids = torch.tensor([prompt], dtype=torch.long, device=device)
    cache = model.alloc_cache(len(prompt) + n_new + 4)
    with torch.inference_mode():
        logits = model(ids, cache, start_pos=0)
    step = StepGraph(model, cache, T=1)
    nt = logits[:, -1, :].argmax(-1, keepdim=True)
    out = [int(nt.item())]
    pos = len(prompt)
    for _ in range(n_new - 1):
        nt = step(nt, pos)[:, -1, :].argmax(-1, keepdim=True)
        out.append(int(nt.item()))
        pos += 1
    return out
