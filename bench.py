#!/usr/bin/env python3
"""Benchmark of the fused QKV + gate-up-SiLU projections on one MI355X.

A step is one pass of the hot path over a Qwen3 decoder stack: for each of
``--layers`` (36) layers, the fused QKV projection then the fused gate-up-SiLU,
each layer with its own weight set (N(0, 0.02) bf16), so the 4.72 GB working
set of Qwen3-4B is far above the 256 MB Infinity Cache. Inputs x ~ N(0, 1)
are resident in HBM before timing starts. The step's 72 launches are captured
once in a HIP graph and replayed.

Headline metric: HBM GB/s at M=1 on Qwen3-4B shapes =
algorithmic bytes per layer pair (2K(N_qkv+2I) + 4MK + 2M(N_qkv+I)) x layers /
step time. Also reported: TFLOP/s at M=2048 (prefill), the dominant kernel's
roofline (per-launch HIP events on its stream), the model's other BASELINE
cells (``cells``: bf16 spec-verify at M=4 with hipBLASLt beside it, int8 at
M=1, 4 and 2048; per-launch µs by graph replay), and the reference's unfused
torch path timed on this host's CPU cores.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 100]
Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, GB/s
# MI355X dense bf16 MFMA, TFLOP/s: 256 CUs x 4 SIMDs x 1024 FLOP/clk x 2.4 GHz
PEAK_BF16_TFLOPS = 2516.6
PEAK_CLOCK_GHZ = 2.4
METRIC = "HBM GB/s (% peak) fused QKV+gate-up-SiLU Qwen3-4B M=1; TFLOPS at M=2048"

# (K, n_q, n_k, I)
SHAPES = {
    "qwen3-0.6b": (1024, 2048, 1024, 3072),
    "qwen3-4b": (2560, 4096, 1024, 9728),
    "qwen3-8b": (4096, 4096, 1024, 12288),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def pair_bytes(M: int, K: int, n_qkv: int, inter: int) -> int:
    """Algorithmic HBM bytes of one (QKV, gate-up) layer pair."""
    return 2 * K * (n_qkv + 2 * inter) + 4 * M * K + 2 * M * (n_qkv + inter)


def gate_up_bytes(M: int, K: int, inter: int) -> int:
    return 2 * K * 2 * inter + 2 * M * K + 2 * M * inter


def pair_flops(M: int, K: int, n_qkv: int, inter: int) -> int:
    return 2 * M * K * (n_qkv + 2 * inter)


class Stack:
    """Per-layer weights and inputs for one shape, resident on the GPU."""

    def __init__(self, torch, shape, layers: int, M: int, seed: int = 0):
        K, n_q, n_k, inter = shape
        self.K, self.n_q, self.n_k, self.I = K, n_q, n_k, inter
        self.n_qkv = n_q + 2 * n_k
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        bf = torch.bfloat16

        def w(rows):
            return (torch.randn(rows, K, generator=g, device="cuda") * 0.02).to(bf)

        self.wqkv = [w(self.n_qkv) for _ in range(layers)]
        self.wg = [w(inter) for _ in range(layers)]
        self.wu = [w(inter) for _ in range(layers)]
        self.set_m(torch, M, seed=seed)

    def set_m(self, torch, M: int, g=None, seed=None):
        """New x rows for M; with `seed`, drawn from a fresh generator of that
        seed (the rows of a Stack built with it, when M matches)."""
        self.M = M
        if seed is not None:
            g = torch.Generator(device="cuda")
            g.manual_seed(seed + 1)
        self.x_attn = torch.randn(M, self.K, generator=g, device="cuda").to(torch.bfloat16)
        self.x_ffn = torch.randn(M, self.K, generator=g, device="cuda").to(torch.bfloat16)


def run_step(stack: Stack, kern) -> None:
    for l in range(len(stack.wqkv)):
        kern.triton_fused_qkv(stack.x_attn, stack.wqkv[l], n_q=stack.n_q, n_k=stack.n_k)
        kern.triton_fused_gate_up_silu(stack.x_ffn, stack.wg[l], stack.wu[l])


def capture(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def time_graph(torch, graph, steps: int, warmup: int) -> float:
    """Seconds per replay over `steps` replays (after `warmup`), bracketed by
    synchronisations."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / 1e3 / steps


def kernel_seconds(torch, launches: list, reps: int) -> float:
    """Average duration (s) of one launch of a kernel: the launches (one per
    layer weight set) are captured in a HIP graph, the graph is replayed
    `reps` times between HIP events on the stream it runs on, and the elapsed
    time is divided by the number of launches. Graph replay keeps the GPU fed
    back-to-back, so no host launch latency is counted."""
    graph = capture(torch, lambda: [fn() for fn in launches])
    sec = time_graph(torch, graph, reps, warm_replays(torch, graph, 2))
    del graph
    return sec / len(launches)


def warm_replays(torch, graph, floor: int) -> int:
    """Replays that make ~100 ms (at least `floor`): after an idle gap the GPU
    clocks need that long to settle (a cold 10 ms window reads 5-9% slow on
    the prefill kernels)."""
    once = time_graph(torch, graph, 1, 1)
    return max(floor, int(0.1 / max(once, 1e-6)))


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "rows_kernel_qwen3-4b_decode_m1.md")


def profiled_traffic(path: str = TRAFFIC_PROFILE):
    """HBM bytes per launch of the dominant kernel from its committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or
    None when the summary is absent."""
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(ln.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """The job's CPU share: the affinity mask, capped by OMP_NUM_THREADS
    (set to the box's per-job share)."""
    aff = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", aff) or aff)
    return max(1, min(aff, share))


def cpu_time_pair(torch, shape, x1, x2, W, reps: int) -> float:
    """Median seconds per (QKV, gate-up) layer pair of the reference's
    unfused torch path (oracle.torch_path) on the host CPU, cycling the
    weight sets W in order, after one warm-up pass."""
    from oracle import torch_path as tp

    K, n_q, n_k, inter = shape
    for wq, wg, wu in W:  # warm-up pass
        tp.torch_qkv(x1, wq, n_q, n_k)
        tp.torch_gate_up_silu(x2, wg, wu)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for wq, wg, wu in W:
            tp.torch_qkv(x1, wq, n_q, n_k)
            tp.torch_gate_up_silu(x2, wg, wu)
        times.append((time.perf_counter() - t0) / len(W))
    return statistics.median(times)


def cpu_baseline(torch, stacks: dict, reps: int) -> dict:
    """The reference's unfused bf16 torch path on the host CPU for each
    {config name: (shape, Stack)}: the inputs are the GPU run's own (the
    Stack's x rows and its layer weight sets, generated on the device from
    the same seed and copied to the host), every weight set cycled once per
    pass, median of `reps` passes. The first entry is the reported value."""
    threads = cpu_threads()
    torch.set_num_threads(threads)
    per = {}
    for name, (shape, stack) in stacks.items():
        K, n_q, n_k, inter = shape
        x1, x2 = stack.x_attn.cpu(), stack.x_ffn.cpu()
        W = [(a.cpu(), b.cpu(), c.cpu()) for a, b, c in zip(stack.wqkv, stack.wg, stack.wu)]
        sec = cpu_time_pair(torch, shape, x1, x2, W, reps)
        per[name] = {"gbs": round(pair_bytes(stack.M, K, n_q + 2 * n_k, inter) / sec / 1e9, 2),
                     "ms_per_layer_pair": round(sec * 1e3, 4), "M": stack.M,
                     "weight_sets": len(W)}
        del W
    first = next(iter(per))
    return {
        "value": per[first]["gbs"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/torch_path.py, the reference's unfused bf16 torch path "
                   f"(F.linear+split, F.silu(F.linear)*F.linear) on the host CPU with the GPU "
                   f"run's inputs (device-generated from seed 0, copied to the host), every "
                   f"layer weight set cycled once per pass, median of {reps} passes; value = "
                   f"{first}; cpu: {cpu_model()}"),
        "configs": per,
    }


def clock_under_load(torch, graph, seconds: float = 0.3) -> dict:
    """The graphics clock while `graph` runs: the graph is replayed for about
    `seconds` while a host thread samples amdsmi's GPU metrics
    (current_gfxclks, one value per XCD) every ~2 ms. Each XCD's figure is
    the median of its samples over the middle 80% of the window; the reported
    clock is the highest of them. The kernels run on every XCD, so the
    highest reading is the conservative one for a fraction of peak: one box
    gave a mean of 1.27 GHz over its XCDs while the prefill ran at the same
    speed as on boxes that read 2.2 GHz, which made an impossible 89% of
    peak at that clock. None when amdsmi is not available."""
    import threading

    try:
        import amdsmi

        amdsmi.amdsmi_init()
        handles = amdsmi.amdsmi_get_processor_handles()
        h = handles[torch.cuda.current_device()] if len(handles) > 1 else handles[0]
    except Exception as e:  # noqa: BLE001 - report, do not fail the bench
        return {"ghz_under_load": None, "method": f"amdsmi unavailable ({type(e).__name__})"}

    def sample():
        m = amdsmi.amdsmi_get_gpu_metrics_info(h)
        v = m.get("current_gfxclks")
        vals = v if isinstance(v, list) else [m.get("current_gfxclk")]
        return [float(c) if isinstance(c, (int, float)) and 0 < c < 10000 else None
                for c in vals]

    once = time_graph(torch, graph, 1, 1)
    reps = max(4, int(seconds / max(once, 1e-6)))
    samples, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            try:
                c = sample()
            except Exception:  # noqa: BLE001
                c = None
            if c and any(v is not None for v in c):
                samples.append(c)
            time.sleep(0.002)

    for _ in range(reps):
        graph.replay()
    t = threading.Thread(target=poll)
    t.start()
    torch.cuda.synchronize()
    stop.set()
    t.join()
    n = len(samples)
    window = samples[n // 10: n - n // 10] if n >= 10 else samples
    per_xcd = []
    for j in range(max((len(c) for c in window), default=0)):
        col = sorted(c[j] for c in window if j < len(c) and c[j] is not None)
        if col:
            per_xcd.append(round(col[len(col) // 2] / 1e3, 3))
    top = max(per_xcd) if per_xcd else None
    return {"ghz_under_load": top, "per_xcd_ghz": per_xcd, "samples": n,
            "method": "amdsmi current_gfxclks sampled every ~2 ms during "
                      f"{reps} prefill graph replays; per XCD the median of the middle 80%, "
                      "reported: the highest XCD"}


def counters_run(torch, kern, shape, layers: int, Mp: int = 2048, blt: bool = False) -> dict:
    """A short fixed sequence for `rocprofv3 --pmc` runs: a plain device copy
    of known size (calibrates FETCH_SIZE / WRITE_SIZE), then three passes of
    the decode (M=1) fused kernels over `layers` cycled weight sets and three
    of the prefill (M=Mp, default 2048) kernels over 4 of them. With `blt`,
    then three passes of torch's F.linear (hipBLASLt) on the same prefill
    contractions (one GEMM over [Wq; Wk; Wv] and one over [Wg; Wu], no
    epilogue), for a side-by-side profile."""
    K, n_q, n_k, inter = shape
    n_qkv = n_q + 2 * n_k
    copy_bytes = 256 << 20
    src = torch.empty(copy_bytes // 2, dtype=torch.bfloat16, device="cuda").normal_()
    dst = torch.empty_like(src)
    stack = Stack(torch, shape, layers, M=1)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(3):
        run_step(stack, kern)
    torch.cuda.synchronize()
    stack.set_m(torch, Mp)
    for _ in range(3):
        for l in range(min(4, layers)):
            kern.triton_fused_qkv(stack.x_attn, stack.wqkv[l], n_q=n_q, n_k=n_k)
            kern.triton_fused_gate_up_silu(stack.x_ffn, stack.wg[l], stack.wu[l])
    torch.cuda.synchronize()
    if blt:
        import torch.nn.functional as F

        cat_g = [torch.cat([stack.wg[l], stack.wu[l]]) for l in range(min(4, layers))]
        torch.cuda.synchronize()
        for _ in range(3):
            for l in range(min(4, layers)):
                F.linear(stack.x_attn, stack.wqkv[l])
                F.linear(stack.x_ffn, cat_g[l])
        torch.cuda.synchronize()
    return {
        "mode": "counters",
        "copy": {"kernel": "bfloat16_copy_kernel", "read_bytes": copy_bytes,
                 "write_bytes": copy_bytes, "launches": 3},
        "gate_up_m1": {"read_bytes": 2 * K * 2 * inter + 2 * K, "write_bytes": 2 * inter,
                       "launches": 3 * layers},
        "qkv_m1": {"read_bytes": 2 * K * n_qkv + 2 * K, "write_bytes": 2 * n_qkv,
                   "launches": 3 * layers},
        f"gate_up_m{Mp}": {"read_bytes": 2 * K * 2 * inter + 2 * Mp * K,
                           "write_bytes": 2 * Mp * inter, "launches": 3 * min(4, layers)},
        f"qkv_m{Mp}": {"read_bytes": 2 * K * n_qkv + 2 * Mp * K,
                       "write_bytes": 2 * Mp * n_qkv, "launches": 3 * min(4, layers)},
    }


def decode_run(torch, n_tok: int, fused_only: bool = False) -> dict:
    """Greedy decode of n_tok tokens after a 128-token prefill on a Qwen3-4B-
    shaped decoder (``llms_amd.harness``, random weights): the reference's
    eager modules (hipBLASLt ``F.linear``, torch RMSNorm), then the same model
    after ``apply_triton_kernels(fuse_norm=True, linear_down_o=True)``; each
    step eagerly and as a replayed HIP graph (``StepGraph``), plus the
    graph-replayed verify step of 4 and 8 draft tokens. Times are wall-clock
    per step with the argmax fed back on the device."""
    from llms_amd.harness import QWEN3_4B, StepGraph, random_model
    from llms_amd.kernels import apply_triton_kernels

    c = QWEN3_4B
    P = 128
    # room for the longest run (verify T = 8: (n_tok + 2) steps of 8) plus
    # StepGraph's scratch positions at the end of the cache
    S = P + (n_tok + 4) * 8 + 16
    assert S <= c.max_position_embeddings
    log(f"decode: building a random Qwen3-4B-shaped model ({c.num_hidden_layers} layers)")
    m = random_model(c, seed=0)
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    prompt = torch.randint(0, c.vocab_size, (1, P), generator=g, device="cuda")

    def prefill():
        cache = m.alloc_cache(S)
        with torch.inference_mode():
            logits = m(prompt, cache, start_pos=0)
        return cache, logits[:, -1:].argmax(-1)

    def eager_ms():
        cache, nt = prefill()
        with torch.inference_mode():
            for i in range(2):  # warm-up steps
                nt = m(nt, cache, start_pos=P + i)[:, -1:].argmax(-1)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(n_tok):
                nt = m(nt, cache, start_pos=P + 2 + i)[:, -1:].argmax(-1)
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_tok * 1e3

    def graph_ms(T: int):
        cache, nt = prefill()
        step = StepGraph(m, cache, T=T)
        ids = nt.repeat(1, T)
        for i in range(2):
            step(ids, P + i * T)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n_tok):
            ids = step(ids, P + (2 + i) * T)[:, -1:].argmax(-1).repeat(1, T)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_tok * 1e3

    out = {"mode": "decode", "model": "qwen3-4b shapes, random weights", "prompt": P,
           "tokens": n_tok, "ms_per_token": {}, "verify_ms_per_step": {}}
    if not fused_only:
        out["ms_per_token"]["reference_eager"] = round(eager_ms(), 3)
        out["ms_per_token"]["reference_graph"] = round(graph_ms(1), 3)
        log("decode: reference path timed; swapping in the fused modules")
    apply_triton_kernels(m, fuse_norm=True, linear_down_o=True)
    if fused_only:
        # only the graph-replayed fused decode step (for a kernel trace of it)
        out["ms_per_token"]["fused_graph"] = round(graph_ms(1), 3)
        out["tokens_per_s"] = {k: round(1e3 / v, 1) for k, v in out["ms_per_token"].items()}
        return out
    out["ms_per_token"]["fused_eager"] = round(eager_ms(), 3)
    out["ms_per_token"]["fused_graph"] = round(graph_ms(1), 3)
    for T in (4, 8):
        out["verify_ms_per_step"][f"fused_graph_T{T}"] = round(graph_ms(T), 3)
    out["tokens_per_s"] = {k: round(1e3 / v, 1) for k, v in out["ms_per_token"].items()}
    return out


def launch_gap_run(torch, kern, reps: int) -> dict:
    """What a decode launch costs besides its bytes (Qwen3-4B, M = 1, graph
    replay): the gap between dependent kernels of a graph (72 one-element
    torch additions per replay, the same count as the decode step's
    launches); the 72-launch decode step over 36 distinct layer weight sets
    (the headline workload) and over one weight set reused by every layer
    (131 MB, within the 256 MB Infinity Cache); and the two fused launches
    alone on 36 sets. One JSON line."""
    K, n_q, n_k, inter = SHAPES["qwen3-4b"]
    n_qkv = n_q + 2 * n_k
    out = {"mode": "launch_gap", "shape": "qwen3-4b", "M": 1}
    z = torch.zeros(1, device="cuda")
    g = capture(torch, lambda: [z.add_(1.0) for _ in range(72)])
    out["tiny_kernel_us"] = round(time_graph(torch, g, reps, 200) / 72 * 1e6, 3)
    del g
    st = Stack(torch, SHAPES["qwen3-4b"], 36, M=1)
    for name, layer in (("step_36_sets", lambda l: l), ("step_1_set", lambda l: 0)):
        g = capture(torch, lambda: [
            (kern.triton_fused_qkv(st.x_attn, st.wqkv[layer(l)], n_q=n_q, n_k=n_k),
             kern.triton_fused_gate_up_silu(st.x_ffn, st.wg[layer(l)], st.wu[layer(l)]))
            for l in range(36)])
        sec = time_graph(torch, g, reps, warm_replays(torch, g, 20))
        out[f"{name}_us"] = round(sec * 1e6, 1)
        out[f"{name}_gbs"] = round(36 * pair_bytes(1, K, n_qkv, inter) / sec / 1e9, 1)
        del g
    out["gate_up_us"] = round(kernel_seconds(torch, [
        lambda l=l: kern.triton_fused_gate_up_silu(st.x_ffn, st.wg[l], st.wu[l]) for l in range(36)],
        reps) * 1e6, 3)
    out["qkv_us"] = round(kernel_seconds(torch, [
        lambda l=l: kern.triton_fused_qkv(st.x_attn, st.wqkv[l], n_q=n_q, n_k=n_k) for l in range(36)],
        reps) * 1e6, 3)
    # what the step would take with no gap: 72 launches' worth of gaps removed
    out["step_minus_gaps_us"] = round(out["step_36_sets_us"] - 72 * out["tiny_kernel_us"], 1)
    return out


# Row-streaming launches (M = 1) whose size is swept at a fixed grid shape:
# (label, K, gate_up, int8, output widths). Each width is a whole number of
# workgroups of the shape the dispatch picks (bf16: 8 waves of one row or row
# pair; int8 with x from L2: 4 waves; K = 4096: x staged in LDS).
LAUNCH_FIT = (
    ("bf16 gate-up, K=2560, 8 waves x 1 row pair", 2560, True, False, (1216, 2432, 4864, 9728, 19456)),
    ("bf16 QKV, K=2560, 8 waves x 1 row", 2560, False, False, (1536, 3072, 6144, 12288, 24576)),
    ("int8 gate-up, K=2560, 4 waves x 1 row pair", 2560, True, True, (1216, 2432, 4864, 9728, 19456)),
    ("bf16 gate-up, K=4096, 8 waves x 1 row pair, x in LDS", 4096, True, False, (1536, 3072, 6144, 12288)),
)


def launch_fit_run(torch, kern, reps: int) -> None:
    """The fixed cost F of a row-streaming launch at a given grid shape: per
    LAUNCH_FIT entry, the M = 1 launch over output widths that double, each
    timed by graph replay over enough distinct weight sets (at least 1.2 GB
    per replay, so the 256 MB Infinity Cache holds none of it between uses),
    and the least-squares line t = F + bytes / B through the points (F in us,
    B in TB/s). A one-element torch kernel in the same kind of graph gives
    the launch floor of any kernel. One JSON line per entry."""
    z = torch.zeros(1, device="cuda")
    g = capture(torch, lambda: [z.add_(1.0) for _ in range(72)])
    print(json.dumps({"mode": "launch_fit", "tiny_kernel_us":
                      round(time_graph(torch, g, reps, 200) / 72 * 1e6, 3)}), flush=True)
    del g
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    for label, K, gu, int8, widths in LAUNCH_FIT:
        pts = []
        x = torch.randn(1, K, generator=gen, device="cuda").to(torch.bfloat16)
        for N in widths:
            mats = 2 if gu else 1
            per = mats * N * K * (1 if int8 else 2) + (mats * N * 4 if int8 else 0)
            sets = int(min(400, max(8, -(-1_200_000_000 // per))))
            if int8:
                q = torch.randint(-127, 128, (sets, mats, N, K), generator=gen, device="cuda",
                                  dtype=torch.int8)
                s = torch.rand(sets, mats, N, generator=gen, device="cuda") * 1e-3 + 1e-4
                if gu:
                    fns = [lambda i=i: kern.fused_gate_up_silu_w8(x, q[i, 0], s[i, 0], q[i, 1], s[i, 1])
                           for i in range(sets)]
                else:
                    fns = [lambda i=i: kern.fused_linear_w8(x, q[i, 0], s[i, 0]) for i in range(sets)]
            else:
                w = torch.randn(sets, mats, N, K, generator=gen, device="cuda",
                                dtype=torch.bfloat16)
                if gu:
                    fns = [lambda i=i: kern.triton_fused_gate_up_silu(x, w[i, 0], w[i, 1])
                           for i in range(sets)]
                else:
                    n_k = N // 6
                    fns = [lambda i=i: kern.triton_fused_qkv(x, w[i, 0], n_q=N - 2 * n_k, n_k=n_k)
                           for i in range(sets)]
            t = kernel_seconds(torch, fns, reps)
            nbytes = per + 2 * K + 2 * N
            pts.append({"N": N, "sets": sets, "bytes": nbytes, "us": round(t * 1e6, 3)})
            del fns
            if int8:
                del q, s
            else:
                del w
            torch.cuda.empty_cache()
        n = len(pts)
        mb = sum(p["bytes"] for p in pts) / n
        mt = sum(p["us"] for p in pts) / n
        sxx = sum((p["bytes"] - mb) ** 2 for p in pts)
        slope = sum((p["bytes"] - mb) * (p["us"] - mt) for p in pts) / sxx  # us per byte
        F = mt - slope * mb
        resid = max(abs(p["us"] - (F + slope * p["bytes"])) for p in pts)
        print(json.dumps({"mode": "launch_fit", "shape": label, "points": pts,
                          "F_us": round(F, 3), "B_tbs": round(1e-6 / slope, 3),
                          "max_residual_us": round(resid, 3)}), flush=True)


NORM_M = (1, 2, 8, 64, 512)


def norm_run(torch, kern, reps: int) -> dict:
    """The RMSNorm prologue fused into the projections (Qwen3-4B QKV and
    gate-up, bf16): per M in NORM_M, the fused call (fused_rmsnorm_qkv /
    fused_rmsnorm_gate_up_silu: one launch in the row-streaming regime, M <=
    2; else the norm kernel, then the projection) against the eager pair the
    engine runs (the reference's RMSNorm module restated in
    llms_amd.kernels._eager, then the fused projection) and the projection
    alone. Graph replay over cycled weight sets (36 up to 64 rows, 4 at 512),
    average per call. One JSON line per M."""
    from llms_amd.kernels import fused_norm as fn
    from llms_amd.kernels._eager import RMSNorm

    K, n_q, n_k, inter = SHAPES["qwen3-4b"]
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    norm = RMSNorm(K).cuda().to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(K, generator=g, device="cuda"))
    gamma = norm.weight.detach()
    for M in NORM_M:
        L = 36 if M <= 64 else 4
        st = Stack(torch, SHAPES["qwen3-4b"], L, M, seed=M)
        out = {"mode": "norm", "M": M, "weight_sets": L}
        with torch.no_grad():
            cases = {
                "qkv_fused": lambda l: fn.fused_rmsnorm_qkv(st.x_attn, gamma, norm.eps, st.wqkv[l],
                                                            n_q=n_q, n_k=n_k),
                "qkv_norm_then_qkv": lambda l: kern.triton_fused_qkv(norm(st.x_attn), st.wqkv[l],
                                                                     n_q=n_q, n_k=n_k),
                "qkv_alone": lambda l: kern.triton_fused_qkv(st.x_attn, st.wqkv[l], n_q=n_q, n_k=n_k),
                "gate_up_fused": lambda l: fn.fused_rmsnorm_gate_up_silu(st.x_ffn, gamma, norm.eps,
                                                                         st.wg[l], st.wu[l]),
                "gate_up_norm_then_gate_up": lambda l: kern.triton_fused_gate_up_silu(
                    norm(st.x_ffn), st.wg[l], st.wu[l]),
                "gate_up_alone": lambda l: kern.triton_fused_gate_up_silu(st.x_ffn, st.wg[l], st.wu[l]),
            }
            for name, fn_l in cases.items():
                t = kernel_seconds(torch, [lambda l=l, f=fn_l: f(l) for l in range(L)], reps)
                out[f"{name}_us"] = round(t * 1e6, 2)
        print(json.dumps(out), flush=True)
        del st
        torch.cuda.empty_cache()
    return {"mode": "norm", "done": True}


def linear_run(torch, kern, M: int, N: int, K: int, reps: int) -> dict:
    """The plain projection y = x W^T (the engine's down / o Linears) over
    weight sets cycled past the Infinity Cache: average launch duration by
    graph replay, and torch's F.linear (hipBLASLt) on the same shape for scale."""
    import torch.nn.functional as F

    sets = max(2, min(32, (600 << 20) // (2 * N * K)))
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    ws = [(torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
          for _ in range(sets)]
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    ours = kernel_seconds(torch, [lambda w=w: kern.fused_linear(x, w) for w in ws], reps)
    ref = kernel_seconds(torch, [lambda w=w: F.linear(x, w) for w in ws], reps)
    flops = 2 * M * N * K
    return {"mode": "linear", "M": M, "N": N, "K": K, "weight_sets": sets,
            "us": round(ours * 1e6, 2), "tflops": round(flops / ours / 1e12, 1),
            "gbs": round((2 * N * K + 2 * M * K + 2 * M * N) / ours / 1e9, 1),
            "hipblaslt_us": round(ref * 1e6, 2)}


def _median_event_us(torch, fn, warmup: int, iters: int) -> float:
    """The reference microbench's timer (src/bench/microbench_fused_qkv.py
    _time_fn): `warmup` calls, then one pair of HIP events around each of
    `iters` calls on the current stream, median in microseconds."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        st[i].record()
        fn()
        en[i].record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) * 1e3 for a, b in zip(st, en))


def ship_gate_run(torch, kern, warmup: int = 50, iters: int = 200) -> dict:
    """The reference's microbench ship gate on the Qwen3-4B shapes at M in
    {1, 5, 8} (tests/test_kernels_fused_qkv.py:286-311,
    tests/test_kernels_fused_ffn.py:238-265; inputs as in
    src/bench/microbench_fused_{qkv,ffn}.py: torch.manual_seed(0), randn bf16
    on the device). QKV: the fused call against eager_3_linears (the formal
    gate) and eager_concat_linear (one F.linear over [Wq; Wk; Wv] + split,
    informational). Gate-up: the fused call against eager
    silu(x Wg^T) * (x Wu^T). pass: fused median <= the gate's median, the
    reference's criterion."""
    import torch.nn.functional as F

    K, n_q, n_k, inter = SHAPES["qwen3-4b"]
    bf = torch.bfloat16
    out = {"mode": "ship_gate", "shape": "qwen3-4b", "warmup": warmup, "iters": iters,
           "timer": "median of per-call HIP events (reference microbench method)",
           "qkv": {}, "gate_up": {}}
    for M in (1, 5, 8):
        torch.manual_seed(0)
        x = torch.randn(M, K, device="cuda", dtype=bf)
        Wq = torch.randn(n_q, K, device="cuda", dtype=bf)
        Wk = torch.randn(n_k, K, device="cuda", dtype=bf)
        Wv = torch.randn(n_k, K, device="cuda", dtype=bf)
        W = torch.cat([Wq, Wk, Wv], dim=0).contiguous()
        e3 = _median_event_us(torch, lambda: (F.linear(x, Wq), F.linear(x, Wk), F.linear(x, Wv)),
                              warmup, iters)
        ec = _median_event_us(torch, lambda: F.linear(x, W).split([n_q, n_k, n_k], dim=-1),
                              warmup, iters)
        fu = _median_event_us(torch, lambda: kern.triton_fused_qkv(x, W, n_q=n_q, n_k=n_k),
                              warmup, iters)
        out["qkv"][f"M={M}"] = {"eager_3_linears_us": round(e3, 2),
                                "eager_concat_linear_us": round(ec, 2),
                                "fused_us": round(fu, 2),
                                "speedup_vs_3_linears": round(e3 / fu, 3),
                                "speedup_vs_concat": round(ec / fu, 3),
                                "pass": fu <= e3}
        del Wq, Wk, Wv, W
        torch.manual_seed(0)
        x = torch.randn(M, K, device="cuda", dtype=bf)
        Wg = torch.randn(inter, K, device="cuda", dtype=bf)
        Wu = torch.randn(inter, K, device="cuda", dtype=bf)
        ee = _median_event_us(torch, lambda: F.silu(F.linear(x, Wg)) * F.linear(x, Wu),
                              warmup, iters)
        fu = _median_event_us(torch, lambda: kern.triton_fused_gate_up_silu(x, Wg, Wu),
                              warmup, iters)
        out["gate_up"][f"M={M}"] = {"eager_us": round(ee, 2), "fused_us": round(fu, 2),
                                    "speedup": round(ee / fu, 3), "pass": fu <= ee}
        del Wg, Wu
    out["pass"] = all(v["pass"] for d in (out["qkv"], out["gate_up"]) for v in d.values())
    return out


# The kernel families profiled under profiles/ besides the default bench's
# decode and prefill grids: (label, model, M, int8, tensor-parallel degree of
# the per-GPU shard, 1 for the whole layer).
PROFILE_SET = [
    ("int8 decode", "qwen3-4b", 1, True, 1),
    ("int8 verify", "qwen3-4b", 4, True, 1),
    ("int8 prefill", "qwen3-4b", 2048, True, 1),
    ("bf16 verify M=3", "qwen3-4b", 3, False, 1),
    ("bf16 verify M=8", "qwen3-4b", 8, False, 1),
    ("8B M=64", "qwen3-8b", 64, False, 1),
    ("8B M=256", "qwen3-8b", 256, False, 1),
    ("8B int8 M=64", "qwen3-8b", 64, True, 1),
    ("8B int8 M=256", "qwen3-8b", 256, True, 1),
    ("8B M=4096", "qwen3-8b", 4096, False, 1),
    ("8B int8 M=4096", "qwen3-8b", 4096, True, 1),
    ("prefill M=8192", "qwen3-4b", 8192, False, 1),
    ("8B TP=2 shard M=512", "qwen3-8b", 512, False, 2),
    ("8B TP=4 shard M=512", "qwen3-8b", 512, False, 4),
    ("8B TP=8 shard M=512", "qwen3-8b", 512, False, 8),
]


def profile_set_run(torch, kern, reps: int, only: str | None = None) -> dict:
    """A fixed sequence for rocprofv3 runs (kernel trace, --pmc passes): each
    PROFILE_SET entry over its own cycled weight sets (36 for decode-sized
    calls, else enough to pass the Infinity Cache), replayed in a HIP graph
    `reps` times after a short warm-up; one JSON line per entry with the
    measured per-launch times."""
    out = {"mode": "profile_set", "entries": []}
    for label, model, M, int8, tp in PROFILE_SET:
        if only is not None and label != only:
            continue
        K, n_q, n_k, inter = shard_shape(model, tp)
        n = n_q + 2 * n_k
        wbytes = (1 if int8 else 2) * K * (n + 2 * inter)
        sets = 36 if M <= 64 else max(4, min(36, (1200 << 20) // wbytes))
        g = torch.Generator(device="cuda")
        g.manual_seed(0)
        x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)

        def w(rows):
            return (torch.randn(rows, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)

        ws = []
        for _ in range(sets):
            t = (w(n), w(inter), w(inter))
            ws.append(tuple(kern.quantize_w8_per_row(v) for v in t) if int8 else t)
        if int8:
            qk = [lambda t=t: kern.fused_qkv_w8(x, t[0][0], t[0][1], n_q=n_q, n_k=n_k) for t in ws]
            gu = [lambda t=t: kern.fused_gate_up_silu_w8(x, t[1][0], t[1][1], t[2][0], t[2][1])
                  for t in ws]
        else:
            qk = [lambda t=t: kern.triton_fused_qkv(x, t[0], n_q=n_q, n_k=n_k) for t in ws]
            gu = [lambda t=t: kern.triton_fused_gate_up_silu(x, t[1], t[2]) for t in ws]
        ent = {"label": label, "model": model, "tp": tp, "M": M,
               "weights": "int8" if int8 else "bf16", "weight_sets": sets}
        for name, launches in (("qkv", qk), ("gate_up", gu)):
            graph = capture(torch, lambda: [fn() for fn in launches])
            sec = time_graph(torch, graph, reps, 2) / len(launches)
            del graph
            ent[f"{name}_us"] = round(sec * 1e6, 2)
        print(json.dumps(ent), flush=True)
        out["entries"].append(ent)
        del ws, qk, gu
        torch.cuda.empty_cache()
    return out


# Every configuration BASELINE.json lists: (model, M, int8).
CONFIGS = ([("qwen3-0.6b", 1, False)]
           + [("qwen3-4b", m, False) for m in (1, 3, 4, 8, 512, 2048, 8192)]
           + [("qwen3-4b", m, True) for m in (1, 4, 2048)]
           + [("qwen3-8b", m, q) for q in (False, True) for m in (1, 4, 16, 64, 256, 4096)])


def config_line(torch, kern, shape, M: int, int8: bool, reps: int, hipblaslt: bool = True) -> dict:
    """Both fused projections of one shape (K, n_q, n_k, I) at M rows: average
    launch duration by graph replay over distinct weight sets (36 for M <= 64,
    else enough to pass the Infinity Cache), GB/s of algorithmic bytes and
    TFLOP/s; for bf16 with `hipblaslt`, torch's F.linear (hipBLASLt) on the
    same contraction (one GEMM over [Wq; Wk; Wv] or [Wg; Wu], no epilogue)
    for scale."""
    import torch.nn.functional as F

    K, n_q, n_k, inter = shape
    n = n_q + 2 * n_k
    wbytes = (1 if int8 else 2) * K * (n + 2 * inter)
    sets = 36 if M <= 64 else max(4, min(36, (1200 << 20) // wbytes))
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)

    def w(rows):
        return (torch.randn(rows, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)

    ws = []
    for _ in range(sets):
        t = (w(n), w(inter), w(inter))
        ws.append(tuple(kern.quantize_w8_per_row(v) for v in t) if int8 else t)
        del t
    if int8:
        qk = [lambda t=t: kern.fused_qkv_w8(x, t[0][0], t[0][1], n_q=n_q, n_k=n_k) for t in ws]
        gu = [lambda t=t: kern.fused_gate_up_silu_w8(x, t[1][0], t[1][1], t[2][0], t[2][1])
              for t in ws]
    else:
        qk = [lambda t=t: kern.triton_fused_qkv(x, t[0], n_q=n_q, n_k=n_k) for t in ws]
        gu = [lambda t=t: kern.triton_fused_gate_up_silu(x, t[1], t[2]) for t in ws]
    tq = kernel_seconds(torch, qk, reps)
    tg = kernel_seconds(torch, gu, reps)
    wb = 1 if int8 else 2
    bq = wb * n * K + (4 * n if int8 else 0) + 2 * M * K + 2 * M * n
    bg = wb * 2 * inter * K + (8 * inter if int8 else 0) + 2 * M * K + 2 * M * inter
    out = {"M": M, "weights": "int8" if int8 else "bf16", "weight_sets": sets,
           "qkv_us": round(tq * 1e6, 2), "qkv_gbs": round(bq / tq / 1e9, 1),
           "qkv_tflops": round(2 * M * K * n / tq / 1e12, 1),
           "gate_up_us": round(tg * 1e6, 2), "gate_up_gbs": round(bg / tg / 1e9, 1),
           "gate_up_tflops": round(2 * M * K * 2 * inter / tg / 1e12, 1)}
    if hipblaslt and not int8:
        cat_q = [t[0] for t in ws]
        cat_g = [torch.cat([t[1], t[2]]) for t in ws]
        out["hipblaslt_qkv_us"] = round(
            kernel_seconds(torch, [lambda c=c: F.linear(x, c) for c in cat_q], reps) * 1e6, 2)
        out["hipblaslt_gate_up_us"] = round(
            kernel_seconds(torch, [lambda c=c: F.linear(x, c) for c in cat_g], reps) * 1e6, 2)
        del cat_g
    del ws, qk, gu
    torch.cuda.empty_cache()
    return out


# BASELINE cells of the bench model reported beside the headline (M, int8):
# spec-verify in bf16, and the int8 decode, verify and prefill configurations
BENCH_CELLS = ((4, False), (1, True), (4, True), (2048, True))


def configs_run(torch, kern, reps: int):
    """Both fused projections on every BASELINE configuration, one JSON line
    each (config_line)."""
    for model, M, int8 in CONFIGS:
        out = {"mode": "config", "model": model}
        out.update(config_line(torch, kern, SHAPES[model], M, int8, reps))
        print(json.dumps(out), flush=True)


# Per-GPU shards of tensor parallelism: QKV column-parallel by heads (n_q /
# tp query and n_k / tp key/value columns), gate-up column-parallel over I
# with Wg and Wu split alike. The rows each GPU computes at the M of the
# decode, verify and prefill configurations.
SHARD_TP = (2, 4, 8)
SHARD_M = (1, 4, 8, 512, 2048)


def shard_shape(model: str, tp: int):
    K, n_q, n_k, inter = SHAPES[model]
    return (K, n_q // tp, n_k // tp, inter // tp)


def shards_run(torch, kern, reps: int):
    """Both fused projections on the per-GPU shard of TP = 2, 4, 8 for
    Qwen3-4B and -8B (one JSON line per model, tp and M), with the layer
    pair's time and its fraction of the HBM (M <= 8) or MFMA (M >= 512)
    peak. One GPU runs one shard: what it shows is each GPU's share of a TP
    layer, without the all-reduce that follows o and down."""
    for model in ("qwen3-4b", "qwen3-8b"):
        for tp in SHARD_TP:
            shape = shard_shape(model, tp)
            K, n_q, n_k, inter = shape
            for M in SHARD_M:
                out = {"mode": "shard", "model": model, "tp": tp, "K": K,
                       "n_qkv": n_q + 2 * n_k, "I": inter}
                out.update(config_line(torch, kern, shape, M, False, reps))
                pair_us = out["qkv_us"] + out["gate_up_us"]
                out["pair_us"] = round(pair_us, 2)
                if M <= 8:
                    gbs = pair_bytes(M, K, n_q + 2 * n_k, inter) / pair_us / 1e3
                    out["pair_gbs"] = round(gbs, 1)
                    out["frac_of_peak"] = round(gbs / PEAK_HBM_GBS, 4)
                else:
                    tf = pair_flops(M, K, n_q + 2 * n_k, inter) / pair_us / 1e6
                    out["pair_tflops"] = round(tf, 1)
                    out["frac_of_peak"] = round(tf / PEAK_BF16_TFLOPS, 4)
                print(json.dumps(out), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 100 untimed steps of ~0.9 ms: the clocks settle before the timed region
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--model", default="qwen3-4b", choices=sorted(SHAPES))
    ap.add_argument("--prefill-m", type=int, default=2048)
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cells", action="store_true",
                    help="skip the other BASELINE cells of the model (verify and int8) that "
                         "the default run reports beside the decode step")
    ap.add_argument("--counters", action="store_true",
                    help="run only the short fixed sequence used for rocprofv3 --pmc runs")
    ap.add_argument("--hipblaslt", action="store_true",
                    help="with --counters: also run torch's F.linear (hipBLASLt) on the "
                         "prefill contractions, for a side-by-side profile")
    ap.add_argument("--decode", action="store_true",
                    help="end-to-end decode on a Qwen3-4B-shaped harness model with random "
                         "weights: reference eager path vs fused modules, eager and "
                         "graph-replayed steps; prints one JSON line")
    ap.add_argument("--decode-tokens", type=int, default=32)
    ap.add_argument("--decode-fused", action="store_true",
                    help="with --decode: only the graph-replayed fused decode step (for a kernel "
                         "trace of that step)")
    ap.add_argument("--launch-gap", action="store_true",
                    help="the graph launch gap (72 tiny kernels) and the M = 1 decode step over "
                         "36 weight sets and over one (cache-resident); prints one JSON line")
    ap.add_argument("--launch-fit", action="store_true",
                    help="the fixed cost of a row-streaming launch at four grid shapes: M = 1 "
                         "over doubling output widths, t = F + bytes / B fitted; one JSON line "
                         "per shape")
    ap.add_argument("--norm", action="store_true",
                    help="the RMSNorm prologue fused into the projections against the eager "
                         "norm + projection, Qwen3-4B at M in 1, 2, 8, 64, 512; one JSON line "
                         "per M")
    ap.add_argument("--configs", action="store_true",
                    help="time both projections on every BASELINE configuration (with "
                         "hipBLASLt for scale); one JSON line per configuration")
    ap.add_argument("--shards", action="store_true",
                    help="time both projections on the per-GPU shards of TP = 2, 4, 8 "
                         "(Qwen3-4B and -8B); one JSON line per shard and M")
    ap.add_argument("--ship-gate", action="store_true",
                    help="the reference's microbench ship gate (fused <= eager at M = 1, 5, 8 "
                         "on Qwen3-4B QKV and gate-up); prints one JSON line")
    ap.add_argument("--profile-set", action="store_true",
                    help="the fixed kernel sequence the profiles/ summaries other than the "
                         "default bench's are taken from (one JSON line per entry)")
    ap.add_argument("--only", metavar="LABEL",
                    help="with --profile-set: run only the entry with this label")
    ap.add_argument("--linear", metavar="M,N,K",
                    help="time only the plain projection (down / o) of this shape over "
                         "cycled weight sets and print one JSON line (profiling aid)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; the fused projections shard "
              "by output columns with no collective inside the path. "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from llms_amd import kernels as kern
    from llms_amd import ops

    ops()  # load the HIP extension or fail loudly
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 2
    dev_name = torch.cuda.get_device_name(0)
    shape = SHAPES[args.model]
    K, n_q, n_k, inter = shape
    n_qkv = n_q + 2 * n_k
    L = args.layers
    if args.counters:
        print(json.dumps(counters_run(torch, kern, shape, L, args.prefill_m, args.hipblaslt)),
              flush=True)
        return 0
    if args.decode:
        print(json.dumps(decode_run(torch, args.decode_tokens, args.decode_fused)), flush=True)
        return 0
    if args.configs:
        configs_run(torch, kern, args.steps)
        return 0
    if args.norm:
        norm_run(torch, kern, args.steps)
        return 0
    if args.launch_gap:
        print(json.dumps(launch_gap_run(torch, kern, args.steps)), flush=True)
        return 0
    if args.launch_fit:
        launch_fit_run(torch, kern, args.steps)
        return 0
    if args.shards:
        shards_run(torch, kern, args.steps)
        return 0
    if args.profile_set:
        if args.only is not None and args.only not in [e[0] for e in PROFILE_SET]:
            print(f"bench.py: no profile-set entry {args.only!r}", file=sys.stderr)
            return 2
        profile_set_run(torch, kern, args.steps, args.only)
        return 0
    if args.ship_gate:
        print(json.dumps(ship_gate_run(torch, kern)), flush=True)
        return 0
    if args.linear:
        M, N, Kl = (int(v) for v in args.linear.split(","))
        print(json.dumps(linear_run(torch, kern, M, N, Kl, args.steps)), flush=True)
        return 0

    # ---------------- decode, M = 1: the headline ----------------
    log(f"device {dev_name}; allocating {L} layer weight sets of {args.model}")
    stack = Stack(torch, shape, L, M=1)
    torch.cuda.synchronize()
    graph = capture(torch, lambda: run_step(stack, kern))
    log("decode graph captured; timing")
    sec = time_graph(torch, graph, args.steps, args.warmup)
    bytes_step = L * pair_bytes(1, K, n_qkv, inter)
    value = bytes_step / sec / 1e9
    log(f"decode M=1: {sec * 1e6:.1f} us/step, {value:.1f} GB/s")

    # eager (no graph) for reference
    for _ in range(2):
        run_step(stack, kern)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(stack, kern)
    torch.cuda.synchronize()
    sec_eager = (time.perf_counter() - t0) / args.steps

    # dominant kernel (gate-up, 76% of the bytes) and QKV, each alone
    gu = [(lambda l=l: kern.triton_fused_gate_up_silu(stack.x_ffn, stack.wg[l], stack.wu[l]))
          for l in range(L)]
    qk = [(lambda l=l: kern.triton_fused_qkv(stack.x_attn, stack.wqkv[l], n_q=n_q, n_k=n_k))
          for l in range(L)]
    d_gu = kernel_seconds(torch, gu, args.steps)
    d_qk = kernel_seconds(torch, qk, args.steps)
    gu_gbs = gate_up_bytes(1, K, inter) / d_gu / 1e9
    qk_gbs = (2 * K * n_qkv + 2 * K + 2 * n_qkv) / d_qk / 1e9
    log(f"gate-up M=1: {d_gu * 1e6:.2f} us/launch {gu_gbs:.1f} GB/s; "
        f"qkv M=1: {d_qk * 1e6:.2f} us/launch {qk_gbs:.1f} GB/s")
    del graph

    # ---------------- prefill ----------------
    prefill = None
    if not args.no_prefill:
        Mp = args.prefill_m
        stack.set_m(torch, Mp)
        torch.cuda.synchronize()
        graph = capture(torch, lambda: run_step(stack, kern))
        psteps = max(3, args.steps // 4)
        psec = time_graph(torch, graph, psteps, warm_replays(torch, graph, max(1, args.warmup // 2)))
        tflops = L * pair_flops(Mp, K, n_qkv, inter) / psec / 1e12
        clk = clock_under_load(torch, graph)
        dp_gu = kernel_seconds(torch, gu, 3)
        dp_qk = kernel_seconds(torch, qk, 3)
        ghz = clk["ghz_under_load"]
        prefill = {
            "M": Mp,
            "tflops": round(tflops, 1),
            "frac_of_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
            "us_per_layer_pair": round(psec / L * 1e6, 2),
            "gate_up_us": round(dp_gu * 1e6, 2),
            "gate_up_tflops": round(2 * Mp * K * 2 * inter / dp_gu / 1e12, 1),
            "qkv_us": round(dp_qk * 1e6, 2),
            "qkv_tflops": round(2 * Mp * K * n_qkv / dp_qk / 1e12, 1),
            "peak_tflops": PEAK_BF16_TFLOPS,
            "clock": clk,
            # the same throughput against the matrix core's peak at the clock
            # measured during the replays (None if the measurement failed)
            "frac_of_peak_at_clock": (round(tflops / (PEAK_BF16_TFLOPS * ghz / PEAK_CLOCK_GHZ), 4)
                                      if ghz else None),
        }
        log(f"prefill M={Mp}: {prefill}")
        del graph

    cpu = None
    if not args.no_cpu:
        # BASELINE configs 1 (this run's decode workload, M = 1) and 0
        # (Qwen3-0.6B, M = 1), on the same device-generated inputs
        log("timing the CPU baseline")
        stack.set_m(torch, 1, seed=0)
        small = Stack(torch, SHAPES["qwen3-0.6b"], L, M=1)
        cpu = cpu_baseline(torch, {f"{args.model} M=1": (shape, stack),
                                   "qwen3-0.6b M=1": (SHAPES["qwen3-0.6b"], small)},
                           args.cpu_reps)
        del small
        log(f"cpu: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['configs']})")

    del stack
    torch.cuda.empty_cache()

    # other BASELINE cells of the same model, in the same run (config_line:
    # graph replay over distinct weight sets; bf16 with hipBLASLt beside)
    cells = None
    if not args.no_cells:
        cells = []
        for M, int8 in BENCH_CELLS:
            c = config_line(torch, kern, shape, M, int8, max(5, args.steps // 4))
            cells.append(c)
            log(f"cell M={M} {c['weights']}: qkv {c['qkv_us']} us, gate-up {c['gate_up_us']} us")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x~N(0,1), W~N(0,0.02) bf16, random-init, fixed seeds",
        "config": {
            "workload": f"{args.model} fused QKV ({K}->{n_qkv}) + gate-up-SiLU "
                        f"({K}->2x{inter}) per layer, M=1 decode, {L} distinct layer weight "
                        f"sets cycled ({L * 2 * K * (n_qkv + 2 * inter) / 1e9:.2f} GB), "
                        "one HIP graph per step",
            "model_shapes": args.model,
            "M": 1,
            "layers": L,
            "bytes_per_step": bytes_step,
        },
        "hbm_frac": round(value / PEAK_HBM_GBS, 4),
        "eager_ms_per_step": round(sec_eager * 1e3, 4),
        "decode_kernels": {
            "gate_up_us": round(d_gu * 1e6, 3),
            "qkv_us": round(d_qk * 1e6, 3),
            "qkv_gbs": round(qk_gbs, 1),
        },
        "roofline": {
            "kernel": "gate-up-SiLU bf16 M=1 (rows_kernel)",
            "bound": "hbm",
            "achieved": round(gu_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / PEAK_HBM_GBS, 4),
            "traffic": profiled_traffic(),
            # not measured in this run: FETCH_SIZE + WRITE_SIZE (copy-
            # calibrated) of the same kernel and workload from the committed
            # rocprofv3 --pmc summary of the profiled build
            "traffic_source": os.path.relpath(TRAFFIC_PROFILE, os.path.dirname(TRAFFIC_PROFILE) + "/.."),
            "algorithmic_bytes": gate_up_bytes(1, K, inter),
            "avg_launch_us": round(d_gu * 1e6, 3),
        },
        "prefill": prefill,
        "cells": cells,
        "cpu_baseline": cpu,
        "device": dev_name,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
