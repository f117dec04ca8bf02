"""Write tests/golden/fixtures.npz: small input/output vectors of the
reference's unfused eager path, computed with torch on the CPU.

The calls are the reference's own (src/engine/attention.py:119-121 via the
stacked form of src/bench/microbench_fused_qkv.py:101-103, and
src/engine/model.py:37); the int8 cases use the task's per-row symmetric
quantisation then the same calls on the dequantised weight. bf16 tensors are
stored as uint16 bit patterns. Regenerate with:

    python tests/golden/make_golden.py

The fixtures pin the oracle (tests/test_golden.py) and the HIP kernels
(tests/test_kernels_gpu.py::test_golden_fixtures) to fixed vectors that do not
depend on the torch version installed at test time.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import torch_path as tp  # noqa: E402

OUT = Path(__file__).resolve().parent / "fixtures.npz"


def b(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    g = torch.Generator().manual_seed(20261201)

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    f: dict[str, np.ndarray] = {}
    # QKV, Qwen3-like GQA split at small dims (n_q = 4 * n_k)
    n_q, n_k = 32, 8
    x, w = rn(3, 64), rn(n_q + 2 * n_k, 64, std=0.1)
    f.update(qkv_x=b(x), qkv_w=b(w), qkv_nq=np.array(n_q), qkv_nk=np.array(n_k),
             qkv_y=b(torch.cat(tp.torch_qkv(x, w, n_q, n_k), -1)))
    x3 = rn(2, 3, 64)
    f.update(qkv3_x=b(x3), qkv3_y=b(torch.cat(tp.torch_qkv(x3, w, n_q, n_k), -1)))
    # gate-up-SiLU
    x, wg, wu = rn(4, 96), rn(40, 96, std=0.1), rn(40, 96, std=0.1)
    f.update(ffn_x=b(x), ffn_wg=b(wg), ffn_wu=b(wu), ffn_y=b(tp.torch_gate_up_silu(x, wg, wu)))
    # unaligned K (rows not 16-byte aligned)
    x, wg, wu = rn(1, 37), rn(12, 37, std=0.3), rn(12, 37, std=0.3)
    f.update(ffn37_x=b(x), ffn37_wg=b(wg), ffn37_wu=b(wu), ffn37_y=b(tp.torch_gate_up_silu(x, wg, wu)))
    # int8 per-row quantisation (with an all-zero row)
    w = rn(16, 64, std=0.05)
    w[5] = 0
    q, s = tp.torch_quantize_w8(w)
    f.update(q8_w=b(w), q8_q=q.numpy(), q8_s=s.numpy())
    # int8 weight-only gate-up and QKV: dequantise then the bf16 calls
    x, wg, wu = rn(2, 128), rn(24, 128, std=0.05), rn(24, 128, std=0.05)
    qg, sg = tp.torch_quantize_w8(wg)
    qu, su = tp.torch_quantize_w8(wu)
    f.update(w8_x=b(x), w8_qg=qg.numpy(), w8_sg=sg.numpy(), w8_qu=qu.numpy(), w8_su=su.numpy(),
             w8_y=b(tp.torch_gate_up_silu_w8(x, qg, sg, qu, su)))
    xq, wq = rn(3, 128), rn(n_q + 2 * n_k, 128, std=0.05)
    qq, sq = tp.torch_quantize_w8(wq)
    f.update(w8q_x=b(xq), w8q_q=qq.numpy(), w8q_s=sq.numpy(),
             w8q_y=b(torch.cat(tp.torch_qkv_w8(xq, qq, sq, n_q, n_k), -1)))
    np.savez(OUT, **f)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(f)} arrays)")


if __name__ == "__main__":
    main()
