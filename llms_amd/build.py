"""Build the native parts of llms_amd in-tree.

Two shared libraries are produced next to this file:

- ``libllms_amd_fp.so``: the HIP kernels for gfx950 and the C ABI declared in
  ``include/llms_amd_fp.h`` (no torch dependency; any FFI can bind it).
- ``_torch_ops.so``: the thin ``torch.ops.llms_amd.*`` custom ops that call
  that C ABI on torch's current HIP stream (links ``libllms_amd_fp.so`` via
  ``$ORIGIN``).

Run ``python -m llms_amd.build`` (or ``__graft_entry__.build()``). hipcc
cross-compiles for gfx950 without a GPU present.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"

CAPI_SO = PKG / "libllms_amd_fp.so"
TORCH_OPS_SO = PKG / "_torch_ops.so"

HIP_SOURCES = ["fp_api.hip", "fp_stream.hip", "fp_rows.hip", "fp_splitk.hip", "fp_tiled.hip",
               "fp_gemm.hip", "fp_scratch.hip", "fp_xpanel.hip"]
HIP_HEADERS = ["fp_common.h", "fp_launch.h"]

# gfx950 only. Packed-fp32 VALU ops (v_pk_*_f32) are disabled for all device
# code: hipcc -O3 would otherwise form them from ordinary float code.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], what: str) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"{what} failed ({proc.returncode}):\n{' '.join(cmd)}\n{out}")
    if out:
        print(out, file=sys.stderr)


def build_capi(verbose: bool = False) -> Path:
    """Compile the HIP kernels + C ABI into ``libllms_amd_fp.so``.

    Each translation unit is compiled in parallel into ``_build/``, then
    linked.
    """
    from concurrent.futures import ThreadPoolExecutor

    if not HIPCC.exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    bdir = PKG / "_build"
    bdir.mkdir(exist_ok=True)
    jobs = []
    for src in HIP_SOURCES:
        obj = bdir / (Path(src).stem + ".o")
        cmd = [str(HIPCC), *HIP_FLAGS, "-c", f"-I{INCLUDE}", f"-I{CSRC}",
               str(CSRC / src), "-o", str(obj)]
        jobs.append((cmd, obj))
    if verbose:
        for cmd, _ in jobs:
            print(" ".join(cmd))
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as ex:
        for fut in [ex.submit(_run, cmd, f"hipcc -c {obj.name}") for cmd, obj in jobs]:
            fut.result()
    tmp = CAPI_SO.with_suffix(".so.tmp")
    _run([str(HIPCC), "--offload-arch=gfx950", "-shared", "-fPIC",
          *[str(o) for _, o in jobs], "-o", str(tmp)], "hipcc link (libllms_amd_fp.so)")
    os.replace(tmp, CAPI_SO)
    return CAPI_SO


def _torch_flags() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    tdir = Path(torch.__file__).resolve().parent
    inc = [tdir / "include", tdir / "include" / "torch" / "csrc" / "api" / "include"]
    cflags = [
        "-O2", "-std=c++17", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in inc], f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
        f"-I{sysconfig.get_paths()['include']}",
    ]
    del cpp_extension  # imported only to fail early if torch is incomplete
    lib = tdir / "lib"
    ldflags = [
        f"-L{lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
        f"-L{ROCM / 'lib'}", "-lamdhip64",
        f"-L{PKG}", "-lllms_amd_fp",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{lib}",
    ]
    return cflags, ldflags


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile the torch custom-op glue into ``_torch_ops.so``."""
    cflags, ldflags = _torch_flags()
    tmp = TORCH_OPS_SO.with_suffix(".so.tmp")
    cmd = ["g++", *cflags, "-shared", str(CSRC / "torch_ops.cpp"), "-o", str(tmp), *ldflags]
    if verbose:
        print(" ".join(cmd))
    _run(cmd, "g++ (_torch_ops.so)")
    os.replace(tmp, TORCH_OPS_SO)
    return TORCH_OPS_SO


def build_all(verbose: bool = False) -> list[Path]:
    """Build the libraries (always recompiles)."""
    return [build_capi(verbose), build_torch_ops(verbose)]


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv):
        print(p)
