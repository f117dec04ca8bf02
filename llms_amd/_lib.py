"""Loaders for the native libraries built by ``llms_amd.build``.

- :func:`capi` returns the ``ctypes`` binding of ``libllms_amd_fp.so`` (the
  C ABI of ``include/llms_amd_fp.h``), with argument and return types set.
- :func:`ops` loads ``_torch_ops.so`` and returns ``torch.ops.llms_amd``.

Both raise :class:`NativeLibraryMissing` when the library has not been built:
there is no fallback path, by design.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

PKG = Path(__file__).resolve().parent
CAPI_SO = PKG / "libllms_amd_fp.so"
TORCH_OPS_SO = PKG / "_torch_ops.so"

_lock = threading.Lock()
_capi: ctypes.CDLL | None = None
_ops = None


class NativeLibraryMissing(RuntimeError):
    """The HIP extension is not built; the fused projections cannot run."""


# (name, argtypes) of every entry point declared in include/llms_amd_fp.h.
_P, _I64, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
CAPI_SIGNATURES: dict[str, list] = {
    "fp_status_string": [ctypes.c_int],
    "fp_abi_version": [],
    "fp_qkv_bf16": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "fp_gate_up_silu_bf16": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "fp_qkv_w8": [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "fp_gate_up_silu_w8": [_P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P],
    "fp_linear_bf16": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "fp_linear_w8": [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P],
    "fp_quantize_w8_per_row": [_P, _I64, _P, _I64, _P, _I64, _I64, _P],
    "fp_workspace_bytes": [_I64, _I64, _I64, ctypes.c_int],
    "fp_qkv_bf16_ws": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_gate_up_silu_bf16_ws": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_linear_bf16_ws": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_workspace_bytes_w8": [_I64, _I64, _I64, ctypes.c_int],
    "fp_qkv_w8_ws": [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_gate_up_silu_w8_ws": [_P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P,
                              _I64, _P],
    "fp_linear_w8_ws": [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_rmsnorm_workspace_bytes": [_I64, _I64, _I64, ctypes.c_int, ctypes.c_int],
    "fp_rmsnorm_qkv_bf16": [_P, _I64, _P, _F, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_rmsnorm_gate_up_silu_bf16": [_P, _I64, _P, _F, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64,
                                     _P, _I64, _P],
    "fp_rmsnorm_qkv_w8": [_P, _I64, _P, _F, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "fp_rmsnorm_gate_up_silu_w8": [_P, _I64, _P, _F, _P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64,
                                   _I64, _P, _I64, _P],
    "fp_rmsnorm_qkv_bf16_noalloc": [_P, _I64, _P, _F, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P],
}

FP_STATUS = {
    0: "FP_OK",
    1: "FP_ERR_NULL",
    2: "FP_ERR_SHAPE",
    3: "FP_ERR_STRIDE",
    4: "FP_ERR_LAUNCH",
    5: "FP_ERR_DEVICE",
    6: "FP_ERR_WORKSPACE",
    7: "FP_ERR_SCRATCH",
}

# FP_SCRATCH_BYTES of include/llms_amd_fp.h: the static scratch of
# fp_rmsnorm_qkv_bf16_noalloc, per GPU.
FP_SCRATCH_BYTES = 32 << 20


def _missing(path: Path) -> NativeLibraryMissing:
    return NativeLibraryMissing(
        f"{path.name} is not built (expected at {path}); build it with "
        "`python -m llms_amd.build` — llms_amd has no non-HIP fallback"
    )


def capi() -> ctypes.CDLL:
    """The ctypes binding of the C ABI (loaded once per process)."""
    global _capi
    with _lock:
        if _capi is None:
            if not CAPI_SO.exists():
                raise _missing(CAPI_SO)
            lib = ctypes.CDLL(str(CAPI_SO))
            for name, argtypes in CAPI_SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = {"fp_status_string": ctypes.c_char_p,
                              "fp_workspace_bytes": ctypes.c_int64,
                              "fp_workspace_bytes_w8": ctypes.c_int64,
                              "fp_rmsnorm_workspace_bytes": ctypes.c_int64}.get(name, ctypes.c_int)
            _capi = lib
        return _capi


def ops():
    """``torch.ops.llms_amd`` after loading ``_torch_ops.so`` (once)."""
    global _ops
    with _lock:
        if _ops is None:
            import torch

            if not TORCH_OPS_SO.exists():
                raise _missing(TORCH_OPS_SO)
            torch.ops.load_library(str(TORCH_OPS_SO))
            _ops = torch.ops.llms_amd
        return _ops


def status_string(code: int) -> str:
    return capi().fp_status_string(code).decode()
