"""llms_amd — MI355X-native (gfx950) fused QKV and gate-up-SiLU projections
for the Qwen3 engine of aaholmes/llms.

- ``llms_amd.kernels``: the drop-in Python surface (reference names).
- ``include/llms_amd_fp.h`` + ``libllms_amd_fp.so``: the C ABI.
- ``torch.ops.llms_amd.*``: the custom ops between the two.
"""

from ._lib import NativeLibraryMissing, capi, ops

__version__ = "0.1.0"

__all__ = ["NativeLibraryMissing", "capi", "ops", "__version__"]
