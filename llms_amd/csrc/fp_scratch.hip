// fp_scratch.hip — the allocation-free entry point fp_rmsnorm_qkv_bf16_noalloc:
// fp_rmsnorm_qkv_bf16 with its workspace taken from a fixed-size device
// array of this library instead of a caller buffer, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops).
//
// The array `scratch` (FP_SCRATCH_BYTES, 256-byte aligned) exists once per
// GPU the library runs on and is held until the process ends. Host code never
// uses its name as an address (on the host it is only a registration
// stand-in): the device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and that address is what
// the kernels get. Every call on a GPU shares that GPU's array and overwrites
// it (the normalised rows, then any split-k partials: both are written in
// full before they are read, so nothing needs clearing between calls); calls
// that can overlap on one GPU (different streams, no ordering) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fp_launch.h"
#include "llms_amd_fp.h"

namespace {

static __device__ __align__(256) unsigned char scratch[FP_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];

// The current device's address of `scratch` (looked up on the first call on
// that device, with it current). FP_ERR_DEVICE if there is no current device
// or the lookup fails.
int device_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FP_ERR_DEVICE;
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = p;
  });
  if (g_err[dev] != hipSuccess || g_ptr[dev] == nullptr) return FP_ERR_DEVICE;
  *out = g_ptr[dev];
  return FP_OK;
}

}  // namespace

extern "C" {

int fp_rmsnorm_qkv_bf16_noalloc(const void* x, int64_t ldx, const void* gamma, float eps,
                                const void* w, int64_t ldw, void* y, int64_t ldy, int64_t M,
                                int64_t n_q, int64_t n_k, int64_t K, void* stream) {
  // argument errors come back exactly as from the workspace entry point,
  // before any device state is touched
  const int st0 = fp::rmsnorm_qkv_args(x, ldx, gamma, eps, w, ldw, y, ldy, M, n_q, n_k, K);
  if (st0 != FP_OK) return st0;
  if (M == 0) return FP_OK;
  const int64_t need = fp_rmsnorm_workspace_bytes(M, n_q + 2 * n_k, K, 0, 0);
  if (need > (int64_t)FP_SCRATCH_BYTES) return FP_ERR_SCRATCH;
  void* ptr = nullptr;
  const int st = device_scratch(&ptr);
  if (st != FP_OK) return st;
  return fp_rmsnorm_qkv_bf16(x, ldx, gamma, eps, w, ldw, y, ldy, M, n_q, n_k, K, ptr,
                             (int64_t)FP_SCRATCH_BYTES, stream);
}

}  // extern "C"
