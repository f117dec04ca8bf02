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
// the kernels get; a stream passed in must belong to the current device.
// Every call on a GPU shares that GPU's array and overwrites it (the
// normalised rows, then any split-k partials: both are written in full before
// they are read, so nothing needs clearing between calls); calls that can
// overlap on one GPU (different streams, no ordering) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fp_launch.h"
#include "llms_amd_fp.h"

namespace {

static __device__ __align__(256) unsigned char scratch[FP_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];

// The address of `scratch` on the device that runs the call: the current
// device, which must also own `stream` when one is given (a stream of another
// GPU would get this GPU's address: FP_ERR_DEVICE instead). Looked up on the
// first successful call on that device, with it current; a failed lookup is
// not remembered, so a later call tries again. FP_ERR_DEVICE if there is no
// current device, the stream's device cannot be read or differs, or the
// lookup fails.
int device_scratch(void* stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FP_ERR_DEVICE;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev)
      return FP_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();  // leave no sticky error for the caller's next call
      return FP_ERR_DEVICE;
    }
    g_ptr[dev] = p;
  }
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
  const int st = device_scratch(stream, &ptr);
  if (st != FP_OK) return st;
  return fp_rmsnorm_qkv_bf16(x, ldx, gamma, eps, w, ldw, y, ldy, M, n_q, n_k, K, ptr,
                             (int64_t)FP_SCRATCH_BYTES, stream);
}

}  // extern "C"
