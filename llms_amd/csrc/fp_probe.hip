// fp_probe.hip — read-only bandwidth probe for the decode roofline (a
// measurement aid, not part of the projection C ABI; bench.py --read-ceiling
// loads it as libllms_amd_probe.so).
//
// The kernel reads a weight-shaped buffer exactly as the row-streaming decode
// kernel (fp_rows.hip) does — a wave owns whole rows of `row_bytes`, reads
// each 1 KB run with one 16-byte load per lane (with the non-temporal hint,
// as those kernels load weights), all of a row's runs in flight from the
// first instruction, 8 waves per workgroup — and does nothing with
// the data but fold it into one word per wave (so the loads stay live). Its
// duration is the floor for a launch that streams that many bytes in that
// pattern: launch, first-byte latency, the HBM stream and the drain.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// U: 1 KB runs per row (row_bytes = U KB). With p1 set, each wave reads its
// row of p0 and the same row of p1 (the gate-up kernel's Wg / Wu pair).
template <int U, bool PAIR>
__global__ __launch_bounds__(512) void read_rows_kernel(const uint8_t* p0, const uint8_t* p1,
                                                        int64_t n_rows, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 8 + wave;
  if (row >= n_rows) return;
  const int64_t off = row * (int64_t)U * 1024 + lane * 16;
  u32x4 v[U], w[PAIR ? U : 1];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p0 + off + u * 1024));
    if constexpr (PAIR)
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p1 + off + u * 1024));
  }
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if constexpr (PAIR) x ^= w[u].x ^ w[u].y ^ w[u].z ^ w[u].w;
  }
  // fold across the wave so only one lane stores
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
  if (lane == 0) sink[row] = x;
}

}  // namespace

extern "C" {

// Reads n_rows rows of row_kb KB from p0 (and, if p1 is not NULL, the same
// rows of p1; both 16-byte aligned) and writes one word per row to sink.
// row_kb must be 2, 4, 5 or 8. Returns 0, 2 for a bad argument, or the
// hipError_t of the launch.
int fp_probe_read_rows(const void* p0, const void* p1, int64_t n_rows, int row_kb, void* sink,
                       void* stream) {
  if (!p0 || !sink || n_rows < 1 || (reinterpret_cast<uintptr_t>(p0) & 15) ||
      (reinterpret_cast<uintptr_t>(p1) & 15))
    return 2;
  const dim3 grid((unsigned)((n_rows + 7) / 8)), block(512);
  const uint8_t* b0 = static_cast<const uint8_t*>(p0);
  const uint8_t* b1 = static_cast<const uint8_t*>(p1);
  uint32_t* s = static_cast<uint32_t*>(sink);
  hipStream_t st = (hipStream_t)stream;
#define FP_PROBE_CASE(U)                                                                      \
  case U:                                                                                    \
    if (b1)                                                                                  \
      hipLaunchKernelGGL((read_rows_kernel<U, true>), grid, block, 0, st, b0, b1, n_rows, s); \
    else                                                                                     \
      hipLaunchKernelGGL((read_rows_kernel<U, false>), grid, block, 0, st, b0, b0, n_rows, s); \
    break;
  switch (row_kb) {
    FP_PROBE_CASE(2)
    FP_PROBE_CASE(4)
    FP_PROBE_CASE(5)
    FP_PROBE_CASE(8)
    default: return 2;
  }
#undef FP_PROBE_CASE
  return (int)hipGetLastError();
}

}  // extern "C"
