// fp_rows.hip — row-streaming fused projections for a single activation row
// (M = 1, the decode step), where the call is one pass over the weights.
//
// Each wave owns whole weight rows (gate-up: row n of Wg and row n of Wu) and
// reads them front to back, one contiguous 1 KB run per wave instruction
// (64 lanes x 16 B = 512 bf16 of one row), so each workgroup streams a
// contiguous stretch of every matrix in address order — measured on MI355X
// ~1 us per gate-up launch faster than gathering 128 B lines of eight rows.
// With one x row the arithmetic is 2 flop per weight byte pair, so the dot
// products run on the VALU (fp32 FMAs of unpacked bf16) and the MFMA pipe is
// not used; lane l accumulates k = 512 j + 8 l .. +7 over the row's chunks j.
// A row ends with a fixed-order wave reduction (DPP within 16-lane rows, then
// the four row sums via readlane), the epilogue at the torch rounding points,
// and one 2-byte store: no LDS reduction, no barrier after the prologue.
// x (K bf16) is staged once per workgroup in LDS while the wave's first
// weight loads are in flight.
// Requirements (checked by rows_supported): M == 1, bf16, 16-byte-aligned
// rows with K % 8 == 0, K <= kRowsMaxK.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kKC = 512;  // k elements per wave instruction (64 lanes x 8)

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wave (wave-uniform result), fixed order.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror: sums of 8
  v += dpp_f32<0x140>(v);  // row_mirror: sums of 16
  return (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))) +
         (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48)));
}

// acc += sum over 8 bf16 pairs (w[e] * x[e]), in e order.
__device__ __forceinline__ float dot8(u32x4 w, u32x4 x, float acc) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xx[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    acc = fmaf(__uint_as_float(ww[d] << 16), __uint_as_float(xx[d] << 16), acc);
    acc = fmaf(__uint_as_float(ww[d] & 0xffff0000u), __uint_as_float(xx[d] & 0xffff0000u), acc);
  }
  return acc;
}

// NW waves per workgroup, R rows per wave, U weight chunks in flight per wave.
template <int NW, int R, int U, bool GATEUP>
__global__ __launch_bounds__(NW * kWave) void rows_kernel(StreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t K = a.K;
  const int J = (int)((K + kKC - 1) / kKC);  // chunks per row
  const int64_t row0 = ((int64_t)blockIdx.x * NW + wave) * R;
  const int64_t left = a.N - row0;
  const int nr = left <= 0 ? 0 : (left < R ? (int)left : R);
  const int T = nr * J;  // chunks of this wave

  // Weight chunks are consumed in issue order: chunk t sits in slot t % U.
  u32x4 wg[U], wu[U];
  int ir = 0, ij = 0;  // (row, chunk) of the next chunk to issue
  auto issue = [&](int u) {
    if (ir < nr) {
      const int64_t row = row0 + ir;
      const int64_t k = (int64_t)ij * kKC + 8 * lane;
      wg[u] = load_bf16x8<true>((const uint16_t*)a.w0 + row * a.ldw0, k, K);
      if constexpr (GATEUP) wu[u] = load_bf16x8<true>((const uint16_t*)a.w1 + row * a.ldw1, k, K);
      if (++ij == J) { ij = 0; ++ir; }
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) issue(u);

  // x[0:K] -> LDS, zero-padded to J * 512
  const int64_t nvec = (int64_t)J * (kKC / 8);
  for (int64_t i = threadIdx.x; i < nvec; i += NW * kWave)
    *reinterpret_cast<u32x4*>(xs + i * 8) = load_bf16x8<true>(a.x, i * 8, K);
  __syncthreads();

  float ag = 0.f, au = 0.f;
  int cr = 0, cj = 0;  // (row, chunk) being consumed
  for (int t0 = 0; t0 < T; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t0 + u < T) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + (int64_t)cj * kKC + 8 * lane);
        ag = dot8(wg[u], xv, ag);
        if constexpr (GATEUP) au = dot8(wu[u], xv, au);
        issue(u);
        if (++cj == J) {
          const float g = wave_sum(ag);
          const float up = GATEUP ? wave_sum(au) : 0.f;
          if (lane == 0)
            a.y[row0 + cr] = (uint16_t)(GATEUP ? gate_up_silu_bits(g, up) : f32_to_bf16_bits(g));
          ag = au = 0.f;
          cj = 0;
          ++cr;
        }
      }
    }
  }
}

template <int NW, int R, int U, bool GATEUP>
int launch_rows_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t per = (int64_t)NW * R;
  const size_t shm = (size_t)((a.K + kKC - 1) / kKC) * kKC * 2;
  hipLaunchKernelGGL((rows_kernel<NW, R, U, GATEUP>), dim3((unsigned)((a.N + per - 1) / per)),
                     dim3(NW * kWave), shm, s, a);
  return (int)hipGetLastError();
}

}  // namespace

bool rows_supported(const StreamArgs& a, bool aligned) {
  return aligned && a.M == 1 && a.K <= kRowsMaxK;
}

// Measured on MI355X (Qwen3-4B, 36 cycled weight sets): one row (pair) per
// wave with its whole row in flight (K = 2560: 5 chunks); gate-up 4 waves per
// workgroup, QKV 8.
template <bool GATEUP>
int launch_rows(const StreamArgs& a, hipStream_t s) {
  if constexpr (GATEUP) return launch_rows_cfg<4, 1, 5, true>(a, s);
  return launch_rows_cfg<8, 1, 5, false>(a, s);
}

template int launch_rows<false>(const StreamArgs&, hipStream_t);
template int launch_rows<true>(const StreamArgs&, hipStream_t);

}  // namespace fp
