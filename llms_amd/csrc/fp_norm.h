// fp_norm.h — the RMSNorm prologue of the fused projections (reference
// src/engine/attention.py:28-33, applied as norm1 -> attention and norm2 ->
// FFN in src/engine/model.py:57-66):
//
//   r     = 1 / sqrt(sum_k float(x[k])^2 / K + eps)      (fp32)
//   xn[k] = bf16(float(gamma[k]) * float(bf16(float(x[k]) * r)))
//
// i.e. torch's x.float(), pow(2).mean(-1), x32 * rsqrt(var + eps), .to(bf16)
// and the bf16 weight product, each rounded where torch rounds. The sum runs
// in a fixed order (per-thread strided chunks, then the wave, then the waves
// in order), so every workgroup that normalises a row gets the same r.
#pragma once

#include "fp_common.h"

namespace fp {

// Sum of v over a workgroup of NT threads; every thread gets the total.
// red: NT / 64 floats of LDS. Contains barriers (uniform control flow only).
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) t += red[w];
  return t;
}

// Sum of squares (each square rounded to fp32, as pow(2) does) of one bf16
// row. VEC: K % 8 == 0 and a 16-byte-aligned row; else element by element.
template <int NT, bool VEC>
__device__ __forceinline__ float row_sumsq(const uint16_t* row, int64_t K, float* red) {
  float s = 0.f;
  if constexpr (VEC) {
    for (int64_t k = (int64_t)threadIdx.x * 8; k < K; k += (int64_t)NT * 8) {
      const u32x4 v = ld16(row + k);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_bits_to_f32(v[j] & 0xffffu), hi = bf16_bits_to_f32(v[j] >> 16);
        s += __fmul_rn(lo, lo);
        s += __fmul_rn(hi, hi);
      }
    }
  } else {
    for (int64_t k = threadIdx.x; k < K; k += NT) {
      const float f = bf16_bits_to_f32(row[k]);
      s += __fmul_rn(f, f);
    }
  }
  return block_sum<NT>(s, red);
}

__device__ __forceinline__ float rms_scale(float sumsq, int64_t K, float eps) {
  return 1.0f / sqrtf(sumsq / (float)K + eps);
}

__device__ __forceinline__ uint32_t norm_bf16(uint32_t xb, uint32_t gb, float r) {
  const float t = round_bf16(__fmul_rn(bf16_bits_to_f32(xb), r));
  return f32_to_bf16_bits(__fmul_rn(bf16_bits_to_f32(gb), t));
}

// Eight packed bf16 of x and gamma -> eight packed normalised bf16.
__device__ __forceinline__ u32x4 norm_bf16x8(u32x4 x, u32x4 g, float r) {
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = norm_bf16(x[j] & 0xffffu, g[j] & 0xffffu, r) |
           (norm_bf16(x[j] >> 16, g[j] >> 16, r) << 16);
  return o;
}

}  // namespace fp
