// fp_common.h — shared device types and helpers for the gfx950 fused
// projection kernels (wave64, MFMA bf16, 16-byte vector memory).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fp {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

constexpr int kWave = 64;

// ---- bf16 <-> fp32, round-to-nearest-even (torch's c10::BFloat16 rule) ----
//
// The hardware pack v_cvt_pk_bf16_f32 rounds every non-NaN fp32 value exactly
// as RNE on the bits (u + 0x7fff + ((u >> 16) & 1)) >> 16 does — checked on
// gfx950 over all 2^32 inputs — and turns a NaN into some NaN; torch gives
// every NaN the canonical bits 0x7fc0, so the stored conversions select that.

// Two fp32 -> two bf16 in one dword (lo in bits 0..15), NaN payloads as the
// hardware leaves them (for intermediate roundings, which are widened again).
__device__ __forceinline__ uint32_t cvt_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t h = cvt_bf16x2(f, f) & 0xffffu;
  return f != f ? 0x7fc0u : h;  // NaN -> canonical qNaN
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// fp32 rounded to the nearest bf16, as fp32 (NaN stays NaN).
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(cvt_bf16x2(f, f) << 16);
}

// Two fp32 -> one dword of packed bf16 (lo in bits 0..15), RNE, canonical NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  uint32_t h = cvt_bf16x2(lo, hi);
  if (lo != lo) h = (h & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) h = (h & 0xffffu) | 0x7fc00000u;
  return h;
}

// ---- wave reduction -------------------------------------------------------

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

// Four int8 of one dword dequantised to bf16(q * s) and returned as two
// packed bf16 pairs (bytes 0,1 and 2,3): fma(q + 128, s, -128 s) is the exact
// product rounded once to fp32, the conversion is RNE.
__device__ __forceinline__ u32x2 dequant4_bf16(uint32_t qword, float s, float n128s) {
  const uint32_t u = qword ^ 0x80808080u;
  const f32x2 lo = {fmaf((float)(u & 0xffu), s, n128s), fmaf((float)((u >> 8) & 0xffu), s, n128s)};
  const f32x2 hi = {fmaf((float)((u >> 16) & 0xffu), s, n128s), fmaf((float)(u >> 24), s, n128s)};
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
               __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2))};
}

// Eight int8 (two dwords) dequantised to eight packed bf16(q * s).
__device__ __forceinline__ u32x4 dequant8_bf16(uint32_t q0, uint32_t q1, float s, float n128s) {
  const u32x2 lo = dequant4_bf16(q0, s, n128s), hi = dequant4_bf16(q1, s, n128s);
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

// ---- epilogues -------------------------------------------------------------

// silu(g) * u with the rounding points of the unfused bf16 torch path:
// g, u are rounded to bf16 (F.linear output), silu is evaluated in fp32 on the
// rounded g and rounded (F.silu output), the product is taken in fp32 on the
// two bf16 operands and rounded (the elementwise mul output).
// The intermediate roundings use the hardware pack (cvt_bf16x2); silu uses
// the fast exp and divide, which give the same bf16 silu(g) as
// g / (1 + expf(-g)) for every bf16 g (checked on gfx950 over all 2^16 bf16
// inputs). The stored value gets torch's canonical NaN.
__device__ __forceinline__ uint32_t gate_up_silu_bits(float acc_g, float acc_u) {
  const uint32_t gu = cvt_bf16x2(acc_g, acc_u);
  const float g = __uint_as_float(gu << 16), u = __uint_as_float(gu & 0xffff0000u);
  const float s = round_bf16(__fdividef(g, 1.0f + __expf(-g)));
  return f32_to_bf16_bits(s * u);
}

// Two outputs of the same epilogue, packed as two bf16 (lo: (g0, u0), hi:
// (g1, u1)); bit-identical to gate_up_silu_bits on each. The conversions of
// the two outputs share each v_cvt_pk_bf16_f32 (one for g and u of an
// output, one for both silu values, one for both products), and NaN
// canonicalisation runs only in waves that hold a NaN.
__device__ __forceinline__ uint32_t gate_up_silu_pair(float g0, float u0, float g1, float u1) {
  const uint32_t a = cvt_bf16x2(g0, u0), b = cvt_bf16x2(g1, u1);
  const float ga = __uint_as_float(a << 16), ua = __uint_as_float(a & 0xffff0000u);
  const float gb = __uint_as_float(b << 16), ub = __uint_as_float(b & 0xffff0000u);
  const uint32_t s = cvt_bf16x2(__fdividef(ga, 1.0f + __expf(-ga)), __fdividef(gb, 1.0f + __expf(-gb)));
  const float ya = __uint_as_float(s << 16) * ua, yb = __uint_as_float(s & 0xffff0000u) * ub;
  uint32_t y = cvt_bf16x2(ya, yb);
  if (__builtin_expect((ya != ya) | (yb != yb), 0)) {
    if (ya != ya) y = (y & 0xffff0000u) | 0x7fc0u;
    if (yb != yb) y = (y & 0xffffu) | 0x7fc00000u;
  }
  return y;
}

// ---- memory ---------------------------------------------------------------

// 16-byte global load (global_load_dwordx4). p must be 16-byte aligned.
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// 16-byte global load with the non-temporal hint (global_load_dwordx4 ... nt):
// for weight streams that are read once per call. Measured on MI355X on a
// read-only kernel with the decode kernels' pattern over 36 cycled weight
// sets (99.6 MB per launch): 17.12 -> 15.63 us.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld8_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

// Eight bf16 starting at element k of a row of length K, zero beyond K.
// ALIGNED: the row base is 16-byte aligned and K % 8 == 0, so a chunk of eight
// starting at a multiple of 8 lies wholly inside or wholly outside the row.
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_bf16x8(const uint16_t* row, int64_t k, int64_t K) {
  if constexpr (ALIGNED) {
    if (k < K) return ld16(row + k);
    return u32x4{0u, 0u, 0u, 0u};
  } else {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (k + e < K) ? (uint32_t)row[k + e] : 0u;
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                 h[6] | (h[7] << 16)};
  }
}

// Sixteen int8 starting at element k of a row of length K, zero beyond K.
// ALIGNED: the row base is 16-byte aligned and K % 16 == 0.
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_i8x16(const int8_t* row, int64_t k, int64_t K) {
  if constexpr (ALIGNED) {
    if (k < K) return ld16(row + k);
    return u32x4{0u, 0u, 0u, 0u};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t kk = k + 4 * d + b;
        const uint32_t byte = (kk < K) ? (uint32_t)(uint8_t)row[kk] : 0u;
        v |= byte << (8 * b);
      }
      w[d] = v;
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
}

// Weight-stream forms of the two loads above: the aligned path uses the
// non-temporal hint (weights are read once per decode-regime call).
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_w_bf16x8(const uint16_t* row, int64_t k, int64_t K) {
  if constexpr (ALIGNED) return k < K ? ld16_nt(row + k) : u32x4{0u, 0u, 0u, 0u};
  return load_bf16x8<false>(row, k, K);
}
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_w_i8x16(const int8_t* row, int64_t k, int64_t K) {
  if constexpr (ALIGNED) return k < K ? ld16_nt(row + k) : u32x4{0u, 0u, 0u, 0u};
  return load_i8x16<false>(row, k, K);
}

// ---- int8 -> bf16 dequantisation ------------------------------------------
//
// w = bf16_rne(fp32(q * s)), bit-identical to (q.float() * s).to(bfloat16):
// the byte is biased to u = q + 128 (xor 0x80), converted exactly with
// v_cvt_f32_ubyteN, and fma(u, s, -128 s) rounds the exact value q*s once
// (-128 s is exact), which is the single fp32 rounding of q.float() * s.
__device__ __forceinline__ void dequant4(uint32_t qword, float s, float neg128s,
                                         float out[4]) {
  const uint32_t u = qword ^ 0x80808080u;
  // (float)(byte n of u) is selected as v_cvt_f32_ubyteN.
  out[0] = fmaf((float)(u & 0xffu), s, neg128s);
  out[1] = fmaf((float)((u >> 8) & 0xffu), s, neg128s);
  out[2] = fmaf((float)((u >> 16) & 0xffu), s, neg128s);
  out[3] = fmaf((float)(u >> 24), s, neg128s);
}

// 8 int8 (two dwords) -> 8 bf16 packed in 4 dwords.
__device__ __forceinline__ u32x4 dequant8(uint32_t q0, uint32_t q1, float s, float neg128s) {
  float a[4], b[4];
  dequant4(q0, s, neg128s, a);
  dequant4(q1, s, neg128s, b);
  return u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]),
               pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// D(16x16, fp32) += A(16x32) * B(32x16), bf16 operands (gfx950 v_mfma_f32_16x16x32_bf16).
// Lane l supplies A row (l % 16) and B column (l % 16), 8 consecutive k of the
// 32-wide k-block selected by (l / 16); D lane l holds rows 4*(l/16)+r, col l%16.
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

}  // namespace fp
