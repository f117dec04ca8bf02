// fp_rows.hip — row-streaming fused projections for one to four activation
// rows (the decode step, short speculative verification), where the call is
// one pass over the weights.
//
// Each wave owns whole weight rows (gate-up: row n of Wg and row n of Wu) and
// reads them front to back, one contiguous 1 KB run per wave instruction
// (64 lanes x 16 B: 512 bf16 or 1024 int8 of one row), so each workgroup
// streams a contiguous stretch of every matrix in address order — measured on
// MI355X ~1 us per gate-up launch faster than gathering 128 B lines of eight
// rows. Lane l holds k = KC j + (KC/64) l .. of chunk j.
// The dot products run on the matrix core with a diagonal trick: lane l
// supplies the same k range to the A operand (its weights) and to the B
// operand (its x), so D[i][i] of v_mfma_f32_16x16x32_bf16 is the partial dot
// product of lanes i, i+16, i+32, i+48; the accumulator carries it over the
// row's chunks and the off-diagonal entries are unused (with one x row the
// matrix core has 16x the work it needs and is still ~7% busy; each further
// x row is one more MFMA per weight chunk with the same A operand). This takes
// the per-element unpack and FMA off the VALU (measured: gate-up 18.3 vs
// 19.1 us bf16, 13.8 vs 16.5 us int8).
// int8 weights are dequantised in registers to bf16(q * s) exactly as the
// dequantise-then-matmul path does (one fp32 rounding of q*s, then RNE to
// bf16 with v_cvt_pk_bf16_f32).
// A row ends with a fixed-order 64-lane sum of the diagonal (DPP within
// 16-lane rows, then the four row sums via readlane), the epilogue at the
// torch rounding points, and one 2-byte store: no LDS reduction, no barrier
// after the prologue.
// x (MM rows of K bf16, zero beyond M) is staged once per workgroup in LDS
// while the wave's first weight loads are in flight — except one row with
// K <= 2560, which each lane reads from L2 chunk by chunk along with the
// weights (no staging, no barrier).
// Requirements (checked by rows_supported): M <= kRowsMaxM, 16-byte-aligned
// rows with K % 8 == 0 (int8: K % 16 == 0), staged x within kRowsMaxLds.
#include "fp_common.h"
#include "fp_launch.h"
#include "fp_norm.h"

namespace fp {

namespace {

// k elements per wave instruction (64 lanes x 16 B)
template <bool W8>
constexpr int kc() { return W8 ? 1024 : 512; }

// Diagonal of a wave's 16x16 MFMA accumulator: lane l holds rows
// 4 (l / 16) + r, column l % 16, so D[i][i] sits in lane 20 (i / 4) + i % 4,
// register i % 4. Returns it there and 0 elsewhere.
__device__ __forceinline__ float diag(f32x4 d, int lane) {
  const int c = lane & 15;
  if ((c >> 2) != (lane >> 4)) return 0.f;
  const int r = c & 3;
  return r == 0 ? d.x : r == 1 ? d.y : r == 2 ? d.z : d.w;
}

// NW waves per workgroup, R rows per wave, U weight chunks in flight per wave,
// MM x rows (the call's M rounded up; the extra rows are zeros in LDS). NORM:
// x is RMS-normalised (a.gamma, a.eps) on its way into LDS. XG (one x row, no
// norm): no LDS staging and no barrier; each lane loads its 16 bytes (int8:
// 32 bytes) of x for a chunk from global memory (L2) together with the
// chunk's weights.
template <int NW, int R, int U, int MM, bool GATEUP, bool W8, bool NORM, bool XG = false>
__global__ __launch_bounds__(NW * kWave) void rows_kernel(StreamArgs a) {
  static_assert(!XG || (MM == 1 && !NORM), "x from global memory: one row, no norm");
  constexpr int KC = kc<W8>();
  constexpr int KL = KC / kWave;  // k elements per lane per chunk
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t K = a.K;
  const int J = (int)((K + KC - 1) / KC);  // chunks per row
  const int64_t row0 = ((int64_t)blockIdx.x * NW + wave) * R;
  const int64_t left = a.N - row0;
  const int nr = left <= 0 ? 0 : (left < R ? (int)left : R);
  const int T = nr * J;  // chunks of this wave

  // Weight chunks are consumed in issue order: chunk t sits in slot t % U.
  u32x4 wg[U], wu[U], xg[XG ? U : 1], xg1[XG && W8 ? U : 1];
  int ir = 0, ij = 0;  // (row, chunk) of the next chunk to issue
  auto issue = [&](int u) {
    if (ir < nr) {
      const int64_t row = row0 + ir;
      const int64_t k = (int64_t)ij * KC + KL * lane;
      if constexpr (XG) {
        xg[u] = load_bf16x8<true>(a.x, k, K);
        if constexpr (W8) xg1[u] = load_bf16x8<true>(a.x, k + 8, K);
      }
      // weights: read once per call, non-temporal; zero past the row's end
      if (k < K) {
        if constexpr (W8) {
          wg[u] = ld16_nt((const int8_t*)a.w0 + row * a.ldw0 + k);
          if constexpr (GATEUP) wu[u] = ld16_nt((const int8_t*)a.w1 + row * a.ldw1 + k);
        } else {
          wg[u] = ld16_nt((const uint16_t*)a.w0 + row * a.ldw0 + k);
          if constexpr (GATEUP) wu[u] = ld16_nt((const uint16_t*)a.w1 + row * a.ldw1 + k);
        }
      } else {
        wg[u] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (GATEUP) wu[u] = u32x4{0u, 0u, 0u, 0u};
      }
      if (++ij == J) { ij = 0; ++ir; }
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) issue(u);

  // x[0:MM, 0:K] -> LDS rows of Kp = J * KC, zero beyond K and beyond M
  const int64_t Kp = (int64_t)J * KC;
  const int64_t nvec = MM * (Kp / 8);
  if constexpr (NORM) {
    // One pass over global memory: the raw x rows and the norm weight (an
    // extra LDS row after the MM x rows) go to LDS while each thread sums
    // the squares of its x elements; then the per-row scales (fixed-order
    // sums, the same in every workgroup) and the rows normalised in place.
    __shared__ float red[MM * NW];
    uint16_t* gs = xs + MM * Kp;
    float s[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) s[m] = 0.f;
    for (int64_t i = threadIdx.x; i < nvec + Kp / 8; i += NW * kWave) {
      const int64_t m = i / (Kp / 8), k = (i - m * (Kp / 8)) * 8;
      u32x4 v = {0, 0, 0, 0};
      if (m < a.M) v = load_bf16x8<true>(a.x + m * a.ldx, k, K);
      else if (m == MM) v = load_bf16x8<true>(a.gamma, k, K);
      *reinterpret_cast<u32x4*>(xs + i * 8) = v;
      if (m < MM) {
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16_bits_to_f32(v[j] & 0xffffu), hi = bf16_bits_to_f32(v[j] >> 16);
          q += __fmul_rn(lo, lo);
          q += __fmul_rn(hi, hi);
        }
#pragma unroll
        for (int j = 0; j < MM; ++j)
          if (m == j) s[j] += q;
      }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) s[m] = wave_sum(s[m]);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MM; ++m) red[m * NW + wave] = s[m];
    }
    __syncthreads();
    float rinv[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += red[m * NW + w];
      rinv[m] = rms_scale(t, K, a.eps);
    }
    for (int64_t i = threadIdx.x; i < nvec; i += NW * kWave) {
      const int64_t m = i / (Kp / 8), k = (i - m * (Kp / 8)) * 8;
      if (m >= a.M) continue;
      float r = rinv[0];
#pragma unroll
      for (int j = 1; j < MM; ++j)
        if (m == j) r = rinv[j];
      u32x4* p = reinterpret_cast<u32x4*>(xs + i * 8);
      *p = norm_bf16x8(*p, *reinterpret_cast<const u32x4*>(gs + k), r);
    }
  } else if constexpr (!XG) {
    for (int64_t i = threadIdx.x; i < nvec; i += NW * kWave) {
      const int64_t m = i / (Kp / 8), k = (i - m * (Kp / 8)) * 8;
      *reinterpret_cast<u32x4*>(xs + i * 8) =
          m < a.M ? load_bf16x8<true>(a.x + m * a.ldx, k, K) : u32x4{0, 0, 0, 0};
    }
  }
  if constexpr (!XG) __syncthreads();

  // int8 row scales of the row being consumed
  float sg = 0.f, su = 0.f;
  auto load_scales = [&](int r) {
    if constexpr (W8) {
      if (r < nr) {
        sg = a.s0[row0 + r];
        if constexpr (GATEUP) su = a.s1[row0 + r];
      }
    }
  };
  load_scales(0);

  f32x4 dg[MM], du[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) dg[m] = du[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  int cr = 0, cj = 0;  // (row, chunk) being consumed
  for (int t0 = 0; t0 < T; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t0 + u < T) {
        const uint16_t* xp = xs + (int64_t)cj * KC + KL * lane;
        if constexpr (W8) {
          const float ng = -128.f * sg;
          const u32x4 g0 = dequant8_bf16(wg[u].x, wg[u].y, sg, ng);
          const u32x4 g1 = dequant8_bf16(wg[u].z, wg[u].w, sg, ng);
          u32x4 u0, u1;
          if constexpr (GATEUP) {
            const float nu = -128.f * su;
            u0 = dequant8_bf16(wu[u].x, wu[u].y, su, nu);
            u1 = dequant8_bf16(wu[u].z, wu[u].w, su, nu);
          }
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            u32x4 xv, xv1;
            if constexpr (XG) {
              xv = xg[u];
              xv1 = xg1[u];
            } else {
              xv = *reinterpret_cast<const u32x4*>(xp + m * Kp);
              xv1 = *reinterpret_cast<const u32x4*>(xp + m * Kp + 8);
            }
            dg[m] = mfma16(g0, xv, dg[m]);
            dg[m] = mfma16(g1, xv1, dg[m]);
            if constexpr (GATEUP) {
              du[m] = mfma16(u0, xv, du[m]);
              du[m] = mfma16(u1, xv1, du[m]);
            }
          }
        } else {
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            u32x4 xv;
            if constexpr (XG) xv = xg[u];
            else xv = *reinterpret_cast<const u32x4*>(xp + m * Kp);
            dg[m] = mfma16(wg[u], xv, dg[m]);
            if constexpr (GATEUP) du[m] = mfma16(wu[u], xv, du[m]);
          }
        }
        issue(u);
        if (++cj == J) {
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            const float g = wave_sum(diag(dg[m], lane));
            const float up = GATEUP ? wave_sum(diag(du[m], lane)) : 0.f;
            dg[m] = du[m] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (lane == 0 && m < a.M)
              a.y[m * a.ldy + row0 + cr] =
                  (uint16_t)(GATEUP ? gate_up_silu_bits(g, up) : f32_to_bf16_bits(g));
          }
          cj = 0;
          ++cr;
          load_scales(cr);
        }
      }
    }
  }
}


// int8 gate-up at one x row without a fused norm: each wave owns one row pair
// of Wg and Wu and reads it 8 bytes per lane per chunk (512 k per wave
// instruction, one MFMA per chunk and matrix), so that K = 2560 fills five
// chunks exactly instead of leaving half of a third 1024-k chunk empty, with
// the whole row pair in flight (U chunks). x comes from L2 chunk by chunk
// (XG, K <= 2560) or is staged once per workgroup in LDS. The dot products
// and the epilogue are those of rows_kernel (MFMA diagonal, fixed-order wave
// sum, torch's rounding points); the dequantisation is the exact
// dequant8_bf16.
template <int NW, int U, bool XG>
__global__ __launch_bounds__(NW * kWave) void rows_gate_up_w8_kernel(StreamArgs a) {
  constexpr int KC = 512, KL = 8;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t K = a.K;
  const int J = (int)((K + KC - 1) / KC);  // chunks per row
  const int64_t row = (int64_t)blockIdx.x * NW + wave;
  const int T = row < a.N ? J : 0;          // chunks of this wave
  const int8_t* g = (const int8_t*)a.w0 + (row < a.N ? row : 0) * a.ldw0;
  const int8_t* u = (const int8_t*)a.w1 + (row < a.N ? row : 0) * a.ldw1;

  // chunk t sits in slot t % U; zero past the row's end
  u32x2 wg[U], wu[U];
  u32x4 xg[XG ? U : 1];
  int ij = 0;
  auto issue = [&](int s) {
    if (ij < T) {
      const int64_t k = (int64_t)ij * KC + KL * lane;
      if constexpr (XG) xg[s] = load_bf16x8<true>(a.x, k, K);
      if (k < K) {
        wg[s] = ld8_nt(g + k);
        wu[s] = ld8_nt(u + k);
      } else {
        wg[s] = u32x2{0u, 0u};
        wu[s] = u32x2{0u, 0u};
      }
      ++ij;
    }
  };
#pragma unroll
  for (int s = 0; s < U; ++s) issue(s);
  if constexpr (!XG) {
    // x[0, 0:K] -> LDS, zero beyond K, while the first weight loads fly
    const int64_t nvec = (int64_t)J * KC / 8;
    for (int64_t i = threadIdx.x; i < nvec; i += NW * kWave)
      *reinterpret_cast<u32x4*>(xs + i * 8) = load_bf16x8<true>(a.x, i * 8, K);
    __syncthreads();
  }
  float sg = 0.f, su = 0.f;
  if (T > 0) {
    sg = a.s0[row];
    su = a.s1[row];
  }
  const float ng = -128.f * sg, nu = -128.f * su;
  f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = dg;
  for (int t0 = 0; t0 < T; t0 += U) {
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int t = t0 + s;
      if (t < T) {
        u32x4 xv;
        if constexpr (XG) xv = xg[s];
        else xv = *reinterpret_cast<const u32x4*>(xs + (int64_t)t * KC + KL * lane);
        dg = mfma16(dequant8_bf16(wg[s].x, wg[s].y, sg, ng), xv, dg);
        du = mfma16(dequant8_bf16(wu[s].x, wu[s].y, su, nu), xv, du);
        issue(s);
      }
    }
  }
  if (T > 0) {
    const float gs = wave_sum(diag(dg, lane));
    const float us = wave_sum(diag(du, lane));
    if (lane == 0) a.y[row] = (uint16_t)gate_up_silu_bits(gs, us);
  }
}

// x rows staged per workgroup: M rounded up to 1, 2 or 4
inline int64_t rows_mm(int64_t M) { return M <= 2 ? M : 4; }

// LDS bytes of the staged x: MM rows of K rounded up to whole chunks, plus
// one such row for the norm weight when the RMSNorm prologue is fused in
template <bool W8>
int64_t rows_lds_bytes(int64_t M, int64_t K, bool norm = false) {
  constexpr int KC = kc<W8>();
  return (rows_mm(M) + (norm ? 1 : 0)) * ((K + KC - 1) / KC) * KC * 2;
}

template <int NW, int R, int U, int MM, bool GATEUP, bool W8>
int launch_rows_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t per = (int64_t)NW * R;
  const size_t shm = (size_t)rows_lds_bytes<W8>(MM, a.K, a.gamma != nullptr);
  const dim3 grid((unsigned)((a.N + per - 1) / per)), block(NW * kWave);
  // One x row with K <= 2560: x straight from L2 into registers instead of
  // an LDS copy behind a barrier (measured on MI355X, bit-identical: bf16 4B
  // QKV 7.46 -> 7.16 us, gate-up 18.20 -> 17.93 us, 0.6B QKV 3.85 -> 3.61 us,
  // gate-up 5.00 -> 4.68 us; int8 4B QKV 6.01 -> 5.73 us, gate-up 13.7-13.9
  // -> 13.34 us, 0.6B QKV 3.53 -> 3.22 us; at K = 4096 (8B) it is even, or
  // for int8 gate-up 5% slower).
  if constexpr (MM == 1) {
    if (!a.gamma && a.K <= 2560) {
      hipLaunchKernelGGL((rows_kernel<NW, R, U, MM, GATEUP, W8, false, true>), grid, block, 0, s, a);
      return (int)hipGetLastError();
    }
  }
  if (a.gamma)
    hipLaunchKernelGGL((rows_kernel<NW, R, U, MM, GATEUP, W8, true>), grid, block, shm, s, a);
  else
    hipLaunchKernelGGL((rows_kernel<NW, R, U, MM, GATEUP, W8, false>), grid, block, shm, s, a);
  return (int)hipGetLastError();
}

// One workgroup per row: the row's scale, then the normalised row.
template <bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, int64_t ldx,
                                                      const uint16_t* gamma, float eps,
                                                      uint16_t* xn, int64_t K) {
  __shared__ float red[256 / kWave];
  const uint16_t* row = x + (int64_t)blockIdx.x * ldx;
  uint16_t* out = xn + (int64_t)blockIdx.x * K;
  const float r = rms_scale(row_sumsq<256, VEC>(row, K, red), K, eps);
  if constexpr (VEC) {
    for (int64_t k = (int64_t)threadIdx.x * 8; k < K; k += 256 * 8)
      *reinterpret_cast<u32x4*>(out + k) = norm_bf16x8(ld16(row + k), ld16(gamma + k), r);
  } else {
    for (int64_t k = threadIdx.x; k < K; k += 256) out[k] = (uint16_t)norm_bf16(row[k], gamma[k], r);
  }
}

}  // namespace

// bf16 takes M <= 2 here (for 3..4 rows the 8-row streaming kernel is
// faster: its MFMA columns hold the x rows), int8 up to kRowsMaxM (the
// dequantisation, shared by all x rows, dominates).
bool rows_fit(int64_t M, int64_t K, bool w8, bool norm) {
  return (w8 ? rows_lds_bytes<true>(M, K, norm) : rows_lds_bytes<false>(M, K, norm)) <= kRowsMaxLds;
}

int launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* gamma, float eps,
                   uint16_t* xn, int64_t M, int64_t K, bool vec, hipStream_t s) {
  if (vec)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, gamma,
                       eps, xn, K);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, gamma,
                       eps, xn, K);
  return (int)hipGetLastError();
}

template <bool W8>
bool rows_supported(const StreamArgs& a, bool aligned) {
  const int64_t max_m = W8 ? kRowsMaxM : 2;
  return aligned && a.M >= 1 && a.M <= max_m &&
         rows_lds_bytes<W8>(a.M, a.K, a.gamma != nullptr) <= kRowsMaxLds;
}

template bool rows_supported<false>(const StreamArgs&, bool);
template bool rows_supported<true>(const StreamArgs&, bool);

// Measured on MI355X (Qwen3-4B and -8B, 24-36 cycled weight sets): the whole
// row in flight (K = 2560: 5 bf16 or 3 int8 chunks); bf16 one row (pair) per
// wave, 8 waves per workgroup; int8 with one x row read from L2 (K <= 2560,
// no fused norm): one row (pair) per wave, 4 waves per workgroup (with the
// non-temporal weight stream: 4B gate-up 12.51 -> 11.75 us against two row
// pairs per wave, QKV 5.85 -> 5.43 us against 8 waves; with x staged in LDS,
// 8B K = 4096, the 4-wave workgroups are 14% slower); otherwise int8 gate-up
// two row pairs per wave and 4 waves up to 2 x rows, one and 8 waves for
// 3..4; x rows rounded up to 1, 2, 4.
template <int MM, bool GATEUP, bool W8>
int launch_rows_m(const StreamArgs& a, hipStream_t s) {
  if constexpr (W8 && GATEUP && MM == 1) {
    // int8 gate-up at one x row: 8-byte chunks, 4 waves, 5 chunks in flight
    // (one box, µs, against the 16-byte chunks of rows_kernel: 4B 11.87-12.07
    // -> 10.91-11.00, 8B 19.71-20.23 -> 18.89-19.89; for QKV they measured
    // even or slower)
    if (!a.gamma) {
      const dim3 grid((unsigned)((a.N + 3) / 4)), block(4 * kWave);
      if (a.K <= 2560) {
        hipLaunchKernelGGL((rows_gate_up_w8_kernel<4, 5, true>), grid, block, 0, s, a);
      } else {
        const size_t shm = (size_t)((a.K + 511) / 512) * 512 * 2;
        hipLaunchKernelGGL((rows_gate_up_w8_kernel<4, 5, false>), grid, block, shm, s, a);
      }
      return (int)hipGetLastError();
    }
  }
  if constexpr (W8) {
    if constexpr (MM == 1)
      if (!a.gamma && a.K <= 2560) return launch_rows_cfg<4, 1, 3, 1, GATEUP, true>(a, s);
    if constexpr (GATEUP && MM <= 2) return launch_rows_cfg<4, 2, 3, MM, true, true>(a, s);
    if constexpr (GATEUP) return launch_rows_cfg<8, 1, 3, MM, true, true>(a, s);
    return launch_rows_cfg<8, 1, 3, MM, false, true>(a, s);
  } else {
    if constexpr (GATEUP) return launch_rows_cfg<8, 1, 5, MM, true, false>(a, s);
    return launch_rows_cfg<8, 1, 5, MM, false, false>(a, s);
  }
}

template <bool GATEUP, bool W8>
int launch_rows(const StreamArgs& a, hipStream_t s) {
  if (a.M == 1) return launch_rows_m<1, GATEUP, W8>(a, s);
  if (a.M == 2) return launch_rows_m<2, GATEUP, W8>(a, s);
  return launch_rows_m<4, GATEUP, W8>(a, s);
}

template int launch_rows<false, false>(const StreamArgs&, hipStream_t);
template int launch_rows<true, false>(const StreamArgs&, hipStream_t);
template int launch_rows<false, true>(const StreamArgs&, hipStream_t);
template int launch_rows<true, true>(const StreamArgs&, hipStream_t);

}  // namespace fp
