// fp_tiled.hip — LDS-tiled MFMA fused projections for the prefill regime
// (M > 64), where the contraction is compute-bound.
//
// Tile = BN weight rows x BM rows of x, k-steps of BK staged through LDS:
//   - Weight rows are the A operand of v_mfma_f32_16x16x32_bf16 and x rows
//     the B operand, so a lane's accumulator holds 4 consecutive output
//     columns of one x row (8-byte stores).
//   - Gate-up tiles interleave 16-row groups of Wg and Wu (gate group, up
//     group, gate group, ...), so g and u of one output sit in the same lane
//     in adjacent accumulators and silu(g)*u is applied in registers.
//   - int8 weights are dequantised (w = bf16(q * s)) on the way into LDS, so
//     the MFMA loop is the bf16 one.
//   - Global -> register prefetch of k-step t+1 overlaps the MFMAs of step t;
//     two LDS buffers, one barrier per k-step.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kPad = 8;  // bf16 elements of padding per LDS row (16 B)

template <int BN, int BM, int BK, int WN, int WM, bool GATEUP, bool W8, bool ALIGNED>
__global__ __launch_bounds__(WN * WM * kWave) void tiled_kernel(StreamArgs a) {
  constexpr int NT = WN * WM * kWave;
  constexpr int TN = BN / WN, TM = BM / WM;   // per-wave tile
  constexpr int FN = TN / 16, FM = TM / 16;   // 16x16 MFMA sub-tiles per wave
  constexpr int LDP = BK + kPad;              // LDS row pitch (elements)
  constexpr int WCH = W8 ? 16 : 8;            // k elements per 16-byte weight chunk
  constexpr int CW = BN * BK / WCH / NT;      // weight chunks per thread per k-step
  constexpr int CX = BM * BK / 8 / NT;        // x chunks per thread per k-step
  static_assert(BN * BK / WCH % NT == 0 && BM * BK / 8 % NT == 0, "tile/threads");
  static_assert(!GATEUP || TN % 32 == 0, "gate-up needs whole gate/up pairs per wave");

  __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN][LDP];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM][LDP];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wn = wave / WM, wm = wave % WM;
  const int li = lane & 15, grp = lane >> 4;

  const int64_t K = a.K;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  // Output column base of this tile; gate-up tiles produce BN/2 columns.
  const int64_t c0 = (int64_t)blockIdx.x * (GATEUP ? BN / 2 : BN);

  // ---- per-thread global chunk assignment (fixed across k-steps) ----
  const char* wsrc[CW];
  bool wok[CW];
  float wsc[CW];
  int wrow_l[CW], wk_l[CW];
#pragma unroll
  for (int j = 0; j < CW; ++j) {
    const int c = tid + j * NT;
    const int t = c / (BK / WCH);
    const int kc = c % (BK / WCH);
    wrow_l[j] = t;
    wk_l[j] = kc * WCH;
    int64_t n;
    bool up = false;
    if constexpr (GATEUP) {
      const int sub = t / 16;
      n = c0 + (sub / 2) * 16 + (t % 16);
      up = (sub & 1) != 0;
    } else {
      n = c0 + t;
    }
    wok[j] = n < a.N;
    const int64_t ns = wok[j] ? n : 0;
    const void* base = up ? a.w1 : a.w0;
    const int64_t ld = up ? a.ldw1 : a.ldw0;
    wsrc[j] = (const char*)base + ns * ld * (W8 ? 1 : 2);
    if constexpr (W8) wsc[j] = wok[j] ? (up ? a.s1 : a.s0)[n] : 0.f;
    else wsc[j] = 0.f;
  }
  const uint16_t* xsrc[CX];
  bool xok[CX];
  int xrow_l[CX], xk_l[CX];
#pragma unroll
  for (int j = 0; j < CX; ++j) {
    const int c = tid + j * NT;
    const int t = c / (BK / 8);
    xrow_l[j] = t;
    xk_l[j] = (c % (BK / 8)) * 8;
    const int64_t m = m0 + t;
    xok[j] = m < a.M;
    xsrc[j] = a.x + (xok[j] ? m : 0) * a.ldx;
  }

  u32x4 rw[CW], rx[CX];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < CW; ++j) {
      const int64_t k = k0 + wk_l[j];
      if constexpr (W8)
        rw[j] = wok[j] ? load_i8x16<ALIGNED>((const int8_t*)wsrc[j], k, K) : u32x4{0, 0, 0, 0};
      else
        rw[j] = wok[j] ? load_bf16x8<ALIGNED>((const uint16_t*)wsrc[j], k, K) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < CX; ++j)
      rx[j] = xok[j] ? load_bf16x8<ALIGNED>(xsrc[j], k0 + xk_l[j], K) : u32x4{0, 0, 0, 0};
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < CW; ++j) {
      if constexpr (W8) {
        const float s = wsc[j], n128s = -128.f * s;
        *reinterpret_cast<u32x4*>(&sW[buf][wrow_l[j]][wk_l[j]]) = dequant8(rw[j].x, rw[j].y, s, n128s);
        *reinterpret_cast<u32x4*>(&sW[buf][wrow_l[j]][wk_l[j] + 8]) = dequant8(rw[j].z, rw[j].w, s, n128s);
      } else {
        *reinterpret_cast<u32x4*>(&sW[buf][wrow_l[j]][wk_l[j]]) = rw[j];
      }
    }
#pragma unroll
    for (int j = 0; j < CX; ++j) *reinterpret_cast<u32x4*>(&sX[buf][xrow_l[j]][xk_l[j]]) = rx[j];
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t nkt = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < nkt) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      u32x4 fa[FN], fb[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i)
        fa[i] = *reinterpret_cast<const u32x4*>(&sW[buf][wn * TN + i * 16 + li][kk * 32 + grp * 8]);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        fb[j] = *reinterpret_cast<const u32x4*>(&sX[buf][wm * TM + j * 16 + li][kk * 32 + grp * 8]);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nkt) sstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const bool y8 = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m0 + wm * TM + j * 16 + li;
    if (m >= a.M) continue;
    uint16_t* yrow = a.y + m * a.ldy;
    if constexpr (GATEUP) {
#pragma unroll
      for (int i = 0; i < FN; i += 2) {
        const int sub = (wn * TN) / 16 + i;  // even: gate group of pair sub/2
        const int64_t nb = c0 + (sub / 2) * 16 + 4 * grp;
        uint32_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = gate_up_silu_bits(acc[i][j][r], acc[i + 1][j][r]);
        if (y8 && nb + 3 < a.N) {
          *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nb + r < a.N) yrow[nb + r] = (uint16_t)h[r];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int64_t nb = c0 + wn * TN + i * 16 + 4 * grp;
        uint32_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16_bits(acc[i][j][r]);
        if (y8 && nb + 3 < a.N) {
          *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nb + r < a.N) yrow[nb + r] = (uint16_t)h[r];
        }
      }
    }
  }
}

template <int BN, int BM, int BK, int WN, int WM, bool GATEUP, bool W8>
int launch_cfg(const StreamArgs& a, bool aligned, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const dim3 grid((unsigned)((a.N + cols - 1) / cols), (unsigned)((a.M + BM - 1) / BM));
  const dim3 block(WN * WM * kWave);
  if (aligned)
    hipLaunchKernelGGL((tiled_kernel<BN, BM, BK, WN, WM, GATEUP, W8, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((tiled_kernel<BN, BM, BK, WN, WM, GATEUP, W8, false>), grid, block, 0, s, a);
  return (int)hipGetLastError();
}

}  // namespace

// bf16 calls that meet gemm_kernel's requirements run there (direct-to-LDS
// loads, XCD-aware order): split across workgroups when the plan says so and
// the caller gave a workspace, else unsplit — except, without the split, up
// to kSplitkMaxM rows against at most 8192 weight rows with K >=
// kSplitkMinKTiled, which give too few tiles for 256 CUs and run the
// in-workgroup split-K tiles, unless a round of tiles with 128-wide k-steps
// has a tile for every CU and one per 20 columns of K (k128_wide: Qwen3-4B
// QKV, 6144 x 2560, at 160-256 rows: 23.0-28.6 -> 17.9-24.4 us; below 160
// rows, and 8B QKV, 4B o and 0.6B o and down, keep the split-K tiles, up to
// 20% faster there), or unless a round of small three-stage tiles fits
// (small_round_tile: 8B QKV at 256 rows 31.6 -> 26.8 us). int8 shapes that
// splitk8_shape() admits run the split-K tiles too, other aligned int8 calls
// with whole 64-wide k-steps run gemm_kernel (both dequantise in registers);
// unaligned rows and K tails run tiled_kernel.
template <bool GATEUP, bool W8>
int launch_tiled(const StreamArgs& a, bool aligned, hipStream_t s) {
  const int64_t wrows = GATEUP ? 2 * a.N : a.N;
  GemmSplit sp;
  if (!W8 && use_gemm_split(a, aligned, GATEUP, &sp)) return launch_gemm_split<GATEUP, false>(a, sp, s);
  if (!W8 && a.M <= kSplitkMaxM && wrows <= kSplitkSmallN && a.K >= kSplitkMinKTiled &&
      splitk_supported(a, aligned, false) && !k128_wide(a.M, a.N, a.K, GATEUP) &&
      small_round_tile(a.M, a.N, a.K, GATEUP) < 0)
    return launch_splitk<GATEUP, false>(a, s);
  if (!W8 && gemm_supported(a, aligned, false)) return launch_gemm<GATEUP, false>(a, s);
  if (W8 && splitk8_shape(a.M, a.N, a.K, GATEUP) && splitk_supported(a, aligned, true))
    return launch_splitk<GATEUP, true>(a, s);
  // int8 that reaches here either suits the in-register gemm or had no
  // workspace to dequantise into: gemm_kernel either way
  if (W8 && gemm_supported(a, aligned, true)) return launch_gemm<GATEUP, true>(a, s);
  return launch_cfg<128, 128, 64, 2, 2, GATEUP, W8>(a, aligned, s);
}

template int launch_tiled<false, false>(const StreamArgs&, bool, hipStream_t);
template int launch_tiled<true, false>(const StreamArgs&, bool, hipStream_t);
template int launch_tiled<false, true>(const StreamArgs&, bool, hipStream_t);
template int launch_tiled<true, true>(const StreamArgs&, bool, hipStream_t);

}  // namespace fp
