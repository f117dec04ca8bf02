// fp_stream.hip — weight-streaming fused projections for the decode /
// spec-verify regime (M <= 64), where every weight byte is used once per call
// and the HBM stream of W is the whole cost.
//
// Mapping (one workgroup = NW waves = one tile of 16 weight rows):
//   - The 16 rows of the tile are the A operand of v_mfma_f32_16x16x32_bf16;
//     x^T (M <= 16*MT columns, zero-padded) is the B operand, so each 16-byte
//     weight load per lane feeds MT MFMAs and the k-reduction happens inside
//     the matrix core. For gate-up the workgroup streams the same 16 rows of
//     Wg and Wu, so g and u of one output land in the same lane.
//   - K is split across the NW waves of the workgroup in interleaved k-blocks
//     (wave w takes blocks w, w+NW, ...), so at any moment the waves of a
//     workgroup read adjacent 64-byte pieces of the same 16 rows.
//   - Each wave double-buffers U k-blocks of loads in registers: the next U
//     blocks are in flight while the current U blocks go through the MFMAs.
//   - The NW partial tiles are summed through LDS in fixed wave order and the
//     epilogue (bf16 store, or silu(g)*u) runs in registers: the fp32
//     intermediate never reaches HBM, and results are bit-reproducible.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

template <int MT, bool W8>
struct Frag {
  u32x4 a0;                    // 16 B of weight row (8 bf16 or 16 int8)
  u32x4 a1;                    // same for the up weights (gate-up only)
  u32x4 xb[MT][W8 ? 2 : 1];    // B operand: 8 bf16 of x per MFMA
};

template <int NW, int MT, int U, bool GATEUP, bool W8, bool ALIGNED>
__global__ __launch_bounds__(NW * kWave) void stream_kernel(StreamArgs a) {
  constexpr int KB = W8 ? 64 : 32;          // k elements per k-block
  constexpr int NACC = MT * (GATEUP ? 2 : 1);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int li = lane & 15;                  // A row / B column within the tile
  const int grp = lane >> 4;                 // which quarter of the k-block
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = n0 + li;
  const bool row_ok = row < a.N;
  const int64_t K = a.K;
  const int64_t nkb = (K + KB - 1) / KB;

  // Weight row pointers (clamped to row 0 when out of range; loads are then
  // replaced by zeros below).
  const int64_t rsafe = row_ok ? row : 0;
  const char* w0row;
  const char* w1row = nullptr;
  if constexpr (W8) {
    w0row = (const char*)a.w0 + rsafe * a.ldw0;
    if constexpr (GATEUP) w1row = (const char*)a.w1 + rsafe * a.ldw1;
  } else {
    w0row = (const char*)a.w0 + rsafe * a.ldw0 * 2;
    if constexpr (GATEUP) w1row = (const char*)a.w1 + rsafe * a.ldw1 * 2;
  }
  float s0 = 0.f, s1 = 0.f;
  if constexpr (W8) {
    s0 = row_ok ? a.s0[row] : 0.f;
    if constexpr (GATEUP) s1 = row_ok ? a.s1[row] : 0.f;
  }
  const float n128s0 = -128.f * s0;
  const float n128s1 = -128.f * s1;

  // x rows this lane feeds into the B operand (column li of each m-subtile).
  const uint16_t* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    xok[mt] = m < a.M;
    xrow[mt] = a.x + (int64_t)(xok[mt] ? m : 0) * a.ldx;
  }

  auto load_block = [&](Frag<MT, W8>& f, int64_t kb) {
    const bool live = kb < nkb;
    const int64_t k = kb * KB + grp * (KB / 4);
    if constexpr (W8) {
      f.a0 = (live && row_ok) ? load_i8x16<ALIGNED>((const int8_t*)w0row, k, K) : u32x4{0, 0, 0, 0};
      if constexpr (GATEUP)
        f.a1 = (live && row_ok) ? load_i8x16<ALIGNED>((const int8_t*)w1row, k, K) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f.xb[mt][0] = (live && xok[mt]) ? load_bf16x8<ALIGNED>(xrow[mt], k, K) : u32x4{0, 0, 0, 0};
        f.xb[mt][1] = (live && xok[mt]) ? load_bf16x8<ALIGNED>(xrow[mt], k + 8, K) : u32x4{0, 0, 0, 0};
      }
    } else {
      f.a0 = (live && row_ok) ? load_bf16x8<ALIGNED>((const uint16_t*)w0row, k, K) : u32x4{0, 0, 0, 0};
      if constexpr (GATEUP)
        f.a1 = (live && row_ok) ? load_bf16x8<ALIGNED>((const uint16_t*)w1row, k, K) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        f.xb[mt][0] = (live && xok[mt]) ? load_bf16x8<ALIGNED>(xrow[mt], k, K) : u32x4{0, 0, 0, 0};
    }
  };

  f32x4 acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_block = [&](const Frag<MT, W8>& f) {
    if constexpr (W8) {
      const u32x4 g_lo = dequant8(f.a0.x, f.a0.y, s0, n128s0);
      const u32x4 g_hi = dequant8(f.a0.z, f.a0.w, s0, n128s0);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = mfma16(g_lo, f.xb[mt][0], acc[mt]);
        acc[mt] = mfma16(g_hi, f.xb[mt][1], acc[mt]);
      }
      if constexpr (GATEUP) {
        const u32x4 u_lo = dequant8(f.a1.x, f.a1.y, s1, n128s1);
        const u32x4 u_hi = dequant8(f.a1.z, f.a1.w, s1, n128s1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[MT + mt] = mfma16(u_lo, f.xb[mt][0], acc[MT + mt]);
          acc[MT + mt] = mfma16(u_hi, f.xb[mt][1], acc[MT + mt]);
        }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16(f.a0, f.xb[mt][0], acc[mt]);
      if constexpr (GATEUP) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[MT + mt] = mfma16(f.a1, f.xb[mt][0], acc[MT + mt]);
      }
    }
  };

  // k-blocks of this wave: wave, wave+NW, ...; processed in chunks of U.
  const int64_t nmine = nkb > wave ? (nkb - wave + NW - 1) / NW : 0;
  const int64_t nchunks = (nmine + U - 1) / U;
  Frag<MT, W8> fa[U], fb[U];
  auto load_chunk = [&](Frag<MT, W8>* f, int64_t c) {
#pragma unroll
    for (int j = 0; j < U; ++j) load_block(f[j], wave + (int64_t)NW * (c * U + j));
  };
  auto compute_chunk = [&](const Frag<MT, W8>* f, int64_t c) {
#pragma unroll
    for (int j = 0; j < U; ++j)
      if (wave + (int64_t)NW * (c * U + j) < nkb) compute_block(f[j]);
  };

  if (nchunks > 0) load_chunk(fa, 0);
  for (int64_t c = 0; c < nchunks; c += 2) {
    if (c + 1 < nchunks) load_chunk(fb, c + 1);
    compute_chunk(fa, c);
    if (c + 1 >= nchunks) break;
    if (c + 2 < nchunks) load_chunk(fa, c + 2);
    compute_chunk(fb, c + 1);
  }

  // Fixed-order cross-wave reduction through LDS, then the epilogue in wave 0.
  __shared__ f32x4 red[NW > 1 ? NW - 1 : 1][NACC][kWave];
  if constexpr (NW > 1) {
    if (wave > 0) {
#pragma unroll
      for (int i = 0; i < NACC; ++i) red[wave - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < NW - 1; ++w)
#pragma unroll
      for (int i = 0; i < NACC; ++i) acc[i] += red[w][i][lane];
  }

  // D lane layout: rows n0 + 4*grp + r (r = 0..3), column m = mt*16 + li.
  const int64_t nb = n0 + 4 * grp;
  const bool vec_ok = (nb + 3 < a.N) && ((a.ldy & 3) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    if (m >= a.M) continue;
    uint32_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (GATEUP)
        h[r] = gate_up_silu_bits(acc[mt][r], acc[MT + mt][r]);
      else
        h[r] = f32_to_bf16_bits(acc[mt][r]);
    }
    uint16_t* yrow = a.y + (int64_t)m * a.ldy;
    if (vec_ok) {
      *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) yrow[nb + r] = (uint16_t)h[r];
    }
  }
}

template <int NW, int MT, int U, bool GATEUP, bool W8>
int launch_stream_mt(const StreamArgs& a, bool aligned, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 15) / 16));
  const dim3 block(NW * kWave);
  if (aligned)
    hipLaunchKernelGGL((stream_kernel<NW, MT, U, GATEUP, W8, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((stream_kernel<NW, MT, U, GATEUP, W8, false>), grid, block, 0, s, a);
  return (int)hipGetLastError();
}

}  // namespace

template <bool GATEUP, bool W8>
int launch_stream(const StreamArgs& a, bool aligned, hipStream_t s) {
  // U: k-blocks in flight per buffer; bf16 gate-up streams two rows per block.
  if (a.M <= 16) return launch_stream_mt<4, 1, (GATEUP ? 4 : 8), GATEUP, W8>(a, aligned, s);
  if (a.M <= 32) return launch_stream_mt<4, 2, 4, GATEUP, W8>(a, aligned, s);
  if (a.M <= 48) return launch_stream_mt<4, 3, 4, GATEUP, W8>(a, aligned, s);
  return launch_stream_mt<4, 4, 2, GATEUP, W8>(a, aligned, s);
}

template int launch_stream<false, false>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<true, false>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<false, true>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<true, true>(const StreamArgs&, bool, hipStream_t);

}  // namespace fp
