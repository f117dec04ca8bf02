// fp_stream.hip — weight-streaming fused projections for the decode /
// spec-verify regime (M <= 64), where every weight byte is used once per call
// and the HBM stream of W is the whole cost.
//
// Memory pattern first: every weight load instruction reads whole 128-byte
// lines — 8 weight rows x 128 B per wave instruction (half-line requests cost
// ~25% of the achieved bandwidth on MI355X). The MFMA mapping is built
// around that:
//   - A workgroup owns a tile of 8 weight rows (for gate-up: the same 8 rows
//     of Wg and of Wu). In a load, lane l reads 16 B of row (l & 7) at chunk
//     c = 4*((l >> 3) & 1) + (l >> 4) of a 128 B line, i.e. rows 0..7 land in
//     MFMA rows i = l & 15 as two halves: MFMA row i holds weight row (i & 7),
//     line half (i >> 3).
//   - v_mfma_f32_16x16x32_bf16 then runs twice per load with two B operands
//     (x for the first and for the second half of the line); MFMA rows 0..7
//     of the first product and rows 8..15 of the second are the wanted partial
//     sums, the other halves are discarded. The MFMA pipe is ~90% idle in this
//     regime, so the doubled MFMA count is free; x^T (M <= 16*MT columns,
//     zero-padded) is the B operand.
//   - K is split across the NW waves of the workgroup, interleaved by k-block
//     (SPLIT 0) or in contiguous ranges (SPLIT 1). Each wave double-buffers U
//     k-blocks of loads in registers.
//   - x is read either from L2 per k-block or, XL, staged once per workgroup
//     in LDS.
//   - The NW partial tiles are summed through LDS in fixed wave order; the
//     epilogue (bf16 store, or silu(g)*u) runs in registers, so the fp32
//     intermediate never reaches HBM and results are bit-reproducible.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

// x vectors per lane per k-block: one per (line half, 8-element sub-chunk);
// packed (XP): one per sub-chunk, lanes 0..7 carrying half 0 and lanes 8..15
// half 1 (needs M <= 8).
template <bool W8, bool XP>
constexpr int x_vectors() { return (W8 ? 2 : 1) * (XP ? 1 : 2); }

template <int MT, bool GATEUP, bool W8, bool XP>
struct Frag {
  static constexpr int XV = x_vectors<W8, XP>();
  u32x4 a0;                               // 16 B of a weight line (8 bf16 or 16 int8)
  u32x4 a1;                               // same for the up weights (gate-up only)
  u32x4 xb[MT][XV];                       // B operands: 8 bf16 of x per vector
};

// Rotate a 4-dword value by 8 lanes within each row of 16 (DPP row_ror:8):
// lane i receives lane (i + 8) mod 16 of its row.
__device__ __forceinline__ u32x4 ror8(u32x4 v) {
  constexpr int kRowRor8 = 0x128;
  return u32x4{(uint32_t)__builtin_amdgcn_mov_dpp((int)v.x, kRowRor8, 0xf, 0xf, false),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v.y, kRowRor8, 0xf, 0xf, false),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v.z, kRowRor8, 0xf, 0xf, false),
               (uint32_t)__builtin_amdgcn_mov_dpp((int)v.w, kRowRor8, 0xf, 0xf, false)};
}

// XL: x is staged once per workgroup in LDS (M rows x K, dynamic shared
// memory) and the B operand is read from there instead of from L2.
// XP: packed x operand for M <= 8 (one x load per sub-chunk; the B operand of
// line half 1 is the half-0 register rotated by 8 lanes).
template <int NW, int MT, int U, int SPLIT, bool GATEUP, bool W8, bool ALIGNED, bool XL,
          bool XP = false>
__global__ __launch_bounds__(NW * kWave) void stream_kernel(StreamArgs a) {
  static_assert(!XP || (MT == 1 && !XL), "packed x needs M <= 8 and x from L2");
  using F = Frag<MT, GATEUP, W8, XP>;
  constexpr int XV = F::XV;
  constexpr int SV = W8 ? 2 : 1;           // 8-element sub-chunks per lane per line half
  constexpr int KB = W8 ? 128 : 64;        // k elements per k-block (one 128 B line)
  constexpr int CK = KB / 8;               // k elements per 16-byte chunk of the line
  constexpr int NM = GATEUP ? 2 : 1;       // weight matrices
  constexpr int NACC = 2 * MT * NM;        // [half][matrix][mt]

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int li = lane & 15;                // MFMA row (A) / column (B)
  const int grp = lane >> 4;               // MFMA k-group
  const int64_t n0 = (int64_t)blockIdx.x * 8;
  const int64_t row = n0 + (lane & 7);     // weight row this lane loads
  const int chunk = 4 * ((lane >> 3) & 1) + grp;
  const bool row_ok = row < a.N;
  const int64_t K = a.K;
  const int64_t nkb = (K + KB - 1) / KB;

  const int64_t rsafe = row_ok ? row : 0;
  const char* w0row = (const char*)a.w0 + rsafe * a.ldw0 * (W8 ? 1 : 2);
  const char* w1row = GATEUP ? (const char*)a.w1 + rsafe * a.ldw1 * (W8 ? 1 : 2) : nullptr;
  float s0 = 0.f, s1 = 0.f;
  if constexpr (W8) {
    s0 = row_ok ? a.s0[row] : 0.f;
    if constexpr (GATEUP) s1 = row_ok ? a.s1[row] : 0.f;
  }
  const float n128s0 = -128.f * s0;
  const float n128s1 = -128.f * s1;

  // x rows this lane feeds into the B operands (column li of each m-subtile;
  // packed: column li & 7, line half li >> 3).
  const uint16_t* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = XP ? (li & 7) : mt * 16 + li;
    xok[mt] = m < a.M;
    xrow[mt] = a.x + (int64_t)(xok[mt] ? m : 0) * a.ldx;
  }
  const int xhalf = XP ? (li >> 3) : 0;

  // k-blocks of this wave
  int64_t kb_first, kb_stride, nmine;
  if constexpr (SPLIT == 0) {
    kb_first = wave;
    kb_stride = NW;
    nmine = nkb > wave ? (nkb - wave + NW - 1) / NW : 0;
  } else {
    const int64_t per = (nkb + NW - 1) / NW;
    kb_first = wave * per;
    kb_stride = 1;
    const int64_t end = kb_first + per < nkb ? kb_first + per : nkb;
    nmine = end > kb_first ? end - kb_first : 0;
  }

  // First k of the 8 x values group grp supplies to the MFMA of line half h,
  // sub-chunk s (int8 lines carry two 8-element sub-chunks per lane).
  auto xk = [&](int64_t kb, int h, int s) -> int64_t {
    return kb * KB + h * (KB / 2) + grp * CK + s * 8;
  };

  auto load_block = [&](F& f, int64_t j) {
    const bool live = j < nmine;
    const int64_t kb = kb_first + j * kb_stride;
    const int64_t kw = kb * KB + chunk * CK;
    const u32x4 z{0, 0, 0, 0};
    if constexpr (W8) {
      f.a0 = (live && row_ok) ? load_w_i8x16<ALIGNED>((const int8_t*)w0row, kw, K) : z;
      if constexpr (GATEUP)
        f.a1 = (live && row_ok) ? load_w_i8x16<ALIGNED>((const int8_t*)w1row, kw, K) : z;
    } else {
      f.a0 = (live && row_ok) ? load_w_bf16x8<ALIGNED>((const uint16_t*)w0row, kw, K) : z;
      if constexpr (GATEUP)
        f.a1 = (live && row_ok) ? load_w_bf16x8<ALIGNED>((const uint16_t*)w1row, kw, K) : z;
    }
    if constexpr (!XL) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < XV; ++v) {
          // packed: v = sub-chunk, half from the lane; else v = h * SV + s
          const int h = XP ? xhalf : v / SV;
          const int s = XP ? v : v % SV;
          f.xb[mt][v] = (live && xok[mt]) ? load_bf16x8<ALIGNED>(xrow[mt], xk(kb, h, s), K) : z;
        }
    }
  };

  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  // B operand for line half h, sub-chunk s of m-subtile mt at this wave's
  // j-th k-block.
  auto xfrag = [&](const F& f, int mt, int h, int s, int64_t j) -> u32x4 {
    if constexpr (XP) {
      return h == 0 ? f.xb[mt][s] : ror8(f.xb[mt][s]);
    } else if constexpr (XL) {
      const int64_t k = xk(kb_first + j * kb_stride, h, s);
      const int m = mt * 16 + li;
      if (!xok[mt] || k >= K) return u32x4{0, 0, 0, 0};
      const uint16_t* p = xs + (int64_t)m * K + k;
      if constexpr (ALIGNED) {
        return *reinterpret_cast<const u32x4*>(p);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (k + e < K) ? (uint32_t)p[e] : 0u;
        return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                     h[6] | (h[7] << 16)};
      }
    } else {
      return f.xb[mt][h * SV + s];
    }
  };

  f32x4 acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // accumulator of (line half h, matrix mat, m-subtile mt)
  auto A = [&](int h, int mat, int mt) -> f32x4& { return acc[(h * NM + mat) * MT + mt]; };

  auto compute_block = [&](const F& f, int64_t j) {
#pragma unroll
    for (int mat = 0; mat < NM; ++mat) {
      const u32x4 w = mat == 0 ? f.a0 : f.a1;
      if constexpr (W8) {
        const float s = mat == 0 ? s0 : s1;
        const float n128s = mat == 0 ? n128s0 : n128s1;
        const u32x4 wlo = dequant8(w.x, w.y, s, n128s);
        const u32x4 whi = dequant8(w.z, w.w, s, n128s);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            A(h, mat, mt) = mfma16(wlo, xfrag(f, mt, h, 0, j), A(h, mat, mt));
            A(h, mat, mt) = mfma16(whi, xfrag(f, mt, h, 1, j), A(h, mat, mt));
          }
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h) A(h, mat, mt) = mfma16(w, xfrag(f, mt, h, 0, j), A(h, mat, mt));
      }
    }
  };

  const int64_t nchunks = (nmine + U - 1) / U;
  F fa[U], fb[U];
  auto load_chunk = [&](F* f, int64_t c) {
#pragma unroll
    for (int j = 0; j < U; ++j) load_block(f[j], c * U + j);
  };
  auto compute_chunk = [&](const F* f, int64_t c) {
#pragma unroll
    for (int j = 0; j < U; ++j)
      if (c * U + j < nmine) compute_block(f[j], c * U + j);
  };

  // Prologue: two chunks of weight loads in flight before anything waits.
  auto prologue = [&]() {
    if (nchunks > 0) load_chunk(fa, 0);
    if (nchunks > 1) load_chunk(fb, 1);
  };
  if constexpr (XL) {
    // Stage x[0:M, 0:K] in LDS: issue the global reads of x, then the first
    // two chunks of weight loads, then write x to LDS (waits only for the x
    // reads, which were issued first).
    const int64_t total = a.M * K;
    constexpr int NT = NW * kWave;
    if constexpr (ALIGNED) {
      const int64_t nvec = total / 8;
      const int64_t per_row = K / 8;
      constexpr int XR = 4;
      for (int64_t base = 0; base < nvec; base += (int64_t)NT * XR) {
        u32x4 t[XR];
#pragma unroll
        for (int r = 0; r < XR; ++r) {
          const int64_t i = base + threadIdx.x + (int64_t)r * NT;
          t[r] = i < nvec ? ld16(a.x + (i / per_row) * a.ldx + (i % per_row) * 8) : u32x4{0, 0, 0, 0};
        }
        if (base == 0) prologue();
#pragma unroll
        for (int r = 0; r < XR; ++r) {
          const int64_t i = base + threadIdx.x + (int64_t)r * NT;
          if (i < nvec) *reinterpret_cast<u32x4*>(xs + i * 8) = t[r];
        }
      }
    } else {
      prologue();
      for (int64_t i = threadIdx.x; i < total; i += NT) xs[i] = a.x[(i / K) * a.ldx + (i % K)];
    }
    __syncthreads();
  } else {
    prologue();
  }
  // Steady state: while one chunk is consumed the other is in flight; a
  // consumed buffer is refilled with the chunk two ahead.
  for (int64_t c = 0; c < nchunks; c += 2) {
    compute_chunk(fa, c);
    if (c + 2 < nchunks) load_chunk(fa, c + 2);
    if (c + 1 >= nchunks) break;
    compute_chunk(fb, c + 1);
    if (c + 3 < nchunks) load_chunk(fb, c + 3);
  }

  // Fixed-order cross-wave reduction through LDS.
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

  // D lane layout: MFMA rows 4*grp + r (r = 0..3), column li. Lanes 0..31
  // hold rows 0..7 (line half 0 of weight rows 0..7) of the first product;
  // lanes 32..63 hold rows 8..15 (half 1 of the same weight rows) of the
  // second. Output row n0 + 4*grp + r (grp < 2) = half 0 (lane) + half 1
  // (lane + 32).
  float sum[NM][MT][4];
#pragma unroll
  for (int mat = 0; mat < NM; ++mat)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float hi = __shfl_down(A(1, mat, mt)[r], 32);
        sum[mat][mt][r] = A(0, mat, mt)[r] + hi;
      }
  if (lane >= 32) return;

  const int64_t nb = n0 + 4 * grp;
  const bool vec_ok = (nb + 3 < a.N) && ((a.ldy & 3) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    if (m >= a.M) continue;
    uint32_t hb[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (GATEUP)
        hb[r] = gate_up_silu_bits(sum[0][mt][r], sum[1][mt][r]);
      else
        hb[r] = f32_to_bf16_bits(sum[0][mt][r]);
    }
    uint16_t* yrow = a.y + (int64_t)m * a.ldy;
    if (vec_ok) {
      *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) yrow[nb + r] = (uint16_t)hb[r];
    }
  }
}

// Dynamic LDS bytes an XL launch needs for x (M rows of K bf16).
inline size_t xl_bytes(const StreamArgs& a) { return (size_t)a.M * (size_t)a.K * 2; }

template <int NW, int MT, int U, int SPLIT, bool GATEUP, bool W8, bool XL, bool XP = false>
int launch_stream_cfg(const StreamArgs& a, bool aligned, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 7) / 8));
  const dim3 block(NW * kWave);
  const size_t shm = XL ? xl_bytes(a) : 0;
  if (aligned)
    hipLaunchKernelGGL((stream_kernel<NW, MT, U, SPLIT, GATEUP, W8, true, XL, XP>), grid, block, shm, s, a);
  else
    hipLaunchKernelGGL((stream_kernel<NW, MT, U, SPLIT, GATEUP, W8, false, XL, XP>), grid, block, shm, s, a);
  return (int)hipGetLastError();
}

}  // namespace

// Configurations measured on MI355X (Qwen3-4B shapes, 36 cycled weight sets):
// 4 waves per 8-row tile with interleaved k-blocks; packed x for M <= 8; the
// gate-up kernel (two weight streams) keeps 4 k-blocks per buffer in flight,
// QKV 2 (QKV's 3x smaller grid is latency-bound and prefers occupancy).
template <bool GATEUP, bool W8>
int launch_stream(const StreamArgs& a, bool aligned, hipStream_t s) {
  // int8 at 2-16 rows with K <= 2560: x staged once per workgroup, all weight
  // loads in flight (fp_xpanel.hip)
  if (W8 && xpanel8_shape(a.M, a.N, a.K, GATEUP) && splitk_supported(a, aligned, true))
    return launch_xpanel8<GATEUP>(a, s);
  // int8 from a few rows: split-K tiles dequantising in registers (fp_splitk.hip)
  if (W8 && splitk8_shape(a.M, a.N, a.K, GATEUP) && splitk_supported(a, aligned, true))
    return launch_splitk<GATEUP, true>(a, s);
  // one or a few rows: contiguous row streaming (fp_rows.hip)
  if (rows_supported<W8>(a, aligned)) return launch_rows<GATEUP, W8>(a, s);
  // bf16 against large weights with a caller workspace: k split across
  // workgroups (fp_gemm.hip)
  GemmSplit sp;
  if (!W8 && use_gemm_split(a, aligned, GATEUP, &sp)) return launch_gemm_split<GATEUP, false>(a, sp, s);
  // bf16 with a nearly full round of small staged tiles (from 48 rows
  // against large weights): fp_gemm.hip
  if (!W8 && small_round_tile(a.M, a.N, a.K, GATEUP) >= 0 && gemm_supported(a, aligned, false))
    return launch_gemm<GATEUP, false>(a, s);
  // bf16 from 3 (small N, e.g. QKV) or 8 rows: split-K tiles (fp_splitk.hip)
  const int64_t wrows = GATEUP ? 2 * a.N : a.N;
  // (wide gate-up from fewer rows: 4 with K > 3072, 6 below. One box, µs,
  // stream -> split-K tiles: Qwen3-8B M = 4 34.0 -> 33.2, M = 6 35.1 -> 32.8,
  // M = 7 36.3-37.4 -> 33.0, M = 3 33.0 -> 34.0; Qwen3-4B M = 7 21.0 -> 20.2,
  // M = 6 even, M = 4 19.3 -> 20.1)
  const int64_t min_m = wrows <= kSplitkSmallN ? kSplitkMinMSmallN
                        : GATEUP               ? (a.K > 3072 ? 4 : 6)
                                               : kSplitkMinM;
  if (!W8 && a.M >= min_m && splitk_supported(a, aligned, false))
    return launch_splitk<GATEUP, false>(a, s);
  // (int8 dequantisation needs registers of its own: 2 k-blocks per buffer)
  constexpr int U8 = (GATEUP && !W8) ? 4 : 2;
  if (a.M <= 8) return launch_stream_cfg<4, 1, U8, 0, GATEUP, W8, false, true>(a, aligned, s);
  if (a.M <= 16) return launch_stream_cfg<4, 1, 2, 0, GATEUP, W8, false>(a, aligned, s);
  if (a.M <= 32) return launch_stream_cfg<4, 2, 2, 0, GATEUP, W8, false>(a, aligned, s);
  if (a.M <= 48) return launch_stream_cfg<4, 3, 2, 0, GATEUP, W8, false>(a, aligned, s);
  return launch_stream_cfg<4, 4, 1, 0, GATEUP, W8, false>(a, aligned, s);
}

template int launch_stream<false, false>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<true, false>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<false, true>(const StreamArgs&, bool, hipStream_t);
template int launch_stream<true, true>(const StreamArgs&, bool, hipStream_t);

}  // namespace fp
