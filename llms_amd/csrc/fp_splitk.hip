// fp_splitk.hip — fused projections for the middle regime (from 3-8 rows up to
// a few hundred): too many x rows for the weight-streaming kernels' register
// budget, too few output tiles for the 256 x 256 prefill tiles to fill 256 CUs
// (QKV has N = 6144: 24 tiles of 256 rows).
//
// A workgroup owns a small output tile: BN weight rows (gate-up: BN/2 rows of
// Wg and BN/2 of Wu, interleaved in 16-row groups) x BM rows of x. A bf16
// QKV tile may hold 24 rows: its second MFMA block then reads 8 rows past
// the tile's (other bytes of the wave's own stage) into accumulator rows
// that are never stored; the matrix core is idle enough in this regime for
// that to cost nothing. Its NW
// waves split K: wave w takes k-steps w, w + NW, w + 2 NW, ... (64 k each),
// each wave with a private ring of NS LDS stages that it fills itself with
// buffer_load_dwordx4 ... lds (8 tile rows x 128 B per instruction, whole
// lines, XOR-swizzled so the fragment reads are conflict-free). The bytes in
// flight therefore live in LDS, not in registers, and the main loop has no
// barrier: a wave only waits for its own loads. After the last step the
// waves' partial tiles are summed through LDS in fixed wave order and the
// epilogue (bf16 store, or silu(g)*u at torch's rounding points) runs on
// wave 0's share of the tile.
// int8 weights (W8) land in LDS as int8 (64 B per row and k-step) and each
// lane dequantises its MFMA A fragment in registers to bf16(q * s), exactly
// as the dequantise-then-matmul path rounds it.
// Requirements (checked by splitk_supported): K % 64 == 0, 16-byte-aligned
// rows, operand byte sizes below 2^31, int8 row scales present.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kBK = 64;                  // k per step
constexpr int kCPR = kBK / 8;            // 16-byte chunks per tile row
constexpr int kRPI = 1024 / (kBK * 2);   // tile rows per load instruction

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & (kCPR - 1); }
__device__ __forceinline__ int swz8(int r) { return (r >> 2) & 3; }

// buffer_load_dwordx4 ... lds: 16 bytes per lane from base + voff + soff into
// LDS at dst + 16 * lane; bytes at or past `nbytes` read as zero. NT: the
// non-temporal hint (cache-policy bit 1), for the weight stream, which a
// call reads once.
template <bool NT = false>
__device__ __forceinline__ void load_lds16(const void* base, int nbytes, lds_ptr_t dst,
                                           uint32_t voff, uint32_t soff) {
  constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, kRsrcFlags), dst, 16,
      voff, soff, 0, NT ? 2 : 0);
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= v only.
constexpr int vmcnt_imm(int v) { return (v & 15) | (7 << 4) | (15 << 8) | ((v >> 4) << 14); }

template <int BN, int BM, int NW, int NS, bool GATEUP, bool W8>
__global__ __launch_bounds__(NW * kWave) void splitk_kernel(StreamArgs a, int n_mt) {
  constexpr int WB = W8 ? 1 : 2;               // bytes per weight element
  constexpr int WROW = kBK * WB;               // bytes of a weight tile row per step
  constexpr int WRPI = 1024 / WROW;            // weight rows per load instruction
  constexpr int WCPR = WROW / 16;              // 16-byte chunks per weight row
  constexpr int FN = (BN + 15) / 16, FM = BM / 16;  // MFMA sub-tiles (the whole tile per wave)
  constexpr int IW = BN / WRPI, IX = BM / kRPI;  // load instructions per stage
  constexpr int kPerStep = IW + IX;
  constexpr int SW = BN * WROW, SX = BM * kBK * 2;  // bytes per wave and stage
  static_assert((BN % 16 == 0 || (BN % 8 == 0 && !GATEUP && !W8)) && BM % 16 == 0 &&
                    BN % WRPI == 0,
                "tile: whole 16-row blocks, or a last half block for bf16 QKV");
  static_assert(!GATEUP || BN % 32 == 0, "gate-up tiles hold whole gate/up 16-row pairs");
  static_assert(NS == 2 || NS == 3, "LDS stages");
  // the partial tiles of waves 1 .. NW-1 are summed in stage 0's space, FC
  // weight fragments (all FM x fragments of each) per pass
  constexpr int FC0 = NW * (SW + SX) / ((NW - 1) * FM * 1024);
  constexpr int FC = FC0 >= FN ? FN : FC0;
  static_assert(FC >= 1, "reduction space");

  // One LDS object per stage (distinct alias scopes: reads of one stage are
  // not ordered after the asynchronous writes into another), each split per
  // wave into the weight rows (SW bytes) then the x rows (SX bytes).
  __shared__ __attribute__((aligned(1024))) char sS0[NW][SW + SX];
  __shared__ __attribute__((aligned(1024))) char sS1[NW][SW + SX];
  __shared__ __attribute__((aligned(1024))) char sS2[NS > 2 ? NW : 1][SW + SX];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int li = lane & 15, grp = lane >> 4;

  const int tm = blockIdx.x % n_mt, tn = blockIdx.x / n_mt;  // M-fastest: W tile reused in L2
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t c0 = (int64_t)tn * (GATEUP ? BN / 2 : BN);  // first output column

  // Weight row t of the tile: output n(t) of matrix Wu when up(t) (gate-up
  // tiles interleave 16-row groups of Wg and Wu).
  auto wrow_n = [&](int t) -> int64_t { return GATEUP ? c0 + (t / 32) * 16 + (t % 16) : c0 + t; };
  auto wrow_up = [&](int t) -> bool { return GATEUP && ((t / 16) & 1); };

  // Per-lane byte offsets of this lane's 16 B in each load instruction (see
  // fp_gemm.hip: a load instruction fills 1 KB of consecutive tile rows; the
  // swizzle is applied on the global side so the LDS writes stay
  // lane-linear). bf16 weight rows (128 B per step): chunk c of row r at
  // c ^ ((r >> 1) & 7); int8 rows (64 B per step): c ^ ((r >> 2) & 3), which
  // keeps the 8-byte fragment reads of 16 rows on distinct banks.
  const int lrow = lane / kCPR, lchunk = lane % kCPR;
  uint32_t woff[IW];
#pragma unroll
  for (int q = 0; q < IW; ++q) {
    const int t = q * WRPI + lane / WCPR;
    const int c = lane % WCPR;
    const int64_t ld = wrow_up(t) ? a.ldw1 : a.ldw0;
    woff[q] = (uint32_t)(wrow_n(t) * ld * WB) + (uint32_t)((c ^ (W8 ? swz8(t) : swz(t))) * 16);
  }
  uint32_t xoff[IX];
#pragma unroll
  for (int q = 0; q < IX; ++q) {
    const int t = q * kRPI + lrow;
    xoff[q] = (uint32_t)((m0 + t) * a.ldx * 2) + (uint32_t)((lchunk ^ swz(t)) * 16);
  }
  const int wbytes0 = (int)((a.N - 1) * a.ldw0 * WB + a.K * WB);
  const int wbytes1 = GATEUP ? (int)((a.N - 1) * a.ldw1 * WB + a.K * WB) : wbytes0;
  const int xbytes = (int)((a.M - 1) * a.ldx * 2 + a.K * 2);
  void* const wptr1 = (void*)(GATEUP ? a.w1 : a.w0);

  // int8: this lane's row scales (rows 16 i + li), zero past N
  float sc[W8 ? FN : 1], nsc[W8 ? FN : 1];
  if constexpr (W8) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int t = 16 * i + li;
      const int64_t n = wrow_n(t);
      sc[i] = n < a.N ? (wrow_up(t) ? a.s1 : a.s0)[n] : 0.f;
      nsc[i] = -128.f * sc[i];
    }
  }

  auto stage = [&](int s) -> char* {
    return s == 0 ? sS0[wave] : (s == 1 ? sS1[wave] : sS2[NS > 2 ? wave : 0]);
  };
  auto issue = [&](int s, int64_t k0) {
    char* t = stage(s);
#pragma unroll
    for (int q = 0; q < IW; ++q) {
      // instruction q holds 16-row groups of one matrix (uniform per instruction)
      const bool up = wrow_up(q * WRPI);
      load_lds16<true>(up ? wptr1 : a.w0, up ? wbytes1 : wbytes0, (lds_ptr_t)(t + q * 1024), woff[q],
                 (uint32_t)(k0 * WB));
    }
#pragma unroll
    for (int q = 0; q < IX; ++q)
      load_lds16(a.x, xbytes, (lds_ptr_t)(t + SW + q * 1024), xoff[q], (uint32_t)(k0 * 2));
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fragment byte offsets (the swizzle of row 16 i + li does not depend on
  // i). k-substep kk: bf16 flips chunk bit 2, int8 chunk bit 1.
  const uint32_t offa = W8 ? (uint32_t)(li * WROW + ((((grp >> 1) ^ swz8(li)) * 16) | ((grp & 1) * 8)))
                           : (uint32_t)(li * WROW + ((grp ^ swz(li)) * 16));
  const uint32_t offb = (uint32_t)(SW + li * kBK * 2 + ((grp ^ swz(li)) * 16));
  auto compute = [&](int s) {
    const char* t = stage(s);
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      const uint32_t oa = offa ^ (uint32_t)(kk * (W8 ? 32 : 64)), ob = offb ^ (uint32_t)(kk * 64);
      u32x4 fa[FN], fb[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        if constexpr (W8) {
          const u32x2 q = *reinterpret_cast<const u32x2*>(t + oa + i * 16 * WROW);
          fa[i] = dequant8_bf16(q.x, q.y, sc[i], nsc[i]);
        } else {
          fa[i] = *reinterpret_cast<const u32x4*>(t + oa + i * 16 * WROW);
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) fb[j] = *reinterpret_cast<const u32x4*>(t + ob + j * 16 * kBK * 2);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
    }
  };

  // This wave's k-steps: w, w + NW, ...; the ring keeps NS - 1 of them in
  // flight while one is consumed.
  const int64_t nkt = a.K / kBK;
  const int64_t mine = nkt > wave ? (nkt - wave + NW - 1) / NW : 0;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < mine) issue(s, (wave + (int64_t)NW * s) * kBK);
  for (int64_t j0 = 0; j0 < mine; j0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int64_t j = j0 + u;
      if (j >= mine) break;
      if (j + NS - 1 < mine) {
        issue((u + NS - 1) % NS, (wave + NW * (j + NS - 1)) * kBK);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * kPerStep));
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
      compute(u);
    }
  }

  // Fixed-order cross-wave sum through LDS (the ring is free now), in passes
  // of FC weight fragments where the partials of a large tile do not fit
  // one stage: each output is still summed in wave order 0, 1, ..., NW - 1.
  float* red = reinterpret_cast<float*>(&sS0[0][0]);
#pragma unroll
  for (int p0 = 0; p0 < FN; p0 += FC) {
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (int i = p0; i < p0 + FC && i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          *reinterpret_cast<f32x4*>(red + (((wave - 1) * FC + i - p0) * FM + j) * 256 + lane * 4) =
              acc[i][j];
    }
    __syncthreads();
    if (wave == 0) {
      for (int w = 0; w < NW - 1; ++w)
#pragma unroll
        for (int i = p0; i < p0 + FC && i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] += *reinterpret_cast<const f32x4*>(
                red + ((w * FC + i - p0) * FM + j) * 256 + lane * 4);
    }
  }
  if (wave != 0) return;

  // Epilogue: D lane holds rows 4*grp + r (weight rows) of column li (x row).
  const bool y8 = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m0 + j * 16 + li;
    if (m >= a.M) continue;
    uint16_t* yrow = a.y + m * a.ldy;
#pragma unroll
    for (int i = 0; i < FN; i += (GATEUP ? 2 : 1)) {
      int64_t nb;
      uint32_t h[4];
      if constexpr (GATEUP) {
        nb = c0 + (i / 2) * 16 + 4 * grp;  // i even: gate group of pair i/2
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = gate_up_silu_bits(acc[i][j][r], acc[i + 1][j][r]);
      } else {
        if (i * 16 + 4 * grp >= BN) continue;  // rows past a 24-row tile
        nb = c0 + i * 16 + 4 * grp;
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16_bits(acc[i][j][r]);
      }
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

template <int BN, int BM, int NW, int NS, bool GATEUP, bool W8>
int launch_splitk_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  hipLaunchKernelGGL((splitk_kernel<BN, BM, NW, NS, GATEUP, W8>), dim3((unsigned)(n_nt * n_mt)),
                     dim3(NW * kWave), 0, s, a, n_mt);
  return (int)hipGetLastError();
}

}  // namespace

bool splitk_supported(const StreamArgs& a, bool aligned, bool w8) {
  constexpr int64_t kLim = (int64_t)1 << 31;
  const int64_t wb = w8 ? 1 : 2;
  if (!aligned || a.K % kBK != 0) return false;
  if (w8 && (!a.s0 || (a.w1 && !a.s1))) return false;
  if ((a.N - 1) * a.ldw0 * wb + a.K * wb >= kLim) return false;
  if (a.w1 && (a.N - 1) * a.ldw1 * wb + a.K * wb >= kLim) return false;
  if ((a.M - 1) * a.ldx * 2 + a.K * 2 >= kLim) return false;
  return true;
}

// Tile tables measured on MI355X (Qwen3-4B and -8B shapes, cycled weight
// sets, warm clocks): the x tile is M rounded up to 16 (up to 64 rows), then
// 64 x 64 tiles; gate-up tiles hold 16 outputs (32 weight rows). int8 (half
// the bytes per weight row, so more rows of LDS per wave) prefers 8 waves.
// Narrow bf16 outputs at up to 16 rows with K >= 2560 (the per-GPU shards
// of tensor parallelism: QKV of at most 2048 columns, gate-up of at most
// 3072; also 0.6B down) have too few tiles for 256 CUs; 8 waves per tile put
// twice the k-steps in flight there. Same-box A/B, µs at M = 4 and 8, 4 -> 8
// waves: 8B QKV 1536 columns 8.1-8.4 -> 6.1-7.0, 768 columns 8.0-8.2 ->
// 5.6-7.2; 8B gate-up 3072 columns 12.5-12.8 -> 11.0-11.7, 1536 columns
// 10.7-11.2 -> 8.8-9.6; 4B QKV 768 and 1536 columns 6.0-6.8 -> 4.6-5.9;
// 0.6B down (1024 x 3072) 6.5-7.0 -> 5.7-6.3. The full Qwen3-4B/8B outputs
// keep 4 waves (8 were 2-14% slower there).
// int8 gate-up over wide outputs (at least 7680 columns, so that 96-row
// tiles number 160 or more: Qwen3-4B and 8B) from 17 rows: 96 weight rows
// (48 outputs) per tile. Every tile reads the x rows of the call again from
// L2, which with 32-row int8 tiles (32 B of weights per x row and k) was 4x
// the weight bytes; 96 rows cut that to 1.3x. Same box, µs, 8B / 4B, against
// the 32- and 64-row tiles: M = 24 33.7 -> 31.5 / 22.9 -> 22.2 (96 x 32, 3
// stages); M = 40 47.5 -> 35.5 / 33.5 -> 25.4 (96 x 48, 3 stages); M = 64
// 51.8 -> 40.4 / 36.7 -> 29.3 (96 x 64); M = 96 81.5 -> 48.5 / 58.6 -> 35.9
// (96 x 96); M = 112 76.7 -> 51.8 / 55.4 -> 38.7 (96 x 112, the LDS full);
// M = 128 78.4 -> 59.6 / 56.2 -> 44.9 (96 x 128 with 3 waves, whose two
// stages fit where 4 waves' do not; two tiles of 64 rows: 78.6 / 56.2).
// Each weight is dequantised once per row tile, so one tile over all the
// rows beats two. At 16 rows 96 x 16 was slower (29.8 / 18.9 against 26.6
// / 18.5).
template <bool GATEUP, bool W8>
int launch_splitk(const StreamArgs& a, hipStream_t s) {
  if constexpr (W8 && GATEUP) {
    if (a.M > 16 && a.N >= 7680) {
      if (a.M <= 32) return launch_splitk_cfg<96, 32, 4, 3, true, true>(a, s);
      if (a.M <= 48) return launch_splitk_cfg<96, 48, 4, 3, true, true>(a, s);
      if (a.M <= 64) return launch_splitk_cfg<96, 64, 4, 2, true, true>(a, s);
      if (a.M <= 96) return launch_splitk_cfg<96, 96, 4, 2, true, true>(a, s);
      if (a.M <= 112) return launch_splitk_cfg<96, 112, 4, 2, true, true>(a, s);
      return launch_splitk_cfg<96, 128, 3, 2, true, true>(a, s);
    }
    if (a.M <= 16) return launch_splitk_cfg<32, 16, 8, 2, true, true>(a, s);
    if (a.M <= 32) return launch_splitk_cfg<32, 32, 4, 3, true, true>(a, s);
    if (a.M <= 64) return launch_splitk_cfg<32, 64, 8, 2, true, true>(a, s);
    return launch_splitk_cfg<64, 64, 4, 2, true, true>(a, s);
  } else if constexpr (W8) {
    if (a.M <= 16) return launch_splitk_cfg<32, 16, 8, 3, false, true>(a, s);
    if (a.M <= 32) return launch_splitk_cfg<32, 32, 8, 2, false, true>(a, s);
    if (a.M <= 64) return launch_splitk_cfg<32, 64, 8, 2, false, true>(a, s);
    return launch_splitk_cfg<64, 64, 4, 2, false, true>(a, s);
  } else if constexpr (GATEUP) {
    // wide gate-up with a short K (Qwen3-4B) at 8-16 rows: 96-row tiles, the
    // same k split and order (bit-identical), a third of the x re-reads (one
    // box, µs: M = 8 20.9 -> 20.3, M = 12 21.4 -> 20.4, M = 16 22.0 -> 21.0;
    // on Qwen3-8B, K = 4096, they measured slower: 32.7 -> 39.1)
    if (a.M <= 16 && a.N >= 7680 && a.K <= 3072)
      return launch_splitk_cfg<96, 16, 4, 2, true, W8>(a, s);
    // ... and at 17-64 rows (203 tiles on Qwen3-4B where 32-row tiles made
    // 608; the two libraries alternated on one box, µs, M = 17, 24, 32, 40,
    // 47: 26.9, 28.2, 30.2, 36.4, 37.3 -> 23.1, 23.6, 24.1, 27.8, 28.2; from
    // 48 rows the staged tiles of fp_gemm.hip take these calls)
    if (a.M <= 64 && a.N >= 7680 && a.K <= 3072)
      return a.M <= 32 ? launch_splitk_cfg<96, 32, 4, 2, true, W8>(a, s)
                       : launch_splitk_cfg<96, 64, 4, 2, true, W8>(a, s);
    if (a.M <= 16)
      return a.N <= 3072 && a.K >= 2560 ? launch_splitk_cfg<32, 16, 8, 2, true, W8>(a, s)
                         : launch_splitk_cfg<32, 16, 4, 3, true, W8>(a, s);
    if (a.M <= 32) return launch_splitk_cfg<32, 32, 8, 2, true, W8>(a, s);
    if (a.M <= 64) return launch_splitk_cfg<32, 64, 4, 3, true, W8>(a, s);
    return launch_splitk_cfg<64, 64, 4, 2, true, W8>(a, s);
  } else {
    // Qwen3-sized QKV (4096 < N <= 6144, K 2048..4096) at up to 16 rows:
    // 24-row tiles with 8 waves, at most 256 of them, one per CU. The two
    // libraries alternated on one box over 36 weight sets (µs): Qwen3-4B (K =
    // 2560) at M = 3, 4, 8, 16 7.77, 7.83, 9.1, 9.55 -> 7.65, 7.65, 8.7, 9.25
    // against 32-row tiles (192 of them; bit-identical, the same k order);
    // Qwen3-8B (K = 4096) at M = 4, 16 11.17, 13.3 -> 10.95, 11.2 against
    // 16-row tiles of 4 waves.
    if (!W8 && a.M <= 16 && splitk24_shape(a.M, a.N, a.K))
      return launch_splitk_cfg<24, 16, 8, 2, false, false>(a, s);
    // ... and at 17-64 rows: 8 waves of 32 x rows to 32 rows, then 4 waves of
    // 64 with three LDS stages (same comparison, Qwen3-8B at M = 32, 48, 64:
    // 15.1, 18.2, 19.0 -> 13.2, 17.1, 17.95 against 32-row tiles)
    if (!W8 && splitk24_shape(a.M, a.N, a.K))
      return a.M <= 32 ? launch_splitk_cfg<24, 32, 8, 2, false, false>(a, s)
                       : launch_splitk_cfg<24, 64, 4, 3, false, false>(a, s);
    // Qwen3-4B-sized QKV (4096 < N <= 8192, K 2048..3072) at up to 16 rows:
    // 32-row tiles with 8 waves (one box, µs at M = 3, 4, 8, 16: 8.11, 8.50,
    // 8.77, 9.85 -> 7.73, 8.02, 8.32, 8.80 against 16-row tiles of 4 waves;
    // on Qwen3-8B, K = 4096, and 0.6B, K = 1024, they measured 3-12% slower)
    if (a.M <= 16 && a.N > 4096 && a.N <= 8192 && a.K >= 2048 && a.K <= 3072)
      return launch_splitk_cfg<32, 16, 8, 2, false, W8>(a, s);
    if (a.M <= 16)
      return a.N <= 2048 && a.K >= 2560 ? launch_splitk_cfg<16, 16, 8, 3, false, W8>(a, s)
                         : launch_splitk_cfg<16, 16, 4, 3, false, W8>(a, s);
    if (a.M <= 32) return launch_splitk_cfg<32, 32, 4, 3, false, W8>(a, s);
    if (a.M <= 64) return launch_splitk_cfg<32, 64, 4, 3, false, W8>(a, s);
    return launch_splitk_cfg<64, 64, 4, 2, false, W8>(a, s);
  }
}

template int launch_splitk<false, false>(const StreamArgs&, hipStream_t);
template int launch_splitk<true, false>(const StreamArgs&, hipStream_t);
template int launch_splitk<false, true>(const StreamArgs&, hipStream_t);
template int launch_splitk<true, true>(const StreamArgs&, hipStream_t);

}  // namespace fp
