// fp_gemm.hip — prefill-regime (M > 64) fused projections as an LDS-tiled
// bf16 MFMA contraction with direct global->LDS loads.
//
//   - Tile = BN weight rows x BM rows of x, k-steps of BK = 64. Weight rows are
//     the A operand of v_mfma_f32_16x16x32_bf16 and x rows the B operand, so a
//     lane's accumulator holds 4 consecutive output columns of one x row.
//   - Operand tiles move HBM/L2 -> LDS with global_load_lds_dwordx4: one wave
//     instruction fills 1 KB of LDS (8 tile rows x 128 B, whole cache lines).
//     The lane -> global address choice realises an XOR-swizzled LDS layout
//     (16-byte chunk c of tile row r lives at chunk c ^ ((r >> 1) & 7)), which
//     keeps the MFMA fragment reads (ds_read_b128) free of bank conflicts.
//   - Two LDS buffers; loads of k-step t+1 are in flight during the MFMAs of
//     step t; one barrier per k-step. No registers stage the operands.
//   - Gate-up tiles interleave 16-row groups of Wg and Wu so g and u of one
//     output sit in adjacent accumulators of one lane; silu(g)*u is applied in
//     registers at the torch rounding points.
//   - Workgroups are remapped so that each XCD (its own L2) runs a contiguous
//     range of tiles, ordered in groups of 8 m-tiles, M-fastest inside a
//     group: the ~32 tiles an XCD runs at once (8 m x 4 n) share their weight
//     and activation panels in its L2.
// Requirements (checked by the dispatcher): bf16, K % 64 == 0, 16-byte-aligned
// rows (the general case runs tiled_kernel).
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kBK = 64;          // k per LDS stage (bf16 unsplit tiles may take 128)
constexpr int kGroupM = 8;       // m-tiles per group of the tile order

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// XOR swizzle of the 16-byte chunks of bf16 tile row r at a k-step of BK:
// 64 (8 chunks per row, chunk c stored at c ^ ((r >> 1) & 7)) or 128 (16
// chunks, at c ^ (r & 15)); either way the 16 rows that one fragment read
// touches land on distinct LDS banks.
template <int BK>
__device__ __forceinline__ int swzk(int r) { return BK == 64 ? (r >> 1) & 7 : r & 15; }
__device__ __forceinline__ int swz8(int r) { return (r >> 2) & 3; }

// buffer_load_dwordx4 ... lds: 16 bytes per lane from base + voff + soff into
// LDS at dst + 16 * lane; bytes at or past `nbytes` read as zero.
// (device-only so the host pass never sees the AMDGPU builtins)
__device__ __forceinline__ void load_lds16(const void* base, int nbytes, lds_ptr_t dst,
                                           uint32_t voff, uint32_t soff) {
  constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, kRsrcFlags), dst, 16,
      voff, soff, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= v only.
constexpr int vmcnt_imm(int v) { return (v & 15) | (7 << 4) | (15 << 8) | ((v >> 4) << 14); }
// ... and for lgkmcnt == 0 (every LDS access of this wave done) as well.
constexpr int vmcnt_lgkm0_imm(int v) { return (v & 15) | (7 << 4) | ((v >> 4) << 14); }

// SPLIT: the grid holds nsplit workgroups per tile, each contracting one
// contiguous range of k-steps, and the fp32 accumulators go to the workspace
// ws[split][m][col] (col: output column n; gate-up: g at n, u at N + n) for
// splitk_reduce_kernel, which sums them in split order.
// W8: int8 weights with per-row scales (a.s0, a.s1). A weight tile row is 64 B
// per k-step in LDS (16 rows per load instruction, chunk c of row r at
// c ^ ((r >> 2) & 3)); each lane turns the 8 int8 of its MFMA A fragment into
// bf16(q * s) in registers (dequant8_bf16: the dequantise-then-matmul
// rounding) before the bf16 MFMA. (The one-tile-per-CU kernel below
// dequantises once per workgroup instead.)
template <int BN, int BM, int WN, int WM, bool GATEUP, int NS, bool SPLIT = false, bool W8 = false,
          int BK = kBK>
__global__ __launch_bounds__(WN * WM * kWave) void gemm_kernel(StreamArgs a, int n_mt, int n_nt,
                                                              int ksteps, float* ws) {
  constexpr int NW = WN * WM;
  constexpr int CPR = BK / 8;                 // 16-byte chunks per tile row
  constexpr int RPI = 1024 / (BK * 2);        // tile rows per load instruction
  static_assert(BK == kBK || (BK == 2 * kBK && !W8 && !SPLIT), "k-step: 64, or 128 for bf16 unsplit");
  constexpr int TN = BN / WN, TM = BM / WM;   // per-wave tile
  constexpr int FN = TN / 16, FM = TM / 16;   // MFMA sub-tiles per wave
  constexpr int WB = W8 ? 1 : 2;              // bytes per weight element
  constexpr int WKE = BK * WB / 2;           // weight LDS row, in 16-bit units
  constexpr int WRPI = W8 ? 16 : RPI;        // weight rows per load instruction
  constexpr int WCPR = W8 ? 4 : CPR;         // 16-byte chunks per weight row
  constexpr int NWI = BN / WRPI;              // weight load instructions per stage
  constexpr int IW = (NWI + NW - 1) / NW;     // ... per wave (the last may be idle)
  constexpr int IX = BM / RPI / NW;          // x load instructions per wave per stage
  static_assert(BN % WRPI == 0 && BM % (RPI * NW) == 0, "tile/waves");
  static_assert(W8 || NWI % NW == 0, "bf16 weight loads spread evenly over the waves");
  // with three stages the waits count a wave's loads per step, so they must
  // be the same for every wave
  static_assert(NS == 2 || NWI % NW == 0, "three stages need even weight loads");
  static_assert(!GATEUP || TN % 32 == 0, "gate-up needs whole gate/up pairs per wave");
  static_assert(NS == 2 || NS == 3, "LDS stages");

  // One LDS object per stage and operand: distinct objects carry distinct
  // alias scopes, so the compiler can see that fragment reads of one stage do
  // not depend on the asynchronous global->LDS writes into another stage
  // (with a single [NS][..] array it waits for all loads before every read).
  __shared__ __attribute__((aligned(1024))) uint16_t sW0[BN][WKE];
  __shared__ __attribute__((aligned(1024))) uint16_t sW1[BN][WKE];
  __shared__ __attribute__((aligned(1024))) uint16_t sW2[NS > 2 ? BN : 1][WKE];
  __shared__ __attribute__((aligned(1024))) uint16_t sX0[BM][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX1[BM][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX2[NS > 2 ? BM : 1][BK];

  const int lane = threadIdx.x & (kWave - 1);
  // wave index as a scalar: load instructions, LDS bases and buffer
  // resources chosen by it stay uniform (no waterfall loops)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wn = wave / WM, wm = wave % WM;
  const int li = lane & 15, grp = lane >> 4;

  // XCD-aware tile order (see file comment); with SPLIT the k-range index is
  // the slowest.
  const int T = (int)gridDim.x;
  int b = blockIdx.x;
  if (T % 8 == 0) b = (b % 8) * (T / 8) + b / 8;
  const int ks = SPLIT ? b / (n_mt * n_nt) : 0;
  b -= ks * n_mt * n_nt;
  // Groups of kGroupM m-tiles, M-fastest inside a group: the 32 tiles an XCD
  // runs at once form an 8 x 4 block (12 operand panels per k-step in its L2)
  // rather than a strip down one weight panel (33 panels once M > 8 tiles).
  const int gbase = (b / (kGroupM * n_nt)) * kGroupM;
  const int gm = n_mt - gbase < kGroupM ? n_mt - gbase : kGroupM;
  const int gin = b - gbase * n_nt;
  const int tm = gbase + gin % gm, tn = gin / gm;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t c0 = (int64_t)tn * (GATEUP ? BN / 2 : BN);  // first output column

  // Load instruction q (q = wave + NW*j) fills tile rows RPI q .. RPI q + RPI-1
  // (RPI = 8 at a k-step of 64, 4 at 128; int8 weights: 16) with
  // buffer_load_dwordx4 ... lds: the matrix base lives in a buffer resource
  // (SGPRs), the k-step in soffset, and each lane carries one 32-bit byte
  // offset (row * stride + chunk). The resource size is the matrix size, so
  // rows past the end read as zeros. The dispatcher guarantees matrix byte
  // sizes below 2^32.
  const int lrow = lane / CPR;                 // row within an instruction's RPI
  const int lchunk = lane % CPR;               // LDS chunk position it fills
  // weight tile row t: output n(t) of matrix Wu when up(t) (gate-up tiles
  // interleave 16-row groups of Wg and Wu)
  auto wrow_n = [&](int t) -> int64_t { return GATEUP ? c0 + (t / 32) * 16 + (t % 16) : c0 + t; };
  auto wrow_up = [&](int t) -> bool { return GATEUP && ((t / 16) & 1); };
  uint32_t woff[IW];
#pragma unroll
  for (int j = 0; j < IW; ++j) {
    const int q = wave + NW * j;
    const int t = q * WRPI + lane / WCPR;
    const int c = lane % WCPR;
    const int64_t ld = wrow_up(t) ? a.ldw1 : a.ldw0;
    woff[j] = (uint32_t)(wrow_n(t) * ld * WB) + (uint32_t)((c ^ (W8 ? swz8(t) : swzk<BK>(t))) * 16);
  }
  uint32_t xoff[IX];
#pragma unroll
  for (int j = 0; j < IX; ++j) {
    const int t = (wave + NW * j) * RPI + lrow;
    xoff[j] = (uint32_t)((m0 + t) * a.ldx * 2) + (uint32_t)((lchunk ^ swzk<BK>(t)) * 16);
  }
  // byte sizes of the buffer resources (rows past them read as zeros)
  const int wbytes0 = (int)((a.N - 1) * a.ldw0 * WB + a.K * WB);
  const int wbytes1 = GATEUP ? (int)((a.N - 1) * a.ldw1 * WB + a.K * WB) : wbytes0;
  const int xbytes = (int)((a.M - 1) * a.ldx * 2 + a.K * 2);
  void* const wptr1 = (void*)(GATEUP ? a.w1 : a.w0);

  // int8: this lane's row scales (weight rows wn * TN + 16 i + li), zero past N
  float sc[W8 ? FN : 1], nsc[W8 ? FN : 1];
  if constexpr (W8) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int t = wn * TN + 16 * i + li;
      const int64_t n = wrow_n(t);
      sc[i] = n < a.N ? (wrow_up(t) ? a.s1 : a.s0)[n] : 0.f;
      nsc[i] = -128.f * sc[i];
    }
  }

  auto issue = [&](uint16_t (*tw)[WKE], uint16_t (*tx)[BK], int64_t k0) {
    const uint32_t kb = (uint32_t)(k0 * 2);
#pragma unroll
    for (int j = 0; j < IW; ++j) {
      const int q = wave + NW * j;
      if (q >= NWI) break;  // uniform per wave
      // gate-up: 16-row groups alternate Wg, Wu; uniform per instruction
      const bool up = wrow_up(q * WRPI);
      load_lds16(up ? wptr1 : a.w0, up ? wbytes1 : wbytes0, (lds_ptr_t)&tw[q * WRPI][0], woff[j],
                 (uint32_t)(k0 * WB));
    }
#pragma unroll
    for (int j = 0; j < IX; ++j)
      load_lds16(a.x, xbytes, (lds_ptr_t)&tx[(wave + NW * j) * RPI][0], xoff[j], kb);
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment addresses: sub-tile i of a wave reads tile row base + 16 i + li,
  // and swzk<BK>() of that row does not depend on i (16 i only touches row bits
  // above the swizzle), so every fragment address is one per-lane byte offset
  // plus the compile-time constants 16 i * 2 BK and the stage base. k-substep
  // kk flips chunk bits 2.. (chunk (4 kk + grp) ^ s = (grp ^ s) ^ 4 kk).
  const int ra = wn * TN + li, rb = wm * TM + li;
  // int8: 8 bytes at chunk 2 kk + (grp >> 1), half grp & 1 (k-substep kk
  // flips chunk bit 1)
  const uint32_t offa =
      W8 ? (uint32_t)(ra * BK + ((((grp >> 1) ^ swz8(ra)) * 16) | ((grp & 1) * 8)))
         : (uint32_t)(ra * BK * 2 + ((grp ^ swzk<BK>(ra)) * 16));
  const uint32_t offb = (uint32_t)(rb * BK * 2 + ((grp ^ swzk<BK>(rb)) * 16));
  auto compute = [&](const uint16_t (*tw)[WKE], const uint16_t (*tx)[BK]) {
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      const uint32_t oa = offa ^ (uint32_t)(kk * (W8 ? 32 : 64)), ob = offb ^ (uint32_t)(kk * 64);
      u32x4 fa[FN], fb[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        if constexpr (W8) {
          const u32x2 q = *reinterpret_cast<const u32x2*>((const char*)tw + oa + i * 16 * BK);
          fa[i] = dequant8_bf16(q.x, q.y, sc[i], nsc[i]);
        } else {
          fa[i] = *reinterpret_cast<const u32x4*>((const char*)tw + oa + i * 16 * BK * 2);
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j)
        fb[j] = *reinterpret_cast<const u32x4*>((const char*)tx + ob + j * 16 * BK * 2);
      // With 8 waves (two per SIMD) the wave issuing MFMAs gets the higher
      // priority, so the SIMD's other wave fits its LDS reads and load issue
      // in between (measured: 4B gate-up M = 2048 180.3 -> 175.9 us, 4B QKV
      // M = 2048 60.0 -> 58.8 us; with one wave per SIMD it costs ~2%).
      if constexpr (NW >= 8) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
      if constexpr (NW >= 8) __builtin_amdgcn_s_setprio(0);
      // keep each k-substep's fragments in one register set (the co-resident
      // wave on the SIMD hides the LDS latency)
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto stw = [&](int s) -> uint16_t (*)[WKE] { return s == 0 ? sW0 : (s == 1 ? sW1 : sW2); };
  auto stx = [&](int s) -> uint16_t (*)[BK] { return s == 0 ? sX0 : (s == 1 ? sX1 : sX2); };

  // Ring of NS stages: k-step k lives in stage k % NS, and while step k is
  // consumed steps k+1 .. k+NS-1 are in flight. After a step, wait until this
  // wave's loads of step k+1 have landed (the NS-2 later steps may stay in
  // flight), then for every wave's.
  constexpr int kPerStep = IW + IX;  // load instructions per wave per step (even loads)
  const int64_t kfirst = (int64_t)ks * ksteps;  // first k-step of this workgroup
  const int64_t nleft = a.K / BK - kfirst;
  const int64_t nkt = SPLIT ? (ksteps < nleft ? (int64_t)ksteps : nleft) : a.K / BK;
  const int64_t kb0 = kfirst * BK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) issue(stw(s), stx(s), kb0 + s * BK);
  if (nkt > NS - 2)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * kPerStep));
  else
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  for (int64_t kt = 0; kt < nkt; kt += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {  // u: compile-time stage of step kt + u
      const int64_t k = kt + u;
      if (k >= nkt) break;
      const bool steady = k + NS - 1 < nkt;
      if (steady) issue(stw((u + NS - 1) % NS), stx((u + NS - 1) % NS), kb0 + (k + NS - 1) * BK);
      compute(stw(u), stx(u));
      if (steady)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * kPerStep));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __syncthreads();
    }
  }

  if constexpr (SPLIT) {
    // fp32 partials: 4 consecutive columns of one x row per lane
    const int64_t wc = GATEUP ? 2 * a.N : a.N;
    // 16-byte partial stores where every column offset is a multiple of 4
    // (gate-up: u at N + n, so N itself must be)
    const bool v16 = (a.N & 3) == 0;
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int64_t m = m0 + wm * TM + j * 16 + li;
      if (m >= a.M) continue;
      float* prow = ws + ((int64_t)ks * a.M + m) * wc;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        int64_t n, col;
        if constexpr (GATEUP) {
          const int sub = (wn * TN) / 16 + i;  // even: gate rows, odd: up rows
          n = c0 + (sub / 2) * 16 + 4 * grp;
          col = (sub & 1) ? a.N + n : n;
        } else {
          n = c0 + wn * TN + i * 16 + 4 * grp;
          col = n;
        }
        if (v16 && n + 3 < a.N) {
          *reinterpret_cast<f32x4*>(prow + col) = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < a.N) prow[col + r] = acc[i][j][r];
        }
      }
    }
    return;
  }

  // ---- epilogue ----
  const bool y8 = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m0 + wm * TM + j * 16 + li;
    if (m >= a.M) continue;
    uint16_t* yrow = a.y + m * a.ldy;
#pragma unroll
    for (int i = 0; i < FN; i += (GATEUP ? 2 : 1)) {
      int64_t nb;
      uint32_t p0, p1;  // packed bf16 of columns nb, nb+1 and nb+2, nb+3
      if constexpr (GATEUP) {
        const int sub = (wn * TN) / 16 + i;  // even: gate group of pair sub/2
        nb = c0 + (sub / 2) * 16 + 4 * grp;
        uint32_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = gate_up_silu_bits(acc[i][j][r], acc[i + 1][j][r]);
        p0 = h[0] | (h[1] << 16);
        p1 = h[2] | (h[3] << 16);
      } else {
        nb = c0 + wn * TN + i * 16 + 4 * grp;
        p0 = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        p1 = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
      }
      if (y8 && nb + 3 < a.N) {
        *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{p0, p1};
      } else {
        const uint32_t h[4] = {p0 & 0xffffu, p0 >> 16, p1 & 0xffffu, p1 >> 16};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < a.N) yrow[nb + r] = (uint16_t)h[r];
      }
    }
  }
}

// The one-tile-per-CU grids (256 x 256, 192 x 256, 320 x 256; k-steps of 64,
// two LDS stages) as a persistent tile loop: one workgroup per CU runs tiles
// b, b + G/8, b + 2G/8, ... of its XCD's contiguous range of the tile order
// (WG g runs on XCD g % 8), so that
//   - the next tile's first k-step is loaded into stage 0 before this tile's
//     epilogue runs, and the load latency hides under the epilogue;
//   - the epilogue stores whole 16-byte chunks of contiguous output columns:
//     each wave passes its accumulators through a private LDS strip of 16 x
//     rows in stage 1 (free once the k loop has ended) and reads them back
//     row-contiguous (stores of 16 rows x 8 bytes per instruction, as the
//     accumulator layout gives, cost 2x the time at the end of a tile);
//   - the gate-up epilogue converts two outputs per v_cvt_pk_bf16_f32
//     (gate_up_silu_pair).
// int8 weights (W8) are dequantised once per workgroup, not per fragment
// read: the raw rows of k-step k + 1 land by DMA in a staging buffer (two,
// 64 B per row each), and during the first half of step k every lane turns
// its 16-byte chunks into bf16(q * s) in the operand stage of step k + 1, as
// the dequantise-then-matmul path rounds them; the MFMAs then read bf16
// fragments exactly as for bf16 weights. Against dequantising each fragment
// in every wave that reads it (2-4x the VALU work, more than the MFMA time),
// 4B QKV at M = 2048 (192 x 256) 77.1 -> 60.8 us, gate-up (256 x 256 plus a
// 256 x 128 tail) 210.5 -> 203 us. The staging needs BN x 128 B of LDS more,
// so 320 x 256 (184 KB) is bf16 only.
// Same k-steps in the same order as gemm_kernel: bit-identical outputs.
// Measured on MI355X against gemm_kernel (4 weight sets cycled): 4B QKV M =
// 2048 (192 x 256) 60.6 -> 54.7 us, M = 8192 (256 x 256) 215.7 -> 210.3 us;
// 4B gate-up M = 8192 711 -> 683 us.
// Four waves (WN x WM = 2 x 2, one wave per SIMD, bf16, an even number of
// k-steps): a wave tile of 96 x 128 reads 30% fewer fragment bytes from LDS
// than the 8-wave 96 x 64, but its 192 accumulators per lane need AGPRs.
// Through the MFMA builtin the compiler then splits them between AGPRs and
// VGPRs and copies them back and forth every k-step (or spills); issued by
// inline asm with the accumulators as "+a" operands they stay in AGPRs, and
// the k loop is the 8-wave one without its odd-count exit (which made the
// compiler double-buffer the fragments). The assembler cannot see what the
// asm statements write, so the accumulators' first and last accesses
// around them are separated by explicit s_nop (24 wait states, more than a
// 16x16x32 MFMA's result latency). Gate-up 192 x 256, bit-identical: 4B M =
// 512 66.3 -> 62.9 us, M = 500 x 9700 70.4 -> 65.2, 8B M = 512 99.9 -> 95.4;
// with 16 k-steps (0.6B, M = 2048) 29.4 -> 30.1, so four waves need at least
// 32. QKV 192 x 256 with four waves is 1-3% faster (4B M = 2048 61.1 -> 60.4
// us) and the 256 x 256 forms slower (4B QKV M = 8192 207 -> 219-225 us), so
// the 192 x 256 tiles run four waves where the step count allows; the 192 x
// 128 tile (96 accumulators per lane) has four waves only.
// With four waves the k-step may also be 128 wide (BK = 128: four 32-wide
// substeps, each one's MFMAs carrying the next one's fragment reads, the
// barrier before the last), for the one-round grids of 96 x 128 and 128 x
// 128 tiles that gemm_kernel would run with 128-wide steps; and small tiles
// may take three or four LDS stages (NS), and then (SPLIT) contract one
// range of k-steps per work item into fp32 partials for
// splitk_reduce_kernel, as gemm_kernel's split form does.
template <int BN, int BM, int WN, int WM, bool GATEUP, bool W8, int BK = kBK, int NS = 2,
          bool SPLIT = false>
__global__ __launch_bounds__(WN * WM * kWave) void gemm_tiles_kernel(StreamArgs a, int n_mt,
                                                                    int n_nt, int nsplit,
                                                                    int per, float* ws) {
  constexpr int NW = WN * WM;
  constexpr int CPR = BK / 8;
  constexpr int RPI = 1024 / (BK * 2);
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 16, FM = TM / 16;
  constexpr int WB = W8 ? 1 : 2;
  constexpr int WRPI = W8 ? 16 : RPI;         // weight rows per load instruction
  constexpr int WCPR = W8 ? 4 : CPR;          // 16-byte chunks per weight row
  constexpr int NWI = BN / WRPI;
  constexpr int IW = (NWI + NW - 1) / NW;
  constexpr int IX = BM / RPI / NW;
  constexpr int NQC = BN * 4;                 // int8: 16-byte chunks per k-step
  constexpr int QCH = (NQC + NW * kWave - 1) / (NW * kWave);  // ... per lane
  constexpr int TNO = GATEUP ? TN / 2 : TN;   // output columns per wave
  constexpr int SROW = TNO + 8;               // LDS strip row stride (elements)
  constexpr int CPRO = TNO / 8;               // 16-byte chunks per strip row
  static_assert(BK == 64 || (BK == 128 && WN * WM == 4 && !W8),
                "32-wide k-substeps: two per k-step, or four with four bf16 waves");
  static_assert(NS == 2 || ((NS == 3 || NS == 4) && WN * WM == 4 && !W8),
                "three or four LDS stages: four bf16 waves");
  static_assert(!SPLIT || NS > 2, "k split across workgroups: the staged four-wave loop");
  static_assert(BN % WRPI == 0 && BM % (RPI * NW) == 0, "tile/waves");
  static_assert(W8 || NWI % NW == 0, "bf16 weight loads spread evenly over the waves");
  static_assert(NQC % kWave == 0, "int8 chunks: whole waves");
  static_assert(!GATEUP || TN % 32 == 0, "gate-up needs whole gate/up pairs per wave");
  static_assert(NW * 16 * SROW * 2 <= BM * BK * 2, "epilogue strips fit in one x stage");
  static_assert(TNO % 8 == 0, "whole 16-byte chunks per strip row");

  // bf16 operand stages (int8 weights are dequantised into sW), and for
  // int8 the raw weight rows of the next k-steps
  __shared__ __attribute__((aligned(1024))) uint16_t sW0[BN][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW1[BN][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW2[NS > 2 ? BN : 1][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW3[NS > 3 ? BN : 1][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX0[BM][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX1[BM][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX2[NS > 2 ? BM : 1][BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX3[NS > 3 ? BM : 1][BK];
  __shared__ __attribute__((aligned(1024))) uint8_t sQ0[W8 ? BN : 1][BK];
  __shared__ __attribute__((aligned(1024))) uint8_t sQ1[W8 ? BN : 1][BK];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wn = wave / WM, wm = wave % WM;
  const int li = lane & 15, grp = lane >> 4;

  // this workgroup's tiles: XCD xcd owns tiles [T xcd / 8, T (xcd + 1) / 8)
  // (SPLIT: work items (k range, tile), the k range slowest)
  const int TT = n_mt * n_nt;
  const int T = TT * (SPLIT ? nsplit : 1);
  const int xcd = (int)blockIdx.x % 8, gx = (int)gridDim.x / 8;
  const int t_end = (int)((int64_t)T * (xcd + 1) / 8);
  int b = (int)((int64_t)T * xcd / 8) + (int)blockIdx.x / 8;
  if (b >= t_end) return;  // uniform per workgroup

  const int wbytes0 = (int)((a.N - 1) * a.ldw0 * WB + a.K * WB);
  const int wbytes1 = GATEUP ? (int)((a.N - 1) * a.ldw1 * WB + a.K * WB) : wbytes0;
  const int xbytes = (int)((a.M - 1) * a.ldx * 2 + a.K * 2);
  void* const wptr1 = (void*)(GATEUP ? a.w1 : a.w0);
  const int lrow = lane / CPR, lchunk = lane % CPR;

  // per-tile state: origin, k range (SPLIT: k-steps kb .. kb + nloc - 1;
  // else all nkt), DMA lane offsets and (int8) the scales of the rows this
  // lane dequantises
  const int64_t nkt = a.K / BK;
  int64_t m0 = 0, c0 = 0, kb = 0, nloc = nkt;
  int ks = 0;
  uint32_t woff[IW], xoff[IX];
  float qs[W8 ? QCH : 1], qn[W8 ? QCH : 1];
  auto wrow_n = [&](int t) -> int64_t { return GATEUP ? c0 + (t / 32) * 16 + (t % 16) : c0 + t; };
  auto wrow_up = [&](int t) -> bool { return GATEUP && ((t / 16) & 1); };
  auto setup = [&](int bb) {
    if constexpr (SPLIT) {
      ks = bb / TT;
      bb -= ks * TT;
      kb = (int64_t)ks * per;
      nloc = nkt - kb < per ? nkt - kb : per;
    }
    const int gbase = (bb / (kGroupM * n_nt)) * kGroupM;
    const int gm = n_mt - gbase < kGroupM ? n_mt - gbase : kGroupM;
    const int gin = bb - gbase * n_nt;
    const int tm = gbase + gin % gm, tn = gin / gm;
    m0 = (int64_t)tm * BM;
    c0 = (int64_t)tn * (GATEUP ? BN / 2 : BN);
#pragma unroll
    for (int j = 0; j < IW; ++j) {
      const int t = (wave + NW * j) * WRPI + lane / WCPR;
      const int c = lane % WCPR;
      const int64_t ld = wrow_up(t) ? a.ldw1 : a.ldw0;
      // int8 rows land unswizzled (the dequantisation pass reads them
      // linearly); bf16 rows in the fragment-read swizzle
      woff[j] = (uint32_t)(wrow_n(t) * ld * WB) + (uint32_t)((W8 ? c : c ^ swzk<BK>(t)) * 16);
    }
#pragma unroll
    for (int j = 0; j < IX; ++j) {
      const int t = (wave + NW * j) * RPI + lrow;
      xoff[j] = (uint32_t)((m0 + t) * a.ldx * 2) + (uint32_t)((lchunk ^ swzk<BK>(t)) * 16);
    }
    if constexpr (W8) {
#pragma unroll
      for (int c = 0; c < QCH; ++c) {
        const int r = (wave * kWave + lane + NW * kWave * c) / 4;
        const int64_t n = wrow_n(r);
        qs[c] = (r < BN && n < a.N) ? (wrow_up(r) ? a.s1 : a.s0)[n] : 0.f;
        qn[c] = -128.f * qs[c];
      }
    }
  };
  // weight rows of k-step k0 / BK: bf16 into an operand stage, int8 into a
  // staging buffer
  // live false: the same instructions with an empty buffer range (they read
  // nothing and land zeros), so that every step issues the same loads
  auto issue_w = [&](void* dst, int64_t k0, bool live = true) {
#pragma unroll
    for (int j = 0; j < IW; ++j) {
      const int q = wave + NW * j;
      if (NWI % NW != 0 && q >= NWI) break;  // uniform per wave
      const bool up = wrow_up(q * WRPI);
      load_lds16(up ? wptr1 : a.w0, live ? (up ? wbytes1 : wbytes0) : 0,
                 (lds_ptr_t)((char*)dst + q * WRPI * BK * WB), woff[j],
                 (uint32_t)((kb * BK + k0) * WB));
    }
  };
  auto issue_x = [&](uint16_t (*tx)[BK], int64_t k0, bool live = true) {
#pragma unroll
    for (int j = 0; j < IX; ++j)
      load_lds16(a.x, live ? xbytes : 0, (lds_ptr_t)&tx[(wave + NW * j) * RPI][0], xoff[j],
                 (uint32_t)((kb * BK + k0) * 2));
  };
  // int8: chunk c of this lane (16 weights of row r, k-range 16 q .. 16 q +
  // 15 of the step) from staging buffer sq to bf16(q * s) in stage tw, in
  // the bf16 fragment-read swizzle; each weight is dequantised once per
  // workgroup (as the dequantise-then-matmul path rounds it)
  auto dq_read = [&](const uint8_t (*sq)[BK], int c) -> u32x4 {
    const int t = wave * kWave + lane + NW * kWave * c;
    return *reinterpret_cast<const u32x4*>((const char*)sq + t * 16);
  };
  auto dq_write = [&](uint16_t (*tw)[BK], int c, u32x4 v) {
    const int t = wave * kWave + lane + NW * kWave * c;
    const int r = t / 4, q = t % 4, sw = swzk<BK>(r);
    *reinterpret_cast<u32x4*>(&tw[r][((2 * q) ^ sw) * 8]) = dequant8_bf16(v.x, v.y, qs[c], qn[c]);
    *reinterpret_cast<u32x4*>(&tw[r][((2 * q + 1) ^ sw) * 8]) =
        dequant8_bf16(v.z, v.w, qs[c], qn[c]);
  };
  // chunk c exists in every lane of this wave (uniform)
  auto dq_has = [&](int c) -> bool { return (wave + NW * c) * kWave < NQC; };

  f32x4 acc[FN][FM];
  const int ra = wn * TN + li, rb = wm * TM + li;
  const uint32_t offa = (uint32_t)(ra * BK * 2 + ((grp ^ swzk<BK>(ra)) * 16));
  const uint32_t offb = (uint32_t)(rb * BK * 2 + ((grp ^ swzk<BK>(rb)) * 16));
  // One k-half's MFMA operands as read from LDS.
  struct Frag {
    u32x4 a[FN];
    u32x4 b[FM];
  };
  auto rd_a = [&](Frag& f, const uint16_t (*tw)[BK], int kk, int i) {
    const uint32_t oa = offa ^ (uint32_t)(kk * 64);
    f.a[i] = *reinterpret_cast<const u32x4*>((const char*)tw + oa + i * 16 * BK * 2);
  };
  auto rd_b = [&](Frag& f, const uint16_t (*tx)[BK], int kk, int j) {
    const uint32_t ob = offb ^ (uint32_t)(kk * 64);
    f.b[j] = *reinterpret_cast<const u32x4*>((const char*)tx + ob + j * 16 * BK * 2);
  };
  // Wave tiles of up to 24 MFMA blocks (192 x 256) keep the plain loop: all
  // of a k-half's reads, then its MFMAs (measured on MI355X, 4B QKV at M =
  // 2048: 60.1 us against 61.6 pipelined; gate-up 320 x 256 175.7 -> 169.5).
  // int8 always pipelines (its dequantisation pass rides in the MFMA block),
  // and so do the four-wave tiles.
  constexpr bool kPipe = W8 || FN * FM > 24 || NW == 4;
  static_assert(NW == 8 || (NW == 4 && !W8), "eight waves, or four for bf16");
  // The MFMAs of k-half f, with the LDS reads of the next k-half (tw, tx,
  // kk) into g spread between them: weight fragment i right after the last
  // MFMA that reads f's fragment i, x fragment j right after the last MFMA
  // that reads f's fragment j (the last row), so g takes f's registers as
  // they free up. A wave's LDS latency hides under its own MFMAs instead of
  // stalling the k-half's first MFMA, and the waves' reads no longer arrive
  // in one burst. With RD false: the MFMAs alone. With DQ (int8): this
  // lane's dequantisation of the next k-step's weights from staging buffer
  // sq into stage dw, its LDS reads at the start and its arithmetic and
  // writes in the middle of the block.
  auto mma = [&](auto RD, auto DQ, const Frag& f, Frag& g, const uint16_t (*tw)[BK],
                 const uint16_t (*tx)[BK], int kk, const uint8_t (*sq)[BK],
                 uint16_t (*dw)[BK]) {
    constexpr bool rd = decltype(RD)::value;
    constexpr bool dq = decltype(DQ)::value;
    u32x4 qv[QCH];
    if constexpr (NW >= 8) __builtin_amdgcn_s_setprio(1);
    if constexpr (dq) {
#pragma unroll
      for (int c = 0; c < QCH; ++c)
        if (dq_has(c)) qv[c] = dq_read(sq, c);
    }
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        if constexpr (NW == 4)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                       : "+a"(acc[i][j])
                       : "v"(f.a[i]), "v"(f.b[j]));
        else
          acc[i][j] = mfma16(f.a[i], f.b[j], acc[i][j]);
        if constexpr (rd)
          if (i == FN - 1) rd_b(g, tx, kk, j);
      }
      if constexpr (rd) rd_a(g, tw, kk, i);
      if constexpr (dq) {
        if (i == FN / 2) {
#pragma unroll
          for (int c = 0; c < QCH; ++c)
            if (dq_has(c)) dq_write(dw, c, qv[c]);
        }
      }
    }
    if constexpr (rd && !dq) {
#pragma unroll
      for (int i = 0; i < FN - 1; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, FM, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (NW >= 8) __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto stw = [&](int st) -> uint16_t (*)[BK] {
    return st == 0 ? sW0 : (st == 1 ? sW1 : (st == 2 ? sW2 : sW3));
  };
  auto stx = [&](int st) -> uint16_t (*)[BK] {
    return st == 0 ? sX0 : (st == 1 ? sX1 : (st == 2 ? sX2 : sX3));
  };
  auto stq = [&](int st) -> uint8_t (*)[BK] { return st == 0 ? sQ0 : sQ1; };
  // a tile's first loads: k-step 0 into stage 0 (int8: the weights of steps
  // 0 and 1 into the staging buffers)
  auto issue_first = [&]() {
    issue_x(sX0, 0);
    if constexpr (W8) {
      issue_w(sQ0, 0);
      if (nkt > 1) issue_w(sQ1, BK);
    } else {
      issue_w(sW0, 0);
    }
  };

  // Four waves: a wait between the accumulators' accesses on either side of
  // it and the MFMA asm statements. The empty asm statements tie every
  // earlier write (the zeroing) to before the s_nop and every later read
  // (an MFMA's or the epilogue's) to after it; asm volatile statements keep
  // their order, so the 24 wait states also separate the asm MFMAs issued
  // before from any read after.
  auto agpr_fence = [&]() {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) asm volatile("" : "+a"(acc[i][j]));
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) asm volatile("" : "+a"(acc[i][j]));
  };
  const bool y16 = ((a.ldy & 7) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
  Frag F, G;
  setup(b);
  issue_first();
  while (true) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // four waves: the zeroed AGPRs settle before an MFMA reads them
    if constexpr (NW == 4) agpr_fence();
    // this tile's first k-step (and the previous tile's output stores)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    if constexpr (kPipe) {
      if constexpr (W8) {
        // step 0's weights into stage 0, then staging buffer 0 takes step 2
#pragma unroll
        for (int c = 0; c < QCH; ++c)
          if (dq_has(c)) dq_write(sW0, c, dq_read(sQ0, c));
        __syncthreads();
        if (nkt > 2) issue_w(sQ0, 2 * BK);
        if (nkt > 1) issue_x(sX1, BK);
      } else if constexpr (NS > 2) {
        // steps 1 .. NS - 1 into their stages (past the last step: empty
        // ranges, so that every step has issued the same loads)
#pragma unroll
        for (int st = 1; st < NS; ++st) {
          const bool live = st < nloc;
          issue_x(stx(st), live ? st * BK : 0, live);
          issue_w(stw(st), live ? st * BK : 0, live);
        }
      } else {
        if (nkt > 1) {
          issue_x(sX1, BK);
          issue_w(sW1, BK);
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) rd_b(F, sX0, 0, j);
#pragma unroll
      for (int i = 0; i < FN; ++i) rd_a(F, sW0, 0, i);
      // k-step k lives in stage k % 2. Its first half's MFMAs run while its
      // second half is read (int8: and step k + 1's weights are dequantised
      // from staging buffer (k + 1) % 2 into stage (k + 1) % 2; on the last
      // step stale bytes into a stage nothing reads); then one barrier
      // (every wave is done reading stage k % 2 and staging buffer
      // (k + 1) % 2, and the loads of step k + 1 have landed) lets step
      // k + 2's loads into that stage (int8: step k + 3's weights into that
      // staging buffer), and the second half's MFMAs run while the first
      // half of step k + 1 is read (on the last step: stale reads, unused).
      // (The loop shape of gemm_kernel: with a different one the compiler
      // double-buffers the accumulators and spills.)
      if constexpr (NW == 4) {
        // the same steps for an even nkt (the launcher checks), without the
        // odd-count exit. With NS = 3 or 4 stages step k lives in stage
        // k % NS, the loads of step k + NS go out after step k's barrier,
        // and the wait before that barrier leaves the loads of steps k + 2
        // .. k + NS - 1 in flight (LPS per wave and step): loads get NS - 1
        // steps to land instead of one. Every step issues its loads, past
        // the last step with an empty range, so that the count of loads in
        // flight is exact, for that wait and for the compiler (which would
        // otherwise wait for all of them before the next stage's reads).
        constexpr int LPS = IW + IX;  // load instructions per wave and k-step
        static_assert((NS - 2) * LPS < 64, "loads in flight within the vmcnt range");
        for (int64_t kt = 0; kt < nloc; kt += NS) {
#pragma unroll
          for (int u = 0; u < NS; ++u) {
            const int64_t k = kt + u;
            if constexpr (NS > 2)
              if (k >= nloc) break;
            mma(std::true_type{}, std::false_type{}, F, G, stw(u), stx(u), 1, sQ0, sW0);
            if constexpr (BK == 128) {
              // substeps 1 and 2 of the four, each reading the next
              mma(std::true_type{}, std::false_type{}, G, F, stw(u), stx(u), 2, sQ0, sW0);
              mma(std::true_type{}, std::false_type{}, F, G, stw(u), stx(u), 3, sQ0, sW0);
            }
            if constexpr (NS > 2) {
              // this wave's loads of step k + 1 have landed and its reads of
              // stage u are done; then a bare barrier (__syncthreads' fence
              // would wait for every load in flight)
              __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm((NS - 2) * LPS));
              __builtin_amdgcn_s_barrier();
            } else {
              __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
              __syncthreads();
            }
            if constexpr (NS > 2) {
              const bool live = k + NS < nloc;
              issue_x(stx(u), live ? (k + NS) * BK : 0, live);
              issue_w(stw(u), live ? (k + NS) * BK : 0, live);
            } else if (k + NS < nloc) {
              issue_x(stx(u), (k + NS) * BK);
              issue_w(stw(u), (k + NS) * BK);
            }
            mma(std::true_type{}, std::false_type{}, G, F, stw((u + 1) % NS), stx((u + 1) % NS), 0,
                sQ0, sW0);
          }
        }
      } else
      for (int64_t kt = 0; kt < nkt; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t k = kt + u;
          if (k >= nkt) break;
          mma(std::true_type{}, std::integral_constant<bool, W8>{}, F, G, stw(u), stx(u), 1,
              stq(u ^ 1), stw(u ^ 1));
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
          __syncthreads();
          if (k + 2 < nkt) {
            issue_x(stx(u), (k + 2) * BK);
            if constexpr (!W8) issue_w(stw(u), (k + 2) * BK);
          }
          if constexpr (W8)
            if (k + 3 < nkt) issue_w(stq(u ^ 1), (k + 3) * BK);
          mma(std::true_type{}, std::false_type{}, G, F, stw(u ^ 1), stx(u ^ 1), 0, sQ0, sW0);
        }
      }
    } else {
      // k-step k lives in stage k % 2; the loads of step k + 1 are in flight
      // while step k is consumed, a k-half's reads before its MFMAs
      for (int64_t kt = 0; kt < nkt; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t k = kt + u;
          if (k >= nkt) break;
          if (k + 1 < nkt) {
            issue_w(stw((u + 1) % 2), (k + 1) * BK);
            issue_x(stx((u + 1) % 2), (k + 1) * BK);
          }
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int i = 0; i < FN; ++i) rd_a(F, stw(u), kk, i);
#pragma unroll
            for (int j = 0; j < FM; ++j) rd_b(F, stx(u), kk, j);
            mma(std::false_type{}, std::false_type{}, F, G, sW0, sX0, kk, sQ0, sW0);
          }
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
          __syncthreads();
        }
      }
    }
    // four waves: the last MFMAs' results land before the epilogue reads them
    if constexpr (NW == 4) agpr_fence();
    // three stages: the empty-range loads of the last steps have landed in
    // every wave before the epilogue strips take stage 1
    if constexpr (NS > 2) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __syncthreads();
    }
    // Both loops: the k-steps in gemm_kernel's order and the same MFMA
    // sequence on the same bf16 operands, so the outputs are bit-identical
    // to it.
    const int bnext = b + gx;
    const bool more = bnext < t_end;
    const int64_t em0 = m0, ec0 = c0;
    const int eks = ks;
    if (more) {
      setup(bnext);
      issue_first();
    }
    if constexpr (SPLIT) {
      // fp32 partials of k range eks into ws[eks][m][col] (col: output
      // column n; gate-up: g at n, u at N + n), 4 consecutive columns of one
      // x row per lane, for splitk_reduce_kernel
      const int64_t wc = GATEUP ? 2 * a.N : a.N;
      const bool v16 = (a.N & 3) == 0;  // as in gemm_kernel's split form
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int64_t m = em0 + wm * TM + j * 16 + li;
        if (m >= a.M) continue;
        float* prow = ws + ((int64_t)eks * a.M + m) * wc;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          int64_t n, col;
          if constexpr (GATEUP) {
            const int sub = (wn * TN) / 16 + i;  // even: gate rows, odd: up rows
            n = ec0 + (sub / 2) * 16 + 4 * grp;
            col = (sub & 1) ? a.N + n : n;
          } else {
            n = ec0 + wn * TN + i * 16 + 4 * grp;
            col = n;
          }
          if (v16 && n + 3 < a.N) {
            *reinterpret_cast<f32x4*>(prow + col) = acc[i][j];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < a.N) prow[col + r] = acc[i][j][r];
          }
        }
      }
      if (!more) break;
      b = bnext;
      continue;
    }
    // ---- epilogue: per wave, 16 x rows at a time through its strip ----
    uint16_t* strip = &sX1[0][0] + wave * 16 * SROW;
    const int64_t nw0 = ec0 + wn * TNO;  // first output column of this wave
#pragma unroll
    for (int j = 0; j < FM; ++j) {
#pragma unroll
      for (int i = 0; i < FN; i += (GATEUP ? 2 : 1)) {
        uint32_t p0, p1;
        int lc;
        if constexpr (GATEUP) {
          p0 = gate_up_silu_pair(acc[i][j][0], acc[i + 1][j][0], acc[i][j][1], acc[i + 1][j][1]);
          p1 = gate_up_silu_pair(acc[i][j][2], acc[i + 1][j][2], acc[i][j][3], acc[i + 1][j][3]);
          lc = (i / 2) * 16 + 4 * grp;
        } else {
          p0 = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
          p1 = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
          lc = i * 16 + 4 * grp;
        }
        *reinterpret_cast<u32x2*>(strip + li * SROW + lc) = u32x2{p0, p1};
      }
      const int64_t mj = em0 + wm * TM + j * 16;
#pragma unroll
      for (int c = lane; c < 16 * CPRO; c += kWave) {
        const int r = c / CPRO, q = c % CPRO;
        const int64_t m = mj + r, n = nw0 + q * 8;
        const u32x4 v = *reinterpret_cast<const u32x4*>(strip + r * SROW + q * 8);
        if (m < a.M) {
          uint16_t* yp = a.y + m * a.ldy + n;
          if (y16 && n + 7 < a.N) {
            *reinterpret_cast<u32x4*>(yp) = v;
          } else {
            const uint32_t h[8] = {v.x & 0xffffu, v.x >> 16, v.y & 0xffffu, v.y >> 16,
                                   v.z & 0xffffu, v.z >> 16, v.w & 0xffffu, v.w >> 16};
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (n + e < a.N) yp[e] = (uint16_t)h[e];
          }
        }
      }
    }
    if (!more) break;
    b = bnext;
  }
}

// Sums the nsplit partial accumulators of each output in split order 0, 1,
// ... (a fixed order: results do not depend on scheduling) and applies the
// epilogue at the torch rounding points. One thread per 4 columns of a row.
template <bool GATEUP>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* ws, int nsplit,
                                                            StreamArgs a) {
  const int64_t nq = (a.N + 3) / 4;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= a.M * nq) return;
  const int64_t m = t / nq, n = (t - m * nq) * 4;
  const int64_t wc = GATEUP ? 2 * a.N : a.N;
  const int64_t plane = a.M * wc;  // floats per split
  const float* p = ws + m * wc + n;
  uint32_t h[4];
  if ((a.N & 3) == 0 && n + 3 < a.N) {  // 16-byte partials (u at N + n)
    f32x4 g = *reinterpret_cast<const f32x4*>(p);
    f32x4 u = GATEUP ? *reinterpret_cast<const f32x4*>(p + a.N) : f32x4{};
    for (int s = 1; s < nsplit; ++s) {
      g += *reinterpret_cast<const f32x4*>(p + s * plane);
      if constexpr (GATEUP) u += *reinterpret_cast<const f32x4*>(p + s * plane + a.N);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) h[r] = GATEUP ? gate_up_silu_bits(g[r], u[r]) : f32_to_bf16_bits(g[r]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (n + r >= a.N) break;
      float g = p[r], u = GATEUP ? p[r + a.N] : 0.f;
      for (int s = 1; s < nsplit; ++s) {
        g += p[s * plane + r];
        if constexpr (GATEUP) u += p[s * plane + r + a.N];
      }
      h[r] = GATEUP ? gate_up_silu_bits(g, u) : f32_to_bf16_bits(g);
    }
  }
  uint16_t* yrow = a.y + m * a.ldy;
  if (((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0) && n + 3 < a.N) {
    *reinterpret_cast<u32x2*>(yrow + n) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < a.N) yrow[n + r] = (uint16_t)h[r];
  }
}

}  // namespace

template <int BN, int BM, int WN, int WM, bool GATEUP, int NS, bool W8 = false, int BK = kBK>
int launch_gemm_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<BN, BM, WN, WM, GATEUP, NS, false, W8, BK>), dim3((unsigned)(n_nt * n_mt)),
                     dim3(WN * WM * kWave), 0, s, a, n_mt, n_nt, 0, (float*)nullptr);
  return (int)hipGetLastError();
}

// The persistent form of a one-tile-per-CU grid: one workgroup per CU (at
// most one per tile).
constexpr int kTilesGrid = 256;
template <int BN, int BM, int WN, int WM, bool GATEUP, bool W8 = false, int BK = kBK, int NS = 2>
int launch_tiles_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  const int64_t tiles = (int64_t)n_nt * n_mt;
  const int grid = tiles < kTilesGrid ? (int)((tiles + 7) / 8 * 8) : kTilesGrid;
  hipLaunchKernelGGL((gemm_tiles_kernel<BN, BM, WN, WM, GATEUP, W8, BK, NS>), dim3((unsigned)grid),
                     dim3(WN * WM * kWave), 0, s, a, n_mt, n_nt, 1, 0, (float*)nullptr);
  return (int)hipGetLastError();
}

// The staged four-wave tiles with k split across workgroups: `used` ranges
// of `per` 128-wide k-steps (the last may be shorter, none empty), fp32
// partials in ws (used planes of M x N, gate-up M x 2N), then the reduce.
template <int BN, int BM, int WN, int WM, bool GATEUP, int NS>
int launch_tiles_split_cfg(const StreamArgs& a, int used, int per, float* ws, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  const int64_t items = (int64_t)n_nt * n_mt * used;
  const int grid = items < kTilesGrid ? (int)((items + 7) / 8 * 8) : kTilesGrid;
  hipLaunchKernelGGL((gemm_tiles_kernel<BN, BM, WN, WM, GATEUP, false, 2 * kBK, NS, true>),
                     dim3((unsigned)grid), dim3(WN * WM * kWave), 0, s, a, n_mt, n_nt, used, per,
                     ws);
  int e = (int)hipGetLastError();
  if (e) return e;
  const int64_t threads = a.M * ((a.N + 3) / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel<GATEUP>, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, s, ws, used, a);
  return (int)hipGetLastError();
}

// Split-K form: at most `nsplit` k-ranges of whole k-steps per tile (the
// count actually used, every range non-empty, is returned through
// *used_split), partials in ws (gemm_splitk_ws_floats floats), then the
// reduce kernel.
inline int64_t gemm_splitk_ksteps(int64_t K, int nsplit) {
  const int64_t nkt = K / kBK;
  return (nkt + nsplit - 1) / nsplit;
}
inline int gemm_splitk_used(int64_t K, int nsplit) {
  const int64_t per = gemm_splitk_ksteps(K, nsplit);
  return (int)((K / kBK + per - 1) / per);
}
template <bool GATEUP>
int64_t gemm_splitk_ws_floats(const StreamArgs& a, int nsplit) {
  return (int64_t)gemm_splitk_used(a.K, nsplit) * a.M * (GATEUP ? 2 * a.N : a.N);
}

template <int BN, int BM, int WN, int WM, bool GATEUP, int NS, bool W8 = false>
int launch_gemm_splitk_cfg(const StreamArgs& a, int nsplit, float* ws, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  const int per = (int)gemm_splitk_ksteps(a.K, nsplit);
  const int used = gemm_splitk_used(a.K, nsplit);
  hipLaunchKernelGGL((gemm_kernel<BN, BM, WN, WM, GATEUP, NS, true, W8>),
                     dim3((unsigned)(n_nt * n_mt * used)), dim3(WN * WM * kWave), 0, s, a, n_mt,
                     n_nt, per, ws);
  int e = (int)hipGetLastError();
  if (e) return e;
  const int64_t threads = a.M * ((a.N + 3) / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel<GATEUP>, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, s, ws, used, a);
  return (int)hipGetLastError();
}

// Whether gemm_kernel can run this call: whole 64-wide k-steps, 16-byte
// aligned rows, every operand's byte size below 2^31 (buffer-resource sizes
// and 32-bit lane offsets); int8 also needs its row scales.
bool gemm_supported(const StreamArgs& a, bool aligned, bool w8) {
  constexpr int64_t kLim = (int64_t)1 << 31;
  const int64_t wb = w8 ? 1 : 2;
  if (!aligned || a.K % kBK != 0) return false;
  if (w8 && (!a.s0 || (a.w1 && !a.s1))) return false;
  if ((a.N - 1) * a.ldw0 * wb + a.K * wb >= kLim) return false;
  if (a.w1 && (a.N - 1) * a.ldw1 * wb + a.K * wb >= kLim) return false;
  if ((a.M - 1) * a.ldx * 2 + a.K * 2 >= kLim) return false;
  return true;
}

// Tiles the dispatcher uses: {weight rows, x rows, workgroups per CU (LDS)}.
// kK*: bf16 tiles with 128-wide k-steps (two LDS stages: 64 KB, 112 KB and
// 128 KB).
enum GemmTile { kT64x32, kT128x64, kT64x128, kT128x128, kT256x256, kT192x256,
                kK64x64, kK96x128, kK128x128, kT320x256, kT192x128, kT160x128,
                kT128x160, kT96x64, kT64x128w, kT96x128, kT160x256 };
struct TileInfo {
  int bn, bm, per_cu;
};
constexpr TileInfo kTiles[] = {{64, 32, 4},   {128, 64, 3},  {64, 128, 2},
                               {128, 128, 2}, {256, 256, 1}, {192, 256, 1},
                               {64, 64, 2},   {96, 128, 1},  {128, 128, 1},
                               {320, 256, 1}, {192, 128, 1}, {160, 128, 1},
                               {128, 160, 1}, {96, 64, 1},   {64, 128, 1},  {96, 128, 1},
                               {160, 256, 1}};
constexpr int kCUs = 256;

int64_t tile_count(int tile, int64_t M, int64_t N, bool gateup) {
  const int64_t cols = gateup ? kTiles[tile].bn / 2 : kTiles[tile].bn;
  return ((N + cols - 1) / cols) * ((M + kTiles[tile].bm - 1) / kTiles[tile].bm);
}

// The tile whose grid fill decides whether to split k (gemm_split_plan): the
// table the split rules were measured against. QKV-sized outputs (<= 8192
// weight rows): 64 x 128 to 768 rows, 128 x 128 to 1536, then 256 x 256;
// outputs of at most 4096 columns: 64 x 128 to 768 rows, then 128 x 128 until
// a 256 x 256 grid fills the chip; gate-up-sized: 128 x 128 to 384 rows,
// 256 x 256 to 768, 128 x 128 to 1536, 256 x 256.
int split_ref_tile(int64_t M, int64_t wrows) {
  if (wrows <= 4096) {
    if (M <= 768) return kT64x128;
    if (tile_count(kT256x256, M, wrows, false) >= kCUs) return kT256x256;
    return kT128x128;
  }
  if (wrows <= 8192) return M <= 768 ? kT64x128 : (M <= 1536 ? kT128x128 : kT256x256);
  if (M <= 384) return kT128x128;
  if (M <= 768) return kT256x256;
  return M <= 1536 ? kT128x128 : kT256x256;
}

// Cost model of an unsplit prefill grid, fitted to warm-clock measurements on
// MI355X (Qwen3-0.6B/4B/8B QKV, gate-up, o and down, M = 256..8192; the
// dispatch it yields is within 0.1% of the best of the candidates below on
// average over those 120 shapes, 4% at worst). A grid's time is set by its busiest CU,
// which runs k = ceil(tiles / 256) tiles; what a tile costs hardly depends on
// how many other CUs are busy. 256 x 256, 192 x 256 and 320 x 256 tiles (one per CU)
// cost k times (per-k-step + per-tile) units; tiles that fit two per CU run
// in pairs: k / 2 pairs and k % 2 single tiles, each with its own per-k-step
// cost (a pair costs ~1.1-1.3 times a single), plus a per-tile cost. Units
// are relative (a common per-shape factor is divided out). 192 x 256 tiles
// (3/4 of the work of 256 x 256) take ~0.92 of the time: they pay where their
// count fills whole rounds (QKV 6144 x 2048: 256 tiles, 69.4 -> 63.0 us).
struct TileCost {
  double single, pair, tile;
};
constexpr TileCost kCost64x128{0.576, 0.598, 0.0};
constexpr TileCost kCost128x128{0.616, 0.765, 1.085};
constexpr TileCost kCost256x256{1.086, 0.0, 7.200};
constexpr TileCost kCost192x256{0.948, 0.0, 4.843};
constexpr TileCost kCost320x256{1.331, 0.0, 7.814};
constexpr double kCostLaunch = 1.925;  // the tail plan's second launch

double grid_cost(int tile, int64_t M, int64_t N, int64_t nkt, bool gateup) {
  const int64_t n = tile_count(tile, M, N, gateup);
  if (n == 0) return 0.0;
  const int64_t k = (n + kCUs - 1) / kCUs;
  const TileCost& c = tile == kT64x128    ? kCost64x128
                      : tile == kT128x128 ? kCost128x128
                      : tile == kT192x256 ? kCost192x256
                      : tile == kT320x256 ? kCost320x256
                                          : kCost256x256;
  if (kTiles[tile].per_cu == 1) return (double)k * ((double)nkt * c.single + c.tile);
  const int64_t pairs = k / 2, singles = k % 2;
  return (double)nkt * ((double)pairs * c.pair + (double)singles * c.single) +
         (double)(pairs + singles) * c.tile;
}

// The unsplit plan: for bf16 weights a single round of k-step-128 tiles where
// one fits (k128_tile); otherwise the cheapest of 64 x 128, 128 x 128,
// 256 x 256, 192 x 256, 320 x 256 (bf16, at most two rounds: 11% more bytes
// per k-step than 256 x 256 for 25% more work, which pays where it saves a
// round: 4B gate-up M = 2048 195.6 -> 184.4 us, M = 1024 116.7 -> 99.5 us;
// 4B QKV M = 3072 104.8 -> 83.8 us), and
// "256 x 256 for whole rounds + a 128 x 128 tail" (nmain > 0: the first
// nmain output columns as whole 256 x 256 rounds, the rest as 128 x 128 tiles
// in a second launch). The tail form turns the last partial round of 256 x
// 256 tiles into 128 x 128 tiles that spread over all CUs (measured 4B
// gate-up M = 2048: 223.6 -> 203.4 us; 4B QKV M = 4096: 142.7 -> 125.9 us).
// Both tiles contract every output over the same k-steps in the same order,
// so each plan's result is bit-identical to the others'. One correction to
// the model: where 128 x 128 tiles would run one per CU and 64 x 128 tiles at
// most two, 64 x 128 is faster on every shape measured (the pair of smaller
// tiles hides latency better than one tile of the same work).
//
// Grids of tiles with 128-wide k-steps: twice the bytes per load round and
// half the per-step waits and barriers of the 64-wide tiles. Measured on
// MI355X (Qwen3-0.6B/4B/8B QKV, o, down and gate-up, M = 160..2048; results
// bit-identical to the 64-wide plans), they win wherever the whole grid runs
// in one round (at most one tile per CU, two for 64 x 64): 4B QKV M = 512
// 37.6 -> 30.2 us (96 x 128), 0.6B QKV M = 512 13.7 -> 9.9 us (64 x 64), 8B
// QKV M = 512 59.5 -> 44.3 us, 4B o M = 1536 48.8 -> 37.6 us; with more
// rounds they lose to the plans above (up to 50% slower). Gate-up only with
// weights under 2^24 elements (0.6B M = 160..640: 13.3 -> 9.5 us; 4B/8B
// gate-up tiles of 128 x 128 run 11-22% slower with 128-wide steps than
// with 64-wide ones). 96 x 128 (QKV-like outputs only: its gate/up pairing
// would need one wave column) where 96 divides N, in place of 128 x 128
// (4-10% faster there; with a partial last tile 5-22% slower). Between 64 x
// 64 and the larger tile, the cost fixed + k-steps x per-step decides,
// where a tile alone on its CU costs more per step the more CUs are busy
// (relative units, fitted to the same measurements).
struct K128Cost {
  double fixed, one, busy, pair;
};
constexpr K128Cost kCostK64x64{0.0, 0.664, 0.199, 0.912};
constexpr K128Cost kCostK96x128{2.065, 1.082, 0.203, 0.0};
constexpr K128Cost kCostK128x128{0.175, 1.134, 0.294, 0.0};

// The k-step-128 tile of a single-round grid for this call, -1 if none.
int k128_tile(int64_t M, int64_t N, int64_t K, bool gateup) {
  if (K % (2 * kBK) != 0) return -1;
  if (gateup && 2 * N * K >= ((int64_t)1 << 24)) return -1;
  const int64_t nkt = K / (2 * kBK);
  const bool use96 = !gateup && N % 96 == 0 && tile_count(kK96x128, M, N, false) <= kCUs;
  int best = -1;
  double cbest = 0.0;
  for (int t : {kK64x64, use96 ? kK96x128 : kK128x128}) {
    const int64_t n = tile_count(t, M, N, gateup);
    if (n > kCUs * kTiles[t].per_cu) continue;
    const K128Cost& c = t == kK64x64 ? kCostK64x64 : t == kK96x128 ? kCostK96x128 : kCostK128x128;
    const double busy = (double)(n < kCUs ? n : kCUs) / kCUs;
    const double step = n > kCUs ? c.pair : c.one + c.busy * busy;
    const double cost = c.fixed + (double)nkt * step;
    if (best < 0 || cost < cbest) best = t, cbest = cost;
  }
  return best;
}

// Whether a single round of k-step-128 tiles (k128_tile) has a tile for
// every CU and at least one tile per 20 columns of K: enough tiles against
// the k loop that splitting k (across or inside workgroups) no longer pays.
bool k128_wide(int64_t M, int64_t N, int64_t K, bool gateup) {
  const int t = k128_tile(M, N, K, gateup);
  if (t < 0) return false;
  const int64_t n = tile_count(t, M, N, gateup);
  return n >= kCUs && n * 20 >= K;
}

// A single round of small four-wave tiles with three LDS stages (bf16,
// 128-wide k-steps, at least 48 rows): 96 x 64 where at most 256 of them
// cover the output, else 64 x 128 with 192-256 tiles (above 512 rows 240-256
// and at least 24 k-steps), either with enough tiles against the k loop: 3
// per k-step for gate-up and for up to 24 k-steps, 6 per k-step above; at
// least 64, 128 with up to 12 k-steps, and up to 128 rows at least 192
// (fewer leave the call to k split across or inside workgroups, to the
// weight-streaming kernels, or to two 64 x 64 tiles per CU); -1 if neither. The third stage gives each k-step's
// loads two steps to land instead of one, and the small tiles keep three
// stages within the LDS (120 and 144 KB). Measured on MI355X over Qwen3
// 0.6B/4B/8B QKV, gate-up, o, down and their tensor-parallel (TP) shards at
// M = 136..2048 (µs, previous plan -> this; hipBLASLt on the same
// contraction in brackets): 8B TP=2 QKV 4096 -> 3072 at M = 512 35.4 -> 25.5
// (24.7); 4B TP=2 QKV 2560 -> 3072 at 512 25.0 -> 18.7 (18.7); 8B TP=8 QKV
// 4096 -> 768 at 2048 34.1 -> 24.4 (24.4); 8B QKV 4096 -> 6144 at 256 31.7 ->
// 26.6 (40.1); 8B TP=8 gate-up 4096 -> 2 x 1536 at 512 35.1 -> 25.7 (24.8);
// 4B TP=4 QKV 2560 -> 1536 at 1024 23.6 -> 17.8; 0.6B o 2048 -> 1024 at 768
// 17.6 -> 12.7; 0.6B down 3072 -> 1024 at 2048 (64 x 128) 27.5 -> 21.7; 8B
// o 4096 -> 4096 at 512 (64 x 128) 32.7 -> 27.9; at 48-128 rows 4B gate-up
// 2560 -> 2 x 9728 at 64 39.4 -> 28.8, 8B gate-up 4096 -> 2 x 12288 at 64
// 50.5 -> 43.9, 8B TP=2 gate-up 4096 -> 2 x 6144 at 128 56.7 -> 34.9 (with
// 64-128 tiles there, or fewer than 48 rows, up to 2x slower). Over 44
// random shapes (M = 48-4096, K = 1024-8192) against the plans before these
// tiles: 8 faster by 10-35%, and the ones slower by 7-13% (few tiles against
// 8-12 k-steps: linear 1024 -> 776 at 768 rows 8.6 -> 9.4 us, QKV 1536 ->
// 1024 at 1536 rows 11.7 -> 13.3 us; 64 x 128 with 204 tiles above 512 rows)
// set the minimum counts above. With 32 k-steps and 96-129
// tiles the split plans were 4-12% faster (8B TP=2 QKV at 192 rows 22.4 vs
// 25.1, 8B o at 192 23.6 vs 25.4), with 76 k-steps 13% (4B down at 768). The
// same tiles with two stages: 96 x 64 on 8B TP=2 QKV at 512 32.2, 64 x 128
// 34.0.
int small_round_tile(int64_t M, int64_t N, int64_t K, bool gateup) {
  if (K % (2 * kBK) != 0 || M < 48) return -1;
  const int64_t nk = K / (2 * kBK);
  int64_t need = (gateup || nk <= 24 ? 3 : 6) * nk;
  if (need < 64) need = 64;
  if (nk <= 12 && need < 128) need = 128;
  if (M <= 128 && need < 192) need = 192;
  const int64_t n1 = tile_count(kT96x64, M, N, gateup);
  if (n1 <= kCUs) return n1 >= need ? kT96x64 : -1;
  const int64_t n2 = tile_count(kT64x128w, M, N, gateup);
  if (n2 > kCUs || n2 < need) return -1;
  return (M <= 512 ? n2 >= 192 : n2 >= 240 && nk >= 24) ? kT64x128w : -1;
}

GemmPlan gemm_plan_unsplit(int64_t M, int64_t N, int64_t K, bool gateup, bool bf16) {
  if (bf16) {
    const int ts = small_round_tile(M, N, K, gateup);
    if (ts >= 0) return GemmPlan{ts, 0};
    // gate-up: one round of 96 x 128 four-wave tiles (96 weight rows, 48
    // outputs; an even number of 128-wide k-steps) on at least 192 CUs:
    // 8B TP=4 gate-up 4096 -> 2 x 3072 at M = 512 57.6 -> 39.5 us (hipBLASLt
    // 35.8), 4B TP=4 2560 -> 2 x 2432 at 512 31.2 -> 27.6 (26.8)
    if (gateup && K % (2 * kBK) == 0 && (K / (2 * kBK)) % 2 == 0) {
      const int64_t n = tile_count(kT96x128, M, N, true);
      if (n >= 192 && n <= kCUs) return GemmPlan{kT96x128, 0};
    }
    const int t = k128_tile(M, N, K, gateup);
    if (t >= 0) return GemmPlan{t, 0};
  }
  const int64_t nkt = K / kBK;
  GemmPlan best{kT64x128, 0};
  double cbest = grid_cost(kT64x128, M, N, nkt, gateup);
  for (int t : {kT128x128, kT256x256, kT192x256, kT320x256}) {
    // 320 x 256 (bf16 only); QKV-like outputs for at most two rounds: beyond,
    // the model underrates it (4B QKV M = 8192 226 against 206 us on 256 x
    // 256). Gate-up at any count (same-box A/B against 256 x 256 and its
    // tail, 4B gate-up: M = 3072 260 -> 248 us, 4096 345 -> 332, 6144 509 ->
    // 483, 8192 668 -> 651).
    if (t == kT320x256 && (!bf16 || (!gateup && tile_count(t, M, N, gateup) > 2 * kCUs))) continue;
    const double c = grid_cost(t, M, N, nkt, gateup);
    if (c < cbest) best = GemmPlan{t, 0}, cbest = c;
  }
  const int64_t cols = gateup ? 128 : 256;  // output columns of a 256 x 256 tile
  const int64_t n_nt = (N + cols - 1) / cols, n_mt = (M + 255) / 256;
  const int64_t rounds = n_nt * n_mt / kCUs;
  const int64_t main_nt = rounds >= 1 ? rounds * kCUs / n_mt : 0;
  if (main_nt > 0 && main_nt < n_nt) {
    const int64_t nmain = main_nt * cols;
    const double c = grid_cost(kT256x256, M, nmain, nkt, gateup) +
                     grid_cost(kT128x128, M, N - nmain, nkt, gateup) + kCostLaunch;
    if (c < cbest) best = GemmPlan{kT256x256, nmain}, cbest = c;
  }
  const auto per_cu = [&](int t) { return (tile_count(t, M, N, gateup) + kCUs - 1) / kCUs; };
  if (best.tile == kT128x128 && per_cu(kT128x128) == 1 && per_cu(kT64x128) <= 2)
    best = GemmPlan{kT64x128, 0};
  // A single round of four-wave tiles (accumulators in AGPRs) on at least
  // 240 CUs: 192 x 128, else 128 x 160 or 160 x 128, with an even number of
  // 128-wide k-steps (192 x 128 also with an even number of at least 32
  // 64-wide ones). Faster than the plan above wherever measured on MI355X
  // (µs, previous plan -> 64-wide steps -> 128-wide steps): 8B gate-up M =
  // 256 80.8 -> 73.4 -> 64.8; gate-up 4096 -> 2 x 6144 at M = 512 73.7 ->
  // 67.2 -> 56.5, 4096 -> 2 x 1536 at M = 2048 66.1 -> 62.9 -> 52.6; QKV 2560
  // -> 3072 at M = 2048 47.7 -> 44.3 -> 38.1, 4096 -> 3072 at M = 2048 66.8
  // -> 63.1 -> 52.7; 128 x 160 for gate-up 2560 -> 2 x 1216 at M = 2048 42.2
  // -> 32.1; 160 x 128 for gate-up 2560 -> 2 x 4864 at M = 512 52.8 -> 36.3.
  // At 204-208 tiles 192 x 128 was 6% faster once and 9% slower once
  // (64-wide steps), at 128 or fewer up to 46% slower.
  if (bf16) {
    const bool k128 = K % (2 * kBK) == 0 && (K / (2 * kBK)) % 2 == 0;
    const auto one_round = [&](int t) {
      const int64_t n = tile_count(t, M, N, gateup);
      return n >= 240 && n <= kCUs;
    };
    if (one_round(kT192x128) && (k128 || (nkt % 2 == 0 && nkt >= 32))) return GemmPlan{kT192x128, 0};
    // gate-up: one round of 160 x 256 four-wave tiles (80 outputs, 64-wide
    // steps) in place of the fewer 192 x 256 ones: 4B gate-up 2560 -> 2 x
    // 9728 at M = 512 62.8-63.1 -> 58.3-58.5 us (244 tiles against 204; with
    // three LDS stages 60.6-61.2)
    if (gateup && nkt % 2 == 0 && nkt >= 32 && one_round(kT160x256)) return GemmPlan{kT160x256, 0};
    if (k128 && one_round(kT128x160)) return GemmPlan{kT128x160, 0};
    if (k128 && one_round(kT160x128)) return GemmPlan{kT160x128, 0};
  }
  // QKV: two nearly whole rounds of 192 x 256 tiles (four waves) over 256 x
  // 256 rounds plus a 128 x 128 tail (same box, µs, bit-identical
  // plans aside: 4B M = 4096 120.7 -> 117.3, 8B M = 4096 178.4 -> 175.6).
  // int8 too, on eight-wave dequantise-once tiles, in place of a 256 x 256
  // round and a 128 x 128 tail of gemm_kernel, which dequantises every
  // fragment in each wave that reads it (same box, bit-identical: 8B M =
  // 4096 202.2 -> 181.6 us, 4B M = 4096 133.1 -> 120.6)
  if (!gateup && nkt % 2 == 0 && nkt >= 32 && best.tile == kT256x256) {
    const int64_t n = tile_count(kT192x256, M, N, false);
    if (n > kCUs && n <= 2 * kCUs && n >= 2 * kCUs - kCUs / 16) return GemmPlan{kT192x256, 0};
  }
  return best;
}

template <bool GATEUP, bool W8>
int launch_gemm(const StreamArgs& a, hipStream_t s) {
  if constexpr (W8 && GATEUP) {
    // int8 gate-up up to 256 rows on one round of 192 x 128 dequantise-once
    // tiles (8 waves of 96 x 32) where it gives 192-256 of them, instead of
    // 128 x 128 gemm_kernel tiles that dequantise each fragment in every wave
    // that reads it. Same box, µs, bit-identical: 8B M = 192 77.0 -> 62.8,
    // M = 256 80.7 -> 67.2; 4B M = 192 49.7 -> 43.3, M = 256 50.4 -> 44.3
    // (at 384 rows, more than a round, 8B 92 -> 117).
    const int64_t n = tile_count(kT192x128, a.M, a.N, true);
    if (a.M <= 256 && n >= 192 && n <= kCUs) return launch_tiles_cfg<192, 128, 2, 4, true, true>(a, s);
  }
  const GemmPlan p = gemm_plan_unsplit(a.M, a.N, a.K, GATEUP, !W8);
  if constexpr (!W8) {
    switch (p.tile) {
      case kT320x256:
        if constexpr (GATEUP) return launch_tiles_cfg<320, 256, 2, 4, true>(a, s);
        return launch_tiles_cfg<320, 256, 4, 2, false>(a, s);
      case kK64x64: return launch_gemm_cfg<64, 64, 2, 2, GATEUP, 2, false, 128>(a, s);
      // The one-per-CU tiles with 128-wide k-steps run as the pipelined
      // four-wave tile loop where their step count is even (measured on
      // MI355X against gemm_kernel, bit-identical, µs: 4B QKV M = 512 30.9
      // -> 27.5, M = 384 30.8 -> 27.2; 8B QKV M = 512 44.1 -> 39.8; 0.6B
      // QKV M = 1024 16.4 -> 14.7, gate-up M = 512 15.7 -> 14.8; other
      // shapes even). 64 x 64 tiles run two per CU in gemm_kernel, which
      // one persistent workgroup per CU does not match (0.6B QKV M = 512
      // 11.9 -> 16.8).
      case kK128x128:
        if ((a.K / (2 * kBK)) % 2 == 0)
          return launch_tiles_cfg<128, 128, 2, 2, GATEUP, false, 2 * kBK>(a, s);
        return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2, false, 128>(a, s);
      case kK96x128:
        if constexpr (!GATEUP) {
          if ((a.K / (2 * kBK)) % 2 == 0)
            return launch_tiles_cfg<96, 128, 2, 2, false, false, 2 * kBK>(a, s);
          return launch_gemm_cfg<96, 128, 2, 2, false, 2, false, 128>(a, s);
        }
        return (int)hipErrorInvalidValue;  // never planned for gate-up
      // Four waves, 128-wide k-steps. 96 x 64 and 64 x 128 with three LDS
      // stages (any step count); 96 x 128 with two (an even step count).
      // Gate-up tiles whose weight rows cannot be split into whole gate/up
      // pairs per wave column take one wave column.
      case kT96x64:
        if (a.K % (2 * kBK) != 0) return (int)hipErrorInvalidValue;  // never planned so
        if constexpr (GATEUP) return launch_tiles_cfg<96, 64, 1, 4, true, false, 2 * kBK, 3>(a, s);
        return launch_tiles_cfg<96, 64, 2, 2, false, false, 2 * kBK, 3>(a, s);
      case kT64x128w:
        if (a.K % (2 * kBK) != 0) return (int)hipErrorInvalidValue;
        if constexpr (GATEUP) return launch_tiles_cfg<64, 128, 1, 4, true, false, 2 * kBK, 3>(a, s);
        return launch_tiles_cfg<64, 128, 2, 2, false, false, 2 * kBK, 3>(a, s);
      case kT96x128:
        if (a.K % (2 * kBK) != 0 || (a.K / (2 * kBK)) % 2 != 0) return (int)hipErrorInvalidValue;
        if constexpr (GATEUP) return launch_tiles_cfg<96, 128, 1, 4, true, false, 2 * kBK>(a, s);
        return launch_tiles_cfg<96, 128, 2, 2, false, false, 2 * kBK>(a, s);
      default: break;
    }
  }
  switch (p.tile) {
    case kT64x128: return launch_gemm_cfg<64, 128, 2, 2, GATEUP, 3, W8>(a, s);
    case kT128x128: return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2, W8>(a, s);
    case kT192x128:
    case kT160x128:
    case kT128x160:
      // four waves, 128-wide k-steps where their count is even (planned
      // only so, except 192 x 128, which may take 64-wide ones)
      if constexpr (!W8) {
        const bool k128 = a.K % (2 * kBK) == 0 && (a.K / (2 * kBK)) % 2 == 0;
        if (p.tile == kT192x128) {
          if (k128) return launch_tiles_cfg<192, 128, 2, 2, GATEUP, false, 2 * kBK>(a, s);
          return launch_tiles_cfg<192, 128, 2, 2, GATEUP, false>(a, s);
        }
        if (!k128) return (int)hipErrorInvalidValue;  // never planned so
        if (p.tile == kT128x160) return launch_tiles_cfg<128, 160, 2, 2, GATEUP, false, 2 * kBK>(a, s);
        // 160 x 128: gate-up needs whole gate/up pairs per wave (one wave column)
        if constexpr (GATEUP) return launch_tiles_cfg<160, 128, 1, 4, true, false, 2 * kBK>(a, s);
        return launch_tiles_cfg<160, 128, 2, 2, false, false, 2 * kBK>(a, s);
      }
      return (int)hipErrorInvalidValue;  // never planned for int8
    case kT160x256:
      // bf16 gate-up, an even number of at least 32 k-steps (planned only
      // so): four waves in one column of 160 weight rows
      if constexpr (GATEUP && !W8)
        if ((a.K / kBK) % 2 == 0 && a.K / kBK >= 32)
          return launch_tiles_cfg<160, 256, 1, 4, true, false>(a, s);
      return (int)hipErrorInvalidValue;
    case kT192x256:
      // bf16 with an even number of at least 32 k-steps: four waves (QKV
      // too, same box, bit-identical: 4B M = 2048 61.1 -> 60.4 us, M = 4096
      // 120.7 -> 117.3; 8B M = 2048 91.2 -> 88.4, M = 4096 178.4 -> 175.6)
      // (int8 keeps eight waves: four measured slower, 8B QKV M = 4096
      // 181.6 -> 198.5 us, 4B M = 2048 61.3 -> 69.0)
      if constexpr (!W8)
        if ((a.K / kBK) % 2 == 0 && a.K / kBK >= 32)
          return launch_tiles_cfg<192, 256, 2, 2, GATEUP, false>(a, s);
      return launch_tiles_cfg<192, 256, 2, 4, GATEUP, W8>(a, s);
    default: break;
  }
  if (p.nmain == 0) return launch_tiles_cfg<256, 256, 4, 2, GATEUP, W8>(a, s);
  StreamArgs m = a;
  m.N = p.nmain;
  int e = launch_tiles_cfg<256, 256, 4, 2, GATEUP, W8>(m, s);
  if (e) return e;
  // the tail: output columns nmain .. N-1 (weight rows and, for int8, their
  // scales from nmain on)
  StreamArgs t = a;
  t.N = a.N - p.nmain;
  if constexpr (W8) {
    t.w0 = static_cast<const int8_t*>(a.w0) + p.nmain * a.ldw0;
    t.s0 = a.s0 + p.nmain;
    if (GATEUP) {
      t.w1 = static_cast<const int8_t*>(a.w1) + p.nmain * a.ldw1;
      t.s1 = a.s1 + p.nmain;
    }
  } else {
    t.w0 = static_cast<const uint16_t*>(a.w0) + p.nmain * a.ldw0;
    if (GATEUP) t.w1 = static_cast<const uint16_t*>(a.w1) + p.nmain * a.ldw1;
  }
  t.y = a.y + p.nmain;
  // int8 gate-up tails on the dequantise-once tile kernel (the 128 x 128
  // gemm_kernel dequantises each weight fragment in every wave that reads
  // it): one round of 192 x 128 tiles where 192-256 of them cover it, else
  // 256 x 128 tiles
  if constexpr (W8 && GATEUP) {
    const int64_t n = tile_count(kT192x128, t.M, t.N, true);
    if (n >= 192 && n <= kCUs) return launch_tiles_cfg<192, 128, 2, 4, true, true>(t, s);
    return launch_tiles_cfg<256, 128, 4, 2, true, true>(t, s);
  }
  return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2, W8>(t, s);
}

// When to split k across workgroups, measured on MI355X over Qwen3-0.6B/4B/8B
// QKV, gate-up, o and down shapes (M = 16..4096). Splitting pays when the
// unsplit grid leaves CUs idle and each tile has a long k loop; it costs the
// fp32 partials' round trip and a second launch. Rules:
//   - at least 32 k-steps (K >= 2048) and 32 x rows (more than 32 rows for
//     outputs wider than 4096 weight rows);
//   - below 128 rows (the weight-streaming regime) only against large
//     weights: >= 64 k-steps and >= 2^24 weight elements (down, 8B o);
//   - from 128 rows while the unsplit grid fills at most half of the
//     chip's workgroup slots, or three quarters with >= 128 k-steps; gate-up
//     (two partial planes) only with >= 128 k-steps.
// Tile by rows: 64 x 32 to 32 rows, 128 x 64 to 128, 128 x 128 (64 x 128
// for outputs of at most 1024 columns) to 1024 rows or narrow outputs,
// 256 x 256 above; splits = slots / tiles rounded, in 2..16 with at least
// 8 k-steps each. No split where a single round of k-step-128 tiles can run
// instead (k128_tile) with K <= 4096 and either at most 3 splits, or at most
// 5 with weights under 2^24 elements and a wide round (k128_wide)
// (measured on two MI355X boxes: 4B QKV M = 256 28.6 -> 18.5-24.4 us, 4B o
// M = 640 35.2 -> 26.6-32.7 us, 8B o M = 1024 49.4-50.0 -> 47.8-48.4 us;
// with 6-8 splits, 4-5 over 8B QKV and o weights, or rounds of few tiles
// against K, such as 0.6B o and down below 256 rows, the split is up to 36%
// faster; 4B o at 448-512 rows, 6 splits, ran 26 us split on both boxes and
// 26 or 31-34 us as a single round).
GemmSplit gemm_split_plan(int64_t M, int64_t N, int64_t K, bool gateup) {
  const GemmSplit none{-1, 1};
  if (M < 32 || K % kBK != 0) return none;
  const int64_t nkt = K / kBK, wrows = gateup ? 2 * N : N;
  if (nkt < 32) return none;
  if (M <= 32 && wrows > 4096) return none;
  if (M < 128) {
    if (nkt < 64 || wrows * K < ((int64_t)1 << 24)) return none;
  } else {
    if (gateup && nkt < 128) return none;
    const int t0 = split_ref_tile(M, wrows);
    const double fill = (double)tile_count(t0, M, N, gateup) / (kCUs * kTiles[t0].per_cu);
    if (!(fill <= 0.5 || (fill < 0.75 && nkt >= 128))) return none;
  }
  int tile;
  if (M <= 32) tile = kT64x32;
  else if (M <= 128) tile = kT128x64;
  else if (M <= 1024 || wrows <= 2048) tile = wrows <= 1024 ? kT64x128 : kT128x128;
  else tile = kT256x256;
  const double want = (double)(kCUs * kTiles[tile].per_cu) / tile_count(tile, M, N, gateup);
  int64_t ns = (int64_t)(want + 0.5);
  ns = ns < 16 ? ns : 16;
  ns = ns < nkt / 8 ? ns : nkt / 8;
  if (ns < 2) return none;
  const int used = gemm_splitk_used(K, (int)ns);
  if (K <= 4096 && k128_tile(M, N, K, gateup) >= 0 &&
      (used <= 3 || (used <= 5 && wrows * K < ((int64_t)1 << 24) && k128_wide(M, N, K, gateup))))
    return none;
  return GemmSplit{tile, used};
}

int64_t gemm_split_ws_floats(const GemmSplit& p, int64_t M, int64_t N, int64_t K, bool gateup) {
  if (p.tile < 0) return 0;
  if (p.tile == kT96x64) return (int64_t)p.nsplit * M * (gateup ? 2 * N : N);
  return (int64_t)gemm_splitk_used(K, p.nsplit) * M * (gateup ? 2 * N : N);
}

GemmSplit gemm_split_plan_bf16(int64_t M, int64_t N, int64_t K, bool gateup) {
  if (small_round_tile(M, N, K, gateup) >= 0) return GemmSplit{-1, 1};
  if (!gateup && splitk24_shape(M, N, K)) return GemmSplit{-1, 1};  // 24-row split-K tiles
  const GemmSplit p = gemm_split_plan(M, N, K, gateup);
  if (p.tile < 0 || K % (2 * kBK) != 0) return p;
  // The staged 96 x 64 four-wave tiles (three LDS stages), k split into
  // ranges of 4 to 32 128-wide steps, as many as one round of at most 256
  // work items allows; ranges above 8 steps only with at least 192 items.
  // Measured on MI355X against the split above (gemm_kernel, 64-wide steps;
  // µs): 8B TP=4 QKV 4096 -> 1536 at M = 256 21.1 -> 17.5, 8B TP=8 QKV
  // 4096 -> 768 at 512 19.8 -> 16.1, 4B o 4096 -> 2560 at 136 22.1 -> 17.7,
  // 4B down 9728 -> 2560 at 128 30.7 -> 25.6, 0.6B down 3072 -> 1024 at 384
  // 17.5 -> 15.0, 4B down at 64 23.9 -> 20.1, 8B QKV 4096 -> 6144 at 64 20.7
  // -> 18.8; with 172-176 items over 12-16 steps (8B o at 96-128 rows, 0.6B
  // down at 512) 4-8% slower, with two rounds of items up to 1.8x.
  const int64_t nk = K / (2 * kBK), n = tile_count(kT96x64, M, N, gateup);
  int64_t ns = kCUs / n;
  ns = ns < 16 ? ns : 16;
  ns = ns < nk / 4 ? ns : nk / 4;
  if (ns < 2) return p;
  const int64_t per = (nk + ns - 1) / ns;
  if (per > 32 || (per > 8 && n * ns < 192)) return p;
  return GemmSplit{kT96x64, (int)((nk + per - 1) / per)};
}

bool use_gemm_split(const StreamArgs& a, bool aligned, bool gateup, GemmSplit* p) {
  if (!a.ws || !gemm_supported(a, aligned, false)) return false;
  *p = gemm_split_plan_bf16(a.M, a.N, a.K, gateup);
  return p->tile >= 0 && gemm_split_ws_floats(*p, a.M, a.N, a.K, gateup) <= a.ws_floats;
}

template <bool GATEUP, bool W8>
int launch_gemm_split(const StreamArgs& a, const GemmSplit& p, hipStream_t s) {
  if constexpr (!W8) {
    if (p.tile == kT96x64) {
      // nsplit ranges of per 128-wide k-steps (gemm_split_plan_bf16)
      const int64_t nk = a.K / (2 * kBK);
      const int per = (int)((nk + p.nsplit - 1) / p.nsplit);
      if (a.K % (2 * kBK) != 0 || (nk + per - 1) / per != p.nsplit) return (int)hipErrorInvalidValue;
      if constexpr (GATEUP) return launch_tiles_split_cfg<96, 64, 1, 4, true, 3>(a, p.nsplit, per, a.ws, s);
      return launch_tiles_split_cfg<96, 64, 2, 2, false, 3>(a, p.nsplit, per, a.ws, s);
    }
  }
  switch (p.tile) {
    case kT64x32: return launch_gemm_splitk_cfg<64, 32, 2, 2, GATEUP, 3, W8>(a, p.nsplit, a.ws, s);
    case kT128x64: return launch_gemm_splitk_cfg<128, 64, 4, 2, GATEUP, 2, W8>(a, p.nsplit, a.ws, s);
    case kT64x128: return launch_gemm_splitk_cfg<64, 128, 2, 2, GATEUP, 3, W8>(a, p.nsplit, a.ws, s);
    case kT128x128: return launch_gemm_splitk_cfg<128, 128, 4, 2, GATEUP, 2, W8>(a, p.nsplit, a.ws, s);
    default: return launch_gemm_splitk_cfg<256, 256, 4, 2, GATEUP, 2, W8>(a, p.nsplit, a.ws, s);
  }
}

template int launch_gemm_split<false, false>(const StreamArgs&, const GemmSplit&, hipStream_t);
template int launch_gemm_split<true, false>(const StreamArgs&, const GemmSplit&, hipStream_t);
template int launch_gemm_split<false, true>(const StreamArgs&, const GemmSplit&, hipStream_t);
template int launch_gemm_split<true, true>(const StreamArgs&, const GemmSplit&, hipStream_t);
template int launch_gemm<false, false>(const StreamArgs&, hipStream_t);
template int launch_gemm<true, false>(const StreamArgs&, hipStream_t);
template int launch_gemm<false, true>(const StreamArgs&, hipStream_t);
template int launch_gemm<true, true>(const StreamArgs&, hipStream_t);

}  // namespace fp
