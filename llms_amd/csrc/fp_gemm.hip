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
//     range of tiles, ordered M-fastest: the ~32 tiles an XCD runs at once
//     share their weight panels and the activation panel in its L2.
// Requirements (checked by the dispatcher): bf16, K % 64 == 0, 16-byte-aligned
// rows (the general case runs tiled_kernel).
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kBK = 64;          // k per LDS stage
constexpr int kCPR = kBK / 8;    // 16-byte chunks per tile row
constexpr int kRPI = 1024 / (kBK * 2);  // tile rows per load instruction

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & (kCPR - 1); }

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

template <int BN, int BM, int WN, int WM, bool GATEUP, int NS>
__global__ __launch_bounds__(WN * WM * kWave) void gemm_kernel(StreamArgs a, int n_mt, int n_nt) {
  constexpr int NW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;   // per-wave tile
  constexpr int FN = TN / 16, FM = TM / 16;   // MFMA sub-tiles per wave
  constexpr int IW = BN / kRPI / NW;          // weight load instructions per wave per stage
  constexpr int IX = BM / kRPI / NW;          // x load instructions per wave per stage
  static_assert(BN % (kRPI * NW) == 0 && BM % (kRPI * NW) == 0, "tile/waves");
  static_assert(!GATEUP || TN % 32 == 0, "gate-up needs whole gate/up pairs per wave");
  static_assert(NS == 2 || NS == 3, "LDS stages");

  // One LDS object per stage and operand: distinct objects carry distinct
  // alias scopes, so the compiler can see that fragment reads of one stage do
  // not depend on the asynchronous global->LDS writes into another stage
  // (with a single [NS][..] array it waits for all loads before every read).
  __shared__ __attribute__((aligned(1024))) uint16_t sW0[BN][kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW1[BN][kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW2[NS > 2 ? BN : 1][kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX0[BM][kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX1[BM][kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sX2[NS > 2 ? BM : 1][kBK];

  const int lane = threadIdx.x & (kWave - 1);
  // wave index as a scalar: load instructions, LDS bases and buffer
  // resources chosen by it stay uniform (no waterfall loops)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wn = wave / WM, wm = wave % WM;
  const int li = lane & 15, grp = lane >> 4;

  // XCD-aware tile order (see file comment), then M-fastest within an XCD.
  const int T = n_mt * n_nt;
  int b = blockIdx.x;
  if (T % 8 == 0) b = (b % 8) * (T / 8) + b / 8;
  const int tm = b % n_mt, tn = b / n_mt;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t c0 = (int64_t)tn * (GATEUP ? BN / 2 : BN);  // first output column

  // Load instruction q (q = wave + NW*j) fills tile rows 8q..8q+7 with
  // buffer_load_dwordx4 ... lds: the matrix base lives in a buffer resource
  // (SGPRs), the k-step in soffset, and each lane carries one 32-bit byte
  // offset (row * stride + chunk). The resource size is the matrix size, so
  // rows past the end read as zeros. The dispatcher guarantees matrix byte
  // sizes below 2^32.
  const int lrow = lane / kCPR;                 // row within an instruction's 8
  const int lchunk = lane % kCPR;               // LDS chunk position it fills
  uint32_t woff[IW];
#pragma unroll
  for (int j = 0; j < IW; ++j) {
    const int q = wave + NW * j;
    const int t = q * kRPI + lrow;
    const int64_t n = GATEUP ? c0 + (t / 32) * 16 + (t % 16) : c0 + t;
    const int64_t ld = (GATEUP && ((t / 16) & 1)) ? a.ldw1 : a.ldw0;
    woff[j] = (uint32_t)(n * ld * 2) + (uint32_t)((lchunk ^ swz(t)) * 16);
  }
  uint32_t xoff[IX];
#pragma unroll
  for (int j = 0; j < IX; ++j) {
    const int t = (wave + NW * j) * kRPI + lrow;
    xoff[j] = (uint32_t)((m0 + t) * a.ldx * 2) + (uint32_t)((lchunk ^ swz(t)) * 16);
  }
  // byte sizes of the buffer resources (rows past them read as zeros)
  const int wbytes0 = (int)((a.N - 1) * a.ldw0 * 2 + a.K * 2);
  const int wbytes1 = GATEUP ? (int)((a.N - 1) * a.ldw1 * 2 + a.K * 2) : wbytes0;
  const int xbytes = (int)((a.M - 1) * a.ldx * 2 + a.K * 2);
  void* const wptr1 = (void*)(GATEUP ? a.w1 : a.w0);

  auto issue = [&](uint16_t (*tw)[kBK], uint16_t (*tx)[kBK], int64_t k0) {
    const uint32_t kb = (uint32_t)(k0 * 2);
#pragma unroll
    for (int j = 0; j < IW; ++j) {
      const int q = wave + NW * j;
      // gate-up: 16-row groups alternate Wg, Wu; uniform per instruction
      const bool up = GATEUP && ((q / 2) & 1);
      load_lds16(up ? wptr1 : a.w0, up ? wbytes1 : wbytes0, (lds_ptr_t)&tw[q * kRPI][0], woff[j],
                 kb);
    }
#pragma unroll
    for (int j = 0; j < IX; ++j)
      load_lds16(a.x, xbytes, (lds_ptr_t)&tx[(wave + NW * j) * kRPI][0], xoff[j], kb);
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment addresses: sub-tile i of a wave reads tile row base + 16 i + li,
  // and swz() of that row does not depend on i (16 i only touches row bits
  // above the swizzle), so every fragment address is one per-lane byte offset
  // plus the compile-time constants 16 i * 128 and the stage base. k-substep
  // kk = 1 flips chunk bit 2 (chunk (4 + grp) ^ s = (grp ^ s) ^ 4).
  const int ra = wn * TN + li, rb = wm * TM + li;
  const uint32_t offa = (uint32_t)(ra * kBK * 2 + ((grp ^ swz(ra)) * 16));
  const uint32_t offb = (uint32_t)(rb * kBK * 2 + ((grp ^ swz(rb)) * 16));
  auto compute = [&](const uint16_t (*tw)[kBK], const uint16_t (*tx)[kBK]) {
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      const uint32_t oa = offa ^ (uint32_t)(kk * 64), ob = offb ^ (uint32_t)(kk * 64);
      u32x4 fa[FN], fb[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i)
        fa[i] = *reinterpret_cast<const u32x4*>((const char*)tw + oa + i * 16 * kBK * 2);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        fb[j] = *reinterpret_cast<const u32x4*>((const char*)tx + ob + j * 16 * kBK * 2);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
      // keep each k-substep's fragments in one register set (the co-resident
      // wave on the SIMD hides the LDS latency)
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto stw = [&](int s) -> uint16_t (*)[kBK] { return s == 0 ? sW0 : (s == 1 ? sW1 : sW2); };
  auto stx = [&](int s) -> uint16_t (*)[kBK] { return s == 0 ? sX0 : (s == 1 ? sX1 : sX2); };

  // Ring of NS stages: k-step k lives in stage k % NS, and while step k is
  // consumed steps k+1 .. k+NS-1 are in flight. After a step, wait until this
  // wave's loads of step k+1 have landed (the NS-2 later steps may stay in
  // flight), then for every wave's.
  constexpr int kPerStep = IW + IX;  // load instructions per wave per step
  const int64_t nkt = a.K / kBK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) issue(stw(s), stx(s), s * kBK);
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
      if (steady) issue(stw((u + NS - 1) % NS), stx((u + NS - 1) % NS), (k + NS - 1) * kBK);
      compute(stw(u), stx(u));
      if (steady)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * kPerStep));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __syncthreads();
    }
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
      uint32_t h[4];
      if constexpr (GATEUP) {
        const int sub = (wn * TN) / 16 + i;  // even: gate group of pair sub/2
        nb = c0 + (sub / 2) * 16 + 4 * grp;
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = gate_up_silu_bits(acc[i][j][r], acc[i + 1][j][r]);
      } else {
        nb = c0 + wn * TN + i * 16 + 4 * grp;
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

}  // namespace

template <int BN, int BM, int WN, int WM, bool GATEUP, int NS>
int launch_gemm_cfg(const StreamArgs& a, hipStream_t s) {
  const int64_t cols = GATEUP ? BN / 2 : BN;
  const int n_nt = (int)((a.N + cols - 1) / cols);
  const int n_mt = (int)((a.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<BN, BM, WN, WM, GATEUP, NS>), dim3((unsigned)(n_nt * n_mt)),
                     dim3(WN * WM * kWave), 0, s, a, n_mt, n_nt);
  return (int)hipGetLastError();
}

#ifndef FP_GEMM_NO_DISPATCH
// Whether gemm_kernel can run this call: bf16 fast path, whole 64-wide
// k-steps, and every operand's byte size below 2^31 (buffer-resource sizes
// and 32-bit lane offsets).
bool gemm_supported(const StreamArgs& a, bool aligned) {
  constexpr int64_t kLim = (int64_t)1 << 31;
  if (!aligned || a.K % kBK != 0) return false;
  if ((a.N - 1) * a.ldw0 * 2 + a.K * 2 >= kLim) return false;
  if (a.w1 && (a.N - 1) * a.ldw1 * 2 + a.K * 2 >= kLim) return false;
  if ((a.M - 1) * a.ldx * 2 + a.K * 2 >= kLim) return false;
  return true;
}

// Tile table for the bf16 prefill path, measured on MI355X with Qwen3-4B and
// -8B shapes. What decides is how many rounds of workgroups a call needs on
// 256 CUs: 256 x 256 tiles (1 workgroup per CU) run best once they fill the
// chip, smaller tiles (2 per CU) win where they save a round. QKV-sized
// outputs (<= 8192 weight rows): 64 x 128 tiles with three stages to 768 rows,
// 128 x 128 to 1536, then 256 x 256. Outputs of at most 4096 columns (the
// down and o projections) keep 128 x 128 to 4096 rows: a 256 x 256 grid
// there is under one round (2048 x 2560 -> 80 tiles). Gate-up-sized: 128 x
// 128 to 384 rows, 256 x 256 to 768 (152-192 tiles, one round), 128 x 128 to
// 1536, 256 x 256.
template <bool GATEUP>
int launch_gemm(const StreamArgs& a, hipStream_t s) {
  const int64_t wrows = GATEUP ? 2 * a.N : a.N;
  if (wrows <= 4096) {
    if (a.M <= 768) return launch_gemm_cfg<64, 128, 2, 2, GATEUP, 3>(a, s);
    if (a.M <= 4096) return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2>(a, s);
    return launch_gemm_cfg<256, 256, 4, 2, GATEUP, 2>(a, s);
  }
  if (wrows <= 8192) {
    if (a.M <= 768) return launch_gemm_cfg<64, 128, 2, 2, GATEUP, 3>(a, s);
    if (a.M <= 1536) return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2>(a, s);
    return launch_gemm_cfg<256, 256, 4, 2, GATEUP, 2>(a, s);
  }
  if (a.M <= 384) return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2>(a, s);
  if (a.M <= 768) return launch_gemm_cfg<256, 256, 4, 2, GATEUP, 2>(a, s);
  if (a.M <= 1536) return launch_gemm_cfg<128, 128, 4, 2, GATEUP, 2>(a, s);
  return launch_gemm_cfg<256, 256, 4, 2, GATEUP, 2>(a, s);
}

template int launch_gemm<false>(const StreamArgs&, hipStream_t);
template int launch_gemm<true>(const StreamArgs&, hipStream_t);
#endif

}  // namespace fp
