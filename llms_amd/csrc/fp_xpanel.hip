// fp_xpanel.hip — int8 weight-only projections at spec-verify row counts (2 to
// 16 rows) with K up to 2560 (Qwen3-4B): x staged once per workgroup in LDS,
// every weight load of a wave issued up front into registers.
//
// A workgroup owns RB blocks of 16 weight rows (gate-up: the 16 Wg rows and
// the 16 Wu rows of one block of 16 outputs) over the whole of K, and all
// the x rows (up to 16; rows past M read as zero):
//   - x, the B operand of v_mfma_f32_16x16x32_bf16, lands in LDS by
//     buffer_load_dwordx4 ... lds as one plane per 64-wide k-step (XR = 16
//     or, at up to 8 rows, 8 rows x 128 B, chunk c of row r at
//     c ^ ((r >> 1) & 7), so the fragment reads of 16 rows hit distinct
//     banks; with 8 staged rows, lanes of B columns 8-15 take zeros). K <=
//     2560 needs at most 80 KB (40 KB with 8 rows), so two (four) workgroups
//     share a CU.
//   - Wave w contracts k-steps w, w + NW, w + 2 NW, ...; before it computes
//     anything it issues the int8 loads of all of them (16 B per lane and
//     row block: row li, k 16 grp .. 16 grp + 15 of the step), so the whole
//     weight stream of the workgroup is in flight at once instead of a few
//     steps of a ring.
//   - Each 16-byte chunk becomes two A fragments, bf16(q * s) exactly as the
//     dequantise-then-matmul path rounds it (dequant8_bf16). The chunk holds
//     k 16 grp + 8 kk .. + 7 for fragment kk, and the x fragment is read at
//     the same k, so each MFMA contracts the same 32 products as a fragment
//     in k order would, in another grouping.
//   - The waves' partial tiles are summed through LDS in wave order 0, 1,
//     ... (fixed: results do not depend on scheduling); wave 0 applies the
//     epilogue (bf16, or silu(g) * u at torch's rounding points) and stores.
// Measured on MI355X against the split-K tiles (fp_splitk.hip), the two
// libraries alternated on one box over 36 cycled weight sets (more than the
// 256 MB Infinity Cache holds), µs: Qwen3-4B int8 QKV (2560 -> 6144) M = 4,
// 8, 16 8.6, 8.9, 9.3 -> 8.2, 8.3, 8.8 (M = 2, against the row kernel: even);
// gate-up (2560 -> 2 x 9728) M = 4 16.3 -> 15.1. Staging 8 x rows instead of
// 16 at M <= 8 (bit-identical; gate-up over 16 sets of 100 MB): 15.5, 15.6,
// 15.9 -> 15.2, 15.3, 15.6 at M = 3, 4, 8. With K = 4096 (Qwen3-8B: 128 KB
// of x, one workgroup per CU), with bf16 weights, and at one row (the row
// kernel) the same kernel measured slower.
// Requirements (checked by the dispatcher): xpanel8_shape(), 16-byte-aligned
// rows, operand byte sizes below 2^31, row scales present.
#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

constexpr int kBK = 64;   // k per step
constexpr int kNK = 40;   // k-steps the x planes hold (K <= 2560)
constexpr int kNSW = 10;  // k-steps per wave (four waves)

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// buffer_load_dwordx4 ... lds: 16 bytes per lane from base + voff + soff into
// LDS at dst + 16 * lane; bytes at or past `nbytes` read as zero.
__device__ __forceinline__ void load_lds16(const void* base, int nbytes, lds_ptr_t dst,
                                           uint32_t voff, uint32_t soff) {
  constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, kRsrcFlags), dst, 16,
      voff, soff, 0, 0);
}

// buffer_load_dwordx4 into registers, with the same range rule.
__device__ __forceinline__ u32x4 load_buf16(const void* base, int nbytes, uint32_t voff,
                                            uint32_t soff) {
  constexpr int kRsrcFlags = 0x00020000;
  return __builtin_amdgcn_raw_buffer_load_b128(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, kRsrcFlags), voff,
      soff, 0);
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= v only.
constexpr int vmcnt_imm(int v) { return (v & 15) | (7 << 4) | (15 << 8) | ((v >> 4) << 14); }

// An offset past every buffer's range (rows past N, steps past K: zeros).
constexpr uint32_t kPastEnd = 0x80000000u;

template <int NW, int RB, int NSW, int XR, bool GATEUP>
__global__ __launch_bounds__(NW * kWave) void xpanel_kernel(StreamArgs a) {
  constexpr int PL = XR * kBK * 2;  // bytes per x plane (XR rows, one k-step)
  static_assert(XR == 8 || XR == 16, "8 or 16 staged x rows");
  static_assert(!GATEUP || RB % 2 == 0, "gate-up blocks come in gate/up pairs");
  static_assert(NW * NSW >= kNK, "every k-step has a wave");
  static_assert(NW * RB * 1024 <= kNK * PL, "the partial tiles fit the x planes");
  static_assert(NSW * RB < 64, "loads in flight within the vmcnt range");
  __shared__ __attribute__((aligned(1024))) char xs[kNK * PL];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int li = lane & 15, grp = lane >> 4;
  const int nkt = (int)(a.K / kBK);

  // x rows 0 .. XR - 1 (past M: zero) into planes 0 .. nkt - 1, this wave's
  // share of the IPP * nkt load instructions (8 rows each)
  constexpr int IPP = XR / 8;
  const int xbytes = (int)((a.M - 1) * a.ldx * 2 + a.K * 2);
  for (int q = wave; q < IPP * nkt; q += NW) {
    const int j = q / IPP, r = (q % IPP) * 8 + lane / 8;
    const uint32_t voff = (uint32_t)(r * a.ldx * 2) + (uint32_t)(((lane & 7) ^ swz(r)) * 16);
    load_lds16(a.x, xbytes, (lds_ptr_t)(xs + j * PL + (q % IPP) * 1024), voff,
               (uint32_t)(j * kBK * 2));
  }

  // this lane's weight row of each block, its scale and byte offset
  const int wbytes0 = (int)((a.N - 1) * a.ldw0 + a.K);
  const int wbytes1 = GATEUP ? (int)((a.N - 1) * a.ldw1 + a.K) : wbytes0;
  void* const wptr1 = (void*)(GATEUP ? a.w1 : a.w0);
  const int rb0 = (int)blockIdx.x * RB;
  uint32_t voff[RB];
  float sc[RB], nsc[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const bool up = GATEUP && (i & 1);
    const int64_t n = GATEUP ? (int64_t)(rb0 / 2 + i / 2) * 16 + li : (int64_t)(rb0 + i) * 16 + li;
    const int64_t ld = up ? a.ldw1 : a.ldw0;
    voff[i] = n < a.N ? (uint32_t)(n * ld + 16 * grp) : kPastEnd;
    sc[i] = n < a.N ? (up ? a.s1 : a.s0)[n] : 0.f;
    nsc[i] = -128.f * sc[i];
  }
  // every weight load of this wave's k-steps (past the last step: nothing)
  u32x4 wq[NSW][RB];
#pragma unroll
  for (int t = 0; t < NSW; ++t) {
    const int j = wave + NW * t;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const bool up = GATEUP && (i & 1);
      wq[t][i] = load_buf16(up ? wptr1 : a.w0, up ? wbytes1 : wbytes0,
                            j < nkt ? voff[i] : kPastEnd, (uint32_t)(j * kBK));
    }
  }
  // this wave's x loads (issued before its weight loads) have landed; then
  // every wave's
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(NSW * RB));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // B column li reads staged row li (8 staged rows: columns 8-15 are zero)
  const int xr = li & (XR - 1);
  const int bo = swz(xr);
  const bool xlive = li < XR;
#pragma unroll
  for (int t = 0; t < NSW; ++t) {
    const int j = wave + NW * t;
    if (j >= nkt) break;  // uniform per wave
    const char* pl = xs + j * PL + xr * 128;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 b = *reinterpret_cast<const u32x4*>(pl + (((2 * grp + kk) ^ bo) * 16));
      if constexpr (XR < 16) b = xlive ? b : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const u32x4 av = kk == 0 ? dequant8_bf16(wq[t][i].x, wq[t][i].y, sc[i], nsc[i])
                                 : dequant8_bf16(wq[t][i].z, wq[t][i].w, sc[i], nsc[i]);
        acc[i] = mfma16(av, b, acc[i]);
      }
    }
  }

  // fixed-order cross-wave sum through LDS (the x planes are free once every
  // wave is past its last step)
  __syncthreads();
  float* red = reinterpret_cast<float*>(xs);
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
      *reinterpret_cast<f32x4*>(red + ((wave - 1) * RB + i) * 256 + lane * 4) = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 0; w < NW - 1; ++w)
#pragma unroll
    for (int i = 0; i < RB; ++i)
      acc[i] += *reinterpret_cast<const f32x4*>(red + (w * RB + i) * 256 + lane * 4);

  // epilogue: lane holds outputs 4 grp .. 4 grp + 3 of each block, x row li
  const int64_t m = li;
  if (m >= a.M) return;
  uint16_t* yrow = a.y + m * a.ldy;
  const bool y8 = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
#pragma unroll
  for (int i = 0; i < RB; i += (GATEUP ? 2 : 1)) {
    const int64_t nb = GATEUP ? (int64_t)(rb0 / 2 + i / 2) * 16 + 4 * grp
                              : (int64_t)(rb0 + i) * 16 + 4 * grp;
    uint32_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      h[r] = GATEUP ? gate_up_silu_bits(acc[i][r], acc[i + 1][r]) : f32_to_bf16_bits(acc[i][r]);
    if (y8 && nb + 3 < a.N) {
      *reinterpret_cast<u32x2*>(yrow + nb) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) yrow[nb + r] = (uint16_t)h[r];
    }
  }
}

}  // namespace

// Four waves of ten k-steps each; QKV (and plain outputs) one block of 16
// rows per workgroup, gate-up one gate/up pair (measured against 8 waves of
// five steps and against two QKV blocks per workgroup: even or slower); 8
// staged x rows up to 8 rows, else 16.
template <int XR, bool GATEUP>
int launch_xpanel_cfg(const StreamArgs& a, hipStream_t s) {
  constexpr int RB = GATEUP ? 2 : 1;
  const int64_t rblocks = GATEUP ? 2 * ((a.N + 15) / 16) : (a.N + 15) / 16;
  hipLaunchKernelGGL((xpanel_kernel<4, RB, kNSW, XR, GATEUP>),
                     dim3((unsigned)((rblocks + RB - 1) / RB)), dim3(4 * kWave), 0, s, a);
  return (int)hipGetLastError();
}
template <bool GATEUP>
int launch_xpanel8(const StreamArgs& a, hipStream_t s) {
  if (a.K % kBK != 0 || a.K / kBK > kNK || a.M < 1 || a.M > 16) return (int)hipErrorInvalidValue;
  return a.M <= 8 ? launch_xpanel_cfg<8, GATEUP>(a, s) : launch_xpanel_cfg<16, GATEUP>(a, s);
}

template int launch_xpanel8<false>(const StreamArgs&, hipStream_t);
template int launch_xpanel8<true>(const StreamArgs&, hipStream_t);

}  // namespace fp
