// fp_launch.h — argument blocks and launcher declarations shared between the
// kernel translation units and the C-ABI dispatch (fp_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fp {

// One fused projection call. Weights are [N, K] row-major; for gate-up w0/w1
// are Wg/Wu (s0/s1 their int8 row scales), for QKV only w0/s0 are used.
// Strides are in elements of the respective buffer.
struct StreamArgs {
  const uint16_t* x;
  int64_t ldx;
  const void* w0;
  int64_t ldw0;
  const void* w1;
  int64_t ldw1;
  const float* s0;
  const float* s1;
  uint16_t* y;
  int64_t ldy;
  int64_t M, N, K;
  // Optional caller workspace for the cross-workgroup split-K contraction
  // (16-byte aligned; NULL / too small: the unsplit kernels run).
  float* ws;
  int64_t ws_floats;
  // Optional RMSNorm prologue of x (fp_norm.h): weight [K] bf16 and eps.
  const uint16_t* gamma;
  float eps;
};

// Weight-streaming kernels (M <= 64). Return the launch's hipError_t.
template <bool GATEUP, bool W8>
int launch_stream(const StreamArgs& a, bool aligned, hipStream_t s);

// Row-streaming kernels for 1 <= M <= kRowsMaxM (fp_rows.hip), bf16 and
// int8, used by launch_stream when rows_supported() holds. x is staged in
// LDS (M rounded up to 1, 2 or 4 rows, K to whole chunks; one more row for
// a fused norm weight): at most kRowsMaxLds bytes.
constexpr int64_t kRowsMaxM = 4;
constexpr int64_t kRowsMaxLds = 65536;
template <bool W8>
bool rows_supported(const StreamArgs& a, bool aligned);
// With a.gamma set, the rows kernel normalises x while staging it (one
// launch for the RMSNorm prologue and the projection).
template <bool GATEUP, bool W8>
int launch_rows(const StreamArgs& a, hipStream_t s);
// Whether M x K fits the rows kernel's x staging, with the norm weight's row
// when norm is set (shape only; alignment and the M limit of rows_supported
// apply on top).
bool rows_fit(int64_t M, int64_t K, bool w8, bool norm);

// RMSNorm prologue on its own (fp_norm.h): xn [M, K] (row stride K) from x.
int launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* gamma, float eps,
                   uint16_t* xn, int64_t M, int64_t K, bool vec, hipStream_t s);

// LDS-tiled MFMA kernels (M > 64). Return the launch's hipError_t.
template <bool GATEUP, bool W8>
int launch_tiled(const StreamArgs& a, bool aligned, hipStream_t s);

// Split-K MFMA tiles for the middle regime (fp_splitk.hip). bf16: used by
// launch_stream from kSplitkMinM rows (kSplitkMinMSmallN for calls with at
// most kSplitkSmallN weight rows; wider gate-up from 4 rows with K > 3072,
// else 6) and by launch_tiled for small-N calls up to
// kSplitkMaxM rows with K >= kSplitkMinKTiled, when splitk_supported() holds.
constexpr int64_t kSplitkMinM = 8;
constexpr int64_t kSplitkMinMSmallN = 3;
constexpr int64_t kSplitkSmallN = 8192;
constexpr int64_t kSplitkMaxM = 256;
constexpr int64_t kSplitkMinKTiled = 2048;
constexpr int64_t kSplitkMaxM8 = 128;
bool splitk_supported(const StreamArgs& a, bool aligned, bool w8);
// Whether an int8 call of this shape (M rows, N outputs) runs the split-K
// tiles (dequantising in registers) rather than the row, streaming or
// dequantise-first paths. Measured on MI355X over Qwen3-4B/8B QKV, gate-up,
// o and down: from 2 rows for gate-up and 3 for other outputs (5 for outputs
// of at most 4096 columns with K <= 8192, where the row kernel holds up to
// 4), up to 128 rows; above 64 rows only with K <= 8192 (the long-K down
// projections keep the dequantise-first path with k split across
// workgroups).
inline bool splitk8_shape(int64_t M, int64_t N, int64_t K, bool gateup) {
  const int64_t min_m = gateup ? 2 : ((N <= 4096 && K <= 8192) ? 5 : 3);
  if (M < min_m || M > kSplitkMaxM8 || K % 64 != 0) return false;
  return M <= 64 || K <= 8192;
}
// int8 shapes that run the unsplit MFMA tiles even where a workspace would
// allow k split across workgroups (the split of fp_api.hip's split8_plan is
// not taken for them): gate-up from 129 to 1024 rows, and one weight stream
// of more than 4096 rows with K <= 2560 from 129 to 512 rows or where its
// tiles are one round of 192 x 256 on at least 3/4 of the CUs (Qwen3-4B QKV).
// Measured on MI355X when the alternative was dequantising into a bf16
// workspace: 8B gate-up at 256 rows 121.7 -> 75.9 us, 4B QKV at 256 33.7 ->
// 28.4 us, 4B QKV at 2048 65.2 -> 60.8 us.
inline bool gemm8_shape(int64_t M, int64_t N, int64_t K, bool gateup) {
  if (M <= kSplitkMaxM8 || K % 64 != 0) return false;
  if (gateup) return M <= 1024;
  if (N <= 4096 || K > 2560) return false;
  const int64_t tiles192 = ((N + 191) / 192) * ((M + 255) / 256);
  return M <= 512 || (tiles192 >= 192 && tiles192 <= 256);
}
template <bool GATEUP, bool W8>
int launch_splitk(const StreamArgs& a, hipStream_t s);
// bf16 QKV-sized calls that run 24-row split-K tiles (at most 256 of them):
// 4096 < N <= 6144 outputs, K from 2048 to 4096, up to 64 rows. k split
// across workgroups (gemm_split_plan_bf16) is not planned for them: on
// Qwen3-8B QKV at 48 and 64 rows it measured 20.4-21.9 µs against 17.3-18.2.
inline bool splitk24_shape(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && M <= 64 && N > 4096 && N <= 6144 && K >= 2048 && K <= 4096;
}

// int8 calls at spec-verify row counts that run fp_xpanel.hip (x staged once
// per workgroup, every weight load of a wave in flight at once): 2 to 16
// rows, K from 2048 to 2560 in whole 64-wide steps, at least 4096 outputs
// (measured on Qwen3-4B QKV and gate-up; with K = 4096 and with bf16 weights
// the split-K tiles stay faster). Needs splitk_supported() as well.
inline bool xpanel8_shape(int64_t M, int64_t N, int64_t K, bool gateup) {
  (void)gateup;
  return M >= 2 && M <= 16 && K % 64 == 0 && K >= 2048 && K <= 2560 && N >= 4096;
}
template <bool GATEUP>
int launch_xpanel8(const StreamArgs& a, hipStream_t s);

// Direct-to-LDS MFMA contraction (fp_gemm.hip; int8 weights dequantised in
// registers), used by launch_tiled when gemm_supported() holds.
bool gemm_supported(const StreamArgs& a, bool aligned, bool w8);
template <bool GATEUP, bool W8>
int launch_gemm(const StreamArgs& a, hipStream_t s);
// The unsplit grid launch_gemm runs: tile (a GemmTile of fp_gemm.hip) and,
// when nmain > 0, whole 256 x 256 rounds over the first nmain output columns
// followed by 128 x 128 tiles over the rest. bf16: whether the tiles with
// 128-wide k-steps (bf16 weights only) are candidates.
struct GemmPlan {
  int tile;
  int64_t nmain;
};
GemmPlan gemm_plan_unsplit(int64_t M, int64_t N, int64_t K, bool gateup, bool bf16);
// Whether the bf16 plan is a single round of tiles with 128-wide k-steps with
// a tile for every CU and one per 20 columns of K (then it beats the split-K
// tiles).
bool k128_wide(int64_t M, int64_t N, int64_t K, bool gateup);
// The tile of a single round of small three-stage tiles for this bf16 call
// (a GemmTile of fp_gemm.hip), -1 if none.
int small_round_tile(int64_t M, int64_t N, int64_t K, bool gateup);
// k split across workgroups — for calls whose tile grid leaves the chip
// partly idle while each tile has a long k loop — with fp32 partials in the
// caller's workspace and a fixed-order reduce (fp_gemm.hip). tile < 0: no
// split for this shape.
struct GemmSplit {
  int tile;
  int nsplit;
};
GemmSplit gemm_split_plan(int64_t M, int64_t N, int64_t K, bool gateup);
// The split of a bf16 call: none where a round of small three-stage tiles
// (small_round_tile) runs instead; with 128-wide k-steps mostly the staged
// 96 x 64 four-wave tiles (tile kT96x64 of fp_gemm.hip, nsplit ranges of
// 128-wide k-steps). int8 calls that split on their int8 weights keep
// gemm_split_plan.
GemmSplit gemm_split_plan_bf16(int64_t M, int64_t N, int64_t K, bool gateup);
int64_t gemm_split_ws_floats(const GemmSplit& p, int64_t M, int64_t N, int64_t K, bool gateup);
// Whether the bf16 call a runs split (plan + workspace large enough).
bool use_gemm_split(const StreamArgs& a, bool aligned, bool gateup, GemmSplit* p);
// W8: int8 weights with row scales, dequantised in registers (the partials
// equal those of the bf16 split over the dequantised weights).
template <bool GATEUP, bool W8>
int launch_gemm_split(const StreamArgs& a, const GemmSplit& p, hipStream_t s);

// Device-side per-row int8 quantisation.
int launch_quantize_w8(const uint16_t* w, int64_t ldw, int8_t* q, int64_t ldq,
                       float* scale, int64_t N, int64_t K, hipStream_t s);

constexpr int64_t kStreamMaxM = 64;

// Argument checks of fp_rmsnorm_qkv_bf16 other than its workspace (the
// fp_status of the first problem, FP_OK if none); nothing touches a device.
int rmsnorm_qkv_args(const void* x, int64_t ldx, const void* gamma, float eps, const void* w,
                     int64_t ldw, const void* y, int64_t ldy, int64_t M, int64_t n_q, int64_t n_k,
                     int64_t K);

}  // namespace fp
