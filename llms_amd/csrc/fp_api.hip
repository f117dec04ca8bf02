// fp_api.hip — the extern "C" entry points of include/llms_amd_fp.h:
// argument validation (before any launch), regime dispatch and the
// per-row int8 quantisation kernel.
#include "llms_amd_fp.h"

#include "fp_common.h"
#include "fp_launch.h"

namespace fp {

namespace {

// One workgroup per weight row: absmax reduction, then quantise the row.
__global__ __launch_bounds__(256) void quantize_w8_kernel(const uint16_t* w, int64_t ldw,
                                                          int8_t* q, int64_t ldq, float* scale,
                                                          int64_t K) {
  const int64_t r = blockIdx.x;
  const uint16_t* wr = w + r * ldw;
  float mx = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) mx = fmaxf(mx, fabsf(bf16_bits_to_f32(wr[k])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float s = mx / 127.0f;
  if (threadIdx.x == 0) scale[r] = s;
  int8_t* qr = q + r * ldq;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
    float v = 0.f;
    if (s > 0.f) v = fminf(fmaxf(rintf(bf16_bits_to_f32(wr[k]) / s), -127.f), 127.f);
    qr[k] = (int8_t)(int)v;
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// rc is the hipError_t of the launch (hipGetLastError right after it).
int launch_status(int rc) {
  if (rc == (int)hipSuccess) return FP_OK;
  const hipError_t e = (hipError_t)rc;
  if (e == hipErrorNoBinaryForGpu || e == hipErrorInvalidDeviceFunction) return FP_ERR_DEVICE;
  return FP_ERR_LAUNCH;
}

template <bool GATEUP, bool W8>
int run(const StreamArgs& a, bool aligned, hipStream_t s) {
  if (a.M == 0) return FP_OK;
  const int rc = (a.M <= kStreamMaxM) ? launch_stream<GATEUP, W8>(a, aligned, s)
                                      : launch_tiled<GATEUP, W8>(a, aligned, s);
  return launch_status(rc);
}

inline int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// int8 calls always dequantise in registers (or once per workgroup into
// LDS in the prefill tiles); no bf16 copy of the weights is ever written.
// With a workspace, the calls whose plan splits k across at least 4
// workgroups (gemm_split_plan: Qwen3 down and o at row counts between 65 and 1792, 8B QKV at 129-256)
// run that split on the int8 weights (gemm_kernel dequantising in registers,
// fp32 partials in the workspace, the fixed-order reduce). Excluded: the
// shapes the int8 split-K tiles take (splitk8_shape) and those the
// in-register prefill tiles take unsplit (gemm8_shape). Measured on MI355X
// against the unsplit dispatch: 8B QKV at 256 rows 44.1 -> 30.9 us, 4B down
// at 128 40.5 -> 26.9 us, 8B down at 256 66.2 -> 46.9 us, 8B o at 256 34.0 ->
// 26.7 us.
inline GemmSplit split8_plan(int64_t M, int64_t N, int64_t K, bool gateup) {
  const GemmSplit none{-1, 1};
  if (K % 64 != 0 || M < 48) return none;
  if (splitk8_shape(M, N, K, gateup) || gemm8_shape(M, N, K, gateup)) return none;
  const GemmSplit p = gemm_split_plan(M, N, K, gateup);
  return p.nsplit >= 4 ? p : none;
}

template <bool GATEUP>
int run_w8(const StreamArgs& a, bool aligned, void* ws, int64_t ws_bytes, hipStream_t s) {
  if (a.M == 0) return FP_OK;
  const GemmSplit p8 = split8_plan(a.M, a.N, a.K, GATEUP);
  if (aligned && p8.tile >= 0 && ws) {
    StreamArgs b = a;
    b.ws = (float*)ws;
    b.ws_floats = ws_bytes / 4;
    if (gemm_split_ws_floats(p8, a.M, a.N, a.K, GATEUP) <= b.ws_floats &&
        gemm_supported(b, true, true))
      return launch_status(launch_gemm_split<GATEUP, true>(b, p8, s));
  }
  StreamArgs b = a;
  b.ws = nullptr;
  b.ws_floats = 0;
  return run<GATEUP, true>(b, aligned, s);
}

int64_t w8_workspace_bytes(int64_t M, int64_t N, int64_t K, bool gateup) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const GemmSplit p8 = split8_plan(M, N, K, gateup);
  return p8.tile >= 0 ? 4 * gemm_split_ws_floats(p8, M, N, K, gateup) : 0;
}

// RMSNorm prologue + projection: one launch on the rows kernel (x normalised
// while it is staged in LDS), else the norm into the workspace and the plain
// dispatch on the normalised rows (any split workspace follows them).
// xaligned: x rows and K fit the vector path; waligned: the weights do.
template <bool GATEUP, bool W8>
int run_norm(StreamArgs a, bool xaligned, bool waligned, void* ws, int64_t ws_bytes,
             hipStream_t s) {
  if (a.M == 0) return FP_OK;
  const bool galigned = al16(a.gamma);
  if (rows_supported<W8>(a, xaligned && waligned && galigned))
    return launch_status(launch_rows<GATEUP, W8>(a, s));
  const int64_t xn_bytes = round_up(a.M * a.K * 2, 256);
  if (!ws || ws_bytes < xn_bytes) return FP_ERR_WORKSPACE;
  uint16_t* xn = (uint16_t*)ws;
  int rc = launch_rmsnorm(a.x, a.ldx, a.gamma, a.eps, xn, a.M, a.K,
                          xaligned && galigned && a.K % 8 == 0, s);
  if (rc) return launch_status(rc);
  StreamArgs b = a;
  b.x = xn;
  b.ldx = a.K;
  b.gamma = nullptr;
  const bool baligned = waligned && a.K % (W8 ? 16 : 8) == 0;
  if constexpr (W8) return run_w8<GATEUP>(b, baligned, (char*)ws + xn_bytes, ws_bytes - xn_bytes, s);
  b.ws = (float*)((char*)ws + xn_bytes);
  b.ws_floats = (ws_bytes - xn_bytes) / 4;
  return run<GATEUP, false>(b, baligned, s);
}

int check_norm(float eps, void* ws, int64_t ws_bytes) {
  if (!(eps >= 0.f) || eps > 3.0e38f) return FP_ERR_SHAPE;
  if (ws_bytes < 0 || (ws && !al16(ws))) return FP_ERR_WORKSPACE;
  return FP_OK;
}

int check_common(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy) {
  if (M < 0 || N < 1 || K < 1) return FP_ERR_SHAPE;
  // grid.x = ceil(N / 16) must fit a 32-bit grid dimension; M tiles likewise.
  if (N > (int64_t)1 << 34 || M > (int64_t)1 << 34) return FP_ERR_SHAPE;
  if (ldx < K || ldy < N) return FP_ERR_STRIDE;
  return FP_OK;
}

}  // namespace

int rmsnorm_qkv_args(const void* x, int64_t ldx, const void* gamma, float eps, const void* w,
                     int64_t ldw, const void* y, int64_t ldy, int64_t M, int64_t n_q, int64_t n_k,
                     int64_t K) {
  if (n_q < 1 || n_k < 0) return FP_ERR_SHAPE;
  int st = check_common(M, n_q + 2 * n_k, K, ldx, ldy);
  if (st) return st;
  if (ldw < K) return FP_ERR_STRIDE;
  if ((st = check_norm(eps, nullptr, 0))) return st;
  if (M > 0 && (!x || !gamma || !w || !y)) return FP_ERR_NULL;
  return FP_OK;
}

}  // namespace fp

using fp::StreamArgs;

extern "C" {

const char* fp_status_string(int status) {
  switch (status) {
    case FP_OK: return "ok";
    case FP_ERR_NULL: return "a required pointer is NULL";
    case FP_ERR_SHAPE: return "shape out of range or inconsistent (M, N, K, n_q, n_k)";
    case FP_ERR_STRIDE: return "row stride smaller than the row length";
    case FP_ERR_LAUNCH: return "HIP kernel launch failed";
    case FP_ERR_DEVICE: return "no gfx950 code object for the current device";
    case FP_ERR_WORKSPACE: return "workspace missing, too small or not 16-byte aligned, or a negative workspace size";
    case FP_ERR_SCRATCH: return "the call needs more than the library's static scratch (FP_SCRATCH_BYTES); use the workspace entry point";
    default: return "unknown fp_status";
  }
}

int fp_abi_version(void) { return (1 << 16) | 5; }

int64_t fp_workspace_bytes(int64_t M, int64_t N, int64_t K, int gate_up) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const fp::GemmSplit p = fp::gemm_split_plan_bf16(M, N, K, gate_up != 0);
  return 4 * fp::gemm_split_ws_floats(p, M, N, K, gate_up != 0);
}

int fp_qkv_bf16_ws(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                   int64_t M, int64_t n_q, int64_t n_k, int64_t K, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  if (n_q < 1 || n_k < 0) return FP_ERR_SHAPE;
  const int64_t N = n_q + 2 * n_k;
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldw < K) return FP_ERR_STRIDE;
  if (workspace_bytes < 0 || (workspace && !fp::al16(workspace))) return FP_ERR_WORKSPACE;
  if (M == 0) return FP_OK;
  if (!x || !w || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, w, ldw, nullptr, 0, nullptr, nullptr,
               (uint16_t*)y, ldy, M, N, K, (float*)workspace, workspace_bytes / 4};
  const bool aligned = (K % 8 == 0) && (ldx % 8 == 0) && (ldw % 8 == 0) &&
                       fp::al16(x) && fp::al16(w);
  return fp::run<false, false>(a, aligned, (hipStream_t)stream);
}

int fp_qkv_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                int64_t M, int64_t n_q, int64_t n_k, int64_t K, void* stream) {
  return fp_qkv_bf16_ws(x, ldx, w, ldw, y, ldy, M, n_q, n_k, K, nullptr, 0, stream);
}

int fp_gate_up_silu_bf16_ws(const void* x, int64_t ldx, const void* wg, int64_t ldwg,
                            const void* wu, int64_t ldwu, void* y, int64_t ldy, int64_t M,
                            int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldwg < K || ldwu < K) return FP_ERR_STRIDE;
  if (workspace_bytes < 0 || (workspace && !fp::al16(workspace))) return FP_ERR_WORKSPACE;
  if (M == 0) return FP_OK;
  if (!x || !wg || !wu || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, wg, ldwg, wu, ldwu, nullptr, nullptr,
               (uint16_t*)y, ldy, M, N, K, (float*)workspace, workspace_bytes / 4};
  const bool aligned = (K % 8 == 0) && (ldx % 8 == 0) && (ldwg % 8 == 0) && (ldwu % 8 == 0) &&
                       fp::al16(x) && fp::al16(wg) && fp::al16(wu);
  return fp::run<true, false>(a, aligned, (hipStream_t)stream);
}

int fp_gate_up_silu_bf16(const void* x, int64_t ldx, const void* wg, int64_t ldwg,
                         const void* wu, int64_t ldwu, void* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, void* stream) {
  return fp_gate_up_silu_bf16_ws(x, ldx, wg, ldwg, wu, ldwu, y, ldy, M, N, K, nullptr, 0,
                                 stream);
}

int64_t fp_workspace_bytes_w8(int64_t M, int64_t N, int64_t K, int gate_up) {
  return fp::w8_workspace_bytes(M, N, K, gate_up != 0);
}

int fp_qkv_w8_ws(const void* x, int64_t ldx, const int8_t* q, int64_t ldq, const float* scale,
                 void* y, int64_t ldy, int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (n_q < 1 || n_k < 0) return FP_ERR_SHAPE;
  const int64_t N = n_q + 2 * n_k;
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldq < K) return FP_ERR_STRIDE;
  if (workspace_bytes < 0 || (workspace && !fp::al16(workspace))) return FP_ERR_WORKSPACE;
  if (M == 0) return FP_OK;
  if (!x || !q || !scale || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, q, ldq, nullptr, 0, scale, nullptr,
               (uint16_t*)y, ldy, M, N, K};
  const bool aligned = (K % 16 == 0) && (ldx % 8 == 0) && (ldq % 16 == 0) &&
                       fp::al16(x) && fp::al16(q);
  return fp::run_w8<false>(a, aligned, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_qkv_w8(const void* x, int64_t ldx, const int8_t* q, int64_t ldq, const float* scale,
              void* y, int64_t ldy, int64_t M, int64_t n_q, int64_t n_k, int64_t K,
              void* stream) {
  return fp_qkv_w8_ws(x, ldx, q, ldq, scale, y, ldy, M, n_q, n_k, K, nullptr, 0, stream);
}

int fp_gate_up_silu_w8_ws(const void* x, int64_t ldx, const int8_t* qg, int64_t ldqg,
                          const float* sg, const int8_t* qu, int64_t ldqu, const float* su,
                          void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                          void* workspace, int64_t workspace_bytes, void* stream) {
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldqg < K || ldqu < K) return FP_ERR_STRIDE;
  if (workspace_bytes < 0 || (workspace && !fp::al16(workspace))) return FP_ERR_WORKSPACE;
  if (M == 0) return FP_OK;
  if (!x || !qg || !sg || !qu || !su || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, qg, ldqg, qu, ldqu, sg, su,
               (uint16_t*)y, ldy, M, N, K};
  const bool aligned = (K % 16 == 0) && (ldx % 8 == 0) && (ldqg % 16 == 0) &&
                       (ldqu % 16 == 0) && fp::al16(x) && fp::al16(qg) && fp::al16(qu);
  return fp::run_w8<true>(a, aligned, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_gate_up_silu_w8(const void* x, int64_t ldx, const int8_t* qg, int64_t ldqg,
                       const float* sg, const int8_t* qu, int64_t ldqu, const float* su,
                       void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  return fp_gate_up_silu_w8_ws(x, ldx, qg, ldqg, sg, qu, ldqu, su, y, ldy, M, N, K, nullptr, 0,
                               stream);
}

int fp_linear_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                   int64_t M, int64_t N, int64_t K, void* stream) {
  return fp_qkv_bf16(x, ldx, w, ldw, y, ldy, M, N, 0, K, stream);
}

int fp_linear_bf16_ws(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  return fp_qkv_bf16_ws(x, ldx, w, ldw, y, ldy, M, N, 0, K, workspace, workspace_bytes, stream);
}

int fp_linear_w8(const void* x, int64_t ldx, const int8_t* q, int64_t ldq, const float* scale,
                 void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  return fp_qkv_w8(x, ldx, q, ldq, scale, y, ldy, M, N, 0, K, stream);
}

int fp_linear_w8_ws(const void* x, int64_t ldx, const int8_t* q, int64_t ldq, const float* scale,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  return fp_qkv_w8_ws(x, ldx, q, ldq, scale, y, ldy, M, N, 0, K, workspace, workspace_bytes,
                      stream);
}

int64_t fp_rmsnorm_workspace_bytes(int64_t M, int64_t N, int64_t K, int gate_up, int int8) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const bool w8 = int8 != 0;
  // Room for the normalised rows always: decode-sized calls usually run as
  // one launch and leave it unused, but take the two-launch path when a
  // pointer or stride misses the 16-byte alignment of that launch. There the
  // plain dispatch (bf16 M <= 2, int8 M <= 4) needs no further workspace.
  int64_t b = fp::round_up(M * K * 2, 256);
  if (M <= (w8 ? fp::kRowsMaxM : 2) && K % (w8 ? 16 : 8) == 0 && fp::rows_fit(M, K, w8, true))
    return b;
  if (w8) return b + fp::w8_workspace_bytes(M, N, K, gate_up != 0);
  return b + 4 * fp::gemm_split_ws_floats(fp::gemm_split_plan_bf16(M, N, K, gate_up != 0), M, N,
                                          K, gate_up != 0);
}

int fp_rmsnorm_qkv_bf16(const void* x, int64_t ldx, const void* gamma, float eps, const void* w,
                        int64_t ldw, void* y, int64_t ldy, int64_t M, int64_t n_q, int64_t n_k,
                        int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  int st = fp::rmsnorm_qkv_args(x, ldx, gamma, eps, w, ldw, y, ldy, M, n_q, n_k, K);
  if (st) return st;
  if ((st = fp::check_norm(eps, workspace, workspace_bytes))) return st;
  if (M == 0) return FP_OK;
  const int64_t N = n_q + 2 * n_k;
  StreamArgs a{(const uint16_t*)x, ldx, w, ldw, nullptr, 0, nullptr, nullptr, (uint16_t*)y, ldy,
               M, N, K, nullptr, 0, (const uint16_t*)gamma, eps};
  const bool xal = K % 8 == 0 && ldx % 8 == 0 && fp::al16(x);
  const bool wal = ldw % 8 == 0 && fp::al16(w);
  return fp::run_norm<false, false>(a, xal, wal, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_rmsnorm_gate_up_silu_bf16(const void* x, int64_t ldx, const void* gamma, float eps,
                                 const void* wg, int64_t ldwg, const void* wu, int64_t ldwu,
                                 void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldwg < K || ldwu < K) return FP_ERR_STRIDE;
  if ((st = fp::check_norm(eps, workspace, workspace_bytes))) return st;
  if (M == 0) return FP_OK;
  if (!x || !gamma || !wg || !wu || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, wg, ldwg, wu, ldwu, nullptr, nullptr, (uint16_t*)y, ldy,
               M, N, K, nullptr, 0, (const uint16_t*)gamma, eps};
  const bool xal = K % 8 == 0 && ldx % 8 == 0 && fp::al16(x);
  const bool wal = ldwg % 8 == 0 && ldwu % 8 == 0 && fp::al16(wg) && fp::al16(wu);
  return fp::run_norm<true, false>(a, xal, wal, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_rmsnorm_qkv_w8(const void* x, int64_t ldx, const void* gamma, float eps, const int8_t* q,
                      int64_t ldq, const float* scale, void* y, int64_t ldy, int64_t M,
                      int64_t n_q, int64_t n_k, int64_t K, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  if (n_q < 1 || n_k < 0) return FP_ERR_SHAPE;
  const int64_t N = n_q + 2 * n_k;
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldq < K) return FP_ERR_STRIDE;
  if ((st = fp::check_norm(eps, workspace, workspace_bytes))) return st;
  if (M == 0) return FP_OK;
  if (!x || !gamma || !q || !scale || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, q, ldq, nullptr, 0, scale, nullptr, (uint16_t*)y, ldy,
               M, N, K, nullptr, 0, (const uint16_t*)gamma, eps};
  const bool xal = K % 16 == 0 && ldx % 8 == 0 && fp::al16(x);
  const bool wal = ldq % 16 == 0 && fp::al16(q);
  return fp::run_norm<false, true>(a, xal, wal, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_rmsnorm_gate_up_silu_w8(const void* x, int64_t ldx, const void* gamma, float eps,
                               const int8_t* qg, int64_t ldqg, const float* sg, const int8_t* qu,
                               int64_t ldqu, const float* su, void* y, int64_t ldy, int64_t M,
                               int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  int st = fp::check_common(M, N, K, ldx, ldy);
  if (st) return st;
  if (ldqg < K || ldqu < K) return FP_ERR_STRIDE;
  if ((st = fp::check_norm(eps, workspace, workspace_bytes))) return st;
  if (M == 0) return FP_OK;
  if (!x || !gamma || !qg || !sg || !qu || !su || !y) return FP_ERR_NULL;
  StreamArgs a{(const uint16_t*)x, ldx, qg, ldqg, qu, ldqu, sg, su, (uint16_t*)y, ldy,
               M, N, K, nullptr, 0, (const uint16_t*)gamma, eps};
  const bool xal = K % 16 == 0 && ldx % 8 == 0 && fp::al16(x);
  const bool wal = ldqg % 16 == 0 && ldqu % 16 == 0 && fp::al16(qg) && fp::al16(qu);
  return fp::run_norm<true, true>(a, xal, wal, workspace, workspace_bytes, (hipStream_t)stream);
}

int fp_quantize_w8_per_row(const void* w, int64_t ldw, int8_t* q, int64_t ldq, float* scale,
                           int64_t N, int64_t K, void* stream) {
  if (N < 0 || K < 1 || N > ((int64_t)1 << 31) - 1) return FP_ERR_SHAPE;
  if (ldw < K || ldq < K) return FP_ERR_STRIDE;
  if (N == 0) return FP_OK;
  if (!w || !q || !scale) return FP_ERR_NULL;
  hipLaunchKernelGGL(fp::quantize_w8_kernel, dim3((unsigned)N), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)w, ldw, q, ldq, scale, K);
  return fp::launch_status((int)hipGetLastError());
}

}  // extern "C"
