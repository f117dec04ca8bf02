/*
 * llms_amd_fp.h — C ABI of the MI355X (gfx950) fused projection kernels.
 *
 * Two fused projections of a Qwen3 decoder layer, each as one contraction
 * over a row-stacked weight:
 *
 *   QKV          y[M, n_q+2*n_k] = x[M,K] . [Wq;Wk;Wv]^T      (split done by the caller, as views)
 *   gate-up-SiLU y[M, N]         = silu(x . Wg^T) * (x . Wu^T)
 *
 * plus per-output-channel symmetric int8 weight-only variants that
 * dequantise w = bf16(float(q) * s[row]) in registers.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers. Element types: bf16 = raw 16-bit
 *     bfloat16 (passed as void*), int8 weights, fp32 scales.
 *   - Matrices are row-major with unit inner stride; ld* is the row
 *     stride in ELEMENTS. Weights use the nn.Linear layout [N, K].
 *   - stream is a hipStream_t (NULL = the legacy default stream). Every call
 *     is asynchronous on that stream; nothing is allocated, freed or
 *     synchronised; calls are reentrant. The *_ws variants also write the
 *     caller's workspace, which must not be used by work that can overlap
 *     the call. The only global state is the per-device address of the
 *     static scratch of fp_rmsnorm_qkv_bf16_noalloc, written once per device.
 *   - Return 0 (FP_OK) on success, a nonzero fp_status otherwise; argument
 *     errors are detected before anything is launched.
 *   - Results are deterministic: the same inputs give bit-identical outputs
 *     on every call (fixed-order reductions, no atomics).
 *
 * Rounding contract (bf16 in, fp32 accumulate, bf16 out):
 *   QKV:      y = bf16(sum_k x*w)
 *   gate-up:  g = bf16(sum x*wg); u = bf16(sum x*wu);
 *             s = bf16(g / (1 + exp(-g)));  y = bf16(s * u)
 *   i.e. the rounding points of the unfused torch path
 *   F.silu(F.linear(x, Wg)) * F.linear(x, Wu) in bfloat16.
 *   int8:     w = bf16(float(q) * s[row]) then the bf16 contract above
 *   (the "dequantise then matmul" path).
 */
#ifndef LLMS_AMD_FP_H
#define LLMS_AMD_FP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fp_status {
  FP_OK = 0,
  FP_ERR_NULL = 1,       /* a required pointer is NULL */
  FP_ERR_SHAPE = 2,      /* M, N, K, n_q, n_k out of range or inconsistent */
  FP_ERR_STRIDE = 3,     /* a row stride is smaller than the row length */
  FP_ERR_LAUNCH = 4,     /* the HIP launch reported an error */
  FP_ERR_DEVICE = 5,     /* no usable gfx950 device for the current context */
  FP_ERR_WORKSPACE = 6,  /* workspace missing or too small where required, not 16-byte
                            aligned, or a negative size */
  FP_ERR_SCRATCH = 7     /* the call needs more than the library's static scratch
                            (FP_SCRATCH_BYTES); use the workspace entry point */
} fp_status;

/* Human-readable text for an fp_status value (static storage). */
const char* fp_status_string(int status);

/* ABI version of this library: (major << 16) | minor. Minor 5 adds
 * fp_rmsnorm_qkv_bf16_noalloc and FP_ERR_SCRATCH, and sizes
 * fp_rmsnorm_workspace_bytes for the normalised rows of every call. */
int fp_abi_version(void);

/*
 * Fused QKV projection.
 * Replaces _qkv_matmul_kernel + the launch in triton_fused_qkv
 * (reference: src/kernels/fused_qkv.py:28-85, :131-145).
 *   x  [M, K]            bf16, row stride ldx
 *   w  [n_q+2*n_k, K]    bf16, row stride ldw  (row-stacked [Wq; Wk; Wv])
 *   y  [M, n_q+2*n_k]    bf16, row stride ldy  (q | k | v column blocks)
 * M >= 0 (M == 0 is a no-op), K >= 1, n_q >= 1, n_k >= 0.
 */
int fp_qkv_bf16(const void* x, int64_t ldx,
                const void* w, int64_t ldw,
                void* y, int64_t ldy,
                int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                void* stream);

/*
 * Fused gate-up-SiLU.
 * Replaces _fused_gate_up_silu_kernel + the launch in
 * triton_fused_gate_up_silu (reference: src/kernels/fused_ffn.py:20-95,
 * :131-150). Wg and Wu stay two separate [N, K] buffers, as in the reference.
 *   y [M, N] = silu(x Wg^T) * (x Wu^T)
 */
int fp_gate_up_silu_bf16(const void* x, int64_t ldx,
                         const void* wg, int64_t ldwg,
                         const void* wu, int64_t ldwu,
                         void* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K,
                         void* stream);

/*
 * int8 weight-only QKV (no reference counterpart: the reference names
 * weight quantisation only as future work, reference DESIGN.md:120).
 *   q [n_q+2*n_k, K] int8 (row stride ldq), scale [n_q+2*n_k] fp32.
 */
int fp_qkv_w8(const void* x, int64_t ldx,
              const int8_t* q, int64_t ldq, const float* scale,
              void* y, int64_t ldy,
              int64_t M, int64_t n_q, int64_t n_k, int64_t K,
              void* stream);

/* int8 weight-only gate-up-SiLU (no reference counterpart, as above). */
int fp_gate_up_silu_w8(const void* x, int64_t ldx,
                       const int8_t* qg, int64_t ldqg, const float* sg,
                       const int8_t* qu, int64_t ldqu, const float* su,
                       void* y, int64_t ldy,
                       int64_t M, int64_t N, int64_t K,
                       void* stream);

/*
 * Plain projection y = x W^T (bf16 out, no split, no epilogue): the MLP
 * `down` and the attention `o` projections next to the fused path. Replaces
 * the eager nn.Linear calls self.down(...) (reference: src/engine/model.py:37)
 * and self.o(...) (reference: src/engine/attention.py:98, :183). Runs the same
 * kernels as fp_qkv_bf16 (which it equals for n_q = N, n_k = 0).
 *   x [M, K] bf16, w [N, K] bf16, y [M, N] bf16.  M >= 0, N >= 1, K >= 1.
 */
int fp_linear_bf16(const void* x, int64_t ldx,
                   const void* w, int64_t ldw,
                   void* y, int64_t ldy,
                   int64_t M, int64_t N, int64_t K,
                   void* stream);

/* int8 weight-only plain projection (no reference counterpart, as above). */
int fp_linear_w8(const void* x, int64_t ldx,
                 const int8_t* q, int64_t ldq, const float* scale,
                 void* y, int64_t ldy,
                 int64_t M, int64_t N, int64_t K,
                 void* stream);

/*
 * Workspace variants of the three bf16 entry points (no reference
 * counterpart: the reference's Triton launches take no workspace). With a
 * workspace of at least fp_workspace_bytes(M, N, K, gate_up) bytes
 * (N = n_q + 2*n_k for QKV, the output width otherwise), calls whose tile
 * grid would leave CUs idle while each tile runs a long k loop split k across
 * workgroups: fp32 partial sums go to the workspace and a second kernel sums
 * them in a fixed order and applies the epilogue (results stay
 * deterministic). A NULL or smaller workspace runs the unsplit kernels of the
 * plain entry points. The workspace must be 16-byte aligned (any hipMalloc or
 * torch allocation is) and is overwritten.
 */
int64_t fp_workspace_bytes(int64_t M, int64_t N, int64_t K, int gate_up);

int fp_qkv_bf16_ws(const void* x, int64_t ldx,
                   const void* w, int64_t ldw,
                   void* y, int64_t ldy,
                   int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                   void* workspace, int64_t workspace_bytes,
                   void* stream);

int fp_gate_up_silu_bf16_ws(const void* x, int64_t ldx,
                            const void* wg, int64_t ldwg,
                            const void* wu, int64_t ldwu,
                            void* y, int64_t ldy,
                            int64_t M, int64_t N, int64_t K,
                            void* workspace, int64_t workspace_bytes,
                            void* stream);

int fp_linear_bf16_ws(const void* x, int64_t ldx,
                      const void* w, int64_t ldw,
                      void* y, int64_t ldy,
                      int64_t M, int64_t N, int64_t K,
                      void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * Workspace variants of the int8 entry points (no reference counterpart).
 * Every int8 call dequantises in registers (in the prefill tiles: once per
 * workgroup into LDS); no bf16 copy of the weights is written anywhere. The
 * workspace serves only the k split across workgroups: for the shapes whose
 * plan splits k over at least 4 workgroups (fp_workspace_bytes_w8(M, N, K,
 * gate_up) > 0: down and o projections at some row counts between 65 and 1792, Qwen3-8B QKV at
 * 129-256), given that much workspace, the split runs with its fp32
 * partials there. Without it those calls run unsplit, with the same
 * contract.
 */
int64_t fp_workspace_bytes_w8(int64_t M, int64_t N, int64_t K, int gate_up);

int fp_qkv_w8_ws(const void* x, int64_t ldx,
                 const int8_t* q, int64_t ldq, const float* scale,
                 void* y, int64_t ldy,
                 int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                 void* workspace, int64_t workspace_bytes,
                 void* stream);

int fp_gate_up_silu_w8_ws(const void* x, int64_t ldx,
                          const int8_t* qg, int64_t ldqg, const float* sg,
                          const int8_t* qu, int64_t ldqu, const float* su,
                          void* y, int64_t ldy,
                          int64_t M, int64_t N, int64_t K,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

int fp_linear_w8_ws(const void* x, int64_t ldx,
                    const int8_t* q, int64_t ldq, const float* scale,
                    void* y, int64_t ldy,
                    int64_t M, int64_t N, int64_t K,
                    void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * RMSNorm prologue fused with the projections (no reference counterpart as a
 * kernel: it replaces the eager pair norm1(x) -> attention q/k/v and
 * norm2(h) -> FFN gate/up, reference src/engine/model.py:57-66 with RMSNorm
 * src/engine/attention.py:28-33). With gamma [K] bf16 and eps:
 *   r     = 1 / sqrt(sum_k x[k]^2 / K + eps)            (fp32)
 *   xn[k] = bf16(gamma[k] * bf16(x[k] * r))
 * and then the contract of the matching projection on xn. Decode-sized calls
 * (the row-streaming regime: bf16 M <= 2, int8 M <= 4, with room for x in
 * LDS) whose x, weights and gamma are 16-byte aligned with row strides that
 * are multiples of 8 (int8 weights: 16) run as one launch that normalises x
 * while staging it and need no workspace. Every other call needs a workspace
 * (the normalised rows, then any split-k partials) and returns
 * FP_ERR_WORKSPACE without one; fp_rmsnorm_workspace_bytes(M, N, K, gate_up,
 * int8) is enough for any pointers and strides of that shape. eps must be
 * finite and >= 0.
 */
int64_t fp_rmsnorm_workspace_bytes(int64_t M, int64_t N, int64_t K, int gate_up, int int8);

int fp_rmsnorm_qkv_bf16(const void* x, int64_t ldx, const void* gamma, float eps,
                        const void* w, int64_t ldw,
                        void* y, int64_t ldy,
                        int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                        void* workspace, int64_t workspace_bytes,
                        void* stream);

int fp_rmsnorm_gate_up_silu_bf16(const void* x, int64_t ldx, const void* gamma, float eps,
                                 const void* wg, int64_t ldwg,
                                 const void* wu, int64_t ldwu,
                                 void* y, int64_t ldy,
                                 int64_t M, int64_t N, int64_t K,
                                 void* workspace, int64_t workspace_bytes,
                                 void* stream);

int fp_rmsnorm_qkv_w8(const void* x, int64_t ldx, const void* gamma, float eps,
                      const int8_t* q, int64_t ldq, const float* scale,
                      void* y, int64_t ldy,
                      int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                      void* workspace, int64_t workspace_bytes,
                      void* stream);

int fp_rmsnorm_gate_up_silu_w8(const void* x, int64_t ldx, const void* gamma, float eps,
                               const int8_t* qg, int64_t ldqg, const float* sg,
                               const int8_t* qu, int64_t ldqu, const float* su,
                               void* y, int64_t ldy,
                               int64_t M, int64_t N, int64_t K,
                               void* workspace, int64_t workspace_bytes,
                               void* stream);

/*
 * Allocation-free variant of fp_rmsnorm_qkv_bf16 (no reference counterpart:
 * for callers that cannot allocate device memory — code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). Same
 * arguments, contract and results as fp_rmsnorm_qkv_bf16, bit for bit, but
 * the workspace is the library's own static device array of FP_SCRATCH_BYTES
 * (one per GPU, held until the process ends; its address is looked up on
 * the first successful call on a device, a failed lookup is retried by the
 * next call). The stream, when not NULL, must belong to the current device
 * (FP_ERR_DEVICE otherwise: the scratch address is per device). Calls whose
 * fp_rmsnorm_workspace_bytes(M, n_q + 2*n_k, K, 0, 0) exceeds FP_SCRATCH_BYTES
 * return FP_ERR_SCRATCH before anything is launched. Every call on a GPU
 * overwrites that GPU's scratch: calls that can overlap on one GPU (streams
 * without ordering between them) race and must be serialised by the caller.
 * Nothing is allocated or freed.
 */
#define FP_SCRATCH_BYTES (32u << 20)

int fp_rmsnorm_qkv_bf16_noalloc(const void* x, int64_t ldx, const void* gamma, float eps,
                                const void* w, int64_t ldw,
                                void* y, int64_t ldy,
                                int64_t M, int64_t n_q, int64_t n_k, int64_t K,
                                void* stream);

/*
 * Per-output-channel symmetric int8 quantisation on the device (the packing
 * step run once at swap time; no reference counterpart).
 *   s[r] = max_k |w[r,k]| / 127   (fp32; rows that are all zero get s = 0)
 *   q[r,k] = clamp(rne(w[r,k] / s[r]), -127, 127)   (0 where s == 0)
 */
int fp_quantize_w8_per_row(const void* w, int64_t ldw,
                           int8_t* q, int64_t ldq, float* scale,
                           int64_t N, int64_t K,
                           void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* LLMS_AMD_FP_H */
