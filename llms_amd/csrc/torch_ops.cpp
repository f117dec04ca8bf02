// torch_ops.cpp — the thin PyTorch-ROCm custom ops over the C ABI of
// include/llms_amd_fp.h. Each op allocates its output (and, for the bf16
// calls that split k across workgroups, the workspace) with torch on the
// tensor's device, takes torch's current HIP stream, and hands plain pointers,
// row strides and sizes to the C ABI; a nonzero fp_status becomes a
// c10::Error (RuntimeError in Python). No computation happens here.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "llms_amd_fp.h"

namespace {

void check_status(int st, const char* fn) {
  TORCH_CHECK(st == FP_OK, fn, " failed: ", fp_status_string(st), " (fp_status ", st, ")");
}

void check_2d(const at::Tensor& t, const char* name, at::ScalarType dt) {
  TORCH_CHECK(t.dim() == 2, name, " must be 2-D, got ", t.dim(), "-D");
  TORCH_CHECK(t.scalar_type() == dt, name, " must be ", c10::toString(dt), ", got ",
              c10::toString(t.scalar_type()));
  TORCH_CHECK(t.size(1) <= 1 || t.stride(1) == 1, name, " must have unit inner stride");
  TORCH_CHECK(t.is_cuda(), name, " must be a HIP device tensor");
}

// Every tensor of a call lives on x's device (the kernels dereference all of
// them there; a host pointer would fault the GPU).
void check_same_device(const at::Tensor& x, const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda() && t.device() == x.device(), name, " must be on ", x.device(),
              ", got ", t.device());
}

// A weight [N, K] of the call: K columns (the x row length), on x's device.
void check_weight(const at::Tensor& x, const at::Tensor& w, const char* name) {
  TORCH_CHECK(w.size(1) == x.size(1), name, " has ", w.size(1), " columns, x has K = ",
              x.size(1));
  check_same_device(x, w, name);
}

// Per-row int8 scales of weight q: contiguous 1-D fp32, one per row, on x's
// device.
void check_scale(const at::Tensor& x, const at::Tensor& s, const at::Tensor& q, const char* name) {
  TORCH_CHECK(s.dim() == 1 && s.scalar_type() == at::kFloat && s.is_contiguous(), name,
              " must be a contiguous 1-D float32 tensor");
  TORCH_CHECK(s.size(0) == q.size(0), name, " has ", s.size(0), " rows, q has ", q.size(0));
  check_same_device(x, s, name);
}

// Gate and up weights of one call have the same shape.
void check_pair(const at::Tensor& g, const at::Tensor& u, const char* gn, const char* un) {
  TORCH_CHECK(g.sizes() == u.sizes(), gn, " ", g.sizes(), " and ", un, " ", u.sizes(),
              " must have the same shape");
}

void* cur_stream(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Split-k workspace for a bf16 call, from torch's caching allocator on the
// current stream (empty when the call does not split).
at::Tensor workspace(const at::Tensor& x, int64_t M, int64_t N, int64_t K, bool gate_up) {
  const int64_t bytes = fp_workspace_bytes(M, N, K, gate_up ? 1 : 0);
  return at::empty({bytes}, x.options().dtype(at::kByte));
}

// Workspace for an int8 call: the fp32 partials where k is split across
// workgroups, empty otherwise (int8 weights are never expanded to bf16).
at::Tensor workspace_w8(const at::Tensor& x, int64_t M, int64_t N, int64_t K, bool gate_up) {
  const int64_t bytes = fp_workspace_bytes_w8(M, N, K, gate_up ? 1 : 0);
  return at::empty({bytes}, x.options().dtype(at::kByte));
}

at::Tensor qkv(const at::Tensor& x, const at::Tensor& w, int64_t n_q, int64_t n_k) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(w, "W_qkv", at::kBFloat16);
  check_weight(x, w, "W_qkv");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = w.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace(x, M, N, K, false);
  check_status(fp_qkv_bf16_ws(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                              y.stride(0), M, n_q, n_k, K, ws.numel() ? ws.data_ptr() : nullptr,
                              ws.numel(), cur_stream(x)),
               "fp_qkv_bf16_ws");
  return y;
}

at::Tensor gate_up_silu(const at::Tensor& x, const at::Tensor& wg, const at::Tensor& wu) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(wg, "Wg", at::kBFloat16);
  check_2d(wu, "Wu", at::kBFloat16);
  check_weight(x, wg, "Wg");
  check_weight(x, wu, "Wu");
  check_pair(wg, wu, "Wg", "Wu");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = wg.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace(x, M, N, K, true);
  check_status(fp_gate_up_silu_bf16_ws(x.data_ptr(), x.stride(0), wg.data_ptr(), wg.stride(0),
                                       wu.data_ptr(), wu.stride(0), y.data_ptr(), y.stride(0), M,
                                       N, K, ws.numel() ? ws.data_ptr() : nullptr, ws.numel(),
                                       cur_stream(x)),
               "fp_gate_up_silu_bf16_ws");
  return y;
}

at::Tensor qkv_w8(const at::Tensor& x, const at::Tensor& q, const at::Tensor& s, int64_t n_q,
                  int64_t n_k) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(q, "q", at::kChar);
  check_weight(x, q, "q");
  check_scale(x, s, q, "scale");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = q.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace_w8(x, M, N, K, false);
  check_status(fp_qkv_w8_ws(x.data_ptr(), x.stride(0), (const int8_t*)q.data_ptr(), q.stride(0),
                            s.data_ptr<float>(), y.data_ptr(), y.stride(0), M, n_q, n_k, K,
                            ws.numel() ? ws.data_ptr() : nullptr, ws.numel(), cur_stream(x)),
               "fp_qkv_w8_ws");
  return y;
}

at::Tensor gate_up_silu_w8(const at::Tensor& x, const at::Tensor& qg, const at::Tensor& sg,
                           const at::Tensor& qu, const at::Tensor& su) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(qg, "qg", at::kChar);
  check_2d(qu, "qu", at::kChar);
  check_weight(x, qg, "qg");
  check_weight(x, qu, "qu");
  check_pair(qg, qu, "qg", "qu");
  check_scale(x, sg, qg, "sg");
  check_scale(x, su, qu, "su");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = qg.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace_w8(x, M, N, K, true);
  check_status(fp_gate_up_silu_w8_ws(x.data_ptr(), x.stride(0), (const int8_t*)qg.data_ptr(),
                                     qg.stride(0), sg.data_ptr<float>(),
                                     (const int8_t*)qu.data_ptr(), qu.stride(0),
                                     su.data_ptr<float>(), y.data_ptr(), y.stride(0), M, N, K,
                                     ws.numel() ? ws.data_ptr() : nullptr, ws.numel(),
                                     cur_stream(x)),
               "fp_gate_up_silu_w8_ws");
  return y;
}

at::Tensor linear(const at::Tensor& x, const at::Tensor& w) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(w, "W", at::kBFloat16);
  check_weight(x, w, "W");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = w.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace(x, M, N, K, false);
  check_status(fp_linear_bf16_ws(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                 y.data_ptr(), y.stride(0), M, N, K,
                                 ws.numel() ? ws.data_ptr() : nullptr, ws.numel(), cur_stream(x)),
               "fp_linear_bf16_ws");
  return y;
}

at::Tensor linear_w8(const at::Tensor& x, const at::Tensor& q, const at::Tensor& s) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(q, "q", at::kChar);
  check_weight(x, q, "q");
  check_scale(x, s, q, "scale");
  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = q.size(0);
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = workspace_w8(x, M, N, K, false);
  check_status(fp_linear_w8_ws(x.data_ptr(), x.stride(0), (const int8_t*)q.data_ptr(), q.stride(0),
                               s.data_ptr<float>(), y.data_ptr(), y.stride(0), M, N, K,
                               ws.numel() ? ws.data_ptr() : nullptr, ws.numel(), cur_stream(x)),
               "fp_linear_w8_ws");
  return y;
}

// ---- RMSNorm prologue fused with the projections ----

void check_gamma(const at::Tensor& x, const at::Tensor& gamma) {
  TORCH_CHECK(gamma.dim() == 1 && gamma.scalar_type() == at::kBFloat16 && gamma.is_contiguous(),
              "norm weight must be a contiguous 1-D bfloat16 tensor");
  TORCH_CHECK(gamma.size(0) == x.size(1), "norm weight has ", gamma.size(0),
              " elements, x has K = ", x.size(1));
  check_same_device(x, gamma, "norm weight");
}

// Workspace for a fused-norm call: what the library asks for (enough for any
// pointers and strides of the shape).
at::Tensor norm_workspace(const at::Tensor& x, int64_t M, int64_t N, int64_t K, bool gate_up,
                          bool int8) {
  const int64_t bytes = fp_rmsnorm_workspace_bytes(M, N, K, gate_up ? 1 : 0, int8 ? 1 : 0);
  return at::empty({bytes}, x.options().dtype(at::kByte));
}

at::Tensor rmsnorm_qkv(const at::Tensor& x, const at::Tensor& gamma, double eps,
                       const at::Tensor& w, int64_t n_q, int64_t n_k) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(w, "W_qkv", at::kBFloat16);
  check_weight(x, w, "W_qkv");
  const int64_t M = x.size(0), K = x.size(1), N = w.size(0);
  check_gamma(x, gamma);
  const c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = norm_workspace(x, M, N, K, false, false);
  check_status(fp_rmsnorm_qkv_bf16(x.data_ptr(), x.stride(0), gamma.data_ptr(), (float)eps,
                                   w.data_ptr(), w.stride(0), y.data_ptr(), y.stride(0), M, n_q,
                                   n_k, K, ws.data_ptr(), ws.numel(), cur_stream(x)),
               "fp_rmsnorm_qkv_bf16");
  return y;
}

at::Tensor rmsnorm_gate_up_silu(const at::Tensor& x, const at::Tensor& gamma, double eps,
                                const at::Tensor& wg, const at::Tensor& wu) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(wg, "Wg", at::kBFloat16);
  check_2d(wu, "Wu", at::kBFloat16);
  check_weight(x, wg, "Wg");
  check_weight(x, wu, "Wu");
  check_pair(wg, wu, "Wg", "Wu");
  const int64_t M = x.size(0), K = x.size(1), N = wg.size(0);
  check_gamma(x, gamma);
  const c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = norm_workspace(x, M, N, K, true, false);
  check_status(fp_rmsnorm_gate_up_silu_bf16(x.data_ptr(), x.stride(0), gamma.data_ptr(),
                                            (float)eps, wg.data_ptr(), wg.stride(0),
                                            wu.data_ptr(), wu.stride(0), y.data_ptr(),
                                            y.stride(0), M, N, K, ws.data_ptr(), ws.numel(),
                                            cur_stream(x)),
               "fp_rmsnorm_gate_up_silu_bf16");
  return y;
}

at::Tensor rmsnorm_qkv_w8(const at::Tensor& x, const at::Tensor& gamma, double eps,
                          const at::Tensor& q, const at::Tensor& s, int64_t n_q, int64_t n_k) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(q, "q", at::kChar);
  check_weight(x, q, "q");
  check_scale(x, s, q, "scale");
  const int64_t M = x.size(0), K = x.size(1), N = q.size(0);
  check_gamma(x, gamma);
  const c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = norm_workspace(x, M, N, K, false, true);
  check_status(fp_rmsnorm_qkv_w8(x.data_ptr(), x.stride(0), gamma.data_ptr(), (float)eps,
                                 (const int8_t*)q.data_ptr(), q.stride(0), s.data_ptr<float>(),
                                 y.data_ptr(), y.stride(0), M, n_q, n_k, K, ws.data_ptr(),
                                 ws.numel(), cur_stream(x)),
               "fp_rmsnorm_qkv_w8");
  return y;
}

at::Tensor rmsnorm_gate_up_silu_w8(const at::Tensor& x, const at::Tensor& gamma, double eps,
                                   const at::Tensor& qg, const at::Tensor& sg,
                                   const at::Tensor& qu, const at::Tensor& su) {
  check_2d(x, "x", at::kBFloat16);
  check_2d(qg, "qg", at::kChar);
  check_2d(qu, "qu", at::kChar);
  check_weight(x, qg, "qg");
  check_weight(x, qu, "qu");
  check_pair(qg, qu, "qg", "qu");
  check_scale(x, sg, qg, "sg");
  check_scale(x, su, qu, "su");
  const int64_t M = x.size(0), K = x.size(1), N = qg.size(0);
  check_gamma(x, gamma);
  const c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty({M, N}, x.options());
  at::Tensor ws = norm_workspace(x, M, N, K, true, true);
  check_status(fp_rmsnorm_gate_up_silu_w8(x.data_ptr(), x.stride(0), gamma.data_ptr(),
                                          (float)eps, (const int8_t*)qg.data_ptr(), qg.stride(0),
                                          sg.data_ptr<float>(), (const int8_t*)qu.data_ptr(),
                                          qu.stride(0), su.data_ptr<float>(), y.data_ptr(),
                                          y.stride(0), M, N, K, ws.data_ptr(), ws.numel(),
                                          cur_stream(x)),
               "fp_rmsnorm_gate_up_silu_w8");
  return y;
}

std::tuple<at::Tensor, at::Tensor> quantize_w8(const at::Tensor& w) {
  check_2d(w, "W", at::kBFloat16);
  const c10::DeviceGuard guard(w.device());
  const int64_t N = w.size(0), K = w.size(1);
  at::Tensor q = at::empty({N, K}, w.options().dtype(at::kChar));
  at::Tensor s = at::empty({N}, w.options().dtype(at::kFloat));
  check_status(fp_quantize_w8_per_row(w.data_ptr(), w.stride(0), (int8_t*)q.data_ptr(),
                                      q.stride(0), s.data_ptr<float>(), N, K, cur_stream(w)),
               "fp_quantize_w8_per_row");
  return {q, s};
}

}  // namespace

TORCH_LIBRARY(llms_amd, m) {
  m.def("qkv(Tensor x, Tensor w_qkv, int n_q, int n_k) -> Tensor");
  m.def("gate_up_silu(Tensor x, Tensor wg, Tensor wu) -> Tensor");
  m.def("qkv_w8(Tensor x, Tensor q, Tensor scale, int n_q, int n_k) -> Tensor");
  m.def("gate_up_silu_w8(Tensor x, Tensor qg, Tensor sg, Tensor qu, Tensor su) -> Tensor");
  m.def("linear(Tensor x, Tensor w) -> Tensor");
  m.def("linear_w8(Tensor x, Tensor q, Tensor scale) -> Tensor");
  m.def("rmsnorm_qkv(Tensor x, Tensor gamma, float eps, Tensor w, int n_q, int n_k) -> Tensor");
  m.def("rmsnorm_gate_up_silu(Tensor x, Tensor gamma, float eps, Tensor wg, Tensor wu) -> Tensor");
  m.def("rmsnorm_qkv_w8(Tensor x, Tensor gamma, float eps, Tensor q, Tensor scale, int n_q, "
        "int n_k) -> Tensor");
  m.def("rmsnorm_gate_up_silu_w8(Tensor x, Tensor gamma, float eps, Tensor qg, Tensor sg, "
        "Tensor qu, Tensor su) -> Tensor");
  m.def("quantize_w8(Tensor w) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(llms_amd, CUDA, m) {
  m.impl("qkv", qkv);
  m.impl("gate_up_silu", gate_up_silu);
  m.impl("qkv_w8", qkv_w8);
  m.impl("gate_up_silu_w8", gate_up_silu_w8);
  m.impl("linear", linear);
  m.impl("linear_w8", linear_w8);
  m.impl("rmsnorm_qkv", rmsnorm_qkv);
  m.impl("rmsnorm_gate_up_silu", rmsnorm_gate_up_silu);
  m.impl("rmsnorm_qkv_w8", rmsnorm_qkv_w8);
  m.impl("rmsnorm_gate_up_silu_w8", rmsnorm_gate_up_silu_w8);
  m.impl("quantize_w8", quantize_w8);
}
