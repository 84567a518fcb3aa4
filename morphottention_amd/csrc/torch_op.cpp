// torch.ops.morphottention.{forward, backward}: the reference op schemas
// (packages/morphottention/csrc/cuda/binder.cpp:6-15) registered on the CUDA
// dispatch key, which PyTorch-ROCm uses for HIP tensors, plus two ops used by
// the autograd Function that carry the forward projection to the backward and
// take the variant bits (masked diagonal, cube projection).
//
// Checks and messages follow packages/morphottention/csrc/cuda/attention/attention.cpp:9-38,64-91.
// Unlike the reference this layer sets a device guard (the reference launches
// on whatever device is current) and honours `causal`.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <vector>

#include "../../include/morphottention.h"

namespace {

void check(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.scalar_type() == at::kHalf, name, " must be float16");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

struct Shape {
  int64_t B, N, D, H, M;
};

Shape check_inputs(const at::Tensor& X, const at::Tensor& W_phi, const at::Tensor& gate_q, const at::Tensor& gate_k,
                   const at::Tensor& W_V, int64_t H, int64_t cube_m) {
  check(X, "X");
  check(W_phi, "W_phi");
  check(gate_q, "gate_q");
  check(gate_k, "gate_k");
  check(W_V, "W_V");
  TORCH_CHECK(X.dim() == 3, "X must be [B, N, D]");
  const int64_t B = X.size(0), N = X.size(1), D = X.size(2);
  TORCH_CHECK(H > 0 && D % H == 0, "D must be divisible by H");
  const int64_t head_dim_v = D / H;
  TORCH_CHECK(W_phi.dim() == 2 && W_phi.size(0) == D && W_phi.size(1) == H * cube_m, "W_phi must be [D, H*cube_m]");
  TORCH_CHECK(W_V.dim() == 2 && W_V.size(0) == D && W_V.size(1) == H * head_dim_v, "W_V must be [D, H*head_dim_v]");
  TORCH_CHECK(gate_q.dim() == 2 && gate_q.size(0) == H && gate_q.size(1) == cube_m, "gate_q must be [H, cube_m]");
  TORCH_CHECK(gate_k.dim() == 2 && gate_k.size(0) == H && gate_k.size(1) == cube_m, "gate_k must be [H, cube_m]");
  for (const at::Tensor* t : {&W_phi, &gate_q, &gate_k, &W_V})
    TORCH_CHECK(t->device() == X.device(), "all tensors must be on the same device as X");
  return {B, N, D, H, cube_m};
}

morpho_stream_t current_stream(const at::Tensor& X) {
  return reinterpret_cast<morpho_stream_t>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(X.device().index()).stream());
}

// The ABI's mode word: bit 0 causal, the other bits the variant
// (MORPHO_MODE_MASK_DIAG, MORPHO_MODE_PROJ_*, MORPHO_MODE_DETERMINISTIC), which
// only the *_train ops take.
int mode_of(bool causal, int64_t variant) {
  TORCH_CHECK((variant & ~(int64_t)(MORPHO_MODE_MASK_DIAG | MORPHO_MODE_PROJ_HARDTANH01 | MORPHO_MODE_PROJ_IDENTITY |
                                    MORPHO_MODE_DETERMINISTIC)) == 0 &&
                  (variant & (MORPHO_MODE_PROJ_HARDTANH01 | MORPHO_MODE_PROJ_IDENTITY)) !=
                      (MORPHO_MODE_PROJ_HARDTANH01 | MORPHO_MODE_PROJ_IDENTITY),
              "variant must combine MORPHO_MODE_MASK_DIAG (2) and MORPHO_MODE_DETERMINISTIC (32) with at most one "
              "of MORPHO_MODE_PROJ_HARDTANH01 (4) and MORPHO_MODE_PROJ_IDENTITY (8), got ", variant);
  return (causal ? MORPHO_MODE_CAUSAL : 0) | (int)variant;
}

void raise_on(int status, const char* what) {
  TORCH_CHECK(status == MORPHO_OK, "morphottention ", what, " failed (", morpho_status_string(status),
              "): ", morpho_last_error());
}

// A workspace size of 0 means the sizes fail the ABI's validation; report its
// reason (empty dimension, unsupported cube_m or head width, problem too
// large). morpho_forward validates the sizes before it looks at any pointer
// or touches the device, so a call without buffers only returns that error.
void raise_size_error(int64_t B, int64_t N, int64_t D, int64_t H, int64_t M, int mode, const char* what) {
  const int st = morpho_forward(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, B, N, D, H, M, 1.0f,
                                mode, nullptr, 0, nullptr);
  raise_on(st == MORPHO_OK ? MORPHO_ERR_INVALID_ARGUMENT : st, what);
}

std::vector<at::Tensor> forward_impl(const at::Tensor& X, const at::Tensor& W_phi, const at::Tensor& gate_q,
                                     const at::Tensor& gate_k, const at::Tensor& W_V, int64_t H, int64_t cube_m,
                                     double scale, bool causal, int64_t variant, bool keep_workspace) {
  const int mode = mode_of(causal, variant);
  const Shape s = check_inputs(X, W_phi, gate_q, gate_k, W_V, H, cube_m);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(X.device());
  auto out = at::empty_like(X);
  auto lse = at::empty({s.B * H, s.N}, X.options().dtype(at::kFloat));
  const size_t ws_bytes = morpho_forward_workspace_size(s.B, s.N, s.D, s.H, s.M);
  if (ws_bytes == 0) raise_size_error(s.B, s.N, s.D, s.H, s.M, mode, "forward");
  auto ws = at::empty({(int64_t)ws_bytes}, X.options().dtype(at::kByte));
  raise_on(morpho_forward(X.data_ptr(), W_phi.data_ptr(), gate_q.data_ptr(), gate_k.data_ptr(), W_V.data_ptr(),
                          out.data_ptr(), lse.data_ptr<float>(), s.B, s.N, s.D, s.H, s.M, (float)scale, mode,
                          ws.data_ptr(), ws_bytes, current_stream(X)),
           "forward");
  if (keep_workspace) return {out, lse, ws};
  return {out, lse};
}

std::vector<at::Tensor> backward_impl(const at::Tensor& grad_out, const at::Tensor& X, const at::Tensor& W_phi,
                                      const at::Tensor& gate_q, const at::Tensor& gate_k, const at::Tensor& W_V,
                                      const at::Tensor& out, const at::Tensor& lse, const at::Tensor* fwd_ws,
                                      int64_t H, int64_t cube_m, double scale, bool causal, int64_t variant) {
  const int mode = mode_of(causal, variant);
  check(grad_out, "grad_out");
  const Shape s = check_inputs(X, W_phi, gate_q, gate_k, W_V, H, cube_m);
  check(out, "out");
  TORCH_CHECK(lse.is_cuda(), "lse must be a CUDA tensor");
  TORCH_CHECK(lse.scalar_type() == at::kFloat, "lse must be float32");
  TORCH_CHECK(lse.is_contiguous(), "lse must be contiguous");
  TORCH_CHECK(grad_out.sizes() == X.sizes(), "grad_out must match X shape [B, N, D]");
  TORCH_CHECK(out.sizes() == X.sizes(), "out must match X shape [B, N, D]");
  TORCH_CHECK(lse.dim() == 2 && lse.size(0) == s.B * H && lse.size(1) == s.N, "lse must be [B*H, N]");
  TORCH_CHECK(grad_out.device() == X.device() && out.device() == X.device() && lse.device() == X.device() &&
                  (!fwd_ws || fwd_ws->device() == X.device()),
              "all tensors must be on the same device as X");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(X.device());
  const void* fwd_ptr = nullptr;
  if (fwd_ws) {
    const size_t need = morpho_forward_workspace_size(s.B, s.N, s.D, s.H, s.M);
    TORCH_CHECK(fwd_ws->is_cuda() && fwd_ws->scalar_type() == at::kByte && fwd_ws->is_contiguous() &&
                    (size_t)fwd_ws->numel() >= need,
                "workspace must be the uint8 CUDA tensor returned by forward_train for these sizes");
    fwd_ptr = fwd_ws->data_ptr();
  }
  auto dX = at::empty_like(X);
  auto dW_phi = at::empty_like(W_phi);
  auto d_gate_q = at::empty_like(gate_q);
  auto d_gate_k = at::empty_like(gate_k);
  auto dW_V = at::empty_like(W_V);
  const size_t ws_bytes = morpho_backward_workspace_size_for_mode(s.B, s.N, s.D, s.H, s.M, fwd_ptr != nullptr, mode);
  if (ws_bytes == 0) raise_size_error(s.B, s.N, s.D, s.H, s.M, mode, "backward");
  auto ws = at::empty({(int64_t)ws_bytes}, X.options().dtype(at::kByte));
  raise_on(morpho_backward(grad_out.data_ptr(), X.data_ptr(), W_phi.data_ptr(), gate_q.data_ptr(), gate_k.data_ptr(),
                           W_V.data_ptr(), out.data_ptr(), lse.data_ptr<float>(), dX.data_ptr(), dW_phi.data_ptr(),
                           d_gate_q.data_ptr(), d_gate_k.data_ptr(), dW_V.data_ptr(), s.B, s.N, s.D, s.H, s.M,
                           (float)scale, mode, fwd_ptr, ws.data_ptr(), ws_bytes, current_stream(X)),
           "backward");
  return {dX, dW_phi, d_gate_q, d_gate_k, dW_V};
}

std::vector<at::Tensor> op_forward(const at::Tensor& X, const at::Tensor& W_phi, const at::Tensor& gate_q,
                                   const at::Tensor& gate_k, const at::Tensor& W_V, int64_t H, int64_t cube_m,
                                   double scale, bool causal) {
  return forward_impl(X, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal, 0, false);
}

std::vector<at::Tensor> op_forward_train(const at::Tensor& X, const at::Tensor& W_phi, const at::Tensor& gate_q,
                                         const at::Tensor& gate_k, const at::Tensor& W_V, int64_t H, int64_t cube_m,
                                         double scale, bool causal, int64_t variant) {
  return forward_impl(X, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal, variant, true);
}

std::vector<at::Tensor> op_backward(const at::Tensor& grad_out, const at::Tensor& X, const at::Tensor& W_phi,
                                    const at::Tensor& gate_q, const at::Tensor& gate_k, const at::Tensor& W_V,
                                    const at::Tensor& out, const at::Tensor& lse, int64_t H, int64_t cube_m,
                                    double scale, bool causal) {
  return backward_impl(grad_out, X, W_phi, gate_q, gate_k, W_V, out, lse, nullptr, H, cube_m, scale, causal, 0);
}

std::vector<at::Tensor> op_backward_train(const at::Tensor& grad_out, const at::Tensor& X, const at::Tensor& W_phi,
                                          const at::Tensor& gate_q, const at::Tensor& gate_k, const at::Tensor& W_V,
                                          const at::Tensor& out, const at::Tensor& lse, const at::Tensor& workspace,
                                          int64_t H, int64_t cube_m, double scale, bool causal, int64_t variant) {
  return backward_impl(grad_out, X, W_phi, gate_q, gate_k, W_V, out, lse, &workspace, H, cube_m, scale, causal,
                       variant);
}

// ---- soft tropical aggregation (no reference op: the reference defines the
// accumulators of morfology/soft_morph.cuh but never wires them)
void check_tau(const at::Tensor& tau, const at::Tensor& X) {
  TORCH_CHECK(tau.is_cuda() && tau.device() == X.device(), "tau must be a CUDA tensor on the device of X");
  TORCH_CHECK(tau.scalar_type() == at::kFloat && tau.numel() == 1 && tau.is_contiguous(),
              "tau must be one contiguous float32 element");
}

// The soft ops also accept MORPHO_MODE_SOFT_EXACT (16) in `variant`.
int soft_mode_of(bool causal, int64_t variant) {
  TORCH_CHECK((variant & MORPHO_MODE_DETERMINISTIC) == 0,
              "MORPHO_MODE_DETERMINISTIC (32) applies to the softmax backward only");
  return mode_of(causal, variant & ~(int64_t)MORPHO_MODE_SOFT_EXACT) | (int)(variant & MORPHO_MODE_SOFT_EXACT);
}

int sgn_of(int64_t sgn) {
  TORCH_CHECK(sgn == 1 || sgn == -1, "sgn must be +1 (dilation) or -1 (erosion), got ", sgn);
  return (int)sgn;
}

std::vector<at::Tensor> op_soft_forward(const at::Tensor& X, const at::Tensor& W_phi, const at::Tensor& gate_q,
                                        const at::Tensor& gate_k, const at::Tensor& W_V, const at::Tensor& tau,
                                        int64_t H, int64_t cube_m, double scale, bool causal, int64_t sgn,
                                        int64_t variant) {
  const int mode = soft_mode_of(causal, variant);
  const int sg = sgn_of(sgn);
  const Shape s = check_inputs(X, W_phi, gate_q, gate_k, W_V, H, cube_m);
  check_tau(tau, X);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(X.device());
  auto out = at::empty_like(X);
  auto zb = at::empty({s.B * H, s.N, s.D / H}, X.options().dtype(at::kFloat));
  const size_t ws_bytes = morpho_soft_forward_workspace_size(s.B, s.N, s.D, s.H, s.M);
  if (ws_bytes == 0) raise_size_error(s.B, s.N, s.D, s.H, s.M, mode & ~MORPHO_MODE_SOFT_EXACT, "soft_forward");
  auto ws = at::empty({(int64_t)ws_bytes}, X.options().dtype(at::kByte));
  raise_on(morpho_soft_forward(X.data_ptr(), W_phi.data_ptr(), gate_q.data_ptr(), gate_k.data_ptr(), W_V.data_ptr(),
                               tau.data_ptr<float>(), out.data_ptr(), zb.data_ptr<float>(), s.B, s.N, s.D, s.H, s.M,
                               (float)scale, mode, sg, ws.data_ptr(), ws_bytes, current_stream(X)),
           "soft_forward");
  return {out, zb, ws};
}

std::vector<at::Tensor> op_soft_backward(const at::Tensor& grad_out, const at::Tensor& X, const at::Tensor& W_phi,
                                         const at::Tensor& gate_q, const at::Tensor& gate_k, const at::Tensor& W_V,
                                         const at::Tensor& tau, const at::Tensor& zb, const at::Tensor& workspace,
                                         int64_t H, int64_t cube_m, double scale, bool causal, int64_t sgn,
                                         int64_t variant) {
  const int mode = soft_mode_of(causal, variant);
  const int sg = sgn_of(sgn);
  check(grad_out, "grad_out");
  const Shape s = check_inputs(X, W_phi, gate_q, gate_k, W_V, H, cube_m);
  check_tau(tau, X);
  TORCH_CHECK(grad_out.sizes() == X.sizes(), "grad_out must match X shape [B, N, D]");
  TORCH_CHECK(zb.is_cuda() && zb.scalar_type() == at::kFloat && zb.is_contiguous() && zb.dim() == 3 &&
                  zb.size(0) == s.B * H && zb.size(1) == s.N && zb.size(2) == s.D / H,
              "zb must be the float32 [B*H, N, D/H] tensor of soft_forward");
  const size_t need = morpho_soft_forward_workspace_size(s.B, s.N, s.D, s.H, s.M);
  TORCH_CHECK(workspace.is_cuda() && workspace.scalar_type() == at::kByte && workspace.is_contiguous() &&
                  (size_t)workspace.numel() >= need,
              "workspace must be the uint8 CUDA tensor returned by soft_forward for these sizes");
  TORCH_CHECK(grad_out.device() == X.device() && zb.device() == X.device() && workspace.device() == X.device(),
              "all tensors must be on the same device as X");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(X.device());
  auto dX = at::empty_like(X);
  auto dW_phi = at::empty_like(W_phi);
  auto d_gate_q = at::empty_like(gate_q);
  auto d_gate_k = at::empty_like(gate_k);
  auto dW_V = at::empty_like(W_V);
  auto dtau = at::empty_like(tau);
  const size_t ws_bytes = morpho_soft_backward_workspace_size(s.B, s.N, s.D, s.H, s.M, 1);
  auto ws = at::empty({(int64_t)ws_bytes}, X.options().dtype(at::kByte));
  raise_on(morpho_soft_backward(grad_out.data_ptr(), X.data_ptr(), W_phi.data_ptr(), gate_q.data_ptr(),
                                gate_k.data_ptr(), W_V.data_ptr(), tau.data_ptr<float>(), zb.data_ptr<float>(),
                                dX.data_ptr(), dW_phi.data_ptr(), d_gate_q.data_ptr(), d_gate_k.data_ptr(),
                                dW_V.data_ptr(), dtau.data_ptr<float>(), s.B, s.N, s.D, s.H, s.M, (float)scale, mode,
                                sg, workspace.data_ptr(), ws.data_ptr(), ws_bytes, current_stream(X)),
           "soft_backward");
  return {dX, dW_phi, d_gate_q, d_gate_k, dW_V, dtau};
}

}  // namespace

TORCH_LIBRARY(morphottention, m) {
  m.def("forward(Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, Tensor W_V, "
        "int H, int cube_m, float scale, bool causal) -> Tensor[]");
  m.def("backward(Tensor grad_out, Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, "
        "Tensor W_V, Tensor out, Tensor lse, int H, int cube_m, float scale, bool causal) -> Tensor[]");
  m.def("forward_train(Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, Tensor W_V, "
        "int H, int cube_m, float scale, bool causal, int variant=0) -> Tensor[]");
  m.def("backward_train(Tensor grad_out, Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, "
        "Tensor W_V, Tensor out, Tensor lse, Tensor workspace, int H, int cube_m, float scale, bool causal, "
        "int variant=0) -> Tensor[]");
  m.def("soft_forward(Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, Tensor W_V, Tensor tau, "
        "int H, int cube_m, float scale, bool causal, int sgn, int variant=0) -> Tensor[]");
  m.def("soft_backward(Tensor grad_out, Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, Tensor W_V, "
        "Tensor tau, Tensor zb, Tensor workspace, int H, int cube_m, float scale, bool causal, int sgn, "
        "int variant=0) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(morphottention, CUDA, m) {
  m.impl("forward", &op_forward);
  m.impl("backward", &op_backward);
  m.impl("forward_train", &op_forward_train);
  m.impl("backward_train", &op_backward_train);
  m.impl("soft_forward", &op_soft_forward);
  m.impl("soft_backward", &op_soft_backward);
}
