// Native host binding of the router's autograd Function (torch C++ extension `moe_mi355._moe_torch`).
//
// The router step is short on the GPU (C2: ~85 us of kernels for fwd + bwd), so its host work shows: the
// Python Function, eight output allocations through Python, the zeroed-workspace lookup and the ctypes
// conversion of ~25 arguments per call add up to more than the kernels on a slow host.  This file does the
// same work in C++: a torch::autograd::Function whose forward allocates the outputs with ATen, takes the
// current HIP stream from c10 and calls moe_router_fwd, and whose backward (run by the autograd engine
// without returning to Python) calls moe_router_bwd.  It calls the same C ABI entry points
// (include/moe_mi355.h) as the ctypes path and launches the same kernels; argument validation with the
// Python error types stays in moe_mi355/router.py.
#include <torch/extension.h>

// In torch's ROCm build GPU tensors carry the device type `cuda`; the HIP guard and stream types that accept
// it are the ones "masquerading as CUDA".
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <hip/hip_runtime_api.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "../../include/moe_mi355.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::Variable;
using torch::autograd::variable_list;

[[noreturn]] void raise_rc(int rc, const char* what) {
  char buf[512];
  buf[0] = 0;
  moe_last_error(buf, sizeof buf);
  if (rc < 0) throw pybind11::value_error(std::string(what) + ": " + buf + " (code " + std::to_string(rc) + ")");
  throw std::runtime_error(std::string(what) + ": " + buf + " (hip error " + std::to_string(rc) + ")");
}

int code_of(const at::Tensor& t) { return t.scalar_type() == at::kBFloat16 ? MOE_BF16 : MOE_F32; }

// The forward's workspace holds a ticket counter that must be zero when a launch starts and that the kernels
// leave at zero: one zero-initialised buffer per (device, stream), reused by every call on that stream (stream
// order serialises them).  Under graph capture each capture takes a fresh slice of a per-device arena instead,
// zeroed and synchronised once outside any capture (on the first eager call): the kernels leave the counter at
// zero after every replay, so that slice serves every replay of its graph, and the graph holds no fill node.
// Captures past the arena's end fall back to a zeroed buffer made inside the capture (a captured fill kernel).
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, at::Tensor> g_ws;
constexpr int64_t kArenaBytes = 32 << 20;
struct CaptureArena {
  at::Tensor buf;
  int64_t used = 0;
};
std::map<int, CaptureArena> g_arena;

at::Tensor fwd_workspace(size_t nbytes, const at::Device& dev, hipStream_t s) {
  const int64_t n = std::max<int64_t>((int64_t)nbytes, 1);
  const auto opts = at::TensorOptions().dtype(at::kByte).device(dev);
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    throw std::runtime_error("moe_router_fwd: hipStreamIsCapturing failed");
  }
  std::lock_guard<std::mutex> lk(g_ws_mu);
  CaptureArena& ar = g_arena[(int)dev.index()];
  if (st != hipStreamCaptureStatusNone) {
    const int64_t n256 = (n + 255) / 256 * 256;
    if (ar.buf.defined() && ar.used + n256 <= kArenaBytes) {
      at::Tensor slice = ar.buf.narrow(0, ar.used, n);
      ar.used += n256;
      return slice;
    }
    return at::zeros({n}, opts);
  }
  if (!ar.buf.defined()) {
    ar.buf = at::zeros({kArenaBytes}, opts);
    if (hipStreamSynchronize(s) != hipSuccess) {  // once: later captures may replay on any stream
      (void)hipGetLastError();
      throw std::runtime_error("moe_router_fwd: hipStreamSynchronize failed");
    }
  }
  auto& buf = g_ws[{(int)dev.index(), s}];
  if (!buf.defined() || buf.numel() < n) buf = at::zeros({n}, opts);
  return buf;
}

struct RouterFn : public torch::autograd::Function<RouterFn> {
  // link_x: x is also returned, as an eighth output, for the layer's expert path to consume.  Its gradient
  // (the expert path's gradient of x) then arrives here as an upstream gradient and is added inside the dx
  // kernel, instead of autograd summing the two contributions to x's gradient in a separate addition.
  static variable_list forward(AutogradContext* ctx, const Variable& x_in, const Variable& gw_in, int64_t k,
                               double aux_coef, double z_coef, const std::optional<Variable>& bias_in, bool link_x) {
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x_in.device());
    const at::Tensor x = x_in.contiguous();
    const at::Tensor gw = gw_in.contiguous();
    const int64_t N = x.size(0), H = x.size(1), E = gw.size(1);
    at::Tensor bias;
    if (bias_in.has_value() && bias_in->defined()) bias = bias_in->detach().to(at::kFloat).contiguous();
    const auto dev = x.device();
    const auto f32 = at::TensorOptions().dtype(at::kFloat).device(dev);
    const auto i64 = at::TensorOptions().dtype(at::kLong).device(dev);
    at::Tensor idx = at::empty({N, k}, i64);
    at::Tensor w = at::empty({N, k}, x.options());
    at::Tensor logits = at::empty({N, E}, f32);
    at::Tensor lse = at::empty({N}, f32);
    at::Tensor cnt = at::empty({E}, i64);
    at::Tensor stats = at::empty({MOE_STATS_HEAD + E}, f32);
    at::Tensor aux = at::empty({}, f32);
    at::Tensor z = at::empty({}, f32);
    if (N == 0) {
      cnt.zero_();
      stats.zero_();
      aux.zero_();
      z.zero_();
    } else {
      const hipStream_t s = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
      const int xdt = code_of(x), wdt = code_of(gw);
      const size_t nbytes = moe_router_fwd_workspace(N, H, E, k, xdt, wdt);
      const at::Tensor ws = fwd_workspace(nbytes, dev, s);
      const int rc = moe_router_fwd(x.data_ptr(), xdt, gw.data_ptr(), wdt,
                                    bias.defined() ? bias.data_ptr<float>() : nullptr, N, H, E, k,
                                    idx.data_ptr<int64_t>(), w.data_ptr(), xdt, logits.data_ptr<float>(),
                                    lse.data_ptr<float>(), cnt.data_ptr<int64_t>(), stats.data_ptr<float>(),
                                    (float)aux_coef, (float)z_coef, aux.data_ptr<float>(), z.data_ptr<float>(),
                                    ws.data_ptr(), nbytes, s);
      if (rc != 0) raise_rc(rc, "moe_router_fwd");
    }
    ctx->save_for_backward({x, gw, logits, idx, cnt});
    ctx->saved_data["aux_coef"] = aux_coef;
    ctx->saved_data["z_coef"] = z_coef;
    ctx->set_materialize_grads(false);
    ctx->mark_non_differentiable({idx, logits, cnt, stats});
    if (link_x) return {idx, w, aux, z, logits, cnt, stats, x_in};
    return {idx, w, aux, z, logits, cnt, stats};
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const bool need_x = ctx->needs_input_grad(0), need_w = ctx->needs_input_grad(1);
    variable_list out(7);
    if (!(need_x || need_w)) return out;
    const auto saved = ctx->get_saved_variables();
    const at::Tensor& x = saved[0];
    const at::Tensor& gw = saved[1];
    const at::Tensor& logits = saved[2];
    const at::Tensor& idx = saved[3];
    const at::Tensor& cnt = saved[4];
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    at::Tensor g_w = grads[1];
    at::Tensor g_aux = grads[2];
    at::Tensor g_z = grads[3];
    // the linked x output's gradient (the expert path's gradient of x), if any
    at::Tensor dx_add;
    if (need_x && grads.size() > 7 && grads[7].defined()) dx_add = grads[7].to(x.scalar_type()).contiguous();
    const float aux_coef = g_aux.defined() ? (float)ctx->saved_data["aux_coef"].toDouble() : 0.f;
    const float z_coef = g_z.defined() ? (float)ctx->saved_data["z_coef"].toDouble() : 0.f;
    int gdt = MOE_F32;
    if (g_w.defined()) {
      g_w = g_w.contiguous();
      if (g_w.scalar_type() != at::kFloat && g_w.scalar_type() != at::kBFloat16) g_w = g_w.to(at::kFloat);
      gdt = code_of(g_w);
    }
    if (g_aux.defined()) g_aux = g_aux.detach().to(at::kFloat).reshape({1}).contiguous();
    if (g_z.defined()) g_z = g_z.detach().to(at::kFloat).reshape({1}).contiguous();
    const int64_t N = x.size(0), H = x.size(1), E = gw.size(1), K = idx.size(1);
    at::Tensor dx = at::empty({N, H}, x.options());
    at::Tensor dw;
    if (N == 0) {
      dw = at::zeros({H, E}, gw.options());
      dx.zero_();
    } else {
      dw = at::empty({H, E}, gw.options());
      const int xdt = code_of(x), wdt = code_of(gw);
      const size_t nbytes = moe_router_bwd_workspace(N, H, E, K, xdt, wdt);
      const at::Tensor ws = at::empty({std::max<int64_t>((int64_t)nbytes, 1)}, x.options().dtype(at::kByte));
      const hipStream_t s = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.device().index()).stream();
      const int rc = moe_router_bwd_acc(x.data_ptr(), xdt, gw.data_ptr(), wdt, logits.data_ptr<float>(),
                                        idx.data_ptr<int64_t>(), g_w.defined() ? g_w.data_ptr() : nullptr, gdt,
                                        cnt.data_ptr<int64_t>(), g_aux.defined() ? g_aux.data_ptr<float>() : nullptr,
                                        g_z.defined() ? g_z.data_ptr<float>() : nullptr, aux_coef, z_coef, N, H, E, K,
                                        dx_add.defined() ? dx_add.data_ptr() : nullptr, dx.data_ptr(), dw.data_ptr(),
                                        ws.data_ptr(), nbytes, s);
      if (rc != 0) raise_rc(rc, "moe_router_bwd");
    }
    if (need_x) out[0] = dx;
    if (need_w) out[1] = dw;
    return out;
  }
};

variable_list router_core(const at::Tensor& x, const at::Tensor& gate_w, int64_t k, double aux_coef,
                          double z_coef, const std::optional<at::Tensor>& bias, bool link_x) {
  return RouterFn::apply(x, gate_w, k, aux_coef, z_coef, bias, link_x);
}

}  // namespace

PYBIND11_MODULE(_moe_torch, m) {
  m.doc() = "Native autograd binding of the fused HIP router (forward and backward over the moe_mi355 C ABI).";
  m.def("router_core", &router_core, "(x, gate_w, k, aux_coef, z_coef, bias) -> (idx, w, aux, z, logits, cnt, stats)",
        pybind11::arg("x"), pybind11::arg("gate_w"), pybind11::arg("k"), pybind11::arg("aux_coef"),
        pybind11::arg("z_coef"), pybind11::arg("bias") = pybind11::none(), pybind11::arg("link_x") = false);
}
