// Host fast path for launch-bound calls (decode shapes): the forward's common case — contiguous
// tensors of one dtype on the current device — validated, allocated and launched in C++, so a
// Python call costs one pybind11 crossing instead of ctypes argument conversion plus three torch
// allocations from Python.  Calls that do not qualify return an empty list and take the general
// Python path (velograd_amd/kernels/__init__.py), which validates and raises.  The kernels are
// the C ABI's (include/velograd_kernels.h); this file only binds them to torch tensors.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "velograd_kernels.h"

namespace {

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return VELOGRAD_DTYPE_F32;
    case at::kHalf: return VELOGRAD_DTYPE_F16;
    case at::kBFloat16: return VELOGRAD_DTYPE_BF16;
    default: return -1;
  }
}

// [y, h, inv_rms] of velograd_rmsnorm_residual_fwd (min_mean_sq == 0) or velograd_rmsnorm_fwd,
// with h the very tensor x when residual is None; [] when the call does not qualify.
std::vector<at::Tensor> forward(const at::Tensor& x, const c10::optional<at::Tensor>& residual,
                                const c10::optional<at::Tensor>& weight, double eps,
                                double min_mean_sq) {
  const int32_t code = dtype_code(x.scalar_type());
  if (code < 0 || !x.is_cuda() || x.dim() == 0 || !x.is_contiguous() || x.numel() == 0) return {};
  if (x.get_device() != c10::hip::current_device()) return {};
  const int64_t d = x.size(-1);
  const int64_t rows = x.numel() / d;
  if (residual.has_value()) {
    const at::Tensor& r = *residual;
    if (r.scalar_type() != x.scalar_type() || !r.is_contiguous() || r.sizes() != x.sizes() ||
        r.device() != x.device())
      return {};
  }
  int32_t wcode = code;
  if (weight.has_value()) {
    const at::Tensor& w = *weight;
    if (w.dim() != 1 || w.size(0) != d || !w.is_contiguous() || w.device() != x.device())
      return {};
    wcode = dtype_code(w.scalar_type());
    if (wcode != code && wcode != VELOGRAD_DTYPE_F32) return {};
  }
  at::Tensor y = at::empty_like(x);
  at::Tensor h = residual.has_value() ? at::empty_like(x) : x;
  std::vector<int64_t> stat(x.sizes().begin(), x.sizes().end() - 1);
  stat.push_back(1);
  at::Tensor inv = at::empty(stat, x.options().dtype(at::kFloat));
  void* stream = c10::hip::getCurrentHIPStream(x.get_device()).stream();
  const void* rp = residual.has_value() ? residual->data_ptr() : nullptr;
  const void* wp = weight.has_value() ? weight->data_ptr() : nullptr;
  void* hp = residual.has_value() ? h.data_ptr() : nullptr;
  // Any nonzero floor (a negative or NaN one included) goes to the entry point that checks it.
  const int32_t rc =
      min_mean_sq != 0.0
          ? velograd_rmsnorm_fwd(x.data_ptr(), rp, wp, y.data_ptr(), hp, inv.data_ptr<float>(),
                                 rows, d, d, d, d, d, code, wcode, (float)eps, (float)min_mean_sq,
                                 stream)
          : velograd_rmsnorm_residual_fwd(x.data_ptr(), rp, wp, y.data_ptr(), hp,
                                          inv.data_ptr<float>(), rows, d, d, d, d, d, code, wcode,
                                          (float)eps, stream);
  if (rc != 0) {
    const std::string msg = std::string("velograd_rmsnorm forward failed (status ") +
                            std::to_string(rc) + "): " + velograd_kernels_last_error();
    if (rc == VELOGRAD_ERR_UNSUPPORTED_DTYPE) throw pybind11::type_error(msg);
    if (rc < 0) throw pybind11::value_error(msg);
    throw std::runtime_error(msg);
  }
  return {y, h, inv};
}

}  // namespace

PYBIND11_MODULE(_fastpath, m) {
  m.doc() = "C++ fast path of the fused RMSNorm + residual forward for launch-bound calls";
  m.def("forward", &forward, "forward(x, residual, weight, eps, min_mean_sq) -> [y, h, inv_rms]",
        pybind11::arg("x"), pybind11::arg("residual"), pybind11::arg("weight"),
        pybind11::arg("eps"), pybind11::arg("min_mean_sq"));
}
