// PyTorch-ROCm extension module `selective_update`: the counterpart of the
// reference's compiled module (csrc/selective_update/bindings.cpp:5-7, host
// code csrc/selective_update/selective_update.cpp:78-130), over the C ABI of
// libssm_mamba_hip.so.
//
//   apply(u, A, B, C, D, delta, delta_bias, h) -> [out, new_h]
//
// keeps the reference's name, argument order, validation messages and
// out-of-place contract (a new state tensor, selective_update.cpp:112-113),
// and adds the device check the reference lacks (a host tensor would reach
// the kernel).  u / delta / B / C may be bfloat16 (one type); A, D,
// delta_bias and h are float32.
//
//   apply_ext(u, A, B, C, D, delta, delta_bias, h, z, delta_softplus,
//             inplace, out) -> [out, new_h]
// adds the fused gate out * silu(z), the softplus switch, optional D /
// delta_bias, an in-place state update (new_h is h) and a caller-given out.
#include "ext_common.h"

#include <vector>

namespace {

using namespace ssm_ext;

std::vector<at::Tensor> apply_impl(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                                   const at::Tensor& C, const OptT& D_, const at::Tensor& delta,
                                   const OptT& bias_, const at::Tensor& h, const OptT& z_,
                                   bool delta_softplus, bool inplace, const OptT& out_) {
  const at::Tensor *D = opt(D_), *bias = opt(bias_), *z = opt(z_), *outp = opt(out_);
  check_dim(u, 2, "u");
  check_dim(A, 2, "A");
  check_dim(B, 2, "B");
  check_dim(C, 2, "C");
  if (D) check_dim(*D, 1, "D");
  check_dim(delta, 2, "delta");
  if (bias) check_dim(*bias, 1, "delta_bias");
  check_dim(h, 3, "h");
  const int64_t batch = h.size(0), dim = h.size(1), nstate = h.size(2);
  TORCH_CHECK(nstate <= 256, "selective_update only supports state_dim <= 256");
  const int io = io_code(u);
  const auto io_t = u.scalar_type();
  check(u, "u", {batch, dim}, "batch_size, num_channels", true, io_t);
  check(A, "A", {dim, nstate}, "num_channels, state_dim", false, io_t);
  check(B, "B", {batch, nstate}, "batch_size, state_dim", true, io_t);
  check(C, "C", {batch, nstate}, "batch_size, state_dim", true, io_t);
  if (D) check(*D, "D", {dim}, "num_channels", false, io_t);
  check(delta, "delta", {batch, dim}, "batch_size, num_channels", true, io_t);
  if (bias) check(*bias, "delta_bias", {dim}, "num_channels", false, io_t);
  check(h, "h", {batch, dim, nstate}, "batch_size, num_channels, state_dim", false, io_t);
  if (z) check(*z, "z", {batch, dim}, "batch_size, num_channels", true, io_t);
  if (outp) check(*outp, "out", {batch, dim}, "batch_size, num_channels", true, io_t);
  c10::hip::HIPGuard guard(u.get_device());
  at::Tensor out = outp ? *outp : at::empty_like(u);
  at::Tensor new_h = inplace ? h : at::empty_like(h);
  ok(ssm_selective_state_update(batch, dim, nstate, io, h.data_ptr<float>(),
                                new_h.data_ptr<float>(), u.data_ptr(), delta.data_ptr(),
                                A.data_ptr<float>(), B.data_ptr(), C.data_ptr(), ptr<float>(D),
                                ptr<float>(bias), ptr(z), delta_softplus ? 1 : 0, out.data_ptr(),
                                stream_of(u)));
  return {out, new_h};
}

std::vector<at::Tensor> apply(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                              const at::Tensor& C, const OptT& D, const at::Tensor& delta,
                              const OptT& delta_bias, const at::Tensor& h) {
  return apply_impl(u, A, B, C, D, delta, delta_bias, h, std::nullopt, true, false, std::nullopt);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  namespace py = pybind11;
  m.doc() = "MI355X selective state update (HIP, gfx950): the reference's selective_update module API";
  m.def("apply", &apply, "Selective update", py::arg("u"), py::arg("A"), py::arg("B"),
        py::arg("C"), py::arg("D"), py::arg("delta"), py::arg("delta_bias"), py::arg("h"));
  m.def("apply_ext", &apply_impl, "Selective update (z gate, softplus switch, in place)",
        py::arg("u"), py::arg("A"), py::arg("B"), py::arg("C"), py::arg("D"), py::arg("delta"),
        py::arg("delta_bias"), py::arg("h"), py::arg("z") = py::none(),
        py::arg("delta_softplus") = true, py::arg("inplace") = false,
        py::arg("out") = py::none());
}
