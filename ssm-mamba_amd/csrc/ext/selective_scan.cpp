// PyTorch-ROCm extension module `selective_scan`: the counterpart of the
// reference's compiled module (csrc/selective_scan/bindings.cpp:5-8, host code
// csrc/selective_scan/selective_scan.cpp:212-380), over the C ABI of
// libssm_mamba_hip.so.
//
//   forward(u, A, B, C, D, delta, delta_bias, h_init=None, length=None,
//           padding_side=None) -> [out, h]
//   backward(u, A, B, C, D, delta, delta_bias, h, h_init, dout, dh_last,
//            length=None, padding_side=None)
//       -> [du, dA, dB, dC, dD, ddelta, ddelta_bias, dh_init]
//
// keep the reference's names, argument order, validation messages and
// padding rule ("right" unless given, selective_scan.cpp:248).  `h` is the
// reference's chunk carry: (batch, dim, nchunks, 2 * state_dim) holding
// (prod a, state) pairs per 128-step chunk (nchunks = ceil(seq_len / 128),
// kernel_config.h:4-10, selective_scan.cpp:270-274), so h[..., -1, 1::2] is
// the final state (ops/selective_scan_interface.py:60).  h is a strided view
// of a channel-contiguous (batch, 8 * nchunks, 2 * state_dim, dim) buffer
// that also holds the state after every 16 steps, which the backward reloads
// (coalesced) instead of recomputing the chunks' states; given any other
// tensor of h's shape (a copy), the backward recomputes those states with the
// forward kernel first.
//
// Extensions used by this package's operator layer:
//   fwd_ext(..., z, delta_softplus, save, out_ungated) with save = 0 (final
//       state (batch, dim, state_dim) only), 1 (states after every 16 steps,
//       (batch, nchunks, state_dim, dim)) or 2 (the reference's pairs, as
//       forward);
//   bwd_ext(..., z, delta_softplus, out_ungated) -> the 8 gradients + dz;
//   u / delta / B / C / z / dout may be bfloat16 (all of one type); D and
//   delta_bias may be None; B and C may be batch-strided views.
#include "ext_common.h"

#include <vector>

namespace {

using namespace ssm_ext;

struct Shape {
  int64_t batch, dim, seqlen, nstate, nchunks;
  int io;
  at::ScalarType io_t;
  int64_t bc_stride;  // 0: contiguous B / C
};

// B and C passed as they are: rows contiguous, the rows of a batch row seqlen
// apart, one batch stride shared by B and C (a channel slice of the
// x-projection output is such a view)
bool bc_batch_strided(const at::Tensor& B, const at::Tensor& C) {
  if (B.dim() != 3 || C.dim() != 3 || B.sizes() != C.sizes()) return false;
  const int64_t batch = B.size(0), n = B.size(1), L = B.size(2);
  for (const at::Tensor* x : {&B, &C}) {
    if (x->stride(2) != 1 || (n > 1 && x->stride(1) != L)) return false;
    if (batch > 1 && x->stride(0) < n * L) return false;
  }
  return batch == 1 || B.stride(0) == C.stride(0);
}

Shape validate(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B, const at::Tensor& C,
               const at::Tensor* D, const at::Tensor& delta, const at::Tensor* bias,
               const at::Tensor* h_init, const at::Tensor* length, const at::Tensor* z) {
  check_dim(u, 3, "u");
  check_dim(A, 2, "A");
  check_dim(B, 3, "B");
  check_dim(C, 3, "C");
  if (D) check_dim(*D, 1, "D");
  check_dim(delta, 3, "delta");
  if (bias) check_dim(*bias, 1, "delta_bias");
  if (h_init) check_dim(*h_init, 3, "h_init");
  if (length) check_dim(*length, 1, "length");
  Shape s;
  s.batch = u.size(0);
  s.dim = u.size(1);
  s.seqlen = u.size(2);
  s.nstate = A.size(1);
  s.nchunks = ssm_scan_nchunks(s.seqlen);
  TORCH_CHECK(s.nstate <= 256, "selective_scan only supports state_dim <= 256");
  s.io = io_code(u);
  s.io_t = u.scalar_type();
  const auto io = s.io_t;
  check(u, "u", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len", true, io);
  check(A, "A", {s.dim, s.nstate}, "num_channels, state_dim", false, io);
  const bool strided = bc_batch_strided(B, C);
  check(B, "B", {s.batch, s.nstate, s.seqlen}, "batch_size, state_dim, seq_len", true, io,
        !strided);
  check(C, "C", {s.batch, s.nstate, s.seqlen}, "batch_size, state_dim, seq_len", true, io,
        !strided);
  s.bc_stride = (s.batch == 1 || B.stride(0) == s.nstate * s.seqlen) ? 0 : B.stride(0);
  if (D) check(*D, "D", {s.dim}, "num_channels", false, io);
  check(delta, "delta", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len", true, io);
  if (bias) check(*bias, "delta_bias", {s.dim}, "num_channels", false, io);
  if (h_init)
    check(*h_init, "h_init", {s.batch, s.dim, s.nstate}, "batch_size, num_channels, state_dim",
          false, io);
  if (length) {
    TORCH_CHECK(length->is_cuda(), "length must be a CUDA tensor");
    TORCH_CHECK(length->scalar_type() == at::kLong, "length must be long tensor");
    TORCH_CHECK(length->is_contiguous(), "length must be contiguous");
    TORCH_CHECK(length->size(0) == s.batch, "length must have shape (batch_size,)");
  }
  if (z) check(*z, "z", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len", true, io);
  return s;
}

bool padding_right_of(const std::optional<std::string>& side) {
  const std::string v = side.value_or("right");
  TORCH_CHECK(v == "right" || v == "left", "padding_side must be \"left\" or \"right\" (got \"",
              v, "\")");
  return v == "right";
}

// the same tensor seen with the given sizes and strides (size-1 axes ignored)
bool has_strides(const at::Tensor& t, at::IntArrayRef sizes, at::IntArrayRef strides) {
  if (t.sizes() != sizes) return false;
  for (int64_t i = 0; i < t.dim(); ++i)
    if (sizes[i] > 1 && t.stride(i) != strides[i]) return false;
  return true;
}

// The reference-shaped view (batch, dim, nchunks, 2 * state_dim) of the pair
// buffer (batch, SSM_REF_SLOTS * nchunks, 2 * state_dim, dim): chunk c is slot
// SSM_REF_SLOTS * c + SSM_REF_SLOTS - 1.
std::vector<int64_t> pair_view_strides(const Shape& s) {
  const int64_t K = ssm_scan_ref_nchunks(s.seqlen), N2 = 2 * s.nstate;
  return {SSM_REF_SLOTS * K * N2 * s.dim, 1, SSM_REF_SLOTS * N2 * s.dim, s.dim};
}
int64_t pair_view_offset(const Shape& s) { return (SSM_REF_SLOTS - 1) * 2 * s.nstate * s.dim; }

// Whether h is exactly the view forward returns: its shape, strides and
// offset into a storage of exactly the pair buffer's size.
bool is_pair_view(const at::Tensor& h, const Shape& s) {
  const int64_t K = ssm_scan_ref_nchunks(s.seqlen), N2 = 2 * s.nstate;
  const auto st = pair_view_strides(s);
  return has_strides(h, {s.batch, s.dim, K, N2}, st) && h.storage_offset() == pair_view_offset(s) &&
         h.storage().nbytes() == (size_t)(s.batch * SSM_REF_SLOTS * K * N2 * s.dim) * sizeof(float);
}

std::vector<at::Tensor> fwd_impl(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                                 const at::Tensor& C, const OptT& D_, const at::Tensor& delta,
                                 const OptT& bias_, const OptT& h_init_, const OptT& length_,
                                 const std::optional<std::string>& padding_side, const OptT& z_,
                                 bool delta_softplus, int64_t save, const OptT& out_ungated_) {
  const at::Tensor *D = opt(D_), *bias = opt(bias_), *h_init = opt(h_init_),
                   *length = opt(length_), *z = opt(z_), *yu = opt(out_ungated_);
  const Shape s = validate(u, A, B, C, D, delta, bias, h_init, length, z);
  TORCH_CHECK(save >= 0 && save <= 2, "save must be 0, 1 or 2");
  if (yu) {
    TORCH_CHECK(z, "out_ungated requires z");
    check(*yu, "out_ungated", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len",
          true, s.io_t);
  }
  const bool pr = padding_right_of(padding_side);
  c10::hip::HIPGuard guard(u.get_device());
  at::Tensor out = at::empty_like(u);
  const auto f32 = u.options().dtype(at::kFloat);
  at::Tensor h, store;
  float *h_chunks = nullptr, *h_last = nullptr;
  if (save == 0) {
    h = at::empty({s.batch, s.dim, s.nstate}, f32);
    h_last = h.data_ptr<float>();
  } else if (save == 1) {
    h = at::empty({s.batch, s.nchunks, s.nstate, s.dim}, f32);
    h_chunks = h.data_ptr<float>();
  } else {
    // the pair layout: SSM_REF_SLOTS slots of 16 steps per 128-step chunk,
    // the chunk's (prod a, state) carry in its last slot
    const int64_t K = ssm_scan_ref_nchunks(s.seqlen), N2 = 2 * s.nstate;
    store = at::empty({s.batch, SSM_REF_SLOTS * K, N2, s.dim}, f32);
    h_chunks = store.data_ptr<float>();
    h = store.as_strided({s.batch, s.dim, K, N2}, pair_view_strides(s), pair_view_offset(s));
  }
  const size_t wsb = ssm_scan_fwd_workspace_bytes(s.batch, s.dim, s.seqlen, s.nstate);
  at::Tensor ws = at::empty({(int64_t)wsb}, u.options().dtype(at::kByte));
  ok(ssm_selective_scan_fwd(
      s.batch, s.dim, s.seqlen, s.nstate, s.io, u.data_ptr(), delta.data_ptr(),
      A.data_ptr<float>(), B.data_ptr(), C.data_ptr(), s.bc_stride, ptr<float>(D),
      ptr<float>(bias), ptr<float>(h_init), ptr<int64_t>(length), pr ? 1 : 0, ptr(z),
      delta_softplus ? 1 : 0, out.data_ptr(), ptr(yu), h_chunks, save == 2 ? 1 : 0, h_last,
      ws.data_ptr(), wsb, stream_of(u)));
  return {out, h};
}

std::vector<at::Tensor> bwd_impl(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                                 const at::Tensor& C, const OptT& D_, const at::Tensor& delta,
                                 const OptT& bias_, const at::Tensor& h_, const OptT& h_init_,
                                 const at::Tensor& dout, const OptT& dh_last_,
                                 const OptT& length_,
                                 const std::optional<std::string>& padding_side, const OptT& z_,
                                 bool delta_softplus, const OptT& out_ungated_) {
  const at::Tensor *D = opt(D_), *bias = opt(bias_), *h_init = opt(h_init_),
                   *length = opt(length_), *z = opt(z_), *yu = opt(out_ungated_),
                   *dh_last = opt(dh_last_);
  check_dim(h_, 4, "h");
  check_dim(dout, 3, "dout");
  const Shape s = validate(u, A, B, C, D, delta, bias, h_init, length, z);
  TORCH_CHECK(!(z && !yu), "backward with z requires out_ungated (the forward's ungated output)");
  TORCH_CHECK(!(yu && !z), "out_ungated requires z");
  if (yu)
    check(*yu, "out_ungated", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len",
          true, s.io_t);
  check(dout, "dout", {s.batch, s.dim, s.seqlen}, "batch_size, num_channels, seq_len", true, s.io_t);
  if (dh_last)
    check(*dh_last, "dh_last", {s.batch, s.dim, s.nstate}, "batch_size, num_channels, state_dim",
          false, s.io_t);
  // the chunk carry: the pair view forward returns (its buffer holds the
  // 16-step states), the state layout of fwd_ext(save=1), or another tensor
  // of the pair view's shape (a copy: the states are recomputed)
  TORCH_CHECK(h_.is_cuda(), "h must be a CUDA tensor");
  TORCH_CHECK(h_.scalar_type() == at::kFloat, "h must be float32 tensor");
  const int64_t K = ssm_scan_ref_nchunks(s.seqlen), N2 = 2 * s.nstate, Dm = s.dim;
  const bool pr = padding_right_of(padding_side);
  c10::hip::HIPGuard guard(u.get_device());
  const float* hp = nullptr;
  at::Tensor states;  // recomputed 16-step states
  int pairs;
  if (is_pair_view(h_, s)) {
    hp = h_.data_ptr<float>() - pair_view_offset(s);  // the start of the pair buffer
    pairs = 1;
  } else if (h_.sizes() == at::IntArrayRef({s.batch, Dm, K, N2})) {
    // the carry alone does not hold the 16-step states the backward reloads:
    // the forward kernel recomputes them (the same kernel and inputs, so the
    // same states as the forward that produced h)
    states = at::empty({s.batch, s.nchunks, s.nstate, Dm}, u.options().dtype(at::kFloat));
    at::Tensor scratch_out = at::empty_like(u);
    const size_t fwsb = ssm_scan_fwd_workspace_bytes(s.batch, s.dim, s.seqlen, s.nstate);
    at::Tensor fws = at::empty({(int64_t)fwsb}, u.options().dtype(at::kByte));
    ok(ssm_selective_scan_fwd(
        s.batch, s.dim, s.seqlen, s.nstate, s.io, u.data_ptr(), delta.data_ptr(),
        A.data_ptr<float>(), B.data_ptr(), C.data_ptr(), s.bc_stride, ptr<float>(D),
        ptr<float>(bias), ptr<float>(h_init), ptr<int64_t>(length), pr ? 1 : 0, ptr(z),
        delta_softplus ? 1 : 0, scratch_out.data_ptr(), nullptr, states.data_ptr<float>(), 0,
        nullptr, fws.data_ptr(), fwsb, stream_of(u)));
    hp = states.data_ptr<float>();
    pairs = 0;
  } else {
    TORCH_CHECK(h_.sizes() == at::IntArrayRef({s.batch, s.nchunks, s.nstate, Dm}) &&
                    h_.is_contiguous(),
                "h must have shape (batch_size, num_channels, num_chunks, 2*state_dim) "
                "(num_chunks = ceil(seq_len / 128)), as returned by forward");
    hp = h_.data_ptr<float>();
    pairs = 0;
  }
  at::Tensor du = at::empty_like(u);
  at::Tensor ddelta = at::empty_like(delta);
  at::Tensor dA = at::empty_like(A);
  at::Tensor dB = at::empty(B.sizes(), B.options());
  at::Tensor dC = at::empty(C.sizes(), C.options());
  at::Tensor dD = D ? at::empty_like(*D) : at::Tensor();
  at::Tensor dbias = bias ? at::empty_like(*bias) : at::Tensor();
  at::Tensor dh_init = h_init ? at::empty_like(*h_init) : at::Tensor();
  at::Tensor dz = z ? at::empty_like(*z) : at::Tensor();
  const size_t wsb = ssm_scan_bwd_workspace_bytes(s.batch, s.dim, s.seqlen, s.nstate);
  at::Tensor ws = at::empty({(int64_t)wsb}, u.options().dtype(at::kByte));
  auto dptr = [](at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; };
  ok(ssm_selective_scan_bwd(
      s.batch, s.dim, s.seqlen, s.nstate, s.io, u.data_ptr(), delta.data_ptr(),
      A.data_ptr<float>(), B.data_ptr(), C.data_ptr(), s.bc_stride, ptr<float>(D),
      ptr<float>(bias), ptr<float>(h_init), ptr<int64_t>(length), pr ? 1 : 0, ptr(z), ptr(yu),
      delta_softplus ? 1 : 0, hp, pairs, dout.data_ptr(), ptr<float>(dh_last),
      du.data_ptr(), ddelta.data_ptr(), dA.data_ptr<float>(), dB.data_ptr(), dC.data_ptr(),
      static_cast<float*>(dptr(dD)), static_cast<float*>(dptr(dbias)),
      static_cast<float*>(dptr(dh_init)), dptr(dz), ws.data_ptr(), wsb, stream_of(u)));
  return {du, dA, dB, dC, dD, ddelta, dbias, dh_init, dz};
}

std::vector<at::Tensor> forward(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                                const at::Tensor& C, const OptT& D, const at::Tensor& delta,
                                const OptT& delta_bias, const OptT& h_init, const OptT& length,
                                const std::optional<std::string>& padding_side) {
  return fwd_impl(u, A, B, C, D, delta, delta_bias, h_init, length, padding_side, std::nullopt,
                  true, 2, std::nullopt);
}

std::vector<at::Tensor> backward(const at::Tensor& u, const at::Tensor& A, const at::Tensor& B,
                                 const at::Tensor& C, const OptT& D, const at::Tensor& delta,
                                 const OptT& delta_bias, const at::Tensor& h, const OptT& h_init,
                                 const at::Tensor& dout, const OptT& dh_last, const OptT& length,
                                 const std::optional<std::string>& padding_side) {
  auto r = bwd_impl(u, A, B, C, D, delta, delta_bias, h, h_init, dout, dh_last, length,
                    padding_side, std::nullopt, true, std::nullopt);
  r.pop_back();  // no dz without the gate
  return r;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  namespace py = pybind11;
  m.doc() = "MI355X selective scan (HIP, gfx950): the reference's selective_scan module API";
  m.def("forward", &forward, "Selective scan forward", py::arg("u"), py::arg("A"), py::arg("B"),
        py::arg("C"), py::arg("D"), py::arg("delta"), py::arg("delta_bias"),
        py::arg("h_init") = py::none(), py::arg("length") = py::none(),
        py::arg("padding_side") = py::none());
  m.def("backward", &backward, "Selective scan backward", py::arg("u"), py::arg("A"),
        py::arg("B"), py::arg("C"), py::arg("D"), py::arg("delta"), py::arg("delta_bias"),
        py::arg("h"), py::arg("h_init"), py::arg("dout"), py::arg("dh_last"),
        py::arg("length") = py::none(), py::arg("padding_side") = py::none());
  m.def("fwd_ext", &fwd_impl, "Selective scan forward (z gate, softplus switch, state layouts)",
        py::arg("u"), py::arg("A"), py::arg("B"), py::arg("C"), py::arg("D"), py::arg("delta"),
        py::arg("delta_bias"), py::arg("h_init"), py::arg("length"), py::arg("padding_side"),
        py::arg("z"), py::arg("delta_softplus"), py::arg("save"), py::arg("out_ungated"));
  m.def("bwd_ext", &bwd_impl, "Selective scan backward (z gate, softplus switch)", py::arg("u"),
        py::arg("A"), py::arg("B"), py::arg("C"), py::arg("D"), py::arg("delta"),
        py::arg("delta_bias"), py::arg("h"), py::arg("h_init"), py::arg("dout"),
        py::arg("dh_last"), py::arg("length"), py::arg("padding_side"), py::arg("z"),
        py::arg("delta_softplus"), py::arg("out_ungated"));
  m.attr("CHUNK") = (int)SSM_CHUNK;
}
