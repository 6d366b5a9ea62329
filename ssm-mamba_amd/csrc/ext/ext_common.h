// Shared host code of the two PyTorch-ROCm extension modules (selective_scan,
// selective_update): validation with the reference's messages, the device
// guard and current stream, and the call into the C ABI of
// libssm_mamba_hip.so (include/ssm_mamba.h).  No device code lives here.
#pragma once

#include <torch/extension.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <optional>
#include <string>

#include "../../../include/ssm_mamba.h"

namespace ssm_ext {

using OptT = std::optional<at::Tensor>;

inline const at::Tensor* opt(const OptT& t) { return (t.has_value() && t->defined()) ? &*t : nullptr; }

template <typename T = void>
inline T* ptr(const at::Tensor* t) {
  return t ? static_cast<T*>(t->data_ptr()) : nullptr;
}

// "<name> must be a <n>D tensor" (csrc/selective_scan/selective_scan.cpp:29-31)
inline void check_dim(const at::Tensor& x, int64_t n, const char* name) {
  TORCH_CHECK(x.dim() == n, name, " must be a ", n, "D tensor");
}

// The reference's CHECK (csrc/selective_scan/selective_scan.cpp:15-27): device,
// element type, contiguity, shape -- in that order and with its wording.
// Streamed tensors may be float32 or bfloat16 here (one type per call).
inline void check(const at::Tensor& x, const char* name, at::IntArrayRef shape,
                  const char* shape_txt, bool stream_dtype, at::ScalarType io,
                  bool need_contig = true) {
  TORCH_CHECK(x.is_cuda(), name, " must be a CUDA tensor");
  if (stream_dtype) {
    TORCH_CHECK(x.scalar_type() == io, name, " must be ",
                io == at::kFloat ? "float32" : "bfloat16", " tensor (the dtype of u)");
  } else {
    TORCH_CHECK(x.scalar_type() == at::kFloat, name, " must be float32 tensor");
  }
  if (need_contig) TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.sizes() == shape, name, " must have shape (", shape_txt, ")");
}

inline int io_code(const at::Tensor& u) {
  TORCH_CHECK(u.is_cuda(), "u must be a CUDA tensor");
  TORCH_CHECK(u.scalar_type() == at::kFloat || u.scalar_type() == at::kBFloat16,
              "u must be float32 or bfloat16 tensor");
  return u.scalar_type() == at::kBFloat16 ? SSM_BF16 : SSM_F32;
}

inline void ok(int rc) {
  TORCH_CHECK(rc == SSM_OK, ssm_last_error());
}

inline void* stream_of(const at::Tensor& x) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(x.get_device()).stream());
}

}  // namespace ssm_ext
