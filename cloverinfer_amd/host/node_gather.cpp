// node_gather.cpp - the "gpu" AttentionNode's payload gather, in native code.
//
// The node receives a decode batch as one small host tensor per item and
// payload (query [Hq, D], key and value [Hkv, D], src/core/nodes.py:203-216,
// src/core/model_adapter.py:382-386); the backend stages all of them in one
// pinned buffer and uploads it with one copy. torch.stack of a list costs
// about 0.3 us per tensor in its checks and dispatch; this module checks the
// same properties through torch's C++ API for some tens of nanoseconds per
// tensor and copies the rows with a parallel memcpy. It is host plumbing of
// the Python backend (torch types are fine here); the paged-attention C ABI
// (include/clover_attn.h) does not depend on it.
#include <torch/extension.h>

#include <ATen/Parallel.h>

#include <algorithm>
#include <cstring>
#include <vector>

namespace {

// Copies ts[i] (each a contiguous CPU tensor of dst's dtype with
// dst.size(1) elements) to row i of dst ([n, row] contiguous CPU); returns
// true. Returns false, having written nothing, when any element of ts is not
// such a tensor (the caller then takes its general path).
bool gather_rows(py::list ts, at::Tensor dst) {
  const int64_t n = (int64_t)PyList_GET_SIZE(ts.ptr());
  if (dst.dim() != 2 || dst.size(0) != n || !dst.is_contiguous() ||
      dst.device().type() != at::kCPU)
    return false;
  const int64_t row = dst.size(1);
  const at::ScalarType dt = dst.scalar_type();
  std::vector<const char *> src((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    PyObject *obj = PyList_GET_ITEM(ts.ptr(), i);  // borrowed
    if (!THPVariable_Check(obj)) return false;
    const at::Tensor &x = THPVariable_Unpack(obj);
    if (x.device().type() != at::kCPU || x.scalar_type() != dt || x.numel() != row ||
        !x.is_contiguous() || x.is_conj() || x.is_neg())
      return false;
    src[(size_t)i] = static_cast<const char *>(x.const_data_ptr());
  }
  const size_t bytes = (size_t)row * dst.element_size();
  char *out = static_cast<char *>(dst.data_ptr());
  at::parallel_for(0, n, 16, [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) std::memcpy(out + (size_t)i * bytes, src[(size_t)i], bytes);
  });
  return true;
}

// Copies the contiguous CPU tensor src into dst (contiguous CPU, same dtype
// and element count) with a parallel memcpy; returns false, having written
// nothing, otherwise.
bool copy_rows(at::Tensor src, at::Tensor dst) {
  if (src.device().type() != at::kCPU || dst.device().type() != at::kCPU ||
      src.scalar_type() != dst.scalar_type() || src.numel() != dst.numel() ||
      !src.is_contiguous() || !dst.is_contiguous() || src.is_conj() || src.is_neg())
    return false;
  const int64_t bytes = src.numel() * (int64_t)src.element_size();
  const char *in = static_cast<const char *>(src.const_data_ptr());
  char *out = static_cast<char *>(dst.data_ptr());
  constexpr int64_t kChunk = 64 << 10;
  at::parallel_for(0, (bytes + kChunk - 1) / kChunk, 1, [&](int64_t b, int64_t e) {
    const int64_t lo = b * kChunk, hi = std::min(bytes, e * kChunk);
    std::memcpy(out + lo, in + lo, (size_t)(hi - lo));
  });
  return true;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "payload gather of the gpu AttentionNode backend";
  m.def("gather_rows", &gather_rows, "copy a list of CPU tensors into the rows of dst");
  m.def("copy_rows", &copy_rows, "copy a contiguous CPU tensor into dst in parallel");
}
