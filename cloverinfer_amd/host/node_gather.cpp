// node_gather.cpp - the "gpu" AttentionNode's batch check and payload gather,
// in native code.
//
// The node receives a decode batch as a list of item dicts with one small
// host tensor per payload (query [Hq, D], key and value [Hkv, D],
// src/core/nodes.py:203-216, src/core/model_adapter.py:382-386); the backend
// checks that the batch is one layer over distinct requests (parse_batch: one
// pass over the dicts instead of several), then stages all payloads in one
// pinned buffer and uploads it with one copy. torch.stack of a list costs
// about 0.3 us per tensor in its checks and dispatch; this module checks the
// same properties through torch's C++ API for some tens of nanoseconds per
// tensor and copies the rows with a parallel memcpy. It is host plumbing of
// the Python backend (torch types are fine here); the paged-attention C ABI
// (include/clover_attn.h) does not depend on it.
#include <torch/extension.h>

#include <ATen/Parallel.h>
#include <pybind11/numpy.h>

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

// The item fields, interned once.
PyObject *key(const char *name) {
  PyObject *k = PyUnicode_InternFromString(name);
  if (k == nullptr) throw py::error_already_set();
  return k;  // kept for the life of the process
}

// One pass over a decode batch (a list of item dicts) for the backend's
// common case: every item of one layer and one score scale (compared as the
// backend's sets compare them), each naming a distinct known request.
// Returns (layer, scale, requests, rows, first, queries, keys, values) with
// rows an int64 array of the requests' table rows and first the row they run
// consecutively from (-1 when they do not), or None whenever the batch is not
// that case (an item that is no dict or lacks a field, an unknown request
// id, two items of one request, mixed layers or scales): the backend's
// general path then takes it and raises its own errors. Errors raised by the
// lookups themselves (an unhashable id) propagate.
py::object parse_batch(py::list items, py::dict requests) {
  static PyObject *const k_layer = key("layer_idx"), *const k_scale = key("score_scale"),
                         *const k_rid = key("request_id"), *const k_q = key("query"),
                         *const k_k = key("key"), *const k_v = key("value"), *const k_row = key("row");
  PyObject *lst = items.ptr();
  const Py_ssize_t n = PyList_GET_SIZE(lst);
  if (n == 0) return py::none();
  py::list reqs(n), qs(n), ks(n), vs(n);
  py::array_t<int64_t> rows(n);
  int64_t *r = rows.mutable_data();
  py::object one = py::float_(1.0);
  py::object layer0, scale0;  // owned: the comparisons below may run Python code
  auto get = [](PyObject *d, PyObject *k) {
    PyObject *x = PyDict_GetItemWithError(d, k);  // borrowed
    if (x == nullptr && PyErr_Occurred()) throw py::error_already_set();
    return x;
  };
  auto same = [](PyObject *a, PyObject *b) {
    const int eq = PyObject_RichCompareBool(a, b, Py_EQ);
    if (eq < 0) throw py::error_already_set();
    return eq == 1;
  };
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject *it = PyList_GET_ITEM(lst, i);
    if (!PyDict_Check(it)) return py::none();
    PyObject *layer = get(it, k_layer), *scale = get(it, k_scale), *rid = get(it, k_rid);
    PyObject *q = get(it, k_q), *k = get(it, k_k), *v = get(it, k_v);
    if (!layer || !rid || !q || !k || !v) return py::none();
    if (scale == nullptr) scale = one.ptr();
    if (i == 0) {
      layer0 = py::reinterpret_borrow<py::object>(layer);
      scale0 = py::reinterpret_borrow<py::object>(scale);
    } else if (!same(layer, layer0.ptr()) || !same(scale, scale0.ptr())) {
      return py::none();
    }
    PyObject *req = get(requests.ptr(), rid);
    if (req == nullptr) return py::none();
    py::object row = py::reinterpret_steal<py::object>(PyObject_GetAttr(req, k_row));
    if (!row) throw py::error_already_set();
    const long long rv = PyLong_AsLongLong(row.ptr());
    if (rv == -1 && PyErr_Occurred()) throw py::error_already_set();
    r[i] = rv;
    PyList_SET_ITEM(reqs.ptr(), i, (Py_INCREF(req), req));
    PyList_SET_ITEM(qs.ptr(), i, (Py_INCREF(q), q));
    PyList_SET_ITEM(ks.ptr(), i, (Py_INCREF(k), k));
    PyList_SET_ITEM(vs.ptr(), i, (Py_INCREF(v), v));
  }
  bool consecutive = true;
  for (Py_ssize_t i = 1; i < n && consecutive; ++i) consecutive = r[i] == r[0] + i;
  if (!consecutive) {  // consecutive rows are distinct; others are checked
    std::vector<int64_t> sorted(r, r + n);
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) return py::none();
  }
  return py::make_tuple(layer0, scale0, reqs, rows, consecutive ? r[0] : (int64_t)-1, qs, ks,
                        vs);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "payload gather of the gpu AttentionNode backend";
  m.def("gather_rows", &gather_rows, "copy a list of CPU tensors into the rows of dst");
  m.def("copy_rows", &copy_rows, "copy a contiguous CPU tensor into dst in parallel");
  m.def("parse_batch", &parse_batch, "one pass over a uniform decode batch of item dicts");
}
