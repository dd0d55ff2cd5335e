// Host-side argument handling for the Python layer (a CPython extension built against torch).
//
// The LMCache and HiCache entry points take lists of cache tensors, one per
// layer and K/V plane (64 for a 32-layer model).  Checking each tensor's type,
// shape, dtype, device and contiguity and collecting its address costs about
// six Python attribute reads per tensor, which made a 256-token LMCache call
// host-bound (about 65 us of host time against 12 us of device time on
// MI355X).  These helpers do the same checks in one C++ pass and return the
// addresses packed as uint64 values for the C ABI of libmusa_aiter_kv_hip.so.
// The Python layer keeps every message and the order in which the checks fail.
// For host <-> device copy batches, int64_column reads the caller's lists of
// offsets and sizes (thousands of ints) into int64 columns and object_index
// numbers the few distinct tensors its entries name.
#include <torch/extension.h>

#include <cstdint>
#include <unordered_map>
#include <vector>

namespace py = pybind11;

namespace {

// Status codes of check_tensors, in the order the checks run for each tensor.
constexpr int kOk = 0, kShape = 1, kDtype = 2, kDevice = 3;

py::bytes pack(const std::vector<uint64_t>& v) {
  return py::bytes(reinterpret_cast<const char*>(v.data()), v.size() * sizeof(uint64_t));
}

// For the tensors in `items`, in order: the first whose type or shape is wrong (not a tensor,
// or sizes != `shape` when `shape` is not None), whose dtype differs from `like`'s, or whose device
// differs from `like`'s.  Returns (status, index of that tensor or -1, index of the first
// non-contiguous tensor or -1, their data pointers packed as uint64; empty unless status is kOk).
py::tuple check_tensors(const py::sequence& items, const py::object& shape, const at::Tensor& like) {
  const py::ssize_t n = py::len(items);
  std::vector<int64_t> want;
  const bool check_shape = !shape.is_none();
  if (check_shape)
    for (const auto& v : shape) want.push_back(v.cast<int64_t>());
  const at::ScalarType dtype = like.scalar_type();
  const at::Device device = like.device();
  std::vector<uint64_t> ptrs;
  ptrs.reserve(static_cast<size_t>(n));
  int64_t noncontig = -1;
  for (py::ssize_t i = 0; i < n; ++i) {
    PyObject* obj = PyList_Check(items.ptr()) ? PyList_GET_ITEM(items.ptr(), i) : nullptr;
    py::object held;
    if (obj == nullptr) {
      held = items[i];
      obj = held.ptr();
    }
    if (!THPVariable_Check(obj)) return py::make_tuple(kShape, i, noncontig, py::bytes());
    const at::Tensor& t = THPVariable_Unpack(obj);
    if (check_shape && t.sizes() != at::IntArrayRef(want)) return py::make_tuple(kShape, i, noncontig, py::bytes());
    if (t.scalar_type() != dtype) return py::make_tuple(kDtype, i, noncontig, py::bytes());
    if (t.device() != device) return py::make_tuple(kDevice, i, noncontig, py::bytes());
    if (noncontig < 0 && !t.is_contiguous()) noncontig = i;
    ptrs.push_back(reinterpret_cast<uint64_t>(t.data_ptr()));
  }
  return py::make_tuple(kOk, -1, noncontig, pack(ptrs));
}

// Addresses base + i * outer_stride + j * inner_stride for i < outer_n, j < inner_n (row-major),
// packed as uint64: the (axis, layer) planes of an LMCache buffer.
py::bytes strided_table(uint64_t base, int64_t outer_stride, int64_t outer_n, int64_t inner_stride, int64_t inner_n) {
  std::vector<uint64_t> v;
  v.reserve(static_cast<size_t>(outer_n > 0 && inner_n > 0 ? outer_n * inner_n : 0));
  for (int64_t i = 0; i < outer_n; ++i)
    for (int64_t j = 0; j < inner_n; ++j)
      v.push_back(base + static_cast<uint64_t>(i * outer_stride + j * inner_stride));
  return pack(v);
}

// The items of a list or tuple of Python ints packed as int64, or None when an item is not an exact
// int (bools and other int subclasses included) or lies outside (-2^61, 2^61): the batch-copy plan
// then checks the items one by one, which reports the reference's error or keeps large values
// exact.  Reading them here takes about 5 ns per item, numpy.fromiter about 30 ns.
py::object int64_column(const py::handle& items) {
  PyObject* const seq = items.ptr();
  if (!PyList_Check(seq) && !PyTuple_Check(seq)) return py::none();
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  PyObject** const item = PySequence_Fast_ITEMS(seq);
  constexpr long long kLimit = 1LL << 61;
  std::vector<int64_t> v(static_cast<size_t>(n));
  for (Py_ssize_t i = 0; i < n; ++i) {
    if (!PyLong_CheckExact(item[i])) return py::none();
    int overflow = 0;
    const long long x = PyLong_AsLongLongAndOverflow(item[i], &overflow);
    if (overflow != 0 || x >= kLimit || x <= -kLimit) return py::none();
    v[static_cast<size_t>(i)] = x;
  }
  return py::bytes(reinterpret_cast<const char*>(v.data()), v.size() * sizeof(int64_t));
}

// For the items of `first` and then `second` (lists or tuples), the index of each among their distinct
// objects by identity, numbered in order of first appearance, packed as int64, and the list of those
// objects.  A copy batch names a few tensors thousands of times; this replaces reading every id()
// into numpy and sorting them.
py::tuple object_index(const py::handle& first, const py::handle& second) {
  for (const py::handle& seq : {first, second})
    if (!PyList_Check(seq.ptr()) && !PyTuple_Check(seq.ptr())) throw py::type_error("expected a list or tuple");
  const Py_ssize_t n1 = PySequence_Fast_GET_SIZE(first.ptr()), n2 = PySequence_Fast_GET_SIZE(second.ptr());
  std::vector<int64_t> index;
  index.reserve(static_cast<size_t>(n1 + n2));
  std::unordered_map<PyObject*, int64_t> seen;
  py::list distinct;
  PyObject* last = nullptr;
  int64_t last_index = -1;
  for (const py::handle& seq : {first, second}) {
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq.ptr());
    PyObject** const item = PySequence_Fast_ITEMS(seq.ptr());
    for (Py_ssize_t i = 0; i < n; ++i) {
      PyObject* const o = item[i];
      if (o != last) {
        const auto found = seen.emplace(o, static_cast<int64_t>(seen.size()));
        if (found.second) distinct.append(py::reinterpret_borrow<py::object>(o));
        last = o;
        last_index = found.first->second;
      }
      index.push_back(last_index);
    }
  }
  return py::make_tuple(py::bytes(reinterpret_cast<const char*>(index.data()), index.size() * sizeof(int64_t)),
                        distinct);
}

}  // namespace

PYBIND11_MODULE(_kv_host, m) {
  m.doc() = "Host-side tensor checks and address tables for the MI355X KV path";
  m.def("check_tensors", &check_tensors, py::arg("items"), py::arg("shape"), py::arg("like"));
  m.def("strided_table", &strided_table);
  m.def("int64_column", &int64_column, py::arg("items"));
  m.def("object_index", &object_index, py::arg("first"), py::arg("second"));
  m.attr("OK") = static_cast<int>(kOk);
  m.attr("SHAPE") = static_cast<int>(kShape);
  m.attr("DTYPE") = static_cast<int>(kDtype);
  m.attr("DEVICE") = static_cast<int>(kDevice);
}
