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

#include "musa_aiter_kv_hip.h"

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

// One LMCache 2 x NL row copy (lmcache_kv_paged_to_buffer_two_x_nl / _buffer_to_paged_two_x_nl)
// checked and launched in one pass: the K/V layer caches [NB, BS, NH, HS] of `kvcaches` (a list of
// two lists) <-> memory [2, NL, M, NH*HS], through musa_aiter_hip_copy_rows_packed (`entry`, its
// address) on `stream`.  Returns -1, having launched nothing, unless every argument is one the fast
// path takes as is: a CUDA memory tensor on the current device (`device`) with contiguous rows and
// dtype float16 / bfloat16 / float32, the reference's contract shapes, contiguous caches of
// memory's dtype and device, and a contiguous one-dimensional int64 slot tensor on that device; the
// Python layer then runs its own checks, which raise the reference's errors.  Otherwise returns the
// HIP status of the launch.  `claims`: address of the scatter's musa_aiter_hip_claims (0 for a
// gather).  Device-resident slots are not range-checked, as in the reference (the kernels skip
// slots outside the caches).
int64_t two_x_nl_rows(const py::handle& kvcaches, const py::handle& memory_obj, const py::handle& slots_obj,
                      int64_t skip, int64_t block_size, int64_t num_heads, int64_t head_size, bool scatter,
                      uint64_t entry, uint64_t claims, uint64_t stream, int64_t device) {
  constexpr int64_t kNo = -1;
  if (!THPVariable_Check(memory_obj.ptr()) || !THPVariable_Check(slots_obj.ptr())) return kNo;
  const at::Tensor& mem = THPVariable_Unpack(memory_obj.ptr());
  const at::Tensor& slots = THPVariable_Unpack(slots_obj.ptr());
  if (!mem.is_cuda() || mem.device().index() != device || mem.dim() != 4 || mem.size(0) != 2) return kNo;
  const at::ScalarType dt = mem.scalar_type();
  if (dt != at::kHalf && dt != at::kBFloat16 && dt != at::kFloat) return kNo;
  if (block_size <= 0 || num_heads <= 0 || head_size <= 0 || mem.size(3) != num_heads * head_size) return kNo;
  if (mem.stride(3) != 1 && mem.size(3) != 1) return kNo;
  if (slots.scalar_type() != at::kLong || slots.dim() != 1 || !slots.is_contiguous() || slots.device() != mem.device())
    return kNo;
  PyObject* const groups = kvcaches.ptr();
  if (!PyList_Check(groups) || PyList_GET_SIZE(groups) != 2) return kNo;
  PyObject* const kl = PyList_GET_ITEM(groups, 0);
  PyObject* const vl = PyList_GET_ITEM(groups, 1);
  if (!PyList_Check(kl) || !PyList_Check(vl)) return kNo;
  const Py_ssize_t nl = PyList_GET_SIZE(kl);
  if (nl <= 0 || PyList_GET_SIZE(vl) != nl || mem.size(1) != nl) return kNo;
  const int64_t t = slots.size(0);
  const int64_t m = mem.size(2);
  if (skip < 0 || (!scatter && skip != 0) || skip + t > m) return kNo;
  if (nl > 64) return kNo;  // the plane tables below hold 2 x 64 planes
  uint64_t caches[128], buffer[128];
  int64_t nb = -1;
  for (int axis = 0; axis < 2; ++axis) {
    PyObject* const grp = axis == 0 ? kl : vl;
    for (Py_ssize_t l = 0; l < nl; ++l) {
      PyObject* const obj = PyList_GET_ITEM(grp, l);
      if (!THPVariable_Check(obj)) return kNo;
      const at::Tensor& c = THPVariable_Unpack(obj);
      if (c.dim() != 4) return kNo;
      if (nb < 0) nb = c.size(0);
      if (nb <= 0 || c.size(0) != nb || c.size(1) != block_size || c.size(2) != num_heads || c.size(3) != head_size ||
          c.scalar_type() != dt || c.device() != mem.device() || !c.is_contiguous())
        return kNo;
      caches[axis * nl + l] = reinterpret_cast<uint64_t>(c.data_ptr());
    }
  }
  const int64_t elt = mem.element_size();
  const int64_t row = num_heads * head_size * elt;
  const uint64_t base = reinterpret_cast<uint64_t>(mem.data_ptr());
  for (int axis = 0; axis < 2; ++axis)
    for (Py_ssize_t l = 0; l < nl; ++l)
      buffer[axis * nl + l] = base + static_cast<uint64_t>((axis * mem.stride(0) + l * mem.stride(1)) * elt);
  const int64_t token_stride = (m > 1 ? mem.stride(2) : mem.size(3)) * elt;
  if (t == 0 && scatter) return 0;
  musa_aiter_hip_copy_rows_call call{};
  call.num_planes = 2 * nl;
  call.num_tokens = t;
  call.row_bytes = row;
  if (scatter) {
    call.src_planes = buffer;
    call.dst_planes = caches;
    call.dst_idx = static_cast<const int64_t*>(slots.data_ptr());
    call.num_rows_out = t;
    call.src_offset = skip;
    call.src_rows = m;
    call.dst_rows = nb * block_size;
    call.src_stride = token_stride;
    call.dst_stride = row;
    call.dedupe = 1;
    call.claims = reinterpret_cast<const musa_aiter_hip_claims*>(claims);
  } else {
    call.src_planes = caches;
    call.dst_planes = buffer;
    call.src_idx = static_cast<const int64_t*>(slots.data_ptr());
    call.num_rows_out = m;
    call.src_rows = nb * block_size;
    call.dst_rows = m;
    call.src_stride = row;
    call.dst_stride = token_stride;
    call.zero_invalid = 1;
  }
  using Entry = int (*)(const musa_aiter_hip_copy_rows_call*, void*);
  return reinterpret_cast<Entry>(entry)(&call, reinterpret_cast<void*>(stream));
}

}  // namespace

PYBIND11_MODULE(_kv_host, m) {
  m.doc() = "Host-side tensor checks and address tables for the MI355X KV path";
  m.def("check_tensors", &check_tensors, py::arg("items"), py::arg("shape"), py::arg("like"));
  m.def("strided_table", &strided_table);
  m.def("int64_column", &int64_column, py::arg("items"));
  m.def("object_index", &object_index, py::arg("first"), py::arg("second"));
  m.def("two_x_nl_rows", &two_x_nl_rows);
  m.attr("OK") = static_cast<int>(kOk);
  m.attr("SHAPE") = static_cast<int>(kShape);
  m.attr("DTYPE") = static_cast<int>(kDtype);
  m.attr("DEVICE") = static_cast<int>(kDevice);
}
