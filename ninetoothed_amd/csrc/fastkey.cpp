// The host side of a Handle call in C++ (ninetoothed_amd._fastkey): its call key, built from the
// tensors' metadata, and the launch of a bound call through a packed entry point.
//
// Handle.__call__ looks a call up among the launchers bound by earlier calls by a key that
// holds, per tensor argument, its dtype, shape, strides, device index and the alignment of
// its data pointer (the data pointer modulo 16).  Built in Python from the tensors'
// attributes that key costs a few microseconds per call, as long as a 512^3 fp32 GEMM;
// here it is one pass over the tensors' C++ metadata.  The key is an opaque bytes object:
// equal bytes mean equal metadata for every tensor, in order.
#include <Python.h>

#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <cstring>
#include <exception>

namespace {

template <typename V>
void put(char*& p, V v) {
  std::memcpy(p, &v, sizeof(V));
  p += sizeof(V);
}

// key(tensors: tuple) -> bytes, or None when an item is not a tensor (the caller's own
// checks then report it).
PyObject* key(PyObject*, PyObject* tensors) {
  if (!PyTuple_Check(tensors)) {
    PyErr_SetString(PyExc_TypeError, "key expects a tuple of tensors");
    return nullptr;
  }
  const Py_ssize_t n = PyTuple_GET_SIZE(tensors);
  // dtype, rank, device type and index, alignment (5 x int16), sizes and strides (int64)
  char buf[2048];
  char* p = buf;
  try {
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* item = PyTuple_GET_ITEM(tensors, i);
    if (!THPVariable_Check(item)) Py_RETURN_NONE;
    const at::Tensor& t = THPVariable_Unpack(item);
    const int64_t dim = t.dim();
    if ((p - buf) + 16 + 16 * dim > (int64_t)sizeof(buf)) Py_RETURN_NONE;
    const c10::Device dev = t.device();
    put<int16_t>(p, (int16_t)t.scalar_type());
    put<int16_t>(p, (int16_t)dim);
    put<int16_t>(p, (int16_t)dev.type());
    put<int16_t>(p, (int16_t)dev.index());
    put<int16_t>(p, (int16_t)(reinterpret_cast<uintptr_t>(t.data_ptr()) & 15));
    const auto sizes = t.sizes();
    const auto strides = t.strides();
    for (int64_t d = 0; d < dim; ++d) put<int64_t>(p, sizes[d]);
    for (int64_t d = 0; d < dim; ++d) put<int64_t>(p, strides[d]);
  }
  } catch (const std::exception&) {  // e.g. a tensor without strides or storage
    Py_RETURN_NONE;
  }
  return PyBytes_FromStringAndSize(buf, p - buf);
}

// call(fn, template, ptr_slots, tensors, value_slots, values) -> int: a library entry point
// `int fn(const int64_t* v)` (the packed forms in nt_mi355x.h) called with `template` (the
// array's constant values, int64 little-endian) after writing each tensor's data pointer
// (0 for None) into its slot and each value into its slot.  Everything per call happens
// here, so a bound launch costs one Python call instead of one conversion per argument.
PyObject* call(PyObject*, PyObject* args) {
  unsigned long long fn = 0;
  Py_buffer tmpl;
  PyObject *ps, *ts, *vs, *vals;
  if (!PyArg_ParseTuple(args, "Ky*O!O!O!O!", &fn, &tmpl, &PyTuple_Type, &ps, &PyTuple_Type, &ts, &PyTuple_Type, &vs,
                        &PyTuple_Type, &vals))
    return nullptr;
  int64_t buf[64];
  const Py_ssize_t n = tmpl.len / (Py_ssize_t)sizeof(int64_t);
  const bool fits = tmpl.len % (Py_ssize_t)sizeof(int64_t) == 0 && n <= 64;
  if (fits) std::memcpy(buf, tmpl.buf, (size_t)tmpl.len);
  PyBuffer_Release(&tmpl);
  if (!fits || fn == 0 || PyTuple_GET_SIZE(ps) != PyTuple_GET_SIZE(ts) || PyTuple_GET_SIZE(vs) != PyTuple_GET_SIZE(vals)) {
    PyErr_SetString(PyExc_ValueError, "call: malformed packed call");
    return nullptr;
  }
  try {
    for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(ps); ++i) {
      const long slot = PyLong_AsLong(PyTuple_GET_ITEM(ps, i));
      PyObject* t = PyTuple_GET_ITEM(ts, i);
      if (slot < 0 || slot >= n) {
        if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "call: slot out of range");
        return nullptr;
      }
      if (t == Py_None) {
        buf[slot] = 0;
      } else if (THPVariable_Check(t)) {
        buf[slot] = (int64_t)reinterpret_cast<uintptr_t>(THPVariable_Unpack(t).data_ptr());
      } else {
        PyErr_SetString(PyExc_TypeError, "call: expected a tensor or None");
        return nullptr;
      }
    }
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
  for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(vs); ++i) {
    const long slot = PyLong_AsLong(PyTuple_GET_ITEM(vs, i));
    const unsigned long long v = PyLong_AsUnsignedLongLongMask(PyTuple_GET_ITEM(vals, i));
    if (PyErr_Occurred()) return nullptr;
    if (slot < 0 || slot >= n) {
      PyErr_SetString(PyExc_ValueError, "call: slot out of range");
      return nullptr;
    }
    buf[slot] = (int64_t)v;
  }
  const int rc = reinterpret_cast<int (*)(const int64_t*)>(static_cast<uintptr_t>(fn))(buf);
  return PyLong_FromLong(rc);
}

PyMethodDef methods[] = {
    {"key", key, METH_O, "Call-key bytes of a tuple of tensors (None if an item is not a tensor)."},
    {"call", call, METH_VARARGS, "Call a packed library entry point with tensors' data pointers and values filled in."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastkey", nullptr, -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__fastkey() { return PyModule_Create(&module); }
