// CPython binding of the VMM allocator's hot path: ensure_resident and the DLPack export behind
// ResidentHandle.as_tensor, as the reference binds them with pyo3 (vmm_src/python.rs:137-221,
// handle.rs:65-110). Each is one C call from Python with no ctypes argument conversion, no ctypes
// objects and no trip through ctypes.pythonapi for the capsule; stagehand_amd.vmm builds the
// Python objects around them. Errors come back as the negated status (a pointer is never
// negative), and the Python side raises through stagehand_amd._native.check, which reads
// sh_last_error on the same thread.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <cstdint>

#include "stagehand_native.h"

namespace {

// The capsule of an export that no consumer took: the DLPack contract renames a consumed
// capsule ("used_dltensor"), so a capsule still named "dltensor" owns its tensor.
void capsule_free(PyObject* cap) {
  if (PyCapsule_IsValid(cap, "dltensor")) {
    auto* t = static_cast<sh_dl_managed_tensor*>(PyCapsule_GetPointer(cap, "dltensor"));
    if (t != nullptr) (void)sh_dl_free(t);
  }
}

bool as_u64(PyObject* o, uint64_t* out) {
  *out = PyLong_AsUnsignedLongLong(o);
  return !(*out == (uint64_t)-1 && PyErr_Occurred());
}

// ensure(vmm, slab, region, stream) -> handle pointer (int > 0), or -status.
PyObject* ensure(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 4) {
    PyErr_SetString(PyExc_TypeError, "ensure(vmm, slab, region, stream)");
    return nullptr;
  }
  uint64_t vmm, slab, region, stream;
  if (!as_u64(args[0], &vmm) || !as_u64(args[1], &slab) || !as_u64(args[2], &region) ||
      !as_u64(args[3], &stream))
    return nullptr;
  if (slab > UINT32_MAX || region > UINT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "slab and region ids are 32-bit");
    return nullptr;
  }
  sh_vmm_handle* h = nullptr;
  int st;
  // A resident region is served with atomics alone; mapping one may wait on the device for an
  // evicted region's last consumer, so the GIL is not held across the call.
  Py_BEGIN_ALLOW_THREADS
  st = sh_vmm_ensure_resident(reinterpret_cast<sh_vmm*>(vmm), (uint32_t)slab, (uint32_t)region,
                              reinterpret_cast<void*>(stream), &h);
  Py_END_ALLOW_THREADS
  if (st != SH_OK) return PyLong_FromLong(-st);
  return PyLong_FromUnsignedLongLong((unsigned long long)(uintptr_t)h);
}

// export(handle, code, bits, shape) -> DLPack capsule "dltensor", or -status.
PyObject* export_(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 4) {
    PyErr_SetString(PyExc_TypeError, "export(handle, code, bits, shape)");
    return nullptr;
  }
  uint64_t handle, code, bits;
  if (!as_u64(args[0], &handle) || !as_u64(args[1], &code) || !as_u64(args[2], &bits)) return nullptr;
  PyObject* seq = PySequence_Fast(args[3], "shape must be a sequence of ints");
  if (seq == nullptr) return nullptr;
  const Py_ssize_t ndim = PySequence_Fast_GET_SIZE(seq);
  if (ndim > 16) {
    Py_DECREF(seq);
    PyErr_SetString(PyExc_ValueError, "at most 16 dimensions");
    return nullptr;
  }
  int64_t dims[16];
  PyObject** items = PySequence_Fast_ITEMS(seq);
  for (Py_ssize_t i = 0; i < ndim; ++i) {
    dims[i] = PyLong_AsLongLong(items[i]);
    if (dims[i] == -1 && PyErr_Occurred()) {
      Py_DECREF(seq);
      return nullptr;
    }
  }
  Py_DECREF(seq);
  sh_dl_managed_tensor* t = nullptr;
  const int st = sh_vmm_handle_export(reinterpret_cast<sh_vmm_handle*>(handle), (uint8_t)code, (uint8_t)bits,
                                      (int32_t)ndim, dims, &t);
  if (st != SH_OK) return PyLong_FromLong(-st);
  PyObject* cap = PyCapsule_New(t, "dltensor", capsule_free);
  if (cap == nullptr) (void)sh_dl_free(t);
  return cap;
}

PyMethodDef kMethods[] = {
    {"ensure", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(ensure)), METH_FASTCALL,
     "sh_vmm_ensure_resident: the handle pointer, or the negated status"},
    {"export", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(export_)), METH_FASTCALL,
     "sh_vmm_handle_export into a DLPack capsule, or the negated status"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_sh_vmm", "VMM hot path (ensure_resident, DLPack export)", -1,
                       kMethods, nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__sh_vmm(void) { return PyModule_Create(&kModule); }
