// _fdp_call: the per-call path of the Python operators into libflashdp_hip.so.
//
// ctypes converts each of fdp_wgrad_clip's 28 arguments through its argtypes
// (about 3 us per call on the MI355X box's host); these METH_FASTCALL
// functions read plain Python ints and floats and call the C ABI directly.
// The checks on shapes, dtypes and devices stay in Python (flashdp4review_amd
// .core.wgrad), which only takes this path for call signatures it has already
// checked; the library validates its arguments again.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <cstdint>

#include "../../../include/flashdp_hip.h"

namespace {

inline bool get_i64(PyObject* o, int64_t* v) {
  *v = PyLong_AsLongLong(o);
  return !(*v == -1 && PyErr_Occurred());
}
inline bool get_u64(PyObject* o, uint64_t* v) {
  *v = PyLong_AsUnsignedLongLongMask(o);
  return !(*v == static_cast<uint64_t>(-1) && PyErr_Occurred());
}
inline bool get_ptr(PyObject* o, void** p) {
  if (o == Py_None) {
    *p = nullptr;
    return true;
  }
  uint64_t v = 0;
  if (!get_u64(o, &v)) return false;
  *p = reinterpret_cast<void*>(static_cast<uintptr_t>(v));
  return true;
}
inline bool get_f32(PyObject* o, float* f) {
  const double d = PyFloat_AsDouble(o);
  if (d == -1.0 && PyErr_Occurred()) return false;
  *f = static_cast<float>(d);
  return true;
}
// (seed, offset), (seed, offset, device counter address) or None
inline bool get_key(PyObject* o, fdp_noise_key* k, bool* has) {
  *has = false;
  if (o == Py_None) return true;
  const Py_ssize_t n = PyTuple_Check(o) ? PyTuple_GET_SIZE(o) : 0;
  if (n != 2 && n != 3) {
    PyErr_SetString(PyExc_TypeError, "noise key must be (seed, offset[, counter]) or None");
    return false;
  }
  uint64_t s = 0, off = 0;
  void* ctr = nullptr;
  if (!get_u64(PyTuple_GET_ITEM(o, 0), &s) || !get_u64(PyTuple_GET_ITEM(o, 1), &off)) return false;
  if (n == 3 && !get_ptr(PyTuple_GET_ITEM(o, 2), &ctr)) return false;
  k->seed = s;
  k->offset = off;
  k->counter = static_cast<const uint64_t*>(ctr);
  *has = true;
  return true;
}

// The arguments shared by both entry points, in fdp_wgrad_clip's order:
// a, b, B, K, M, N, stride_ab, lda, stride_bb, ldb, layout, dtype, C, clamp,
// out_scale, noise_scale, noise_key, out, ldo, out_dtype, flags
struct Common {
  void *a, *b, *out;
  int64_t i[8];  // B, K, M, N, stride_ab, lda, stride_bb, ldb
  int64_t layout, dtype, ldo, out_dtype, flags;
  float C, clamp, out_scale, noise_scale;
  fdp_noise_key key;
  bool has_key;
};
constexpr Py_ssize_t kCommon = 21;

bool parse_common(PyObject* const* a, Common* c) {
  if (!get_ptr(a[0], &c->a) || !get_ptr(a[1], &c->b)) return false;
  for (int j = 0; j < 8; ++j)
    if (!get_i64(a[2 + j], &c->i[j])) return false;
  return get_i64(a[10], &c->layout) && get_i64(a[11], &c->dtype) && get_f32(a[12], &c->C) &&
         get_f32(a[13], &c->clamp) && get_f32(a[14], &c->out_scale) &&
         get_f32(a[15], &c->noise_scale) && get_key(a[16], &c->key, &c->has_key) &&
         get_ptr(a[17], &c->out) && get_i64(a[18], &c->ldo) && get_i64(a[19], &c->out_dtype) &&
         get_i64(a[20], &c->flags);
}

// wgrad(<common 21>, workspace, workspace_bytes, stream) -> status
PyObject* wgrad(PyObject*, PyObject* const* args, Py_ssize_t n) {
  if (n != kCommon + 3) {
    PyErr_SetString(PyExc_TypeError, "wgrad: wrong number of arguments");
    return nullptr;
  }
  Common c;
  void *ws = nullptr, *stream = nullptr;
  uint64_t wsb = 0;
  if (!parse_common(args, &c) || !get_ptr(args[kCommon], &ws) ||
      !get_u64(args[kCommon + 1], &wsb) || !get_ptr(args[kCommon + 2], &stream))
    return nullptr;
  int st;
  Py_BEGIN_ALLOW_THREADS;
  st = fdp_wgrad_clip(c.a, c.b, c.i[0], c.i[1], c.i[2], c.i[3], c.i[4], c.i[5], c.i[6], c.i[7],
                      int(c.layout), int(c.dtype), c.C, c.clamp, nullptr, c.out_scale, nullptr,
                      c.noise_scale, c.has_key ? &c.key : nullptr, c.out, c.ldo, int(c.out_dtype),
                      nullptr, nullptr, int(c.flags), ws, size_t(wsb), stream);
  Py_END_ALLOW_THREADS;
  return PyLong_FromLong(st);
}

// wgrad_bias(<common 21>, bias_out, bias_dtype, bias_scale, bias_noise_scale,
//            bias_noise_key, workspace, workspace_bytes, stream) -> status
PyObject* wgrad_bias(PyObject*, PyObject* const* args, Py_ssize_t n) {
  if (n != kCommon + 8) {
    PyErr_SetString(PyExc_TypeError, "wgrad_bias: wrong number of arguments");
    return nullptr;
  }
  Common c;
  fdp_bias_out bias{};
  int64_t bdt = 0;
  fdp_noise_key bkey{};
  bool has_bkey = false;
  void *ws = nullptr, *stream = nullptr;
  uint64_t wsb = 0;
  if (!parse_common(args, &c) || !get_ptr(args[kCommon], &bias.out) ||
      !get_i64(args[kCommon + 1], &bdt) || !get_f32(args[kCommon + 2], &bias.out_scale) ||
      !get_f32(args[kCommon + 3], &bias.noise_scale) ||
      !get_key(args[kCommon + 4], &bkey, &has_bkey) || !get_ptr(args[kCommon + 5], &ws) ||
      !get_u64(args[kCommon + 6], &wsb) || !get_ptr(args[kCommon + 7], &stream))
    return nullptr;
  bias.out_dtype = int(bdt);
  bias.noise_key = has_bkey ? &bkey : nullptr;
  int st;
  Py_BEGIN_ALLOW_THREADS;
  st = fdp_wgrad_bias_clip(c.a, c.b, c.i[0], c.i[1], c.i[2], c.i[3], c.i[4], c.i[5], c.i[6],
                           c.i[7], int(c.layout), int(c.dtype), c.C, c.clamp, nullptr,
                           c.out_scale, nullptr, c.noise_scale, c.has_key ? &c.key : nullptr,
                           c.out, c.ldo, int(c.out_dtype), nullptr, nullptr, int(c.flags), &bias,
                           ws, size_t(wsb), stream);
  Py_END_ALLOW_THREADS;
  return PyLong_FromLong(st);
}

PyMethodDef kMethods[] = {
    {"wgrad", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(wgrad)), METH_FASTCALL,
     "fdp_wgrad_clip without stats or injected noise; returns the status"},
    {"wgrad_bias", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(wgrad_bias)),
     METH_FASTCALL, "fdp_wgrad_bias_clip without stats or injected noise; returns the status"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_fdp_call",
                       "Per-call path of the operators into libflashdp_hip.so", -1, kMethods,
                       nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__fdp_call(void) { return PyModule_Create(&kModule); }
