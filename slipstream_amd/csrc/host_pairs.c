/* Host-side packing of a copy_blocks / swap_blocks mapping (a Python dict of
 * src -> dst block ids) into an int64 [n][2] buffer, with the id checks and the
 * independence test of the one-launch path, in one pass over the dict.
 *
 * The reference takes the mapping as a dict (attention_ref.py:92-94,
 * block_manager.py:196-200, :220-225, :297-298). Turning 2048 dict entries into a
 * numpy array (two np.fromiter passes), range-checking it and testing independence
 * with numpy cost about 100 us per call, twice the copy itself; here it is a few
 * microseconds. Host code only: no device call, no torch type.
 *
 * pack(mapping, addr, cap, n_src, n_dst, check) -> (n, independent)
 *   mapping  dict of int -> int, keys the source blocks, values the destinations
 *   addr     address of at least cap int64 pairs (a pinned staging buffer)
 *   n_src    blocks of the source cache (ids must lie in [0, n_src))
 *   n_dst    blocks of the destination cache
 *   check    compute `independent` (the pairs may all run in one launch: distinct
 *            destinations, none of them another pair's source); 0 returns 1
 * Raises ValueError for an id outside its cache (same message as the numpy path),
 * TypeError for a non-integer id, OverflowError past int64.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>

/* Stamps per block for the independence test: stamp[b] == epoch marks b in the
 * current call, so no clearing per call (cleared on wraparound and on growth). */
static uint32_t* g_src_stamp = NULL;
static uint32_t* g_dst_stamp = NULL;
static int64_t g_stamp_cap = 0;
static uint32_t g_epoch = 0;

static int stamps_reserve(int64_t n) {
  if (n <= g_stamp_cap) return 0;
  uint32_t* a = (uint32_t*)calloc((size_t)n, sizeof(uint32_t));
  uint32_t* b = (uint32_t*)calloc((size_t)n, sizeof(uint32_t));
  if (!a || !b) {
    free(a);
    free(b);
    PyErr_NoMemory();
    return -1;
  }
  free(g_src_stamp);
  free(g_dst_stamp);
  g_src_stamp = a;
  g_dst_stamp = b;
  g_stamp_cap = n;
  g_epoch = 0;
  return 0;
}

static uint32_t next_epoch(void) {
  if (++g_epoch == 0) { /* wrapped: old stamps could match again */
    for (int64_t i = 0; i < g_stamp_cap; ++i) g_src_stamp[i] = g_dst_stamp[i] = 0;
    g_epoch = 1;
  }
  return g_epoch;
}

static int as_id(PyObject* o, long long* out) {
  if (!PyLong_Check(o)) {
    /* numpy integers and other index types */
    PyObject* idx = PyNumber_Index(o);
    if (!idx) return -1;
    *out = PyLong_AsLongLong(idx);
    Py_DECREF(idx);
  } else {
    *out = PyLong_AsLongLong(o);
  }
  return (*out == -1 && PyErr_Occurred()) ? -1 : 0;
}

static PyObject* pack(PyObject* self, PyObject* args) {
  (void)self;
  PyObject* mapping;
  unsigned long long addr;
  Py_ssize_t cap;
  long long n_src, n_dst;
  int check;
  if (!PyArg_ParseTuple(args, "O!KnLLp", &PyDict_Type, &mapping, &addr, &cap, &n_src, &n_dst, &check)) return NULL;
  const Py_ssize_t n = PyDict_Size(mapping);
  if (n > cap) {
    PyErr_Format(PyExc_ValueError, "pack: %zd pairs for a buffer of %zd", n, cap);
    return NULL;
  }
  if (n > 0 && addr == 0) {
    PyErr_SetString(PyExc_ValueError, "pack: null buffer");
    return NULL;
  }
  int64_t* buf = (int64_t*)(uintptr_t)addr;
  Py_ssize_t pos = 0, i = 0;
  PyObject *k, *v;
  while (PyDict_Next(mapping, &pos, &k, &v)) {
    long long s, d;
    if (as_id(k, &s) < 0 || as_id(v, &d) < 0) return NULL;
    if (s < 0 || s >= n_src) {
      PyErr_Format(PyExc_ValueError, "source block %lld outside [0, %lld)", s, n_src);
      return NULL;
    }
    if (d < 0 || d >= n_dst) {
      PyErr_Format(PyExc_ValueError, "destination block %lld outside [0, %lld)", d, n_dst);
      return NULL;
    }
    buf[2 * i] = s;
    buf[2 * i + 1] = d;
    ++i;
  }
  int indep = 1;
  if (check && n > 0) {
    const int64_t need = n_src > n_dst ? n_src : n_dst;
    if (stamps_reserve(need) < 0) return NULL;
    const uint32_t e = next_epoch();
    for (Py_ssize_t j = 0; j < n; ++j) g_src_stamp[buf[2 * j]] = e;
    for (Py_ssize_t j = 0; j < n && indep; ++j) {
      const int64_t s = buf[2 * j], d = buf[2 * j + 1];
      if (g_dst_stamp[d] == e) indep = 0;              /* a second write of d */
      g_dst_stamp[d] = e;
      if (g_src_stamp[d] == e && s != d) indep = 0;    /* d is another pair's source */
    }
  }
  return Py_BuildValue("(ni)", n, indep);
}

static PyMethodDef methods[] = {
    {"pack", pack, METH_VARARGS, "pack(mapping, addr, cap, n_src, n_dst, check) -> (n, independent)"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_host_pairs", "Packing of block-id mappings.", -1,
                                    methods};

PyMODINIT_FUNC PyInit__host_pairs(void) { return PyModule_Create(&module); }
