// Host packer for one step's attention inputs (CPython extension module
// microserve_amd._step_pack).
//
// The runner's context builders (microserve/engine/model_runner.py:124-216)
// walk the scheduled sequences in Python and write every element to the
// device on its own.  mskv_build_step_inputs expands one packed host buffer
// on the GPU instead; this module fills that buffer in one pass over the
// sequences, reading their Python lists directly rather than through
// generator expressions (a batch of 256 decodes holds ~5,600 block ids).
//
// pack(seqs, block_size) -> (bytes, total_q, max_seqlen_q, ntab, max_table_len)
//   bytes: int64 token ids of the scheduled positions, then int32 first
//   positions [nseq], cu_seqlens_q [nseq + 1], table offsets [nseq + 1] and
//   the concatenated block tables [ntab].
// Sequences are duck-typed: token_ids, num_computed_tokens,
// num_scheduled_tokens and block_table (microserve/engine/sequence.py:19-50).
// Errors follow the reference's list indexing: IndexError for a scheduled
// position past the token list or past the block table.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <climits>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

PyObject* g_computed;   // "num_computed_tokens"
PyObject* g_scheduled;  // "num_scheduled_tokens"
PyObject* g_table;      // "block_table"
PyObject* g_ids;        // "token_ids"

bool attr_ll(PyObject* o, PyObject* name, long long& v) {
  PyObject* a = PyObject_GetAttr(o, name);
  if (!a) return false;
  v = PyLong_AsLongLong(a);
  Py_DECREF(a);
  return !(v == -1 && PyErr_Occurred());
}

struct Row {
  long long start = 0, n = 0;
  PyObject* ids = nullptr;  // new reference
  PyObject* tab = nullptr;  // new reference, a list or tuple (PySequence_Fast)
  Py_ssize_t tlen = 0;
};

struct Rows {
  std::vector<Row> v;
  ~Rows() {
    for (Row& r : v) {
      Py_XDECREF(r.ids);
      Py_XDECREF(r.tab);
    }
  }
};

// element i of a sequence as a C long long (lists and tuples without a call)
bool item_ll(PyObject* seq, Py_ssize_t i, long long& v) {
  PyObject* it;
  if (PyList_CheckExact(seq)) {
    it = PyList_GET_ITEM(seq, i);
    v = PyLong_AsLongLong(it);
    return !(v == -1 && PyErr_Occurred());
  }
  if (PyTuple_CheckExact(seq)) {
    it = PyTuple_GET_ITEM(seq, i);
    v = PyLong_AsLongLong(it);
    return !(v == -1 && PyErr_Occurred());
  }
  it = PySequence_GetItem(seq, i);
  if (!it) return false;
  v = PyLong_AsLongLong(it);
  Py_DECREF(it);
  return !(v == -1 && PyErr_Occurred());
}

bool put_i32(long long v, char* dst) {
  if (v < INT32_MIN || v > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "value does not fit int32");
    return false;
  }
  const int32_t x = (int32_t)v;
  std::memcpy(dst, &x, 4);
  return true;
}

PyObject* pack(PyObject*, PyObject* args) {
  PyObject* seqs_obj;
  long long bs;
  if (!PyArg_ParseTuple(args, "OL", &seqs_obj, &bs)) return nullptr;
  if (bs <= 0) {
    PyErr_SetString(PyExc_ValueError, "block_size must be positive");
    return nullptr;
  }
  PyObject* seqs = PySequence_Fast(seqs_obj, "seqs must be a sequence");
  if (!seqs) return nullptr;
  const Py_ssize_t nseq = PySequence_Fast_GET_SIZE(seqs);
  PyObject** items = PySequence_Fast_ITEMS(seqs);
  Rows rows;
  rows.v.resize((size_t)nseq);
  bool ok = true;
  for (Py_ssize_t i = 0; i < nseq && ok; ++i) {
    Row& r = rows.v[(size_t)i];
    ok = attr_ll(items[i], g_computed, r.start) && attr_ll(items[i], g_scheduled, r.n);
    if (!ok) break;
    PyObject* t = PyObject_GetAttr(items[i], g_table);
    if (!t) { ok = false; break; }
    r.tab = PySequence_Fast(t, "block_table must be a sequence");
    Py_DECREF(t);
    if (!r.tab) { ok = false; break; }
    r.tlen = PySequence_Fast_GET_SIZE(r.tab);
    r.ids = PyObject_GetAttr(items[i], g_ids);
    if (!r.ids) ok = false;
  }
  Py_DECREF(seqs);
  if (!ok) return nullptr;
  // the checks of the Python builder, in its order
  for (const Row& r : rows.v)
    if (r.start < 0 || r.n < 0) {
      PyErr_SetString(PyExc_ValueError, "negative num_computed_tokens or num_scheduled_tokens");
      return nullptr;
    }
  for (const Row& r : rows.v)
    if (r.n > 0 && (r.start + r.n - 1) / bs >= r.tlen) {
      PyErr_SetString(PyExc_IndexError, "list index out of range (block_table shorter than "
                                        "the scheduled positions)");
      return nullptr;
    }
  long long total_q = 0, max_q = 0, ntab = 0, max_tlen = 0, max_end = 0;
  for (const Row& r : rows.v) {
    const Py_ssize_t nids = PySequence_Size(r.ids);
    if (nids < 0) return nullptr;
    if (r.start + r.n > nids) {
      PyErr_SetString(PyExc_IndexError, "list index out of range (token_ids shorter than "
                                        "the scheduled positions)");
      return nullptr;
    }
    total_q += r.n;
    if (r.n > max_q) max_q = r.n;
    ntab += r.tlen;
    if (r.tlen > max_tlen) max_tlen = r.tlen;
    if (r.start + r.n > max_end) max_end = r.start + r.n;
  }
  if (max_end > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "positions beyond int32");
    return nullptr;
  }
  // cu_seqlens_q and the table offsets are int32 on the device
  if (total_q > INT32_MAX || ntab > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "step too large for int32 offsets");
    return nullptr;
  }
  const long long o_start = 8 * total_q, o_cu = o_start + 4 * (long long)nseq;
  const long long o_toff = o_cu + 4 * ((long long)nseq + 1), o_tab = o_toff + 4 * ((long long)nseq + 1);
  const long long nbytes = o_tab + 4 * ntab;
  PyObject* out = PyBytes_FromStringAndSize(nullptr, (Py_ssize_t)(nbytes > 8 ? nbytes : 8));
  if (!out) return nullptr;
  char* p = PyBytes_AS_STRING(out);
  std::memset(p, 0, (size_t)(nbytes > 8 ? nbytes : 8));
  // cu_seqlens_q[0] and the first table offset stay 0
  long long tok = 0, cu = 0, toff = 0;
  for (Py_ssize_t i = 0; i < nseq; ++i) {
    const Row& r = rows.v[(size_t)i];
    for (long long k = 0; k < r.n; ++k) {
      long long id;
      if (!item_ll(r.ids, (Py_ssize_t)(r.start + k), id)) { Py_DECREF(out); return nullptr; }
      std::memcpy(p + 8 * (tok + k), &id, 8);
    }
    tok += r.n;
    const int32_t st = (int32_t)r.start;
    std::memcpy(p + o_start + 4 * i, &st, 4);
    cu += r.n;
    const int32_t c32 = (int32_t)cu;
    std::memcpy(p + o_cu + 4 * (i + 1), &c32, 4);
    PyObject** tv = PySequence_Fast_ITEMS(r.tab);
    for (Py_ssize_t k = 0; k < r.tlen; ++k) {
      const long long b = PyLong_AsLongLong(tv[k]);
      if ((b == -1 && PyErr_Occurred()) || !put_i32(b, p + o_tab + 4 * (toff + k))) {
        Py_DECREF(out);
        return nullptr;
      }
    }
    toff += r.tlen;
    if (!put_i32(toff, p + o_toff + 4 * (i + 1))) { Py_DECREF(out); return nullptr; }
  }
  return Py_BuildValue("(NLLLL)", out, total_q, max_q, ntab, max_tlen);
}

PyMethodDef kMethods[] = {
    {"pack", pack, METH_VARARGS,
     "pack(seqs, block_size) -> (bytes, total_q, max_seqlen_q, ntab, max_table_len)"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_step_pack",
                       "Host packer of one step's attention inputs.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__step_pack(void) {
  g_computed = PyUnicode_InternFromString("num_computed_tokens");
  g_scheduled = PyUnicode_InternFromString("num_scheduled_tokens");
  g_table = PyUnicode_InternFromString("block_table");
  g_ids = PyUnicode_InternFromString("token_ids");
  if (!g_computed || !g_scheduled || !g_table || !g_ids) return nullptr;
  return PyModule_Create(&kModule);
}
