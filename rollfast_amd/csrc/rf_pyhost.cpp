// rf_pyhost.cpp -- native host fast path of the fused step (CPython module
// rollfast_amd._lib._rfhost).
//
// A fused step over a tree whose structure, params and moment objects are
// those of the previous step only needs new grad pointers in the leaf table.
// Doing that in Python costs about 1.6 us per leaf (pytree walks, weakref and
// pointer checks); here it is one joint walk of the four trees and one pass
// over the cached rows, in C++.
//
//   gather(grads, mu, nu, params) -> (g, mu, nu, p) leaf lists, or None
//       Joint walk in the flattening order of rollfast_amd._tree (dicts by
//       sorted keys, lists and tuples in order; None and MaskedNode are
//       leaves of the grads tree).  mu / nu / params are taken as they are
//       at each grads leaf.  Returns None (the caller falls back to the
//       Python walk) for any container it does not handle or any mismatch.
//
//   updates_out(grads, g, mu, rows, table_address[, cache]) -> updates tree
//       Update-only mode: the f32 outputs of a refreshed table (one device
//       buffer, a view per leaf) and the updates tree (see py_updates_out);
//       with `cache`, the buffers of earlier calls that nothing else still
//       references are written again instead of allocated.
//
//   apply_rows(params, updates) -> packed rf_apply_leaf rows and the params
//       tree for rollfast.apply_updates (see py_apply_rows).
//
//   refresh(g, mu, nu, p, rows, table_address, device) -> bool
//       rows[j] = (i, mref, vref, pref, bufrefs, bufptrs, grad_dtype, size, vec)
//       Checks that leaf i's moment and param objects are the cached ones
//       (weak references), that their buffers still have the cached device
//       pointers, and that grad i is a contiguous tensor of the cached dtype,
//       size and device (16-byte aligned when the row was); then writes its
//       pointer into row j of the rf_adam8_leaf table at table_address.
//       Returns False at the first difference (the table may then be partly
//       rewritten: the caller rebuilds it).
#include <Python.h>

#include <torch/csrc/autograd/python_variable.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include <ATen/ATen.h>

#include "rfadam8.h"

namespace {

PyObject* g_masked_node_type = nullptr;  // rollfast_amd._base.MaskedNode

bool is_aux(PyObject* x)
{
    return x == Py_None || (g_masked_node_type && PyObject_TypeCheck(x, (PyTypeObject*)g_masked_node_type));
}

bool is_grad_leaf(PyObject* x)
{
    return x == Py_None || THPVariable_Check(x) ||
           (g_masked_node_type && PyObject_TypeCheck(x, (PyTypeObject*)g_masked_node_type));
}

// Appends the grads leaves and the other trees' subtrees at those positions.
// Returns 1 on success, 0 for "not handled here" (no Python error set), -1 on
// a Python error.
int walk(PyObject* g, PyObject* m, PyObject* v, PyObject* p, PyObject* lg, PyObject* lm, PyObject* lv, PyObject* lp)
{
    if (is_grad_leaf(g)) {
        if (PyList_Append(lg, g) || PyList_Append(lm, m) || PyList_Append(lv, v)) return -1;
        if (lp && PyList_Append(lp, p)) return -1;
        return 1;
    }
    if (PyDict_CheckExact(g)) {
        if (!PyDict_CheckExact(m) || !PyDict_CheckExact(v) || (lp && !PyDict_CheckExact(p))) return 0;
        const Py_ssize_t n = PyDict_Size(g);
        if (PyDict_Size(m) != n || PyDict_Size(v) != n || (lp && PyDict_Size(p) != n)) return 0;
        PyObject* keys = PyDict_Keys(g);
        if (!keys) return -1;
        if (PyList_Sort(keys) < 0) {  // keys that do not sort: leave it to the Python walk
            Py_DECREF(keys);
            PyErr_Clear();
            return 0;
        }
        int rc = 1;
        for (Py_ssize_t k = 0; k < n && rc == 1; ++k) {
            PyObject* key = PyList_GET_ITEM(keys, k);
            PyObject* cg = PyDict_GetItemWithError(g, key);
            PyObject* cm = cg ? PyDict_GetItemWithError(m, key) : nullptr;
            PyObject* cv = cm ? PyDict_GetItemWithError(v, key) : nullptr;
            PyObject* cp = (cv && lp) ? PyDict_GetItemWithError(p, key) : nullptr;
            if (!cg || !cm || !cv || (lp && !cp)) {
                rc = PyErr_Occurred() ? -1 : 0;
                break;
            }
            rc = walk(cg, cm, cv, cp, lg, lm, lv, lp);
        }
        Py_DECREF(keys);
        return rc;
    }
    const bool is_list = PyList_CheckExact(g), is_tuple = PyTuple_CheckExact(g);
    if (is_list || is_tuple) {
        auto same = [&](PyObject* x) { return is_list ? PyList_CheckExact(x) : PyTuple_CheckExact(x); };
        if (!same(m) || !same(v) || (lp && !same(p))) return 0;
        const Py_ssize_t n = PySequence_Fast_GET_SIZE(g);
        if (PySequence_Fast_GET_SIZE(m) != n || PySequence_Fast_GET_SIZE(v) != n ||
            (lp && PySequence_Fast_GET_SIZE(p) != n))
            return 0;
        for (Py_ssize_t k = 0; k < n; ++k) {
            const int rc = walk(PySequence_Fast_GET_ITEM(g, k), PySequence_Fast_GET_ITEM(m, k),
                                PySequence_Fast_GET_ITEM(v, k), lp ? PySequence_Fast_GET_ITEM(p, k) : nullptr, lg,
                                lm, lv, lp);
            if (rc != 1) return rc;
        }
        return 1;
    }
    return 0;  // custom nodes, namedtuples, OrderedDicts: the Python walk
}

PyObject* py_gather(PyObject*, PyObject* args)
{
    PyObject *g, *m, *v, *p;
    if (!PyArg_ParseTuple(args, "OOOO", &g, &m, &v, &p)) return nullptr;
    const bool has_p = p != Py_None;
    PyObject* lg = PyList_New(0);
    PyObject* lm = PyList_New(0);
    PyObject* lv = PyList_New(0);
    PyObject* lp = has_p ? PyList_New(0) : nullptr;
    PyObject* out = nullptr;
    if (lg && lm && lv && (!has_p || lp)) {
        const int rc = walk(g, m, v, has_p ? p : nullptr, lg, lm, lv, lp);
        if (rc == 1) {
            out = PyTuple_Pack(4, lg, lm, lv, has_p ? lp : Py_None);
        } else if (rc == 0) {
            out = Py_None;
            Py_INCREF(out);
        }
    }
    Py_XDECREF(lg);
    Py_XDECREF(lm);
    Py_XDECREF(lv);
    Py_XDECREF(lp);
    return out;
}

// The live object behind a weak reference, or nullptr (borrowed).
PyObject* deref(PyObject* ref)
{
    if (ref == Py_None) return nullptr;
    PyObject* o = PyWeakref_GetObject(ref);
    return o == Py_None ? nullptr : o;
}

bool tensor_ptr(PyObject* o, uintptr_t* out)
{
    if (!o || !THPVariable_Check(o)) return false;
    *out = (uintptr_t)THPVariable_Unpack(o).data_ptr();
    return true;
}

PyObject* py_refresh(PyObject*, PyObject* args)
{
    PyObject *lg, *lm, *lv, *lp, *rows;
    unsigned long long table_addr = 0;
    int device = 0;
    if (!PyArg_ParseTuple(args, "O!O!O!OO!Ki", &PyList_Type, &lg, &PyList_Type, &lm, &PyList_Type, &lv, &lp,
                          &PyList_Type, &rows, &table_addr, &device))
        return nullptr;
    if (lp != Py_None && !PyList_Check(lp)) {
        PyErr_SetString(PyExc_TypeError, "params leaves must be a list or None");
        return nullptr;
    }
    const Py_ssize_t n = PyList_GET_SIZE(lg);
    if (PyList_GET_SIZE(lm) != n || PyList_GET_SIZE(lv) != n || (lp != Py_None && PyList_GET_SIZE(lp) != n))
        Py_RETURN_FALSE;
    auto* table = (rf_adam8_leaf*)(uintptr_t)table_addr;
    const Py_ssize_t nrows = PyList_GET_SIZE(rows);
    Py_ssize_t live = 0;  // leaves that are neither passthrough in mu nor in the grads
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject* g = PyList_GET_ITEM(lg, i);
        PyObject* m = PyList_GET_ITEM(lm, i);
        const bool pass = g == Py_None || m == Py_None ||
                          (g_masked_node_type && (PyObject_TypeCheck(g, (PyTypeObject*)g_masked_node_type) ||
                                                  PyObject_TypeCheck(m, (PyTypeObject*)g_masked_node_type)));
        live += pass ? 0 : 1;
    }
    if (live != nrows) Py_RETURN_FALSE;
    for (Py_ssize_t j = 0; j < nrows; ++j) {
        PyObject* row = PyList_GET_ITEM(rows, j);
        if (!PyTuple_Check(row) || PyTuple_GET_SIZE(row) != 9) {
            PyErr_SetString(PyExc_TypeError, "bad row record");
            return nullptr;
        }
        const Py_ssize_t i = PyLong_AsSsize_t(PyTuple_GET_ITEM(row, 0));
        if (i < 0 || i >= n) {
            if (PyErr_Occurred()) return nullptr;
            Py_RETURN_FALSE;
        }
        PyObject* m = PyList_GET_ITEM(lm, i);
        PyObject* v = PyList_GET_ITEM(lv, i);
        if (deref(PyTuple_GET_ITEM(row, 1)) != m || deref(PyTuple_GET_ITEM(row, 2)) != v) Py_RETURN_FALSE;
        PyObject* pref = PyTuple_GET_ITEM(row, 3);
        if (pref != Py_None && (lp == Py_None || deref(pref) != PyList_GET_ITEM(lp, i))) Py_RETURN_FALSE;
        // same objects, same storage (a `.data` swap changes the pointer)
        PyObject* bufrefs = PyTuple_GET_ITEM(row, 4);
        PyObject* bufptrs = PyTuple_GET_ITEM(row, 5);
        const Py_ssize_t nb = PyTuple_GET_SIZE(bufrefs);
        if (PyTuple_GET_SIZE(bufptrs) != nb) Py_RETURN_FALSE;
        for (Py_ssize_t b = 0; b < nb; ++b) {
            uintptr_t ptr = 0;
            if (!tensor_ptr(deref(PyTuple_GET_ITEM(bufrefs, b)), &ptr)) Py_RETURN_FALSE;
            if ((unsigned long long)ptr != PyLong_AsUnsignedLongLong(PyTuple_GET_ITEM(bufptrs, b))) {
                if (PyErr_Occurred()) return nullptr;
                Py_RETURN_FALSE;
            }
        }
        PyObject* g = PyList_GET_ITEM(lg, i);
        if (!THPVariable_Check(g)) Py_RETURN_FALSE;
        const at::Tensor& t = THPVariable_Unpack(g);
        const long want_dtype = PyLong_AsLong(PyTuple_GET_ITEM(row, 6));
        const long long want_size = PyLong_AsLongLong(PyTuple_GET_ITEM(row, 7));
        const int vec = PyObject_IsTrue(PyTuple_GET_ITEM(row, 8));
        if (PyErr_Occurred()) return nullptr;
        const at::ScalarType st = t.scalar_type();
        const bool dtype_ok = (want_dtype == RF_F32 && st == at::kFloat) || (want_dtype == RF_BF16 && st == at::kBFloat16) ||
                              (want_dtype == RF_F16 && st == at::kHalf);
        if (!dtype_ok || !t.is_cuda() || t.get_device() != device || t.numel() != want_size || !t.is_contiguous())
            Py_RETURN_FALSE;
        const uintptr_t gp = (uintptr_t)t.data_ptr();
        if (vec && (gp & 15u)) Py_RETURN_FALSE;
        table[j].grad = (const void*)gp;
    }
    Py_RETURN_TRUE;
}

// Rebuilds the containers of `g` (the grads tree, walked as in walk()) with
// leaf k replaced by vals[k].  New reference, or nullptr with an error set.
PyObject* rebuild(PyObject* g, PyObject* vals, Py_ssize_t& k)
{
    if (is_grad_leaf(g)) {
        PyObject* v = PyList_GET_ITEM(vals, k++);
        Py_INCREF(v);
        return v;
    }
    if (PyDict_CheckExact(g)) {
        PyObject* keys = PyDict_Keys(g);
        if (!keys || PyList_Sort(keys) < 0) {
            Py_XDECREF(keys);
            return nullptr;
        }
        PyObject* out = PyDict_New();
        for (Py_ssize_t i = 0; out && i < PyList_GET_SIZE(keys); ++i) {
            PyObject* key = PyList_GET_ITEM(keys, i);
            PyObject* c = rebuild(PyDict_GetItem(g, key), vals, k);
            if (!c || PyDict_SetItem(out, key, c) < 0) Py_CLEAR(out);
            Py_XDECREF(c);
        }
        Py_DECREF(keys);
        return out;
    }
    const bool is_list = PyList_CheckExact(g);
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(g);
    PyObject* out = is_list ? PyList_New(n) : PyTuple_New(n);
    for (Py_ssize_t i = 0; out && i < n; ++i) {
        PyObject* c = rebuild(PySequence_Fast_GET_ITEM(g, i), vals, k);
        if (!c) {
            Py_CLEAR(out);
            break;
        }
        if (is_list) PyList_SET_ITEM(out, i, c);
        else PyTuple_SET_ITEM(out, i, c);
    }
    return out;
}

// An earlier call's output (cache entry [flat, views]) that may be written
// again: no Python reference to its views but the entry's own, no tensor but
// the buffer and its views on the buffer's storage (so no alias survives
// from a tree the caller still holds), and views of the grads' shapes.
bool reusable(PyObject* entry, PyObject* lg, PyObject* rows)
{
    PyObject* flat_obj = PyList_GET_ITEM(entry, 0);
    PyObject* views = PyList_GET_ITEM(entry, 1);
    const Py_ssize_t nrows = PyList_GET_SIZE(rows);
    if (PyList_GET_SIZE(views) != nrows) return false;  // (the buffer object itself is never handed out)
    const at::Tensor& flat = THPVariable_Unpack(flat_obj);
    if (flat.storage().use_count() != 1 + nrows) return false;
    for (Py_ssize_t j = 0; j < nrows; ++j) {
        PyObject* v = PyList_GET_ITEM(views, j);
        if (Py_REFCNT(v) != 1) return false;
        const Py_ssize_t i = PyLong_AsSsize_t(PyTuple_GET_ITEM(PyList_GET_ITEM(rows, j), 0));
        if (!THPVariable_Unpack(v).sizes().equals(THPVariable_Unpack(PyList_GET_ITEM(lg, i)).sizes())) return false;
    }
    return true;
}

constexpr Py_ssize_t UPDATES_CACHE = 2;  // output buffers kept for reuse (one may still be held by the caller)

// updates_out(grads, lg, lm, rows, table_address[, cache]) -> updates tree
//
// Update-only (Optax) mode after a successful refresh(): one f32 device
// buffer holds every row's updates (each leaf 16-byte aligned), row j's
// `updates` pointer is set to its slice and the updates tree is the grads
// tree with, per leaf, that slice viewed in the grad's shape, or the
// passthrough leaf (the moment's MaskedNode / None, else the grad's).
// `cache` (a list owned by the caller, at most UPDATES_CACHE entries
// [flat buffer, views]): a reusable entry (see reusable()) gives its buffer
// and view objects to this call instead of a new allocation and nrows new
// views; a new buffer is appended to it, the oldest entry dropped.  The
// kernel that writes the buffer again is stream-ordered after whatever read
// it before, as with the caching allocator's reuse.
PyObject* py_updates_out(PyObject*, PyObject* args)
{
    PyObject *g, *lg, *lm, *rows;
    PyObject* cache = nullptr;
    unsigned long long table_addr = 0;
    if (!PyArg_ParseTuple(args, "OO!O!O!K|O!", &g, &PyList_Type, &lg, &PyList_Type, &lm, &PyList_Type, &rows,
                          &table_addr, &PyList_Type, &cache))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(lg);
    const Py_ssize_t nrows = PyList_GET_SIZE(rows);
    auto* table = (rf_adam8_leaf*)(uintptr_t)table_addr;
    std::vector<int64_t> off((size_t)nrows);
    int64_t total = 0;
    for (Py_ssize_t j = 0; j < nrows; ++j) {
        off[(size_t)j] = total;
        total += (table[j].size + 3) / 4 * 4;
    }
    PyObject* vals = PyList_New(n);
    if (!vals) return nullptr;
    for (Py_ssize_t i = 0; i < n; ++i) {  // passthrough leaves (utils of the Python path)
        PyObject* gi = PyList_GET_ITEM(lg, i);
        PyObject* mi = PyList_GET_ITEM(lm, i);
        PyObject* v = is_aux(mi) ? mi : gi;
        Py_INCREF(v);
        PyList_SET_ITEM(vals, i, v);
    }
    PyObject* entry = nullptr;  // the cache entry this call writes (borrowed)
    if (nrows > 0 && cache) {
        const at::Tensor& g0 = THPVariable_Unpack(PyList_GET_ITEM(lg, PyLong_AsSsize_t(PyTuple_GET_ITEM(
                                                                          PyList_GET_ITEM(rows, 0), 0))));
        for (Py_ssize_t c = 0; c < PyList_GET_SIZE(cache) && !entry; ++c) {
            PyObject* e = PyList_GET_ITEM(cache, c);
            if (PyList_CheckExact(e) && PyList_GET_SIZE(e) == 2 && reusable(e, lg, rows) &&
                THPVariable_Unpack(PyList_GET_ITEM(e, 0)).device() == g0.device())
                entry = e;
        }
        if (entry) {
            PyObject* views = PyList_GET_ITEM(entry, 1);
            for (Py_ssize_t j = 0; j < nrows; ++j) {
                const Py_ssize_t i = PyLong_AsSsize_t(PyTuple_GET_ITEM(PyList_GET_ITEM(rows, j), 0));
                PyObject* v = PyList_GET_ITEM(views, j);
                table[j].updates = THPVariable_Unpack(v).data_ptr<float>();
                Py_INCREF(v);
                PyList_SetItem(vals, i, v);
            }
        }
    }
    if (nrows > 0 && !entry) {
        const at::Tensor& g0 = THPVariable_Unpack(PyList_GET_ITEM(lg, PyLong_AsSsize_t(PyTuple_GET_ITEM(
                                                                          PyList_GET_ITEM(rows, 0), 0))));
        at::Tensor flat = at::empty({total}, g0.options().dtype(at::kFloat));
        PyObject* views = cache ? PyList_New(nrows) : nullptr;
        if (cache && !views) {
            Py_DECREF(vals);
            return nullptr;
        }
        for (Py_ssize_t j = 0; j < nrows; ++j) {
            const Py_ssize_t i = PyLong_AsSsize_t(PyTuple_GET_ITEM(PyList_GET_ITEM(rows, j), 0));
            const at::Tensor& gi = THPVariable_Unpack(PyList_GET_ITEM(lg, i));
            at::Tensor view = flat.as_strided(gi.sizes(), gi.strides(), off[(size_t)j]);  // gi is contiguous
            table[j].updates = view.data_ptr<float>();
            PyObject* obj = THPVariable_Wrap(std::move(view));
            if (!obj) {
                Py_XDECREF(views);
                Py_DECREF(vals);
                return nullptr;
            }
            if (views) {
                Py_INCREF(obj);
                PyList_SET_ITEM(views, j, obj);
            }
            PyList_SetItem(vals, i, obj);  // steals obj, drops the passthrough placeholder
        }
        if (cache) {
            PyObject* flat_obj = THPVariable_Wrap(std::move(flat));
            PyObject* e = flat_obj ? PyList_New(2) : nullptr;
            if (!e) {
                Py_XDECREF(flat_obj);
                Py_DECREF(views);
                Py_DECREF(vals);
                return nullptr;
            }
            PyList_SET_ITEM(e, 0, flat_obj);
            PyList_SET_ITEM(e, 1, views);
            if (PyList_Append(cache, e) < 0 ||
                (PyList_GET_SIZE(cache) > UPDATES_CACHE && PySequence_DelItem(cache, 0) < 0)) {
                Py_DECREF(e);
                Py_DECREF(vals);
                return nullptr;
            }
            Py_DECREF(e);
        }
    }
    Py_ssize_t k = 0;
    PyObject* out = rebuild(g, vals, k);
    Py_DECREF(vals);
    return out;
}

// apply_rows(params, updates) -> (rows bytes, n rows, device, new params tree) or None
//
// rollfast.apply_updates' walk (utils.py:648-708): the params tree drives,
// updates are taken at its leaves; None / MaskedNode on either side is left
// alone.  Every other leaf pair must be a contiguous f32 / bf16 param and a
// contiguous f32 update of the same size on one device: the row records
// (rf_apply_leaf) come back packed, with param_index = the leaf's position.
// The returned params tree has new containers around the same tensors.
// None means "not handled here" (other containers, dtypes or layouts): the
// Python walk then does the conversions and raises the errors.
struct ApplyWalk {
    std::string rows;
    int64_t leaf = 0;
    int device = -1;
};

// Returns a new reference to the rebuilt subtree; nullptr with no error set
// for "not handled here", nullptr with an error set on failure.
PyObject* apply_walk(PyObject* p, PyObject* u, ApplyWalk& w)
{
    if (!is_aux(p) && !THPVariable_Check(p) && !PyDict_CheckExact(p) && !PyList_CheckExact(p) && !PyTuple_CheckExact(p))
        return nullptr;  // other leaves and containers (namedtuples, custom nodes): the Python walk
    if (is_aux(p) || THPVariable_Check(p)) {
        const int64_t i = w.leaf++;
        if (!is_aux(p) && !is_aux(u)) {
            if (!THPVariable_Check(p) || !THPVariable_Check(u)) return nullptr;
            const at::Tensor& tp = THPVariable_Unpack(p);
            const at::Tensor& tu = THPVariable_Unpack(u);
            const at::ScalarType sp = tp.scalar_type();
            if ((sp != at::kFloat && sp != at::kBFloat16 && sp != at::kHalf) || tu.scalar_type() != at::kFloat)
                return nullptr;
            if (!tp.is_cuda() || !tu.is_cuda() || tp.get_device() != tu.get_device()) return nullptr;
            if (w.device < 0) w.device = tp.get_device();
            if (tp.get_device() != w.device) return nullptr;
            if (!tp.is_contiguous() || !tu.is_contiguous() || tp.numel() != tu.numel()) return nullptr;
            if (i > INT32_MAX) return nullptr;
            rf_apply_leaf row{};
            row.param = tp.data_ptr();
            row.updates = (const float*)tu.data_ptr();
            row.bits = nullptr;
            row.size = tp.numel();
            row.param_dtype = sp == at::kBFloat16 ? RF_BF16 : (sp == at::kHalf ? RF_F16 : RF_F32);
            row.param_index = (int32_t)i;
            w.rows.append((const char*)&row, sizeof(row));
        }
        Py_INCREF(p);
        return p;
    }
    if (PyDict_CheckExact(p)) {
        if (!PyDict_CheckExact(u) || PyDict_Size(u) != PyDict_Size(p)) return nullptr;
        PyObject* keys = PyDict_Keys(p);
        if (!keys) return nullptr;
        if (PyList_Sort(keys) < 0) {
            Py_DECREF(keys);
            PyErr_Clear();
            return nullptr;
        }
        PyObject* out = PyDict_New();
        const Py_ssize_t n = PyList_GET_SIZE(keys);
        for (Py_ssize_t k = 0; out && k < n; ++k) {
            PyObject* key = PyList_GET_ITEM(keys, k);
            PyObject* cp = PyDict_GetItemWithError(p, key);
            PyObject* cu = cp ? PyDict_GetItemWithError(u, key) : nullptr;
            PyObject* c = (cp && cu) ? apply_walk(cp, cu, w) : nullptr;
            if (!c || PyDict_SetItem(out, key, c) < 0) {
                Py_XDECREF(c);
                Py_CLEAR(out);
                break;
            }
            Py_DECREF(c);
        }
        Py_DECREF(keys);
        return out;
    }
    const bool is_list = PyList_CheckExact(p);
    if (is_list ? !PyList_CheckExact(u) : !PyTuple_CheckExact(u)) return nullptr;
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(p);
    if (PySequence_Fast_GET_SIZE(u) != n) return nullptr;
    PyObject* out = is_list ? PyList_New(n) : PyTuple_New(n);
    for (Py_ssize_t k = 0; out && k < n; ++k) {
        PyObject* c = apply_walk(PySequence_Fast_GET_ITEM(p, k), PySequence_Fast_GET_ITEM(u, k), w);
        if (!c) {
            Py_CLEAR(out);
            break;
        }
        if (is_list) PyList_SET_ITEM(out, k, c);
        else PyTuple_SET_ITEM(out, k, c);
    }
    return out;
}

PyObject* py_apply_rows(PyObject*, PyObject* args)
{
    PyObject *p, *u;
    if (!PyArg_ParseTuple(args, "OO", &p, &u)) return nullptr;
    ApplyWalk w;
    PyObject* tree = apply_walk(p, u, w);
    if (!tree) {
        if (PyErr_Occurred()) return nullptr;
        Py_RETURN_NONE;
    }
    PyObject* rows = PyBytes_FromStringAndSize(w.rows.data(), (Py_ssize_t)w.rows.size());
    if (!rows) {
        Py_DECREF(tree);
        return nullptr;
    }
    PyObject* out = Py_BuildValue("(NnnN)", rows, (Py_ssize_t)(w.rows.size() / sizeof(rf_apply_leaf)),
                                  (Py_ssize_t)w.device, tree);
    return out;
}

PyObject* py_set_masked_node_type(PyObject*, PyObject* t)
{
    if (!PyType_Check(t)) {
        PyErr_SetString(PyExc_TypeError, "expected a type");
        return nullptr;
    }
    Py_XDECREF(g_masked_node_type);
    Py_INCREF(t);
    g_masked_node_type = t;
    Py_RETURN_NONE;
}

PyMethodDef methods[] = {
    {"gather", py_gather, METH_VARARGS, "joint walk of (grads, mu, nu, params); None if not handled"},
    {"refresh", py_refresh, METH_VARARGS, "rewrite the grad pointers of a cached leaf table; False on a mismatch"},
    {"updates_out", py_updates_out, METH_VARARGS, "update-only mode: output buffers and the updates tree"},
    {"apply_rows", py_apply_rows, METH_VARARGS, "apply_updates' leaf table and rebuilt params tree; None if not handled"},
    {"set_masked_node_type", py_set_masked_node_type, METH_O, "the MaskedNode class (a grads leaf)"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_rfhost", "native host fast path of the fused step", -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__rfhost(void) { return PyModule_Create(&module); }
