// The `pdscope_layer_dispatch` extension module: the native decode MoE tail
// (pack -> submit -> join -> stage -> merge) behind the interface of
// native/native_layer_dispatch.cpp:49-142, so the reference driver's loader
// (benchmarks/pdscope_compare.py:39-52: glob, spec_from_file_location,
// exec_module, hasattr submit_and_merge) loads it unchanged.
//
//   submit_group(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr,
//                count_ptr, selected_ptr, coeff_ptr, ids) -> None
//   finish_and_merge(pool, block_ptr, rows, row_bytes, scratch, out, tokens,
//                    weights) -> out
//   submit_and_merge(pool, layer, row_ptr, rows, row_bytes, packed_ptr,
//                    block_ptr, scratch, count_ptr, selected_ptr, coeff_ptr,
//                    ids, out, tokens, weights) -> out
//
// Host packing is pdscope_dispatch_pack and the stage + merge is
// pdscope_stage_merge (one hipMemcpyAsync of the CPU block into `scratch`
// and the rows added into `out` at `tokens` in bf16, in row order) on the
// current stream of `out`'s device; both come from libpdscope_moe.so.  Every
// pointer and tensor is borrowed from the caller and `out` is updated in
// place and returned.  `pool` (submit / sync) and `layer` (forward_task) are
// the caller's CPU expert queue objects, called exactly as the reference
// calls them, with the GIL held throughout.  Shape and device errors raise
// RuntimeError with the reference's messages.  Plain CPython API: no torch
// headers; tensors are used through their Python attributes.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <dlfcn.h>
#include <limits.h>
#include <stdlib.h>

#include <cstdint>
#include <string>
#include <vector>

namespace {

typedef int (*pack_fn)(const void *, int64_t, int64_t, void *, int32_t *, int64_t *, float *, const int64_t *);
typedef int (*merge_fn)(const void *, int64_t, int64_t, void *, void *, const int64_t *, const void *, int64_t,
                        void *);
typedef const char *(*error_fn)(void);

pack_fn g_pack = nullptr;
merge_fn g_merge = nullptr;
error_fn g_error = nullptr;
PyObject *g_torch = nullptr;      // the torch module
PyObject *g_bf16 = nullptr;       // torch.bfloat16
PyObject *g_int64 = nullptr;      // torch.int64

PyObject *runtime_error(const char *msg) {
    PyErr_SetString(PyExc_RuntimeError, msg);
    return nullptr;
}

PyObject *library_error(const char *what) {
    std::string msg = std::string(what) + ": " + (g_error ? g_error() : "unknown error");
    PyErr_SetString(PyExc_RuntimeError, msg.c_str());
    return nullptr;
}

// libpdscope_moe.so beside this module's resolved file (a symlink placed
// where the reference's loader looks resolves to the package directory),
// else the one pdscope_amd._lib names.
bool load_library() {
    void *handle = nullptr;
    Dl_info info;
    if (dladdr(reinterpret_cast<void *>(&load_library), &info) && info.dli_fname) {
        char resolved[PATH_MAX];
        if (realpath(info.dli_fname, resolved)) {
            std::string dir(resolved);
            dir = dir.substr(0, dir.find_last_of('/'));
            handle = dlopen((dir + "/libpdscope_moe.so").c_str(), RTLD_NOW | RTLD_LOCAL);
        }
    }
    if (!handle) {
        PyObject *mod = PyImport_ImportModule("pdscope_amd._lib");
        if (!mod) return false;
        PyObject *path = PyObject_GetAttrString(mod, "LIB_PATH");
        Py_DECREF(mod);
        PyObject *text = path ? PyObject_Str(path) : nullptr;
        Py_XDECREF(path);
        if (!text) return false;
        const char *p = PyUnicode_AsUTF8(text);
        if (p) handle = dlopen(p, RTLD_NOW | RTLD_LOCAL);
        Py_DECREF(text);
    }
    if (!handle) {
        PyErr_Format(PyExc_ImportError, "pdscope_layer_dispatch: libpdscope_moe.so not loadable (%s); build it with "
                                        "`python -m pdscope_amd.build`", dlerror());
        return false;
    }
    g_pack = reinterpret_cast<pack_fn>(dlsym(handle, "pdscope_dispatch_pack"));
    g_merge = reinterpret_cast<merge_fn>(dlsym(handle, "pdscope_stage_merge"));
    g_error = reinterpret_cast<error_fn>(dlsym(handle, "pdscope_last_error"));
    if (!g_pack || !g_merge || !g_error) {
        PyErr_SetString(PyExc_ImportError, "pdscope_layer_dispatch: libpdscope_moe.so lacks the dispatch entry points");
        return false;
    }
    return true;
}

// ids (any sequence of ints) -> int64 vector
bool read_ids(PyObject *seq, std::vector<int64_t> &ids) {
    PyObject *fast = PySequence_Fast(seq, "ids must be a sequence of expert ids");
    if (!fast) return false;
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(fast);
    ids.resize(static_cast<size_t>(n));
    for (Py_ssize_t i = 0; i < n; ++i) {
        ids[static_cast<size_t>(i)] = PyLong_AsLongLong(PySequence_Fast_GET_ITEM(fast, i));
        if (ids[static_cast<size_t>(i)] == -1 && PyErr_Occurred()) {
            Py_DECREF(fast);
            return false;
        }
    }
    Py_DECREF(fast);
    return true;
}

// truth value of tensor attribute `name`; -1 with an exception set on error
int flag(PyObject *t, const char *name) {
    PyObject *v = PyObject_GetAttrString(t, name);
    if (!v) return -1;
    const int r = PyObject_IsTrue(v);
    Py_DECREF(v);
    return r;
}

// integer result of a zero-argument tensor method
bool int_method(PyObject *t, const char *name, long long &out) {
    PyObject *v = PyObject_CallMethod(t, name, nullptr);
    if (!v) return false;
    out = PyLong_AsLongLong(v);
    Py_DECREF(v);
    return !(out == -1 && PyErr_Occurred());
}

bool same_object_attr(PyObject *t, const char *name, PyObject *want, int &eq) {
    PyObject *v = PyObject_GetAttrString(t, name);
    if (!v) return false;
    eq = PyObject_RichCompareBool(v, want, Py_EQ);
    Py_DECREF(v);
    return eq >= 0;
}

// device index of a CUDA tensor
bool device_index(PyObject *t, long long &index) { return int_method(t, "get_device", index); }

bool check_cuda(PyObject *scratch, PyObject *out, PyObject *tokens, PyObject *weights, bool &ok) {
    ok = true;
    for (PyObject *t : {scratch, out, tokens, weights}) {
        const int c = flag(t, "is_cuda");
        if (c < 0) return false;
        ok = ok && c;
    }
    return true;
}

// pdscope_dispatch_pack + layer.forward_task + pool.submit
PyObject *do_submit(PyObject *pool, PyObject *layer, long long row_ptr, long long rows, long long row_bytes,
                    long long packed_ptr, long long block_ptr, long long count_ptr, long long selected_ptr,
                    long long coeff_ptr, const std::vector<int64_t> &ids) {
    if (g_pack(reinterpret_cast<const void *>(row_ptr), rows, row_bytes, reinterpret_cast<void *>(packed_ptr),
               reinterpret_cast<int32_t *>(count_ptr), reinterpret_cast<int64_t *>(selected_ptr),
               reinterpret_cast<float *>(coeff_ptr), ids.data()) != 0)
        return library_error("pdscope_dispatch_pack");
    // one packed call for the whole layer group
    PyObject *task = PyObject_CallMethod(layer, "forward_task", "LiLLLLO", count_ptr, 1, selected_ptr, coeff_ptr,
                                         packed_ptr, block_ptr, Py_False);
    if (!task) return nullptr;
    PyObject *r = PyObject_CallMethod(pool, "submit", "O", task);
    Py_DECREF(task);
    return r;
}

// scratch size check, then stage + merge on the current stream of out's device
PyObject *do_stage_merge(long long block_ptr, long long rows, long long row_bytes, PyObject *scratch, PyObject *out,
                         PyObject *tokens, PyObject *weights) {
    long long numel = 0, esize = 0;
    if (!int_method(scratch, "numel", numel) || !int_method(scratch, "element_size", esize)) return nullptr;
    if (numel * esize != rows * row_bytes) return runtime_error("scratch buffer must match the packed block");
    int eq = 0;
    for (PyObject *t : {scratch, out, weights}) {
        if (!same_object_attr(t, "dtype", g_bf16, eq)) return nullptr;
        if (!eq) return runtime_error("scratch, out and weights must be bf16");
    }
    long long dev = 0, d = 0;
    if (!device_index(out, dev)) return nullptr;
    for (PyObject *t : {scratch, tokens, weights}) {
        if (!device_index(t, d)) return nullptr;
        if (d != dev) return runtime_error("scratch/out/tokens/weights must be on one device");
    }
    long long out_dim = 0, out_rows = 0, out_cols = 0;
    if (!int_method(out, "dim", out_dim)) return nullptr;
    const int out_contig = [&] {
        PyObject *v = PyObject_CallMethod(out, "is_contiguous", nullptr);
        if (!v) return -1;
        const int r = PyObject_IsTrue(v);
        Py_DECREF(v);
        return r;
    }();
    if (out_contig < 0) return nullptr;
    if (out_dim == 2) {
        PyObject *s0 = PyObject_CallMethod(out, "size", "i", 0);
        PyObject *s1 = s0 ? PyObject_CallMethod(out, "size", "i", 1) : nullptr;
        if (!s1) {
            Py_XDECREF(s0);
            return nullptr;
        }
        out_rows = PyLong_AsLongLong(s0);
        out_cols = PyLong_AsLongLong(s1);
        Py_DECREF(s0);
        Py_DECREF(s1);
    }
    if (out_dim != 2 || !out_contig || out_cols * 2 != row_bytes)
        return runtime_error("out must be a contiguous [tokens, hidden] tensor of the block's row width");
    // the merge reads contiguous int64 token indices and bf16 weights
    PyObject *tok = PyObject_CallMethod(tokens, "to", "O", g_int64);
    PyObject *tokc = tok ? PyObject_CallMethod(tok, "contiguous", nullptr) : nullptr;
    Py_XDECREF(tok);
    PyObject *wc = tokc ? PyObject_CallMethod(weights, "contiguous", nullptr) : nullptr;
    PyObject *cur = nullptr, *stream = nullptr;
    PyObject *result = nullptr;
    long long tn = 0, wn = 0, tok_ptr = 0, w_ptr = 0, s_ptr = 0, o_ptr = 0, h_stream = 0;
    if (!wc) goto done;
    if (!int_method(tokc, "numel", tn) || !int_method(wc, "numel", wn)) goto done;
    if (tn != rows || wn != rows) {
        runtime_error("tokens and weights must hold one entry per packed row");
        goto done;
    }
    if (!int_method(tokc, "data_ptr", tok_ptr) || !int_method(wc, "data_ptr", w_ptr) ||
        !int_method(scratch, "data_ptr", s_ptr) || !int_method(out, "data_ptr", o_ptr))
        goto done;
    {
        PyObject *cuda = PyObject_GetAttrString(g_torch, "cuda");
        if (!cuda) goto done;
        cur = PyObject_CallMethod(cuda, "current_stream", "L", dev);
        Py_DECREF(cuda);
    }
    if (!cur) goto done;
    stream = PyObject_GetAttrString(cur, "cuda_stream");
    if (!stream) goto done;
    h_stream = PyLong_AsLongLong(stream);
    if (h_stream == -1 && PyErr_Occurred()) goto done;
    if (g_merge(reinterpret_cast<const void *>(block_ptr), rows, row_bytes, reinterpret_cast<void *>(s_ptr),
                reinterpret_cast<void *>(o_ptr), reinterpret_cast<const int64_t *>(tok_ptr),
                reinterpret_cast<const void *>(w_ptr), out_rows, reinterpret_cast<void *>(h_stream)) != 0) {
        library_error("pdscope_stage_merge");
        goto done;
    }
    Py_INCREF(out);
    result = out;
done:
    Py_XDECREF(stream);
    Py_XDECREF(cur);
    Py_XDECREF(wc);
    Py_XDECREF(tokc);
    return result;
}

PyObject *submit_group(PyObject *, PyObject *args) {
    PyObject *pool, *layer, *ids_obj;
    long long row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr, coeff_ptr;
    if (!PyArg_ParseTuple(args, "OOLLLLLLLLO", &pool, &layer, &row_ptr, &rows, &row_bytes, &packed_ptr, &block_ptr,
                          &count_ptr, &selected_ptr, &coeff_ptr, &ids_obj))
        return nullptr;
    std::vector<int64_t> ids;
    if (!read_ids(ids_obj, ids)) return nullptr;
    if (rows < 1 || row_bytes < 2 || row_bytes % 2 != 0) return runtime_error("invalid decode pack shape");
    if (static_cast<long long>(ids.size()) != rows)
        return runtime_error("expert id count must match the packed row count");
    return do_submit(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr,
                     coeff_ptr, ids);
}

PyObject *finish_and_merge(PyObject *, PyObject *args) {
    PyObject *pool, *scratch, *out, *tokens, *weights;
    long long block_ptr, rows, row_bytes;
    if (!PyArg_ParseTuple(args, "OLLLOOOO", &pool, &block_ptr, &rows, &row_bytes, &scratch, &out, &tokens, &weights))
        return nullptr;
    bool on_device = false;
    if (!check_cuda(scratch, out, tokens, weights, on_device)) return nullptr;
    if (!on_device) return runtime_error("scratch/out/tokens/weights must live on the CUDA device");
    PyObject *r = PyObject_CallMethod(pool, "sync", nullptr);
    if (!r) return nullptr;
    Py_DECREF(r);
    return do_stage_merge(block_ptr, rows, row_bytes, scratch, out, tokens, weights);
}

PyObject *submit_and_merge(PyObject *, PyObject *args) {
    PyObject *pool, *layer, *scratch, *ids_obj, *out, *tokens, *weights;
    long long row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr, coeff_ptr;
    if (!PyArg_ParseTuple(args, "OOLLLLLOLLLOOOO", &pool, &layer, &row_ptr, &rows, &row_bytes, &packed_ptr,
                          &block_ptr, &scratch, &count_ptr, &selected_ptr, &coeff_ptr, &ids_obj, &out, &tokens,
                          &weights))
        return nullptr;
    std::vector<int64_t> ids;
    if (!read_ids(ids_obj, ids)) return nullptr;
    if (rows < 1 || row_bytes < 2 || row_bytes % 2 != 0) return runtime_error("invalid decode pack shape");
    if (static_cast<long long>(ids.size()) != rows)
        return runtime_error("expert id count must match the packed row count");
    bool on_device = false;
    if (!check_cuda(scratch, out, tokens, weights, on_device)) return nullptr;
    if (!on_device) return runtime_error("scratch/out/tokens/weights must live on the CUDA device");
    PyObject *r = do_submit(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr,
                            coeff_ptr, ids);
    if (!r) return nullptr;
    Py_DECREF(r);
    r = PyObject_CallMethod(pool, "sync", nullptr);
    if (!r) return nullptr;
    Py_DECREF(r);
    return do_stage_merge(block_ptr, rows, row_bytes, scratch, out, tokens, weights);
}

PyMethodDef methods[] = {
    {"submit_and_merge", submit_and_merge, METH_VARARGS,
     "Native decode MoE tail: submit, join, stage and merge in one call"},
    {"submit_group", submit_group, METH_VARARGS,
     "Pack and submit the decode CPU group to the native queue without joining it"},
    {"finish_and_merge", finish_and_merge, METH_VARARGS,
     "Join the native queue, stage the packed block and scatter it into the output"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef module_def = {PyModuleDef_HEAD_INIT, "pdscope_layer_dispatch",
                          "Native decode MoE tail on the gfx950 library (reference: native/native_layer_dispatch.cpp)",
                          -1, methods, nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit_pdscope_layer_dispatch(void) {
    if (!load_library()) return nullptr;
    g_torch = PyImport_ImportModule("torch");
    if (!g_torch) return nullptr;
    g_bf16 = PyObject_GetAttrString(g_torch, "bfloat16");
    g_int64 = g_bf16 ? PyObject_GetAttrString(g_torch, "int64") : nullptr;
    if (!g_int64) return nullptr;
    return PyModule_Create(&module_def);
}
