// pdscope_amd._records: the base type of the ledger's immutable key records
// (ExpertKey, LoadTicket in pdscope_amd/cache.py).
//
// The ledger hashes and compares these records several times per routed
// expert on every layer call (its maps are keyed by them).  A record computes
// its field tuple and that tuple's hash once, at construction; this base
// stores both in C fields (_t, _h) and answers hash() and ==/!= from them in
// C, with no Python frame per lookup.  Equality holds only between records of
// the same class with equal field tuples (a record never equals a plain
// tuple); the other comparisons are left to the subclass.
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <structmember.h>

#include <cstddef>

namespace {

struct HashedRecord {
    PyObject_HEAD
    Py_hash_t hash;
    PyObject *fields;
};

Py_hash_t record_hash(PyObject *self) {
    const Py_hash_t h = reinterpret_cast<HashedRecord *>(self)->hash;
    return h == -1 ? -2 : h;  // -1 signals an error to the interpreter
}

PyObject *record_richcompare(PyObject *a, PyObject *b, int op) {
    if ((op != Py_EQ && op != Py_NE) || Py_TYPE(a) != Py_TYPE(b)) Py_RETURN_NOTIMPLEMENTED;
    bool equal;
    if (a == b) {
        equal = true;
    } else {
        auto *x = reinterpret_cast<HashedRecord *>(a);
        auto *y = reinterpret_cast<HashedRecord *>(b);
        if (!x->fields || !y->fields) {
            PyErr_SetString(PyExc_TypeError, "record compared before its fields were set");
            return nullptr;
        }
        if (x->hash != y->hash) {
            equal = false;
        } else {
            const int r = PyObject_RichCompareBool(x->fields, y->fields, Py_EQ);
            if (r < 0) return nullptr;
            equal = r == 1;
        }
    }
    if (equal == (op == Py_EQ)) Py_RETURN_TRUE;
    Py_RETURN_FALSE;
}

int record_traverse(PyObject *self, visitproc visit, void *arg) {
    Py_VISIT(reinterpret_cast<HashedRecord *>(self)->fields);
    return 0;
}

int record_clear(PyObject *self) {
    Py_CLEAR(reinterpret_cast<HashedRecord *>(self)->fields);
    return 0;
}

void record_dealloc(PyObject *self) {
    PyObject_GC_UnTrack(self);
    record_clear(self);
    Py_TYPE(self)->tp_free(self);
}

PyMemberDef record_members[] = {
    {const_cast<char *>("_h"), T_PYSSIZET, offsetof(HashedRecord, hash), 0,
     const_cast<char *>("hash of the field tuple, set once at construction")},
    {const_cast<char *>("_t"), T_OBJECT_EX, offsetof(HashedRecord, fields), 0,
     const_cast<char *>("the record's field tuple, set once at construction")},
    {nullptr, 0, 0, 0, nullptr},
};

PyTypeObject record_type = {PyVarObject_HEAD_INIT(nullptr, 0) "pdscope_amd._records.HashedRecord"};

PyModuleDef module_def = {
    PyModuleDef_HEAD_INIT, "_records",
    "Base type of the ledger's key records: hash and equality from cached fields, in C.", -1, nullptr,
};

}  // namespace

PyMODINIT_FUNC PyInit__records(void) {
    record_type.tp_basicsize = sizeof(HashedRecord);
    record_type.tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_BASETYPE | Py_TPFLAGS_HAVE_GC;
    record_type.tp_doc = "Record with a cached field tuple (_t) and hash (_h); hash and ==/!= in C.";
    record_type.tp_new = PyType_GenericNew;
    record_type.tp_hash = record_hash;
    record_type.tp_richcompare = record_richcompare;
    record_type.tp_traverse = record_traverse;
    record_type.tp_clear = record_clear;
    record_type.tp_dealloc = record_dealloc;
    record_type.tp_members = record_members;
    if (PyType_Ready(&record_type) < 0) return nullptr;
    PyObject *m = PyModule_Create(&module_def);
    if (!m) return nullptr;
    Py_INCREF(&record_type);
    if (PyModule_AddObject(m, "HashedRecord", reinterpret_cast<PyObject *>(&record_type)) < 0) {
        Py_DECREF(&record_type);
        Py_DECREF(m);
        return nullptr;
    }
    return m;
}
