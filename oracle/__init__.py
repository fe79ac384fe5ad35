"""Python access to the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the checker. The product
(``rccl_amd``) never imports it.

Every function mirrors one C function in ``oracle.c``; see that file for the
reference file:line each one restates. Arrays are numpy arrays; sorting
functions work on copies and return them.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

# Key kinds (numbering equals include/rccl_hip.h).
KEY_KINDS = {
    "u32": 0, "i32": 1, "f32": 2, "u64": 3, "i64": 4, "f64": 5,
    "u8": 6, "i8": 7, "u16": 8, "i16": 9,
}
KIND_DTYPES = {
    "u32": np.uint32, "i32": np.int32, "f32": np.float32,
    "u64": np.uint64, "i64": np.int64, "f64": np.float64,
    "u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16,
}
SET_OPS = {"union": 0, "intersection": 1, "difference": 2, "symmetric_difference": 3}

_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        c = ctypes
        lib.oracle_splitmix64.restype = c.c_uint64
        lib.oracle_splitmix64.argtypes = [c.c_uint64]
        lib.oracle_radix_ordered.restype = c.c_uint64
        lib.oracle_radix_ordered.argtypes = [c.c_int, c.c_int, c.c_uint64]
        lib.oracle_radix_digit_source.restype = c.c_uint64
        lib.oracle_radix_digit_source.argtypes = [c.c_int, c.c_int, c.c_uint64]
        lib.oracle_radix_sort.restype = c.c_int
        lib.oracle_radix_sort.argtypes = [c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                          c.c_size_t, c.c_size_t, c.c_uint, c.c_uint]
        lib.oracle_merge.restype = c.c_int
        lib.oracle_merge.argtypes = [c.c_int, c.c_int, c.c_void_p, c.c_void_p, c.c_size_t,
                                     c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p,
                                     c.c_void_p, c.c_size_t]
        lib.oracle_merge_sort.restype = c.c_int
        lib.oracle_merge_sort.argtypes = [c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                          c.c_size_t, c.c_size_t]
        lib.oracle_set_op.restype = c.c_longlong
        lib.oracle_set_op.argtypes = [c.c_int, c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                      c.c_size_t, c.c_void_p, c.c_void_p, c.c_size_t,
                                      c.c_void_p, c.c_void_p, c.c_size_t]
        lib.oracle_record_sort.restype = c.c_int
        lib.oracle_record_sort.argtypes = [c.c_uint, c.c_void_p, c.c_void_p, c.c_size_t,
                                           c.c_size_t]
        lib.oracle_unique.restype = c.c_longlong
        lib.oracle_unique.argtypes = [c.c_int, c.c_uint, c.c_void_p, c.c_void_p, c.c_size_t]
        lib.oracle_reduce_by_key.restype = c.c_longlong
        lib.oracle_reduce_by_key.argtypes = [c.c_int, c.c_uint, c.c_int, c.c_void_p, c.c_void_p,
                                             c.c_void_p, c.c_void_p, c.c_size_t]
        lib.oracle_prob_or.restype = c.c_double
        lib.oracle_prob_or.argtypes = [c.c_double, c.c_double]
        lib.oracle_sort_unstable_u32.restype = c.c_int
        lib.oracle_sort_unstable_u32.argtypes = [c.c_void_p, c.c_size_t]
        lib.oracle_par_sort_unstable_u32.restype = c.c_int
        lib.oracle_par_sort_unstable_u32.argtypes = [c.c_void_p, c.c_size_t, c.c_int]
        lib.oracle_stable_sort_pairs_u64_u32.restype = c.c_int
        lib.oracle_stable_sort_pairs_u64_u32.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t,
                                                         c.c_int]
        lib.oracle_merge_pairs_u32.restype = c.c_int
        lib.oracle_merge_pairs_u32.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p,
                                               c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p]
        lib.oracle_std_set_op_u64.restype = c.c_longlong
        lib.oracle_std_set_op_u64.argtypes = [c.c_int, c.c_void_p, c.c_size_t, c.c_void_p,
                                              c.c_size_t, c.c_void_p]
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _vbytes(values):
    return 0 if values is None else values.dtype.itemsize


def splitmix64(x: int) -> int:
    return _load().oracle_splitmix64(x)


def radix_ordered(kind: str, descending: bool, raw: int) -> int:
    return _load().oracle_radix_ordered(KEY_KINDS[kind], int(descending), raw)


def radix_digit_source(kind: str, descending: bool, raw: int) -> int:
    return _load().oracle_radix_digit_source(KEY_KINDS[kind], int(descending), raw)


def radix_sort(kind, keys, values=None, descending=False, begin_bit=0, end_bit=None):
    keys = np.ascontiguousarray(keys, dtype=KIND_DTYPES[kind]).copy()
    values = None if values is None else np.ascontiguousarray(values).copy()
    if end_bit is None:
        end_bit = keys.dtype.itemsize * 8
    rc = _load().oracle_radix_sort(KEY_KINDS[kind], int(descending), _ptr(keys), _ptr(values),
                                   _vbytes(values), keys.size, begin_bit, end_bit)
    if rc != 0:
        raise ValueError("invalid radix sort arguments")
    return (keys, values) if values is not None else keys


def merge(kind, a_keys, b_keys, a_values=None, b_values=None, descending=False):
    dt = KIND_DTYPES[kind]
    a_keys = np.ascontiguousarray(a_keys, dtype=dt)
    b_keys = np.ascontiguousarray(b_keys, dtype=dt)
    out = np.empty(a_keys.size + b_keys.size, dtype=dt)
    out_v = None
    if a_values is not None:
        a_values = np.ascontiguousarray(a_values)
        b_values = np.ascontiguousarray(b_values, dtype=a_values.dtype)
        out_v = np.empty(out.size, dtype=a_values.dtype)
    rc = _load().oracle_merge(KEY_KINDS[kind], int(descending), _ptr(a_keys), _ptr(a_values),
                              a_keys.size, _ptr(b_keys), _ptr(b_values), b_keys.size,
                              _ptr(out), _ptr(out_v), _vbytes(a_values))
    if rc != 0:
        raise ValueError("invalid merge arguments")
    return (out, out_v) if out_v is not None else out


def merge_sort(kind, keys, values=None, descending=False):
    keys = np.ascontiguousarray(keys, dtype=KIND_DTYPES[kind]).copy()
    values = None if values is None else np.ascontiguousarray(values).copy()
    rc = _load().oracle_merge_sort(KEY_KINDS[kind], int(descending), _ptr(keys), _ptr(values),
                                   _vbytes(values), keys.size)
    if rc != 0:
        raise ValueError("invalid merge sort arguments")
    return (keys, values) if values is not None else keys


def set_op(op, kind, a_keys, b_keys, a_values=None, b_values=None, descending=False,
           count_only=False):
    dt = KIND_DTYPES[kind]
    a_keys = np.ascontiguousarray(a_keys, dtype=dt)
    b_keys = np.ascontiguousarray(b_keys, dtype=dt)
    if a_values is not None:
        a_values = np.ascontiguousarray(a_values)
    if b_values is not None:
        b_values = np.ascontiguousarray(b_values, dtype=a_values.dtype)
    lib = _load()
    if count_only:
        n = lib.oracle_set_op(SET_OPS[op], KEY_KINDS[kind], int(descending), _ptr(a_keys), None,
                              a_keys.size, _ptr(b_keys), None, b_keys.size, None, None, 0)
        if n < 0:
            raise ValueError("invalid set operation arguments")
        return int(n)
    out = np.empty(a_keys.size + b_keys.size, dtype=dt)
    out_v = None if a_values is None else np.empty(out.size, dtype=a_values.dtype)
    n = lib.oracle_set_op(SET_OPS[op], KEY_KINDS[kind], int(descending), _ptr(a_keys),
                          _ptr(a_values), a_keys.size, _ptr(b_keys), _ptr(b_values),
                          b_keys.size, _ptr(out), _ptr(out_v), _vbytes(a_values))
    if n < 0:
        raise ValueError("invalid set operation arguments")
    out = out[:n]
    return (out, out_v[:n]) if out_v is not None else out


def sort_unstable_u32(keys):
    """std::sort of a copy of u32 `keys` (the slice::sort_unstable substitute
    of the CPU baseline; oracle_sort.cpp)."""
    k = np.ascontiguousarray(keys, dtype=np.uint32).copy()
    if _load().oracle_sort_unstable_u32(_ptr(k), k.size) != 0:
        raise ValueError("oracle_sort_unstable_u32 failed")
    return k


def par_sort_unstable_u32(keys, threads):
    """Parallel sort of a copy of u32 `keys` on `threads` threads (the
    parallel-sort substitute of the CPU baseline; oracle_sort.cpp)."""
    k = np.ascontiguousarray(keys, dtype=np.uint32).copy()
    if _load().oracle_par_sort_unstable_u32(_ptr(k), k.size, int(threads)) != 0:
        raise ValueError("oracle_par_sort_unstable_u32 failed")
    return k


def stable_sort_pairs_u64_u32(keys, values, threads=1):
    """Stable sort by key of copies of u64 `keys` and u32 `values` on
    `threads` threads (the stable sort_by_key / par_sort substitute of the CPU
    baseline; oracle_sort.cpp). Returns (keys, values)."""
    k = np.ascontiguousarray(keys, dtype=np.uint64).copy()
    v = np.ascontiguousarray(values, dtype=np.uint32).copy()
    if k.size != v.size:
        raise ValueError("keys and values differ in length")
    if _load().oracle_stable_sort_pairs_u64_u32(_ptr(k), _ptr(v), k.size, int(threads)) != 0:
        raise ValueError("oracle_stable_sort_pairs_u64_u32 failed")
    return k, v


def merge_pairs_u32(a, av, b, bv):
    """std::merge of u32 keys with u32 payloads, first input first on ties
    (the two-pointer merge substitute of the CPU baseline)."""
    a, av, b, bv = (np.ascontiguousarray(x, dtype=np.uint32) for x in (a, av, b, bv))
    out = np.empty(a.size + b.size, dtype=np.uint32)
    outv = np.empty_like(out)
    if _load().oracle_merge_pairs_u32(_ptr(a), _ptr(av), a.size, _ptr(b), _ptr(bv), b.size,
                                      _ptr(out), _ptr(outv)) != 0:
        raise ValueError("oracle_merge_pairs_u32 failed")
    return out, outv


def std_set_op_u64(op, a, b):
    """std::set_* over sorted u64 multisets (the host_set_by substitute of
    the CPU baseline). Returns the output keys."""
    a, b = (np.ascontiguousarray(x, dtype=np.uint64) for x in (a, b))
    out = np.empty(a.size + b.size, dtype=np.uint64)
    n = _load().oracle_std_set_op_u64(SET_OPS[op], _ptr(a), a.size, _ptr(b), b.size, _ptr(out))
    if n < 0:
        raise ValueError("oracle_std_set_op_u64 failed")
    return out[:n]


def record_sort(rows, payloads=None):
    """Stable ascending lexicographic sort of a copy of `rows` (an (n, arity)
    u32 array) and `payloads` (n items or None); returns (rows, payloads)."""
    r = np.ascontiguousarray(rows, dtype=np.uint32).copy()
    if r.ndim != 2:
        raise ValueError("rows must be a 2-D (n, arity) array")
    p = None if payloads is None else np.ascontiguousarray(payloads).copy()
    if _load().oracle_record_sort(r.shape[1], _ptr(r), _ptr(p), _vbytes(p), r.shape[0]) != 0:
        raise ValueError("oracle_record_sort: arity outside 2..6")
    return r, p


GROUP_OPS = {"natural_bag_add": 1, "boolean_or": 2, "independent_probability_or": 3}
GROUP_VALUE_DTYPES = {"natural_bag_add": np.uint64, "boolean_or": np.uint8,
                      "independent_probability_or": np.float64}


def _key_args(keys, kind):
    """(kind code, arity, contiguous array) for scalar keys of `kind` or an
    (n, arity) u32 row array (kind None)."""
    if kind is None:
        k = np.ascontiguousarray(keys, dtype=np.uint32)
        return KEY_KINDS["u32"], k.shape[1], k
    return KEY_KINDS[kind], 1, np.ascontiguousarray(keys)


def unique(keys, kind=None):
    """Stable adjacent unique of scalar keys (kind given) or rows (kind None)."""
    code, arity, k = _key_args(keys, kind)
    out = np.empty_like(k)
    n = _load().oracle_unique(code, arity, _ptr(k), _ptr(out), len(k))
    if n < 0:
        raise ValueError("oracle_unique: invalid key")
    return out[:n]


def reduce_by_key(keys, values, op, kind=None):
    """(run keys, run aggregates) of adjacent equal keys; op is one of
    GROUP_OPS."""
    code, arity, k = _key_args(keys, kind)
    v = np.ascontiguousarray(values, dtype=GROUP_VALUE_DTYPES[op])
    out_k = np.empty_like(k)
    out_v = np.empty_like(v)
    n = _load().oracle_reduce_by_key(code, arity, GROUP_OPS[op], _ptr(k), _ptr(v), _ptr(out_k),
                                     _ptr(out_v), len(k))
    if n < 0:
        raise ValueError("oracle_reduce_by_key: invalid key or operator")
    return out_k[:n], out_v[:n]


def prob_or(l: float, r: float) -> float:
    return _load().oracle_prob_or(l, r)
