"""ctypes binding of the CPU oracle (liboracle_attention.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_attention.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "liboracle_attention.so"], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    fp, sz, u8p = ctypes.POINTER(ctypes.c_float), ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint8)
    for name in ("oracle_ref_attention_heads", "oracle_pa_attention_f32_heads"):
        f = getattr(lib, name)
        f.restype = ctypes.c_bool
        f.argtypes = [fp, fp, fp, sz, sz, sz, sz, u8p, fp, fp, sz, sz]
    for name in ("oracle_pa_attention_f32_multi_kv", "oracle_ref_attention_multi_kv"):
        f = getattr(lib, name)
        f.restype = ctypes.c_bool
        f.argtypes = [fp, sz, sz, fp, fp, sz, sz, sz, sz, u8p, sz, fp, fp, sz, sz, sz]
    lib.oracle_attention_heads_checked.restype = ctypes.c_int
    lib.oracle_attention_heads_checked.argtypes = [fp, sz, fp, sz, fp, sz, sz, sz, u8p, sz,
                                                   ctypes.c_int, sz, sz, ctypes.c_int, fp]
    lib.oracle_encoder_mask.restype = ctypes.c_int
    lib.oracle_encoder_mask.argtypes = [sz, sz, sz, sz, ctypes.c_int, u8p]
    lib.oracle_retained_count.restype = sz
    lib.oracle_retained_count.argtypes = [sz, sz, ctypes.c_int]
    lib.oracle_threaded_attention.restype = ctypes.c_bool
    lib.oracle_threaded_attention.argtypes = [ctypes.c_int, ctypes.c_int, fp, sz, fp, fp, sz, sz,
                                              sz, sz, ctypes.c_int, sz, sz, sz, fp]
    _lib = lib
    return lib


def _f(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)) if a is not None else None


def _f32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))


def _mask(x):
    if x is None:
        return None
    return np.ascontiguousarray(np.asarray(x).reshape(-1)).astype(np.uint8)


def heads(query, keys, values, qheads, kvheads, dim, nkeys, allowed=None, h_first=0,
          h_end=None, binary32=False):
    """p9_ref_attention_heads (exact) or pa_attention_f32_heads (binary32):
    returns (ok, out[(h_end-h_first)*dim])."""
    lib = load()
    h_end = qheads if h_end is None else h_end
    q, k, v, m = _f32(query), _f32(keys), _f32(values), _mask(allowed)
    scratch = np.zeros(max(nkeys, 1), np.float32)
    out = np.zeros(max((h_end - h_first) * dim, 1), np.float32)
    fn = lib.oracle_pa_attention_f32_heads if binary32 else lib.oracle_ref_attention_heads
    ok = fn(_f(q), _f(k), _f(v), qheads, kvheads, dim, nkeys, _u(m), _f(scratch), _f(out),
            h_first, h_end)
    return bool(ok), out[:max(h_end - h_first, 0) * dim]


def multi_kv(query, nq, q_stride, keys, values, qheads, kvheads, dim, nkeys, allowed,
             mask_stride, o_stride, kh_first, kh_end, binary32=False):
    """The multi-query contract: one single-query call per query."""
    lib = load()
    q, k, v, m = _f32(query), _f32(keys), _f32(values), _mask(allowed)
    scratch = np.zeros(max(nkeys, 1), np.float32)
    out = np.zeros(max(nq * o_stride, 1), np.float32)
    fn = lib.oracle_pa_attention_f32_multi_kv if binary32 else lib.oracle_ref_attention_multi_kv
    ok = fn(_f(q), nq, q_stride, _f(k), _f(v), qheads, kvheads, dim, nkeys, _u(m), mask_stride,
            _f(scratch), _f(out), o_stride, kh_first, kh_end)
    return bool(ok), out[:nq * o_stride]


def attention_heads_checked(query, keys, values, kv_heads, head_dim, allowed=None, heads=None):
    """kernels::reference::attention_heads: (status, out)."""
    lib = load()
    q, k, v = _f32(query), _f32(keys), _f32(values)
    m = _mask(allowed) if allowed is not None else np.zeros(1, np.uint8)
    h0, h1 = (0, 0) if heads is None else heads
    qheads = q.size // head_dim if head_dim else 0
    n = (h1 - h0) if heads is not None else qheads
    out = np.zeros(max(n * head_dim, 1), np.float32)
    rc = lib.oracle_attention_heads_checked(
        _f(q), q.size, _f(k), k.size, _f(v), v.size, kv_heads, head_dim, _u(m),
        m.size if allowed is not None else 0, int(allowed is not None), h0, h1,
        int(heads is not None), _f(out))
    return rc, out[:max(n, 0) * head_dim]


def encoder_mask(first_key, count, query, window=None):
    lib = load()
    out = np.zeros(max(count, 1), np.uint8)
    rc = lib.oracle_encoder_mask(first_key, count, query, window or 0, int(window is not None),
                                 _u(out))
    if rc != 0:
        return None
    return out[:count].astype(bool)


def retained_count(count, window=None):
    return int(load().oracle_retained_count(count, window or 0, int(window is not None)))


def threaded(query, nq, keys, values, qheads, kvheads, dim, nkeys, causal, first_key=0,
             first_query=0, window=0, threads=1, binary32=False):
    """The engine-threaded CPU path over nq queries: (ok, out[nq*qheads*dim])."""
    lib = load()
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.zeros(nq * qheads * dim, np.float32)
    ok = lib.oracle_threaded_attention(int(binary32), threads, _f(q), nq, _f(k), _f(v), qheads,
                                       kvheads, dim, nkeys, int(causal), first_key, first_query,
                                       window, _f(out))
    return bool(ok), out
