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
    lib.oracle_xorshift_units.restype = None
    lib.oracle_xorshift_units.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_float, sz,
                                          fp]
    lib.oracle_ref_attention_heads_checker.restype = ctypes.c_bool
    lib.oracle_ref_attention_heads_checker.argtypes = [fp, fp, fp, sz, sz, sz, sz, u8p, fp, fp,
                                                       sz, sz]
    lib.oracle_ref_attention_heads_softcap.restype = ctypes.c_bool
    lib.oracle_ref_attention_heads_softcap.argtypes = [fp, fp, fp, sz, sz, sz, sz, u8p, fp, fp,
                                                       sz, sz, ctypes.c_float]
    lib.oracle_threaded_attention_sample.restype = ctypes.c_bool
    lib.oracle_threaded_attention_sample.argtypes = [ctypes.c_int, ctypes.c_int, fp, sz, sz, fp,
                                                     fp, sz, sz, sz, sz, ctypes.c_int, sz, sz, sz,
                                                     fp]
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
          h_end=None, binary32=False, checker=False, softcap=0.0):
    """p9_ref_attention_heads (exact), its bit-identical checker form
    (checker=True), pa_attention_f32_heads (binary32) or the exact path with a
    logit soft-cap (softcap > 0): returns (ok, out[(h_end-h_first)*dim])."""
    lib = load()
    h_end = qheads if h_end is None else h_end
    q, k, v, m = _f32(query), _f32(keys), _f32(values), _mask(allowed)
    scratch = np.zeros(max(nkeys, 1), np.float32)
    out = np.zeros(max((h_end - h_first) * dim, 1), np.float32)
    args = [_f(q), _f(k), _f(v), qheads, kvheads, dim, nkeys, _u(m), _f(scratch), _f(out),
            h_first, h_end]
    if softcap:
        assert not (binary32 or checker)
        ok = lib.oracle_ref_attention_heads_softcap(*args, softcap)
    else:
        fn = (lib.oracle_pa_attention_f32_heads if binary32 else
              lib.oracle_ref_attention_heads_checker if checker else
              lib.oracle_ref_attention_heads)
        ok = fn(*args)
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
             first_query=0, window=0, threads=1, binary32=False, checker=False, query_step=1):
    """The engine-threaded CPU path over nq queries: (ok, out[nq*qheads*dim]).
    checker=True runs the exact path's bit-identical fast form (finite value
    rows), for checking full-size outputs; the default is the form timed as
    the CPU baseline."""
    lib = load()
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.zeros(nq * qheads * dim, np.float32)
    variant = 1 if binary32 else (2 if checker else 0)
    ok = lib.oracle_threaded_attention_sample(variant, threads, _f(q), nq, query_step, _f(k),
                                              _f(v), qheads,
                                       kvheads, dim, nkeys, int(causal), first_key, first_query,
                                       window, _f(out))
    return bool(ok), out


class _CacheStruct(ctypes.Structure):
    _fields_ = [("width", ctypes.c_size_t), ("context", ctypes.c_size_t),
                ("window", ctypes.c_size_t), ("has_window", ctypes.c_int),
                ("max_bytes", ctypes.c_size_t), ("total", ctypes.c_size_t),
                ("start", ctypes.c_size_t), ("len", ctypes.c_size_t), ("cap", ctypes.c_size_t),
                ("keys", ctypes.POINTER(ctypes.c_float)),
                ("values", ctypes.POINTER(ctypes.c_float))]


def _cache_lib():
    lib = load()
    if not getattr(lib, "_cache_bound", False):
        cp, sz = ctypes.POINTER(_CacheStruct), ctypes.c_size_t
        fp, szp = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_size_t)
        for name, res, args in (
                ("oracle_cache_init", ctypes.c_int, [cp, sz, sz, sz, sz, ctypes.c_int, sz]),
                ("oracle_cache_free", None, [cp]),
                ("oracle_cache_retained", sz, [cp]),
                ("oracle_cache_append", ctypes.c_int, [cp, fp, fp, sz, szp, szp]),
                ("oracle_cache_rollback", None, [cp, sz, sz]),
                ("oracle_cache_keep", None, [cp, sz, sz, sz]),
                ("oracle_cache_commit", None, [cp])):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        lib._cache_bound = True
    return lib


class OracleCache:
    """The LayerCache restatement (oracle_cache_*). Pending records are
    (old_len, old_total) with old_len in floats, as the engine keeps them."""

    def __init__(self, kv_heads, head_dim, context, window, max_bytes):
        self.lib = _cache_lib()
        self.c = _CacheStruct()
        self.status = self.lib.oracle_cache_init(ctypes.byref(self.c), kv_heads, head_dim,
                                                 context, window or 0, int(window is not None),
                                                 max_bytes)

    def __del__(self):
        try:
            self.lib.oracle_cache_free(ctypes.byref(self.c))
        except Exception:
            pass

    @property
    def total(self):
        return self.c.total

    def retained(self):
        return int(self.lib.oracle_cache_retained(ctypes.byref(self.c)))

    def first_position(self):
        return self.c.total - self.retained()

    def rows(self):
        """(keys, values) of the retained rows, [retained][width] copies."""
        w, s, n = self.c.width, self.c.start, self.c.len
        if n == s:
            return np.zeros((0, w), np.float32), np.zeros((0, w), np.float32)
        k = np.ctypeslib.as_array(self.c.keys, shape=(n,))[s:].reshape(-1, w).copy()
        v = np.ctypeslib.as_array(self.c.values, shape=(n,))[s:].reshape(-1, w).copy()
        return k, v

    def append(self, keys, values, n):
        k, v = _f32(keys), _f32(values)
        old_len, old_total = ctypes.c_size_t(), ctypes.c_size_t()
        rc = self.lib.oracle_cache_append(ctypes.byref(self.c), _f(k), _f(v), n,
                                          ctypes.byref(old_len), ctypes.byref(old_total))
        return rc, (old_len.value, old_total.value)

    def rollback(self, pending):
        self.lib.oracle_cache_rollback(ctypes.byref(self.c), pending[0], pending[1])

    def keep(self, pending, tokens):
        self.lib.oracle_cache_keep(ctypes.byref(self.c), pending[0], pending[1], tokens)

    def commit(self):
        self.lib.oracle_cache_commit(ctypes.byref(self.c))


def _transform_lib():
    lib = load()
    if not getattr(lib, "_transform_bound", False):
        fp, sz = ctypes.POINTER(ctypes.c_float), ctypes.c_size_t
        lib.oracle_rms_norm.restype = None
        lib.oracle_rms_norm.argtypes = [fp, fp, sz, ctypes.c_float, fp]
        lib.oracle_rope.restype = ctypes.c_bool
        lib.oracle_rope.argtypes = [fp, sz, sz, sz, ctypes.c_float, fp, fp]
        lib.oracle_libm_digest.restype = ctypes.c_uint64
        lib.oracle_libm_digest.argtypes = [ctypes.c_int]
        lib._transform_bound = True
    return lib


def rms_norm(x, scale, eps):
    """p9_ref_rms_norm over one row."""
    lib = _transform_lib()
    x = _f32(x)
    s = _f32(scale) if scale is not None else None
    out = np.zeros(x.size, np.float32)
    lib.oracle_rms_norm(_f(x), _f(s) if s is not None else None, x.size, eps, _f(out))
    return out


def rope(x, dim, position, base, factors=None):
    """p9_ref_rope over whole heads: (ok, out)."""
    lib = _transform_lib()
    x = _f32(x)
    f = _f32(factors) if factors is not None else None
    out = np.zeros(x.size, np.float32)
    ok = lib.oracle_rope(_f(x), x.size // dim, dim, position, base,
                         _f(f) if f is not None else None, _f(out))
    return bool(ok), out


def libm_digest(which):
    """0: powf, 1: sincosf (see oracle_libm_digest)."""
    return int(_transform_lib().oracle_libm_digest(which))


def head_transform(raw_q, raw_k, raw_v, qheads, kvheads, dim, position, query_scale, key_scale,
                   eps, base, factors=None):
    """HeadTransform::prepare (src/engine/attention.rs:102-156) for one token:
    per-head norms, then rotation of Q and K; V = norm(raw V or raw K)."""
    q = np.concatenate([rms_norm(h, query_scale, eps) for h in _f32(raw_q).reshape(qheads, dim)])
    k = np.concatenate([rms_norm(h, key_scale, eps) for h in _f32(raw_k).reshape(kvheads, dim)])
    src = raw_v if raw_v is not None else raw_k
    v = np.concatenate([rms_norm(h, None, eps) for h in _f32(src).reshape(kvheads, dim)])
    okq, q = rope(q, dim, position, base, factors)
    okk, k = rope(k, dim, position, base, factors)
    return okq and okk, q, k, v


def _block_lib():
    lib = _transform_lib()
    if not getattr(lib, "_block_bound", False):
        fp, sz = ctypes.POINTER(ctypes.c_float), ctypes.c_size_t
        lib.oracle_matvec.restype = None
        lib.oracle_matvec.argtypes = [fp, fp, sz, sz, fp]
        lib.oracle_add.restype = None
        lib.oracle_add.argtypes = [fp, fp, sz, fp]
        lib._block_bound = True
    return lib


def matvec(matrix, x, rows, cols):
    """p9_ref_matvec: [rows] f32."""
    lib = _block_lib()
    m, v = _f32(matrix), _f32(x)
    out = np.zeros(rows, np.float32)
    lib.oracle_matvec(_f(m), _f(v), rows, cols, _f(out))
    return out


def add(a, b):
    lib = _block_lib()
    a, b = _f32(a), _f32(b)
    out = np.zeros(a.size, np.float32)
    lib.oracle_add(_f(a), _f(b), a.size, _f(out))
    return out


def attention_output(attended, weights, post_scale, eps, residual, rows, cols):
    """The output block of one token (src/engine/attention.rs:866-884):
    (projected, residual + rms_norm(projected, post_scale, eps))."""
    projected = matvec(weights, attended, rows, cols)
    return projected, add(residual, rms_norm(projected, post_scale, eps))


def xorshift_units(state, n, scale=1.0):
    """n values of the reference tests' xorshift64 stream from `state`
    (oracle_xorshift_units); returns (values, the advanced state)."""
    st = ctypes.c_uint64(state)
    out = np.empty(n, np.float32)
    load().oracle_xorshift_units(ctypes.byref(st), np.float32(scale), n, _f(out))
    return out, int(st.value)
