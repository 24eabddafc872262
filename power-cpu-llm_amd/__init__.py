"""Python loader and host-side mirror of the gfx950 attention backend.

The product is the C-ABI library libpcl_attention.so (include/pcl_attention.h).
This module binds it with ctypes and mirrors the reference engine's attention
interface on top of it, so callers and tests use the reference's names and
error behaviour:

  HipKernels.attention / attention_heads / attention_multi / attention_multi_kv
      FmaKernels' attention methods (src/kernels/quantized/power9_fma.rs:158-255)
      with the binary32 wrappers' validation (src/kernels/quantized/int8.rs:
      489-663); errors raise AttentionError with the kind of
      kernels::reference::Error (src/kernels/reference.rs:6-11).
  Context
      the device-resident entry: device pointers, descriptor masks, two KV
      segments, launches on a stream.
  LayerCache
      the engine's LayerCache (src/engine/attention.rs:244-311) with its K/V
      rows in device memory, producing attention descriptors over them.
  HeadTransform
      the engine's HeadTransform (src/engine/attention.rs:51-243): Q/K/V head
      norms and rotary positions on the device, fused with the cache append.

There is no CPU fallback: without the built library every entry raises.
"""
import ctypes
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpcl_attention.so")

OK, INVALID_SHAPE, INVALID_PARAMETER, NON_FINITE_VALUE, RESOURCE_LIMIT = 0, 1, 2, 3, 4
ERROR_NAMES = {INVALID_SHAPE: "InvalidShape", INVALID_PARAMETER: "InvalidParameter",
               NON_FINITE_VALUE: "NonFiniteValue", RESOURCE_LIMIT: "ResourceLimit"}
(KERNEL_AUTO, KERNEL_SPLIT_KV, KERNEL_TILED, KERNEL_TILED_SPLIT, KERNEL_PIPE_KV,
 KERNEL_SPREAD_KV, KERNEL_FAN_KV) = 0, 1, 2, 3, 4, 6, 7
# every explicit kernel choice (5 is retired and refused)
KERNELS = (KERNEL_SPLIT_KV, KERNEL_TILED, KERNEL_TILED_SPLIT, KERNEL_PIPE_KV, KERNEL_SPREAD_KV,
           KERNEL_FAN_KV)
KERNEL_NAMES = {KERNEL_SPLIT_KV: "split_kv", KERNEL_TILED: "tiled",
                KERNEL_TILED_SPLIT: "tiled_split", KERNEL_PIPE_KV: "pipe_kv",
                KERNEL_SPREAD_KV: "spread_kv", KERNEL_FAN_KV: "fan_kv"}

# Every symbol include/pcl_attention.h declares.
EXPORTS = (
    "pcl_hip_attention_f32_heads",
    "pcl_hip_attention_f32_multi_kv",
    "pcl_attention_heads",
    "pcl_attention_multi_kv",
    "pcl_context_create",
    "pcl_context_create_on_stream",
    "pcl_context_destroy",
    "pcl_context_stream",
    "pcl_attention_launch",
    "pcl_attention_launch_noalloc",
    "pcl_attention_workspace_bytes",
    "pcl_context_reserve",
    "pcl_context_sync",
    "pcl_attention_resolve_kernel",
    "pcl_context_set_wait_limit",
    "pcl_debug_set_epoch_counter",
    "pcl_context_set_timing",
    "pcl_context_timing",
    "pcl_kv_cache_create",
    "pcl_kv_cache_destroy",
    "pcl_kv_cache_reserve_rows",
    "pcl_kv_cache_total_tokens",
    "pcl_kv_cache_retained_tokens",
    "pcl_kv_cache_view",
    "pcl_kv_cache_read",
    "pcl_kv_cache_append",
    "pcl_kv_cache_rollback",
    "pcl_kv_cache_keep",
    "pcl_kv_cache_commit",
    "pcl_kv_cache_encoder_desc",
    "pcl_kv_cache_decoder_desc",
    "pcl_kv_cache_shared_desc",
    "pcl_kv_cache_advance",
    "pcl_head_transform_create",
    "pcl_head_transform_destroy",
    "pcl_head_transform_prepare",
    "pcl_head_transform_query",
    "pcl_kv_cache_append_transformed",
    "pcl_kv_cache_attend_token",
    "pcl_attention_output",
    "pcl_version",
)


class AttentionError(Exception):
    """kernels::reference::Error: kind is InvalidShape, InvalidParameter or
    NonFiniteValue; the layer cache adds engine::Error::ResourceLimit."""

    def __init__(self, code):
        self.code = code
        self.kind = ERROR_NAMES.get(code, "Unknown(%d)" % code)
        super().__init__(self.kind)


class PclDesc(ctypes.Structure):
    """pcl_attention_desc."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride", ctypes.c_int64), ("nq", ctypes.c_int64),
        ("k0", ctypes.c_void_p), ("v0", ctypes.c_void_p), ("n0", ctypes.c_int64),
        ("k1", ctypes.c_void_p), ("v1", ctypes.c_void_p), ("n1", ctypes.c_int64),
        ("qheads", ctypes.c_int64), ("kvheads", ctypes.c_int64), ("dim", ctypes.c_int64),
        ("kh_first", ctypes.c_int64), ("kh_end", ctypes.c_int64),
        ("mask", ctypes.c_void_p), ("mask_stride", ctypes.c_int64),
        ("causal", ctypes.c_int32), ("window", ctypes.c_int64),
        ("first_key", ctypes.c_int64), ("first_query", ctypes.c_int64),
        ("q_scale", ctypes.c_float),
        ("out", ctypes.c_void_p), ("o_stride", ctypes.c_int64),
        ("kernel", ctypes.c_int32), ("softcap", ctypes.c_float),
    ]


class PclPending(ctypes.Structure):
    """pcl_kv_pending (PendingKv, src/engine/attention.rs:263-266), in tokens."""
    _fields_ = [("old_len", ctypes.c_int64), ("old_total", ctypes.c_int64)]


_lib = None


def library_path():
    return LIB_PATH


def load():
    """The loaded library; raises if it was not built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("libpcl_attention.so is not built: run power-cpu-llm_amd/build.py "
                           "(or __graft_entry__.build())")
    # One HIP runtime per process. PyTorch bundles its own libamdhip64 and
    # loads it under a different file name; if this library's ROCm runtime
    # were loaded first, torch would load a second one and fail to see the
    # GPU. Importing torch first makes this library bind to torch's runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    fp, vp, sz, u8p = (ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_size_t,
                       ctypes.POINTER(ctypes.c_uint8))
    lib.pcl_hip_attention_f32_heads.restype = ctypes.c_bool
    lib.pcl_hip_attention_f32_heads.argtypes = [fp, fp, fp, sz, sz, sz, sz, u8p, fp, fp, sz, sz]
    lib.pcl_hip_attention_f32_multi_kv.restype = ctypes.c_bool
    lib.pcl_hip_attention_f32_multi_kv.argtypes = [fp, sz, sz, fp, fp, sz, sz, sz, sz, u8p, sz,
                                                   fp, fp, sz, sz, sz]
    lib.pcl_attention_heads.restype = ctypes.c_int
    lib.pcl_attention_heads.argtypes = [fp, sz, fp, sz, fp, sz, sz, sz, u8p, sz, ctypes.c_int,
                                        sz, sz, ctypes.c_int, fp]
    lib.pcl_attention_multi_kv.restype = ctypes.c_int
    lib.pcl_attention_multi_kv.argtypes = [ctypes.POINTER(fp), sz, sz, fp, sz, fp, sz, sz, sz,
                                           ctypes.POINTER(u8p), sz, sz, sz, fp]
    lib.pcl_context_create.restype = ctypes.c_int
    lib.pcl_context_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
    lib.pcl_context_create_on_stream.restype = ctypes.c_int
    lib.pcl_context_create_on_stream.argtypes = [ctypes.c_int, vp, ctypes.POINTER(vp)]
    lib.pcl_context_destroy.restype = None
    lib.pcl_context_destroy.argtypes = [vp]
    lib.pcl_context_stream.restype = vp
    lib.pcl_context_stream.argtypes = [vp]
    lib.pcl_attention_launch.restype = ctypes.c_int
    lib.pcl_attention_launch.argtypes = [vp, ctypes.POINTER(PclDesc)]
    lib.pcl_attention_launch_noalloc.restype = ctypes.c_int
    lib.pcl_attention_launch_noalloc.argtypes = [vp, ctypes.POINTER(PclDesc)]
    lib.pcl_attention_workspace_bytes.restype = sz
    lib.pcl_attention_workspace_bytes.argtypes = [ctypes.POINTER(PclDesc)]
    lib.pcl_context_reserve.restype = ctypes.c_int
    lib.pcl_context_reserve.argtypes = [vp, sz]
    lib.pcl_context_sync.restype = ctypes.c_int
    lib.pcl_context_sync.argtypes = [vp, ctypes.POINTER(ctypes.c_int)]
    lib.pcl_attention_resolve_kernel.restype = ctypes.c_int
    lib.pcl_attention_resolve_kernel.argtypes = [ctypes.POINTER(PclDesc)]
    lib.pcl_context_set_wait_limit.restype = ctypes.c_int
    lib.pcl_context_set_wait_limit.argtypes = [vp, ctypes.c_int]
    lib.pcl_context_set_timing.restype = ctypes.c_int
    lib.pcl_context_set_timing.argtypes = [vp, ctypes.c_int]
    lib.pcl_context_timing.restype = ctypes.c_int
    lib.pcl_context_timing.argtypes = [vp, ctypes.POINTER(ctypes.c_double),
                                       ctypes.POINTER(ctypes.c_int64)]
    i64, i64p = ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)
    pend = ctypes.POINTER(PclPending)
    dp = ctypes.POINTER(PclDesc)
    for name, res, args in (
            ("pcl_kv_cache_create", ctypes.c_int, [vp, i64, i64, i64, i64, sz,
                                                   ctypes.POINTER(vp)]),
            ("pcl_kv_cache_destroy", None, [vp]),
            ("pcl_kv_cache_reserve_rows", ctypes.c_int, [vp, i64]),
            ("pcl_kv_cache_total_tokens", i64, [vp]),
            ("pcl_kv_cache_retained_tokens", i64, [vp]),
            ("pcl_kv_cache_view", ctypes.c_int, [vp, ctypes.POINTER(vp), ctypes.POINTER(vp),
                                                 i64p, i64p]),
            ("pcl_kv_cache_read", ctypes.c_int, [vp, i64, i64, vp, vp]),
            ("pcl_kv_cache_append", ctypes.c_int, [vp, vp, vp, i64, pend]),
            ("pcl_kv_cache_rollback", ctypes.c_int, [vp, pend]),
            ("pcl_kv_cache_keep", ctypes.c_int, [vp, pend, i64]),
            ("pcl_kv_cache_commit", ctypes.c_int, [vp]),
            ("pcl_kv_cache_encoder_desc", ctypes.c_int, [vp, pend, dp]),
            ("pcl_kv_cache_decoder_desc", ctypes.c_int, [vp, vp, vp, i64, dp]),
            ("pcl_kv_cache_shared_desc", ctypes.c_int, [vp, vp, pend, i64, dp]),
            ("pcl_kv_cache_advance", ctypes.c_int, [vp, i64, pend]),
            ("pcl_head_transform_create", ctypes.c_int,
             [vp, i64, i64, i64, ctypes.c_int, fp, fp, ctypes.c_float, ctypes.c_float, fp,
              ctypes.POINTER(vp)]),
            ("pcl_head_transform_destroy", None, [vp]),
            ("pcl_head_transform_prepare", ctypes.c_int, [vp, vp, vp, vp, i64, i64, vp, vp, vp]),
            ("pcl_head_transform_query", ctypes.c_int, [vp, vp, i64, i64, vp]),
            ("pcl_kv_cache_append_transformed", ctypes.c_int,
             [vp, vp, vp, vp, vp, i64, vp, pend]),
            ("pcl_kv_cache_attend_token", ctypes.c_int,
             [vp, vp, vp, vp, vp, ctypes.c_float, ctypes.c_int, vp, vp, pend]),
            ("pcl_attention_output", ctypes.c_int,
             [vp, vp, i64, i64, vp, i64, vp, ctypes.c_float, vp, vp, vp])):
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib.pcl_version.restype = ctypes.c_char_p
    lib.pcl_version.argtypes = []
    _lib = lib
    return lib


def _fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u8ptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def _f32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))


def _bools(x):
    return np.ascontiguousarray(np.asarray(x, dtype=bool).reshape(-1)).astype(np.uint8)


class HipKernels:
    """The attention half of an FmaKernels table whose `attention` and
    `attention_multi` pointers are this library's entries (a new
    `Request::HipF32` backend; src/kernels/quantized/power9_fma.rs:83-125)."""

    name = "hip-f32"

    def __init__(self):
        self.lib = load()

    def attention(self, query, keys, values, kv_heads, head_dim, allowed=None):
        """FmaKernels::attention (power9_fma.rs:160-170)."""
        return self.attention_heads(query, keys, values, kv_heads, head_dim, allowed, None)

    def attention_heads(self, query, keys, values, kv_heads, head_dim, allowed=None, heads=None):
        """FmaKernels::attention_heads (power9_fma.rs:237-255) through
        attention_with (int8.rs:596-663). heads: None or (start, end)."""
        q, k, v = _f32(query), _f32(keys), _f32(values)
        mask = _bools(allowed) if allowed is not None else np.zeros(1, np.uint8)
        h0, h1 = (0, 0) if heads is None else (int(heads[0]), int(heads[1]))
        qheads = q.size // head_dim if head_dim and q.size % head_dim == 0 else 0
        nout = max(h1 - h0, 0) if heads is not None else qheads
        out = np.zeros(max(nout * head_dim, 1), np.float32)
        rc = self.lib.pcl_attention_heads(
            _fptr(q), q.size, _fptr(k), k.size, _fptr(v), v.size, kv_heads, head_dim,
            _u8ptr(mask), mask.size if allowed is not None else 0, int(allowed is not None),
            h0, h1, int(heads is not None), _fptr(out))
        if rc != OK:
            raise AttentionError(rc)
        return out[:nout * head_dim]

    def attention_multi(self, queries, keys, values, kv_heads, head_dim, masks=None):
        """FmaKernels::attention_multi (power9_fma.rs:174-192)."""
        return self.attention_multi_kv(queries, keys, values, kv_heads, head_dim, masks,
                                       (0, kv_heads))

    def attention_multi_kv(self, queries, keys, values, kv_heads, head_dim, masks=None,
                           kv=None):
        """FmaKernels::attention_multi_kv (power9_fma.rs:197-232) through
        attention_multi_with (int8.rs:489-573). Returns one array per query."""
        qs = [_f32(x) for x in queries]
        if not qs:
            return []
        qlen = qs[0].size
        if any(x.size != qlen for x in qs):
            raise AttentionError(INVALID_SHAPE)
        k, v = _f32(keys), _f32(values)
        kv0, kv1 = (0, kv_heads) if kv is None else (int(kv[0]), int(kv[1]))
        width = kv_heads * head_dim
        nkeys = k.size // width if width else 0
        if masks is not None:
            ms = [_bools(m) for m in masks]
            if len(ms) != len(qs) or any(m.size != ms[0].size for m in ms):
                raise AttentionError(INVALID_SHAPE)
            mask_len = ms[0].size
            mptrs = (ctypes.POINTER(ctypes.c_uint8) * len(ms))(*[_u8ptr(m) for m in ms])
        else:
            ms, mask_len, mptrs = None, 0, None
        group = qlen // head_dim // kv_heads if head_dim and kv_heads else 0
        olen = max(kv1 - kv0, 0) * group * head_dim
        out = np.zeros(max(len(qs) * olen, 1), np.float32)
        qptrs = (ctypes.POINTER(ctypes.c_float) * len(qs))(*[_fptr(x) for x in qs])
        rc = self.lib.pcl_attention_multi_kv(
            qptrs, len(qs), qlen, _fptr(k), k.size, _fptr(v), v.size, kv_heads, head_dim,
            mptrs, mask_len, kv0, kv1, _fptr(out))
        del nkeys
        if rc != OK:
            raise AttentionError(rc)
        return [out[i * olen:(i + 1) * olen].copy() for i in range(len(qs))]


def raw_heads(query, keys, values, qheads, kvheads, dim, nkeys, allowed, h_first, h_end):
    """The AttentionF32 entry itself: (ok, out)."""
    lib = load()
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.zeros(max((h_end - h_first) * dim, 1), np.float32)
    m = _bools(allowed) if allowed is not None else None
    ok = lib.pcl_hip_attention_f32_heads(_fptr(q), _fptr(k), _fptr(v), qheads, kvheads, dim,
                                         nkeys, _u8ptr(m) if m is not None else None, None,
                                         _fptr(out), h_first, h_end)
    return bool(ok), out[:max(h_end - h_first, 0) * dim]


def raw_multi_kv(query, nq, q_stride, keys, values, qheads, kvheads, dim, nkeys, allowed,
                 mask_stride, o_stride, kh_first, kh_end):
    """The AttentionMulti entry itself: (ok, out[nq*o_stride])."""
    lib = load()
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.zeros(max(nq * o_stride, 1), np.float32)
    m = _bools(allowed) if allowed is not None else None
    ok = lib.pcl_hip_attention_f32_multi_kv(
        _fptr(q), nq, q_stride, _fptr(k), _fptr(v), qheads, kvheads, dim, nkeys,
        _u8ptr(m) if m is not None else None, mask_stride, None, _fptr(out), o_stride,
        kh_first, kh_end)
    return bool(ok), out[:nq * o_stride]


def set_host_wait_limit(polls):
    """pcl_context_set_wait_limit(NULL, polls): the wait bound of the context
    the host-pointer entries use (0 = the default); those entries rerun a
    launch whose waits ran out with the pipelined kernel."""
    rc = load().pcl_context_set_wait_limit(None, int(polls))
    if rc != OK:
        raise AttentionError(rc)


class Context:
    """The device-resident entry (pcl_context). Pointers are device addresses
    (ints); torch tensors work through data_ptr(). stream None: the context
    owns a new stream; otherwise a hipStream_t handle (0 = null stream), e.g.
    torch.cuda.current_stream().cuda_stream."""

    def __init__(self, device=0, stream=None):
        self.lib = load()
        self.handle = ctypes.c_void_p()
        # caches and transforms made on this context: closed before it
        self._children = weakref.WeakSet()
        if stream is None:
            rc = self.lib.pcl_context_create(device, ctypes.byref(self.handle))
        else:
            rc = self.lib.pcl_context_create_on_stream(device, ctypes.c_void_p(stream or None),
                                                       ctypes.byref(self.handle))
        if rc != OK:
            raise AttentionError(rc)

    def close(self):
        if self.handle:
            for child in list(self._children):
                child.close()
            self.lib.pcl_context_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return self.lib.pcl_context_stream(self.handle)

    @staticmethod
    def desc(**kw):
        d = PclDesc()
        d.q_scale = 1.0
        for k, v in kw.items():
            setattr(d, k, v)
        return d

    def launch(self, desc):
        rc = self.lib.pcl_attention_launch(self.handle, ctypes.byref(desc))
        if rc != OK:
            raise AttentionError(rc)

    def launch_noalloc(self, desc):
        """pcl_attention_launch_noalloc: the same launch with the partials in
        the GPU's fixed scratch array (no allocation; calls on one GPU must
        not overlap)."""
        rc = self.lib.pcl_attention_launch_noalloc(self.handle, ctypes.byref(desc))
        if rc != OK:
            raise AttentionError(rc)

    def reserve(self, nbytes):
        rc = self.lib.pcl_context_reserve(self.handle, nbytes)
        if rc != OK:
            raise AttentionError(rc)

    def workspace_bytes(self, desc):
        return self.lib.pcl_attention_workspace_bytes(ctypes.byref(desc))

    def resolve_kernel(self, desc):
        return self.lib.pcl_attention_resolve_kernel(ctypes.byref(desc))

    def set_wait_limit(self, polls):
        """pcl_context_set_wait_limit: bound of the spread decode's waits
        between workgroups (0 = the default)."""
        rc = self.lib.pcl_context_set_wait_limit(self.handle, int(polls))
        if rc != OK:
            raise AttentionError(rc)

    def set_timing(self, enable):
        rc = self.lib.pcl_context_set_timing(self.handle, int(bool(enable)))
        if rc != OK:
            raise AttentionError(rc)

    def timing(self):
        """Wait; returns ((stream_ms, combine_ms), (stream_launches,
        combine_launches)) accumulated since the last call."""
        ms = (ctypes.c_double * 2)(0.0, 0.0)
        n = (ctypes.c_int64 * 2)(0, 0)
        rc = self.lib.pcl_context_timing(self.handle, ms, n)
        if rc != OK:
            raise AttentionError(rc)
        return (ms[0], ms[1]), (n[0], n[1])

    def attention_output(self, attended_ptr, n, in_width, weights_ptr, out_width,
                         post_scale_ptr, epsilon, residual_ptr, projected_ptr, result_ptr):
        """The attention output block (src/engine/attention.rs:866-884) on
        device rows: projected = W . attended (W [out][in]), result =
        residual + rms_norm(projected, post_scale, epsilon)."""
        rc = self.lib.pcl_attention_output(
            self.handle, ctypes.c_void_p(attended_ptr), int(n), int(in_width),
            ctypes.c_void_p(weights_ptr), int(out_width), ctypes.c_void_p(post_scale_ptr),
            float(epsilon), ctypes.c_void_p(residual_ptr), ctypes.c_void_p(projected_ptr),
            ctypes.c_void_p(result_ptr))
        if rc != OK:
            raise AttentionError(rc)

    def sync(self):
        """Wait; returns the device error flag (cleared)."""
        err = ctypes.c_int(0)
        rc = self.lib.pcl_context_sync(self.handle, ctypes.byref(err))
        if rc != OK:
            raise AttentionError(rc)
        return err.value


class LayerCache:
    """LayerCache (src/engine/attention.rs:244-311) with its K/V in device
    memory: token-major [tokens][kv_heads][head_dim] f32 rows on the
    context's device, copies on the context's stream. Methods keep the
    engine's names; append() is the K/V half of encode_in_place
    (attention.rs:949-1080) and returns the PendingKv record that rollback,
    keep and the descriptors take. Limits raise AttentionError
    ("ResourceLimit") as check_stage does (attention.rs:507-560)."""

    def __init__(self, ctx, kv_heads, head_dim, context, window, max_bytes):
        self.ctx = ctx
        self.lib = ctx.lib
        self.kv_heads, self.head_dim = int(kv_heads), int(head_dim)
        self.handle = ctypes.c_void_p()
        rc = self.lib.pcl_kv_cache_create(ctx.handle, self.kv_heads, self.head_dim,
                                          int(context), int(window or 0), int(max_bytes),
                                          ctypes.byref(self.handle))
        if rc != OK:
            raise AttentionError(rc)
        ctx._children.add(self)

    def reserve_rows(self, rows):
        """Room for `rows` rows in the device buffers now (grow-only; between
        steps), so that appends up to that many rows do not reallocate."""
        self._check(self.lib.pcl_kv_cache_reserve_rows(self.handle, int(rows)))

    def close(self):
        if self.handle:
            self.lib.pcl_kv_cache_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != OK:
            raise AttentionError(rc)

    def total_tokens(self):
        return self.lib.pcl_kv_cache_total_tokens(self.handle)

    def retained_tokens(self):
        return self.lib.pcl_kv_cache_retained_tokens(self.handle)

    def view(self):
        """(keys_ptr, values_ptr, rows, first_position) of the retained rows."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        rows, first = ctypes.c_int64(), ctypes.c_int64()
        self._check(self.lib.pcl_kv_cache_view(self.handle, ctypes.byref(k), ctypes.byref(v),
                                               ctypes.byref(rows), ctypes.byref(first)))
        return k.value or 0, v.value or 0, rows.value, first.value

    def read(self, first, rows):
        """Retained rows [first, first+rows) of K and V as host arrays."""
        width = self.kv_heads * self.head_dim
        keys = np.zeros(max(rows * width, 1), np.float32)
        values = np.zeros(max(rows * width, 1), np.float32)
        self._check(self.lib.pcl_kv_cache_read(self.handle, int(first), int(rows),
                                               keys.ctypes.data, values.ctypes.data))
        return keys[:rows * width], values[:rows * width]

    def append(self, keys_ptr, values_ptr, n):
        pending = PclPending()
        self._check(self.lib.pcl_kv_cache_append(self.handle, ctypes.c_void_p(keys_ptr),
                                                 ctypes.c_void_p(values_ptr), int(n),
                                                 ctypes.byref(pending)))
        return pending

    def append_transformed(self, transform, raw_q_ptr, raw_k_ptr, raw_v_ptr, n, q_out_ptr):
        """The step's raw projections through `transform` (a HeadTransform):
        prepared K/V rows appended, prepared queries written to q_out."""
        pending = PclPending()
        self._check(self.lib.pcl_kv_cache_append_transformed(
            self.handle, transform.handle, ctypes.c_void_p(raw_q_ptr),
            ctypes.c_void_p(raw_k_ptr), ctypes.c_void_p(raw_v_ptr or None), int(n),
            ctypes.c_void_p(q_out_ptr), ctypes.byref(pending)))
        return pending

    def attend_token(self, transform, raw_q_ptr, raw_k_ptr, raw_v_ptr, q_out_ptr, out_ptr,
                     q_scale=1.0, kernel=KERNEL_AUTO):
        """One decode token: its raw projections through `transform`, K/V
        appended, prepared queries to q_out, and the attention of the token
        over the cache into out ([qheads][dim]), in one call (the transform
        folded into the pipelined decode's launch where that kernel runs)."""
        pending = PclPending()
        self._check(self.lib.pcl_kv_cache_attend_token(
            self.handle, transform.handle, ctypes.c_void_p(raw_q_ptr),
            ctypes.c_void_p(raw_k_ptr), ctypes.c_void_p(raw_v_ptr or None), float(q_scale),
            int(kernel), ctypes.c_void_p(q_out_ptr), ctypes.c_void_p(out_ptr),
            ctypes.byref(pending)))
        return pending

    def advance(self, n):
        """A shared-K/V layer's step (encode_shared_in_place's position move)."""
        pending = PclPending()
        self._check(self.lib.pcl_kv_cache_advance(self.handle, int(n), ctypes.byref(pending)))
        return pending

    def rollback(self, pending):
        self._check(self.lib.pcl_kv_cache_rollback(self.handle, ctypes.byref(pending)))

    def keep(self, pending, tokens):
        self._check(self.lib.pcl_kv_cache_keep(self.handle, ctypes.byref(pending), int(tokens)))

    def commit(self):
        self._check(self.lib.pcl_kv_cache_commit(self.handle))

    def encoder_desc(self, pending, **kw):
        """Descriptor of the encoder pass of the step `pending`; kw sets the
        query, output and head fields."""
        d = Context.desc(**kw)
        self._check(self.lib.pcl_kv_cache_encoder_desc(self.handle, ctypes.byref(pending),
                                                       ctypes.byref(d)))
        return d

    def decoder_desc(self, canvas_keys_ptr, canvas_values_ptr, n, **kw):
        d = Context.desc(**kw)
        self._check(self.lib.pcl_kv_cache_decoder_desc(
            self.handle, ctypes.c_void_p(canvas_keys_ptr or None),
            ctypes.c_void_p(canvas_values_ptr or None), int(n), ctypes.byref(d)))
        return d

    def shared_desc(self, source, source_pending, n, **kw):
        d = Context.desc(**kw)
        self._check(self.lib.pcl_kv_cache_shared_desc(self.handle, source.handle,
                                                      ctypes.byref(source_pending), int(n),
                                                      ctypes.byref(d)))
        return d


class HeadTransform:
    """HeadTransform (src/engine/attention.rs:51-243) on the device. Scales
    and factors are host arrays; prepare()/query() take device pointers of
    [n][heads][dim] rows, token i at position `position + i`."""

    def __init__(self, ctx, qheads, kv_heads, head_dim, query_scale, key_scale, epsilon, base,
                 factors=None, sliding=False):
        self.ctx = ctx
        self.lib = ctx.lib
        qs, ks = _f32(query_scale), _f32(key_scale)
        fs = _f32(factors) if factors is not None else None
        self._keep = (qs, ks, fs)
        self.handle = ctypes.c_void_p()
        rc = self.lib.pcl_head_transform_create(
            ctx.handle, int(qheads), int(kv_heads), int(head_dim), int(bool(sliding)), _fptr(qs),
            _fptr(ks), float(epsilon), float(base), _fptr(fs) if fs is not None else None,
            ctypes.byref(self.handle))
        if rc != OK:
            raise AttentionError(rc)
        ctx._children.add(self)

    def close(self):
        if self.handle:
            self.lib.pcl_head_transform_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare(self, raw_q_ptr, raw_k_ptr, raw_v_ptr, n, position, q_out_ptr, k_out_ptr,
                v_out_ptr):
        rc = self.lib.pcl_head_transform_prepare(
            self.handle, ctypes.c_void_p(raw_q_ptr), ctypes.c_void_p(raw_k_ptr),
            ctypes.c_void_p(raw_v_ptr or None), int(n), int(position),
            ctypes.c_void_p(q_out_ptr), ctypes.c_void_p(k_out_ptr), ctypes.c_void_p(v_out_ptr))
        if rc != OK:
            raise AttentionError(rc)

    def query(self, raw_q_ptr, n, position, q_out_ptr):
        rc = self.lib.pcl_head_transform_query(self.handle, ctypes.c_void_p(raw_q_ptr), int(n),
                                               int(position), ctypes.c_void_p(q_out_ptr))
        if rc != OK:
            raise AttentionError(rc)
