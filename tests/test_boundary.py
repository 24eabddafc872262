"""The C ABI boundary on the CPU: the library loads, exports every symbol
include/pcl_attention.h declares, and rejects what the reference wrappers
reject before any device work (no GPU needed for these paths)."""
import ctypes
import functools
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pcl_attention.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pcl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pcl):
    lib = pcl.load()
    names = declared_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(pcl.EXPORTS)
    assert b"gfx950" in lib.pcl_version()


def test_library_is_built_for_gfx950_only(pcl):
    data = open(pcl.library_path(), "rb").read()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def test_checked_wrapper_rejects_shapes_before_device_work(pcl):
    # attention_with (src/kernels/quantized/int8.rs:607-636) validation
    k = pcl.HipKernels()
    q = np.ones(32, np.float32)
    kv = np.ones(64, np.float32)
    cases = [
        (lambda: k.attention(q, kv, kv, 0, 32), "InvalidShape"),          # kv heads 0
        (lambda: k.attention(q, kv, kv, 1, 0), "InvalidShape"),           # dim 0
        (lambda: k.attention(q[:24], kv[:24], kv[:24], 1, 24), "InvalidShape"),  # dim % 16
        (lambda: k.attention(q, kv, kv[:32], 1, 32), "InvalidShape"),     # len(V) != len(K)
        (lambda: k.attention(q, kv[:48], kv[:48], 1, 32), "InvalidShape"),  # K not whole rows
        (lambda: k.attention(np.ones(48, np.float32), kv, kv, 2, 16), "InvalidShape"),  # 3 % 2
        (lambda: k.attention(q, kv, kv, 1, 32, [True]), "InvalidShape"),  # mask length
        (lambda: k.attention(q, kv, kv, 1, 32, [False, False]), "InvalidParameter"),
        (lambda: k.attention_heads(q, kv, kv, 1, 32, None, (0, 2)), "InvalidShape"),
        (lambda: k.attention_heads(q, kv, kv, 1, 32, None, (1, 0)), "InvalidShape"),
        (lambda: k.attention(np.full(32, np.nan, np.float32), kv, kv, 1, 32), "NonFiniteValue"),
        (lambda: k.attention_multi_kv([q], kv, kv, 1, 32, None, (0, 0)), "InvalidShape"),
        (lambda: k.attention_multi_kv([q], kv, kv, 1, 32, None, (0, 2)), "InvalidShape"),
        (lambda: k.attention_multi([q, q], kv, kv, 1, 32, [[True, False], [False, False]]),
         "InvalidParameter"),
        (lambda: k.attention_multi([q], kv, kv, 1, 32, [[True]]), "InvalidShape"),
        (lambda: k.attention_multi([np.full(32, np.inf, np.float32)], kv, kv, 1, 32),
         "NonFiniteValue"),
    ]
    for fn, kind in cases:
        with pytest.raises(pcl.AttentionError) as e:
            fn()
        assert e.value.kind == kind
    assert k.attention_multi([], kv, kv, 1, 32) == []


def test_raw_entries_reject_geometry_before_device_work(pcl):
    one = np.ones(64, np.float32)
    assert not pcl.raw_heads(one, one, one, 2, 1, 32, 1, None, 1, 3)[0]   # h_end > qheads
    assert not pcl.raw_heads(one, one, one, 2, 1, 32, 1, None, 2, 1)[0]   # h_first > h_end
    assert not pcl.raw_heads(one, one, one, 2, 0, 32, 1, None, 0, 1)[0]   # kvheads 0
    assert not pcl.raw_heads(one, one, one, 3, 2, 16, 1, None, 0, 1)[0]   # qheads % kvheads
    assert not pcl.raw_heads(one, one, one, 1, 1, 1024, 1, None, 0, 1)[0]  # dim > 512
    assert not pcl.raw_multi_kv(one, 1, 32, one, one, 2, 1, 16, 1, None, 1, 32, 1, 1)[0]
    assert not pcl.raw_multi_kv(one, 1, 16, one, one, 2, 1, 16, 1, None, 1, 32, 0, 1)[0]


def test_descriptor_validation_on_the_host(pcl):
    # workspace sizing and kernel choice run on the host only
    d = pcl.Context.desc(q=16, q_stride=16 * 256, nq=1, k0=16, v0=16, n0=32768, qheads=16,
                         kvheads=8, dim=256, kh_first=0, kh_end=8, causal=1, first_query=32767,
                         out=16, o_stride=16 * 256)
    lib = pcl.load()
    # a long cache streams through the pipelined kernel
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    assert lib.pcl_attention_workspace_bytes(ctypes.byref(d)) > 0
    d.dim, d.q_stride, d.o_stride = 512, 16 * 512, 16 * 512
    # also at head dim 512 (two score waves, two value waves)
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.window = 1024  # five chunks per head: short, so at d512 the spread form
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.window = 200  # one chunk: spread as well (its slices write the output)
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.window = 0  # 128 chunks x 8 KV heads: beyond the spread bound, pipelined
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.window = 8192  # 32 chunks x 8 KV heads: 256 items, beyond it, fanned
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_FAN_KV
    # one chunk of 64 KV heads at d512: 1024 slices, beyond it: four-phase
    d.qheads, d.kvheads, d.kh_end, d.window = 64, 64, 64, 200
    d.q_stride = d.o_stride = 64 * 512
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPLIT_KV
    d.qheads, d.kvheads, d.kh_end = 16, 8, 8
    d.q_stride = d.o_stride = 16 * 512
    d.window = 1024
    d.dim, d.q_stride, d.o_stride = 256, 16 * 256, 16 * 256
    # up to head dim 256 a short decode (4 chunks x 8 KV heads) spreads each
    # chunk over 8 workgroups
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.kernel = pcl.KERNEL_PIPE_KV  # forced choices are kept where the kernel exists
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.kernel = pcl.KERNEL_FAN_KV
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_FAN_KV
    d.kernel = 5  # retired
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1
    d.kernel = pcl.KERNEL_PIPE_KV
    d.dim, d.q_stride, d.o_stride = 512, 16 * 512, 16 * 512
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.kernel = pcl.KERNEL_SPREAD_KV  # the one-wave-slice spread form at d512
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.dim, d.q_stride, d.o_stride, d.window = 256, 16 * 256, 16 * 256, 0
    # 128 chunks x 8 KV heads is beyond the spread bound: pipelined
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.window = 1024
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.dim, d.q_stride, d.o_stride = 512, 16 * 512, 16 * 512
    d.kernel = 8  # no such kernel
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1
    d.kernel, d.dim, d.q_stride, d.o_stride = 0, 256, 16 * 256, 16 * 256
    d.dim = 24
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1
    d.dim = 256
    # the optional logit soft-cap: 0 (either sign) is off, a normal positive
    # value is on; negative, subnormal and non-finite caps are rejected
    for cap, valid in ((0.0, True), (-0.0, True), (30.0, True), (1e30, True), (-1.0, False),
                       (1e-40, False), (3e38, False), (float("inf"), False),
                       (float("nan"), False)):
        d.softcap = cap
        assert (lib.pcl_attention_resolve_kernel(ctypes.byref(d)) != -1) == valid, cap
    d.softcap = 0.0
    # the reference's probe shapes (8 queries over every key): the global
    # layer (16/2/512, 3194 keys) fanned, the sliding one (16/8/256, 1279
    # keys) spread; 32 queries at head dim 256 (two row blocks' worth of
    # rows, 416 items) fanned, over 8192 keys (1024 items) chunk-split tiled
    d.causal, d.window, d.first_query = 0, 0, 0
    d.nq, d.n0, d.kvheads, d.kh_end = 8, 3194, 2, 2
    d.dim, d.q_stride, d.o_stride = 512, 16 * 512, 16 * 512
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_FAN_KV
    d.nq, d.n0, d.kvheads, d.kh_end = 8, 1279, 8, 8
    d.dim, d.q_stride, d.o_stride = 256, 16 * 256, 16 * 256
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_SPREAD_KV
    d.nq, d.n0 = 32, 3194
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_FAN_KV
    d.n0 = 8192
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_TILED_SPLIT
    d.causal = 1
    d.dim, d.nq, d.first_query, d.window, d.n0 = 256, 4096, 0, 0, 4096
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_TILED
    d.first_key = 5000  # no query sees a key
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1
    # size limits (every grid below 2^31 work-items): 2^30 keys, and
    # 2^22 rows x KV heads; calls beyond them are split by the caller
    d.first_key, d.nq, d.first_query, d.n0 = 0, 1, (1 << 30) - 1, 1 << 30
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_PIPE_KV
    d.n0, d.first_query = (1 << 30) + 1, 1 << 30
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1
    d.n0, d.nq, d.first_query = 4096, (1 << 22) // 16, 0  # x group 2 x 8 KV heads
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == pcl.KERNEL_TILED
    d.nq += 1
    assert lib.pcl_attention_resolve_kernel(ctypes.byref(d)) == -1


def test_product_path_has_no_cpu_fallback():
    src = open(os.path.join(ROOT, "power-cpu-llm_amd", "__init__.py")).read()
    assert "oracle" not in src.replace("the oracle", "")
    for name in os.listdir(os.path.join(ROOT, "power-cpu-llm_amd", "csrc")):
        text = open(os.path.join(ROOT, "power-cpu-llm_amd", "csrc", name)).read()
        assert "oracle" not in text


@functools.lru_cache(maxsize=None)
def _resource_remarks(source):
    """Device-only compile of one kernel source with the library's flags,
    returning {kernel symbol: VGPR spill count} from the compiler's
    kernel-resource-usage remarks."""
    import subprocess
    import sys
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "power-cpu-llm_amd"))
    try:
        import build as hip_build
    finally:
        sys.path.pop(0)
    flags = [f for f in hip_build.FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory() as tmp:
        res = subprocess.run([hip_build.HIPCC] + flags + [
            "--cuda-device-only", "-c", "-Rpass-analysis=kernel-resource-usage",
            os.path.join(ROOT, "power-cpu-llm_amd", "csrc", source),
            "-o", os.path.join(tmp, "k.o")], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    spills, name = {}, None
    for line in res.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"VGPRs Spill: (\d+)", line)
        if m and name:
            spills[name] = int(m.group(1))
    return spills


@pytest.mark.parametrize("source,kernel", [
    ("tiled.hip", "_ZN3pcl12tiled_kernelILi256ELi8ELb0EEEvNS_6ParamsEii"),
    ("tiled_wide.hip", "_ZN3pcl17tiled_wide_kernelILb0EEEvNS_6ParamsEii"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb0ELi2ELb0ELb0EEEvNS_6ParamsE"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi2ELb0ELb0EEEvNS_6ParamsE"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi4ELb0ELb0EEEvNS_6ParamsE"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi2ELb1ELb0EEEvNS_6ParamsE"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi4ELb1ELb0EEEvNS_6ParamsE"),
    # whole-chunk launches (no per-key path)
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi2ELb1ELb1EEEvNS_6ParamsE"),
    ("spread_kv.hip", "_ZN3pcl16spread_kv_kernelILi256ELb1ELb0ELb1ELi4ELb1ELb1EEEvNS_6ParamsE"),
    ("pipe_kv.hip", "_ZN3pcl14pipe_kv_kernelILi256ELi1ELb1ELb0ELb0EEEvNS_6ParamsEi"),
    ("pipe_kv.hip", "_ZN3pcl14pipe_kv_kernelILi512ELi1ELb1ELb1ELb0EEEvNS_6ParamsEi"),
    # the same with a one-token step's head transform folded in
    ("pipe_kv.hip", "_ZN3pcl14pipe_kv_kernelILi256ELi1ELb1ELb0ELb1EEEvNS_6ParamsEi"),
    ("pipe_kv.hip", "_ZN3pcl14pipe_kv_kernelILi512ELi1ELb1ELb1ELb1EEEvNS_6ParamsEi"),
    ("fan_kv.hip", "_ZN3pcl13fan_kv_kernelILi256ELb1ELb0ELb1ELi1EEEvNS_6ParamsEi"),
    ("fan_kv.hip", "_ZN3pcl13fan_kv_kernelILi256ELb0ELb1ELb0ELi1EEEvNS_6ParamsEi"),
    # launches of few items, each item's output dims split
    ("fan_kv.hip", "_ZN3pcl13fan_kv_kernelILi256ELb1ELb0ELb0ELi2EEEvNS_6ParamsEi"),
    ("fan_kv.hip", "_ZN3pcl13fan_kv_kernelILi512ELb1ELb0ELb0ELi2EEEvNS_6ParamsEi"),
    ("fan_kv.hip", "_ZN3pcl13fan_kv_kernelILi512ELb1ELb0ELb0ELi4EEEvNS_6ParamsEi"),
    # the decode step's output projection and the prompt's head transform
    ("output_block.hip", "_ZN3pcl22project_row_lds_kernelENS_11BlockParamsEi"),
    ("head_transform.hip", "_ZN3pcl21head_transform_kernelILi256ELi16EEEvNS_15TransformParamsE"),
    ("head_transform.hip", "_ZN3pcl21head_transform_kernelILi512ELi8EEEvNS_15TransformParamsE"),
])
def test_hot_kernels_do_not_spill_registers(source, kernel):
    # a spill in these kernels costs every tile or block: the prefill once
    # hoisted 32 accumulator addresses out of its tile loop and spilled them
    # (4-5 % of the 4K prefill); keep all three at zero VGPR spills
    if not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc absent")
    spills = _resource_remarks(source)
    assert kernel in spills, sorted(spills)
    assert spills[kernel] == 0
