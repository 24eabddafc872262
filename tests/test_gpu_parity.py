"""GPU parity of the gfx950 attention backend against the CPU oracle.

Ports the reference's attention tests to this backend (names follow them),
checks BASELINE.json's five configs against the exact oracle within 1e-4
max-abs with the same argmax per (query, head) row, and checks the
size-independent properties the design promises (every kernel gives the
same bits; head, query and KV-head ranges do not change results).
"""
import math
import os

import numpy as np
import pytest

from helpers import Rng, normals, prescale, row_argmax_agree

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


@pytest.fixture(scope="module")
def kernels(pcl):
    return pcl.HipKernels()


@pytest.fixture(scope="module")
def ctx(pcl, torch):
    c = pcl.Context(0, torch.cuda.current_stream().cuda_stream)
    yield c
    c.close()


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def assert_parity(got, want, dim, tol=TOL):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got))
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert err <= tol, "max abs error %.3g" % err
    ok, mismatches = row_argmax_agree(got, want, dim)
    assert ok, "argmax differs in %d rows (row, top-1 minus top-2 margin): %s" % (
        len(mismatches), mismatches[:20])
    return err


# ---- the engine interface (host pointers), reference tests ported ---------

TWIN_GEOMETRIES = [
    (16, 8, 256, 37), (16, 2, 512, 5), (4, 4, 16, 1), (2, 1, 32, 64), (6, 3, 48, 6),
    (4, 2, 80, 7), (8, 2, 144, 3), (2, 1, 320, 130), (6, 2, 16, 9), (9, 3, 32, 2),
    (10, 2, 48, 11), (8, 1, 16, 1), (4, 1, 96, 3), (16, 2, 512, 130),
]


def test_attention_f32_matches_reference_on_twin_geometries(kernels, oracle):
    # src/kernels/quantized/int8/tests.rs:399-476, against the exact oracle
    rng = Rng(0xa77e)
    for qheads, kvh, dim, nkeys in TWIN_GEOMETRIES:
        query = rng.units(qheads * dim, 0.5)
        keys = rng.units(nkeys * kvh * dim, 0.5)
        values = rng.units(nkeys * kvh * dim)
        mask = np.array([t % 3 != 1 or nkeys == 1 for t in range(nkeys)])
        for allowed in (None, mask):
            got = kernels.attention(query, keys, values, kvh, dim, allowed)
            ok, want = oracle.heads(query, keys, values, qheads, kvh, dim, nkeys, allowed)
            assert ok
            assert_parity(got, want, dim)
            assert np.all(np.abs(got - want) <= 2e-5 * (1.0 + np.abs(want)))
        bad = values.copy()
        bad[(nkeys - 1) * kvh * dim + dim - 1] = np.inf
        bad_keys = keys.copy()
        bad_keys[dim - 1] = np.nan
        with pytest.raises(Exception) as e:
            kernels.attention(query, keys, bad, kvh, dim, None)
        assert getattr(e.value, "kind", "") == "NonFiniteValue"
        with pytest.raises(Exception) as e:
            kernels.attention(query, bad_keys, values, kvh, dim, None)
        assert getattr(e.value, "kind", "") == "NonFiniteValue"


def test_attention_rejects_bad_shapes_masks_and_overflow(kernels, pcl):
    q = np.ones(32, np.float32)
    kv = np.ones(32, np.float32)
    with pytest.raises(pcl.AttentionError) as e:
        kernels.attention(q, kv, kv, 1, 32, [False])
    assert e.value.kind == "InvalidParameter"
    with pytest.raises(pcl.AttentionError) as e:
        kernels.attention(q[:24], kv[:24], kv[:24], 1, 24, None)
    assert e.value.kind == "InvalidShape"
    big = np.full(32, np.finfo(np.float32).max, np.float32)
    with pytest.raises(pcl.AttentionError) as e:
        kernels.attention(big, big, kv, 1, 32, None)
    assert e.value.kind == "NonFiniteValue"


def test_attention_head_ranges_match_full_attention(kernels, oracle):
    # int8/tests.rs:594-659: every head range is that slice, bitwise
    rng = Rng(0x7f4a7c159e3779b9)
    for qheads, kvh, dim, nkeys in [(16, 8, 32, 7), (8, 1, 64, 33), (4, 2, 16, 1),
                                    (6, 2, 48, 5), (9, 3, 16, 2)]:
        query = rng.units(qheads * dim)
        keys = rng.units(nkeys * kvh * dim)
        values = rng.units(nkeys * kvh * dim)
        mask = np.array([t % 3 != 1 or t == 0 for t in range(nkeys)])
        for allowed in (None, mask):
            full = kernels.attention(query, keys, values, kvh, dim, allowed)
            ok, want = oracle.heads(query, keys, values, qheads, kvh, dim, nkeys, allowed)
            assert_parity(full, want, dim)
            for a in range(qheads):
                for b in range(a, qheads + 1):
                    part = kernels.attention_heads(query, keys, values, kvh, dim, allowed, (a, b))
                    assert np.array_equal(bits(part), bits(full[a * dim:b * dim])), (a, b)
            with pytest.raises(Exception):
                kernels.attention_heads(query, keys, values, kvh, dim, allowed, (0, qheads + 1))


def test_concurrent_head_range_calls_share_one_upload_and_see_rewrites(kernels, oracle):
    # the engine's fan-out of one position (src/engine/attention.rs:755-777):
    # concurrent calls, one query head each, over the same read-only K/V;
    # every head equals the full call bitwise, and after the calls return a
    # rewrite of the same buffers is seen by the next fan-out
    import concurrent.futures
    qheads, kvh, dim, nkeys = 16, 8, 256, 3000
    g = np.random.default_rng(0xFA11)
    q = prescale(g.standard_normal(qheads * dim, dtype=np.float32), dim)
    k = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    v = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    pool = concurrent.futures.ThreadPoolExecutor(qheads)
    for rewrite in range(3):
        if rewrite:
            k[:] = g.standard_normal(k.size, dtype=np.float32)  # same buffers, new contents
            v[:] = g.standard_normal(v.size, dtype=np.float32)
        full = kernels.attention(q, k, v, kvh, dim, None)
        parts = list(pool.map(
            lambda h: kernels.attention_heads(q, k, v, kvh, dim, None, (h, h + 1)),
            range(qheads)))
        got = np.concatenate(parts)
        assert np.array_equal(bits(got), bits(full)), rewrite
        ok, want = oracle.heads(q, k, v, qheads, kvh, dim, nkeys)
        assert ok
        assert_parity(got, want, dim)
    pool.shutdown()


def test_host_entry_keeps_the_bits_when_spread_waits_run_out(pcl, kernels):
    # the engine-facing entry's context with a one-poll wait bound: the
    # waves of its 2K decode (the spread kernel) stop waiting for each other
    # and form the missing scores themselves: the same bits as at the default
    # bound
    qheads, kvh, dim, nkeys = 16, 8, 256, 2048
    g = np.random.default_rng(0x3A17)
    q = prescale(g.standard_normal(qheads * dim, dtype=np.float32), dim)
    k = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    v = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    want = kernels.attention(q, k, v, kvh, dim, None)
    pcl.set_host_wait_limit(1)
    try:
        got = kernels.attention(q, k, v, kvh, dim, None)
    finally:
        pcl.set_host_wait_limit(0)
    assert np.array_equal(bits(got), bits(want))


def test_attention_multi_matches_single_queries(kernels):
    # int8/tests.rs:661-706
    rng = Rng(0x51ed270b)
    for qheads, kvh, dim, nkeys, nq in [(16, 8, 32, 9, 5), (8, 1, 64, 33, 3), (4, 2, 16, 2, 7),
                                        (16, 2, 48, 1, 1)]:
        queries = [rng.units(qheads * dim) for _ in range(nq)]
        keys = rng.units(nkeys * kvh * dim)
        values = rng.units(nkeys * kvh * dim)
        masks = [np.array([t <= nkeys // 2 + i or t == 0 for t in range(nkeys)])
                 for i in range(nq)]
        for masked in (False, True):
            m = masks if masked else None
            multi = kernels.attention_multi(queries, keys, values, kvh, dim, m)
            for i, q in enumerate(queries):
                single = kernels.attention(q, keys, values, kvh, dim, m[i] if m else None)
                assert np.array_equal(bits(multi[i]), bits(single))


def test_attention_multi_kv_ranges_match_single_queries(kernels, oracle):
    # int8/tests.rs:708-768: sliding windows, more keys than one block
    rng = Rng(0x7a11ed)
    for qheads, kvh, dim, nkeys, nq, window in [(16, 2, 512, 150, 6, 40),
                                                (16, 8, 256, 300, 5, 130),
                                                (4, 2, 16, 37, 9, 5)]:
        queries = [rng.units(qheads * dim) for _ in range(nq)]
        keys = rng.units(nkeys * kvh * dim)
        values = rng.units(nkeys * kvh * dim)
        masks = [np.array([t <= nkeys - nq + i and t + window > nkeys - nq + i
                           for t in range(nkeys)]) for i in range(nq)]
        group = qheads // kvh
        for masked in (False, True):
            m = masks if masked else None
            singles = [kernels.attention(q, keys, values, kvh, dim, m[i] if m else None)
                       for i, q in enumerate(queries)]
            for i, q in enumerate(queries):
                ok, want = oracle.heads(q, keys, values, qheads, kvh, dim, nkeys,
                                        m[i] if m else None)
                assert_parity(singles[i], want, dim)
            for kv in [(0, kvh), (0, 1), (kvh - 1, kvh)]:
                part = kernels.attention_multi_kv(queries, keys, values, kvh, dim, m, kv)
                for i, single in enumerate(singles):
                    want = single[kv[0] * group * dim:kv[1] * group * dim]
                    assert np.array_equal(bits(part[i]), bits(want)), (kv, i, masked)


def test_attention_multi_throughput_shapes(kernels, oracle):
    # the shapes and inputs of int8/tests.rs:770-809 (queries unit() * 0.1,
    # no mask): 1279 and 3194 keys end inside a chunk; every query row
    # matches the exact oracle, and the multi call equals single calls
    rng = Rng(7)
    for qheads, kvh, dim, nkeys, nq in [(16, 8, 256, 1279, 8), (16, 2, 512, 3194, 8)]:
        queries = [rng.units_c(qheads * dim, 0.1) for _ in range(nq)]
        keys = rng.units_c(nkeys * kvh * dim)
        values = rng.units_c(nkeys * kvh * dim)
        multi = kernels.attention_multi(queries, keys, values, kvh, dim, None)
        for i, q in enumerate(queries):
            ok, want = oracle.heads(q, keys, values, qheads, kvh, dim, nkeys, None)
            assert ok
            assert_parity(multi[i], want, dim)
        for i in (0, nq - 1):
            single = kernels.attention(queries[i], keys, values, kvh, dim, None)
            assert np.array_equal(bits(multi[i]), bits(single)), (dim, i)


def run_threads(fn, args, timeout=60.0):
    """Runs fn(*a) for every a in args on its own thread; re-raises the first
    failure (ctypes releases the GIL, so the library calls overlap)."""
    import threading
    errors = []

    def body(a):
        try:
            fn(*a)
        except BaseException as e:  # reported on the main thread
            errors.append(e)

    threads = [threading.Thread(target=body, args=(a,)) for a in args]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    if errors:
        raise errors[0]


def test_concurrent_workers_on_disjoint_head_ranges_match_one_call(kernels):
    # the engine's decode fan-out (src/engine/attention.rs:755-777): up to N
    # workers call the AttentionF32 entry at once, each on its own head range
    # of one position, over shared read-only K/V (kernels.rs:230-231)
    qheads, kvh, dim, nkeys = 16, 8, 256, 1500
    g = np.random.default_rng(0xC0C0)
    q = prescale(g.standard_normal(qheads * dim, dtype=np.float32), dim)
    k = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    v = g.standard_normal(nkeys * kvh * dim, dtype=np.float32)
    allowed = np.arange(nkeys) > nkeys - 1 - 700
    full = kernels.attention(q, k, v, kvh, dim, allowed)
    got = {}

    def worker(h0, h1):
        got[(h0, h1)] = [kernels.attention_heads(q, k, v, kvh, dim, allowed, (h0, h1))
                         for _ in range(4)]

    run_threads(worker, [(2 * i, 2 * i + 2) for i in range(8)] + [(0, qheads), (5, 11)])
    assert len(got) == 10
    for (h0, h1), outs in got.items():
        for out in outs:
            assert np.array_equal(bits(out), bits(full[h0 * dim:h1 * dim])), (h0, h1)


def test_a_context_per_thread_gives_the_single_context_bits(pcl, torch, ctx):
    # "a context per thread" re-entrancy: each worker owns a device context
    # (and its stream and workspace), launches over the shared device K/V,
    # and reads its own output; kernels alternate between workers
    qheads, kvh, dim, nq, nkeys = 16, 8, 256, 3, 5000
    g = np.random.default_rng(0xC0DE)
    dev = torch.device("cuda:0")
    q = torch.from_numpy(prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32),
                                  dim)).to(dev)
    k = torch.from_numpy(g.standard_normal((nkeys, kvh, dim), dtype=np.float32)).to(dev)
    v = torch.from_numpy(g.standard_normal((nkeys, kvh, dim), dtype=np.float32)).to(dev)
    workers = 6
    outs = [torch.full((nq, qheads * dim), float("nan"), device=dev) for _ in range(workers + 1)]
    torch.cuda.synchronize()

    def desc(c, out, kernel):
        return c.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=nq, qheads=qheads,
                      kvheads=kvh, dim=dim, kh_first=0, kh_end=kvh, causal=1, window=0,
                      first_key=0, first_query=nkeys - nq, k0=k.data_ptr(), v0=v.data_ptr(),
                      n0=nkeys, out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)

    ctx.launch(desc(ctx, outs[workers], pcl.KERNEL_SPLIT_KV))
    assert ctx.sync() == 0
    kernels = (pcl.KERNEL_PIPE_KV, pcl.KERNEL_SPLIT_KV, pcl.KERNEL_FAN_KV)

    def worker(i):
        c = pcl.Context(0)
        try:
            for r in range(5):
                c.launch(desc(c, outs[i], kernels[(i + r) % len(kernels)]))
                assert c.sync() == 0
        finally:
            c.close()

    run_threads(worker, [(i,) for i in range(workers)])
    want = bits(outs[workers].cpu().numpy())
    for i in range(workers):
        assert np.array_equal(bits(outs[i].cpu().numpy()), want), i


def test_attention_score_bounds_handle_holes_and_query_tails(kernels, oracle):
    # int8/tests.rs:1118-1177: holes, wholly masked blocks, disjoint masks
    rng = Rng(0x78124)
    qheads, kvh, nkeys = 3, 3, 259
    for dim in (48, 256, 512):
        keys = rng.units(nkeys * kvh * dim)
        values = np.array([0.0 if i % 13 == 0 else (-0.0 if i % 13 == 1 else rng.unit())
                           for i in range(nkeys * kvh * dim)], np.float32)
        for nq in (1, 2, 3, 5):
            queries = [rng.units(qheads * dim, 0.1) for _ in range(nq)]
            lives = {0: [5, 7, 13, 17], 1: [129, 131, 139], 2: [255, 257], 3: [258]}
            masks = [np.isin(np.arange(nkeys), lives[i % 4]) for i in range(nq)]
            got = kernels.attention_multi_kv(queries, keys, values, kvh, dim, masks, (0, kvh))
            for i in range(nq):
                single = kernels.attention(queries[i], keys, values, kvh, dim, masks[i])
                assert np.array_equal(bits(got[i]), bits(single)), (dim, nq, i)
                ok, want = oracle.heads(queries[i], keys, values, qheads, kvh, dim, nkeys,
                                        masks[i])
                assert_parity(single, want, dim)


def test_raw_entries_report_bad_geometry(pcl):
    ok, _ = pcl.raw_heads(np.ones(32), np.ones(32), np.ones(32), 2, 1, 16, 1, None, 1, 3)
    assert not ok  # h_end > qheads
    ok, _ = pcl.raw_heads(np.ones(24), np.ones(24), np.ones(24), 1, 1, 24, 1, None, 0, 1)
    assert not ok  # dim % 16
    ok, out = pcl.raw_heads(np.ones(32), np.ones(32), np.ones(32), 2, 1, 16, 1, None, 1, 1)
    assert ok and out.size == 0  # empty head range
    ok, _ = pcl.raw_multi_kv(np.ones(32), 1, 32, np.ones(32), np.ones(32), 2, 1, 16, 1, None, 1,
                             32, 1, 1)
    assert not ok  # empty KV-head range


# ---- device descriptors: every kernel gives the same bits ------------------

def run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal=0, window=0, first_key=0,
             first_query=0, mask=None, split_at=None, kv=None, q_scale=1.0, softcap=None,
             noalloc=False):
    """One device launch over numpy inputs (through the allocation-free
    entry with noalloc); returns (out, error flag)."""
    dev = torch.device("cuda:0")
    nq = q.shape[0]
    nkeys = k.shape[0]
    kv = kv or (0, kvh)
    group = qheads // kvh
    olen = (kv[1] - kv[0]) * group * dim
    tq = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    out = torch.full((nq, olen), float("nan"), device=dev)
    kw = dict(q=tq.data_ptr(), q_stride=qheads * dim, nq=nq, qheads=qheads, kvheads=kvh,
              dim=dim, kh_first=kv[0], kh_end=kv[1], causal=causal, window=window,
              first_key=first_key, first_query=first_query, out=out.data_ptr(), o_stride=olen,
              kernel=kernel, q_scale=q_scale)
    if softcap is not None:
        kw["softcap"] = softcap
    keep = [tq, out]
    if split_at is None:
        tk = torch.from_numpy(np.ascontiguousarray(k)).to(dev)
        tv = torch.from_numpy(np.ascontiguousarray(v)).to(dev)
        kw.update(k0=tk.data_ptr(), v0=tv.data_ptr(), n0=nkeys)
        keep += [tk, tv]
    else:
        parts = [torch.from_numpy(np.ascontiguousarray(x)).to(dev)
                 for x in (k[:split_at], v[:split_at], k[split_at:], v[split_at:])]
        kw.update(k0=parts[0].data_ptr(), v0=parts[1].data_ptr(), n0=split_at,
                  k1=parts[2].data_ptr(), v1=parts[3].data_ptr(), n1=nkeys - split_at)
        keep += parts
    if mask is not None:
        tm = torch.from_numpy(np.ascontiguousarray(mask, dtype=np.uint8)).to(dev)
        kw.update(mask=tm.data_ptr(), mask_stride=nkeys)
        keep.append(tm)
    d = ctx.desc(**kw)
    if noalloc:
        ctx.launch_noalloc(d)
    else:
        ctx.launch(d)
    err = ctx.sync()
    return out.cpu().numpy(), err


DESC_CASES = [
    # qheads, kvh, dim, nq, nkeys, causal, window, first_query
    (16, 8, 256, 1, 2048, 1, 0, 2047),
    (16, 8, 256, 1, 700, 1, 100, 699),
    (16, 2, 512, 1, 3000, 1, 0, 2999),
    (16, 2, 512, 7, 900, 1, 0, 893),
    (16, 8, 256, 300, 300, 1, 0, 0),
    (16, 8, 256, 200, 1200, 1, 130, 1000),
    (16, 8, 256, 64, 600, 0, 0, 0),
    (8, 2, 128, 100, 500, 1, 0, 400),
    (4, 4, 64, 70, 333, 1, 33, 263),
    (6, 3, 48, 20, 90, 1, 0, 70),
    (10, 2, 80, 33, 517, 1, 0, 484),
    (16, 16, 16, 9, 1000, 1, 17, 991),
    # 4 row blocks x 8 KV heads x 9 chunks = 288 chunk items: on 256 CUs the
    # chunk-split kernel runs the last chunk as single-wave workgroups
    (16, 8, 64, 256, 2304, 0, 0, 0),
    (16, 8, 128, 256, 2304, 1, 700, 2048),
    # the same last round fanned over a workgroup's eight waves: at a padded
    # head dim (208 -> 256), and over two spans (17 chunks: the fanned chunk
    # writes its partial for the combine instead of merging the output)
    (16, 8, 208, 256, 2304, 1, 0, 2048),
    (16, 8, 256, 256, 4352, 0, 0, 0),
    # ... and with padding rows in the last 16-row unit (500 rows)
    (16, 8, 256, 250, 2304, 0, 0, 0),
    (16, 8, 256, 250, 2304, 1, 0, 2054),
    # head dim 512 (and 320, padded to 512) through the wave-pair tiled
    # kernel, one pass and one chunk per block
    (16, 2, 512, 100, 700, 1, 0, 600),
    (16, 2, 512, 40, 5000, 1, 0, 4960),
    # its chunk-split launches whose last round runs fanned: a padded head
    # dim (320) with causal rows in the last chunk, and two spans (the
    # fanned chunk writes its partial for the combine)
    (16, 2, 320, 256, 2304, 1, 0, 2048),
    (16, 2, 512, 256, 4352, 0, 0, 0),
    (8, 2, 320, 70, 400, 1, 130, 330),
]


@pytest.mark.parametrize("case", DESC_CASES, ids=lambda c: "x".join(map(str, c)))
def test_every_kernel_gives_identical_bits(torch, ctx, oracle, case):
    qheads, kvh, dim, nq, nkeys, causal, window, fq = case
    g = np.random.default_rng(sum(case))
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    outs = {}
    for kernel in (1, 2, 3, 4, 6, 7):
        outs[kernel], err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal,
                                     window, 0, fq)
        assert err == 0
    for kernel in (2, 3, 4, 6, 7):
        assert np.array_equal(bits(outs[1]), bits(outs[kernel])), kernel
    for i in sorted({0, nq // 2, nq - 1}):
        m = oracle.encoder_mask(0, nkeys, fq + i, window or None) if causal else None
        ok, want = oracle.heads(q[i], k, v, qheads, kvh, dim, nkeys, m)
        assert ok
        assert_parity(outs[1][i], want, dim)


SOFTCAP_CASES = [
    # qheads, kvh, dim, nq, nkeys, causal, window, first_query
    (16, 8, 256, 1, 2048, 1, 0, 2047),      # short decode (spread under AUTO)
    (16, 8, 256, 1, 9000, 1, 0, 8999),      # pipelined decode, two spans
    (16, 2, 512, 1, 3000, 1, 0, 2999),      # head dim 512 decode
    (16, 8, 256, 300, 300, 1, 0, 0),        # tiled prefill
    (16, 8, 128, 256, 2304, 1, 700, 2048),  # chunk-split launch with its tail
    (16, 2, 512, 100, 700, 1, 0, 600),      # wave-pair tiled kernel
]


@pytest.mark.parametrize("cap", [4.0, 1.5])
@pytest.mark.parametrize("case", SOFTCAP_CASES, ids=lambda c: "x".join(map(str, c)))
def test_softcap_every_kernel_identical_and_matches_the_oracle(torch, ctx, oracle, case, cap):
    # the descriptor's optional logit soft-cap: every kernel applies the same
    # f32 cap to the raw scores (bitwise equal results), within the contract
    # of the oracle's exact path with the f64 cap, and the cap takes effect
    qheads, kvh, dim, nq, nkeys, causal, window, fq = case
    g = np.random.default_rng(sum(case) + int(cap * 10))
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim) * np.float32(2.0)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    outs = {}
    for kernel in (0, 1, 2, 3, 4, 6, 7):
        outs[kernel], err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal,
                                     window, 0, fq, softcap=cap)
        assert err == 0
    for kernel in (1, 2, 3, 4, 6, 7):
        assert np.array_equal(bits(outs[0]), bits(outs[kernel])), kernel
    plain, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, 0, causal, window, 0, fq)
    assert err == 0 and np.max(np.abs(plain - outs[0])) > 1e-3
    for i in sorted({0, nq // 2, nq - 1}):
        m = oracle.encoder_mask(0, nkeys, fq + i, window or None) if causal else None
        ok, want = oracle.heads(q[i], k, v, qheads, kvh, dim, nkeys, m, softcap=cap)
        assert ok
        assert_parity(outs[0][i], want, dim)


def test_softcap_off_is_bitwise_inert(torch, ctx):
    # 0 and -0 are off: the same bits as a descriptor that never set the
    # field, for every kernel; a huge cap stays within rounding of off
    for case in (SOFTCAP_CASES[0], SOFTCAP_CASES[3], SOFTCAP_CASES[5]):
        qheads, kvh, dim, nq, nkeys, causal, window, fq = case
        g = np.random.default_rng(sum(case))
        q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
        k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        for kernel in (0, 4, 6, 2):
            base, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal, window,
                                 0, fq)
            assert err == 0
            for cap in (0.0, -0.0):
                got, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal,
                                    window, 0, fq, softcap=cap)
                assert err == 0 and np.array_equal(bits(got), bits(base)), (kernel, cap)
            huge, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal, window,
                                 0, fq, softcap=1e30)
            assert err == 0 and np.max(np.abs(huge - base)) < 1e-6, kernel


def test_spread_waits_give_up_at_the_host_limit_and_keep_the_bits(pcl, torch, ctx, oracle):
    # a limit of one poll on the spread decode's waits for the other
    # workgroups' scores: the waits run out while the items still run, and
    # each wave then forms the missing score blocks itself by the same chain,
    # so the device entry returns the pipelined kernel's bits with no error
    # bit (one chunk: the output straight from the item workgroups; several:
    # through the launch's merge workgroups); back at the default limit the
    # same context reproduces them too
    qheads, kvh, dim = 16, 8, 256
    g = np.random.default_rng(77)
    for nkeys in (2048, 1024, 256, 200):
        q = prescale(g.standard_normal((1, qheads * dim), dtype=np.float32), dim)
        k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        want, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_PIPE_KV, 1, 0, 0,
                             nkeys - 1)
        assert err == 0
        other = pcl.Context(0, torch.cuda.current_stream().cuda_stream)
        try:
            with pytest.raises(pcl.AttentionError) as e:
                other.set_wait_limit(-1)
            assert e.value.kind == "InvalidParameter"
            other.set_wait_limit(1)
            for _ in range(2):
                got, err = run_desc(torch, other, q, k, v, qheads, kvh, dim,
                                    pcl.KERNEL_SPREAD_KV, 1, 0, 0, nkeys - 1)
                assert err == 0, (nkeys, err)
                assert np.array_equal(bits(got), bits(want)), nkeys
            other.set_wait_limit(0)
            got, err = run_desc(torch, other, q, k, v, qheads, kvh, dim, pcl.KERNEL_SPREAD_KV, 1,
                                0, 0, nkeys - 1)
            assert err == 0
            assert np.array_equal(bits(got), bits(want))
        finally:
            other.close()
        ok, ref = oracle.heads(q[0], k, v, qheads, kvh, dim, nkeys,
                               oracle.encoder_mask(0, nkeys, nkeys - 1, None))
        assert ok
        assert_parity(want[0], ref, dim)


def test_wide_spread_waits_give_up_and_keep_the_bits(pcl, torch, ctx, oracle):
    # the head-dim-512 spread decode under a one-poll wait limit: every
    # slice forms the blocks whose words have not arrived itself, and the
    # output keeps the pipelined kernel's bits (one chunk and several)
    qheads, kvh, dim = 16, 2, 512
    g = np.random.default_rng(512)
    for nkeys in (2048, 200):
        q = prescale(g.standard_normal((1, qheads * dim), dtype=np.float32), dim)
        k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
        want, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_PIPE_KV, 1, 0, 0,
                             nkeys - 1)
        assert err == 0
        other = pcl.Context(0, torch.cuda.current_stream().cuda_stream)
        try:
            other.set_wait_limit(1)
            for _ in range(2):
                got, err = run_desc(torch, other, q, k, v, qheads, kvh, dim,
                                    pcl.KERNEL_SPREAD_KV, 1, 0, 0, nkeys - 1)
                assert err == 0, (nkeys, err)
                assert np.array_equal(bits(got), bits(want)), nkeys
        finally:
            other.close()
        ok, ref = oracle.heads(q[0], k, v, qheads, kvh, dim, nkeys,
                               oracle.encoder_mask(0, nkeys, nkeys - 1, None))
        assert ok
        assert_parity(want[0], ref, dim)


def test_spread_epochs_across_a_counter_wrap(pcl, torch, ctx):
    # the device's epoch counter set just below a wrap of its low 32 bits:
    # the launches before and after the wrap (when the workspace's published
    # words are zeroed again) keep the pipelined kernel's bits, through a
    # context's workspace and through the allocation-free scratch
    lib = pcl.load()
    qheads, kvh, dim, nkeys = 16, 8, 256, 2048
    g = np.random.default_rng(0xE90C)
    q = prescale(g.standard_normal((1, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    want, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_PIPE_KV, 1, 0, 0,
                         nkeys - 1)
    assert err == 0
    for noalloc in (False, True):
        assert lib.pcl_debug_set_epoch_counter(0, (5 << 32) | 0xFFFFFFFD) == 0
        for i in range(6):
            got, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_SPREAD_KV, 1,
                                0, 0, nkeys - 1, noalloc=noalloc)
            assert err == 0, (noalloc, i)
            assert np.array_equal(bits(got), bits(want)), (noalloc, i)


SPREAD_FORM_CASES = [
    # qheads, kvh, dim, nq, nkeys, first_query. The spread decode's launch
    # forms on a 256-CU MI355X: two-wave workgroups with every request up
    # front (at most one 32-dim slice per CU), four-wave workgroups of two
    # slices (two slices per CU), two-wave workgroups in the compiler's order
    # (up to three per CU); each in the local form when the (KV head, unit)
    # groups come in whole eights (8 KV heads here), otherwise (4 KV heads)
    # the three-dimensional grid
    (16, 8, 256, 1, 1024, 1023),  # 32 items, 256 slices: two-wave, early
    (16, 8, 256, 1, 2048, 2047),  # 64 items, 512 slices: four-wave
    (16, 8, 256, 1, 3072, 3071),  # 96 items, 768 slices: two-wave, compiler order
    (16, 8, 208, 1, 2048, 2047),  # head dim below the padded 256: four-wave
    (16, 8, 128, 1, 4096, 4095),  # 128 items, 512 slices at d128: four-wave
    (16, 8, 128, 1, 2000, 1999),  # ragged last chunk at d128: two-wave, early
    (8, 4, 64, 4, 1500, 1496),    # d64, four queries of two heads per KV head
    # the local form (each (KV head, unit) group's workgroups on one XCD)
    # with two groups per XCD: 16 queries, two 16-row units per KV head
    (16, 8, 128, 16, 1000, 984),
    # head dim 512: one-wave slices, 16 per item, items dealt to XCDs
    (16, 2, 512, 1, 2048, 2047),  # 16 items, one slice per CU
    (16, 2, 512, 1, 4096, 4095),  # 32 items, two per CU
    (16, 2, 512, 1, 6000, 5999),  # 48 items (three per CU), ragged last chunk
    (16, 2, 320, 1, 2000, 1999),  # a head dim below the padded 512
    (16, 2, 512, 1, 200, 199),    # one chunk: the output straight from the slices
    (16, 2, 512, 2, 1500, 1498),  # two queries of eight heads per KV head
    (8, 1, 512, 3, 1000, 997),    # two 16-row units, one with padding rows
]


@pytest.mark.parametrize("case", SPREAD_FORM_CASES, ids=lambda c: "x".join(map(str, c)))
def test_spread_forms_match_the_pipelined_kernel_and_the_oracle(pcl, torch, ctx, oracle, case):
    qheads, kvh, dim, nq, nkeys, fq = case
    g = np.random.default_rng(sum(case))
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    got, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_SPREAD_KV, 1, 0, 0, fq)
    assert err == 0
    ref, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_PIPE_KV, 1, 0, 0, fq)
    assert err == 0
    assert np.array_equal(bits(got), bits(ref))
    for i in range(nq):
        ok, want = oracle.heads(q[i], k, v, qheads, kvh, dim, nkeys,
                                oracle.encoder_mask(0, nkeys, fq + i, None))
        assert ok
        assert_parity(got[i], want, dim)


SPREAD_WINDOW_CASES = [
    # qheads, kvh, dim, nq, nkeys, window: the query is the last key. A
    # sliding layer's steady state: the window starts and ends inside chunks
    # (and inside tiles), so partial chunks mix whole tiles, partial tiles
    # and tiles with no allowed key
    (16, 8, 256, 1, 32668, 1024),  # five chunks, both ends partial
    (16, 8, 256, 1, 32668, 600),   # three chunks
    (16, 8, 256, 1, 4100, 1000),   # window start 3100: mid-tile
    (16, 8, 256, 1, 4096, 1024),   # aligned: four whole chunks
    (16, 8, 256, 1, 3000, 33),     # one partial chunk after another's last key
    (16, 8, 128, 2, 2000, 700),    # two queries: rows of one unit see different ranges
    (16, 2, 512, 1, 5000, 1500),   # head dim 512
    (16, 2, 512, 1, 2077, 300),
]


@pytest.mark.parametrize("case", SPREAD_WINDOW_CASES, ids=lambda c: "x".join(map(str, c)))
def test_spread_windows_inside_chunks_match_the_pipelined_kernel_and_the_oracle(
        pcl, torch, ctx, oracle, case):
    qheads, kvh, dim, nq, nkeys, window = case
    fq = nkeys - nq
    g = np.random.default_rng(sum(case))
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    got, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_SPREAD_KV, 1, window,
                        0, fq)
    assert err == 0
    ref, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_PIPE_KV, 1, window,
                        0, fq)
    assert err == 0
    assert np.array_equal(bits(got), bits(ref))
    auto, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, pcl.KERNEL_AUTO, 1, window, 0, fq)
    assert err == 0
    assert np.array_equal(bits(auto), bits(ref))
    for i in range(nq):
        ok, want = oracle.heads(q[i], k, v, qheads, kvh, dim, nkeys,
                                oracle.encoder_mask(0, nkeys, fq + i, window))
        assert ok
        assert_parity(got[i], want, dim)


def test_split_launch_tail_with_masks_segments_and_kv_ranges(torch, ctx, oracle):
    # the canvas shape (4 row blocks x 8 KV heads x 9 chunks = 288 items on
    # 256 CUs) leaves one chunk's items for a last round, which runs as
    # pipelined-kernel items: with an explicit mask and the canvas K/V as a
    # second segment every kernel keeps the bits (a 5-head sub-range, 180
    # items, takes no tail and is checked the same way)
    qheads, kvh, dim, nq, nkeys = 16, 8, 256, 256, 2304
    g = np.random.default_rng(0x7A11)
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    mask = g.random((nq, nkeys)) < 0.7
    mask[:, -1] = True
    outs = {}
    for kernel in (1, 2, 3, 4, 6, 7):
        for kv in [(0, kvh), (2, 7)]:
            out, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, mask=mask,
                                split_at=nkeys - nq, kv=kv)
            assert err == 0
            outs[(kernel, kv)] = out
    for kv in [(0, kvh), (2, 7)]:
        for kernel in (2, 3, 4, 6, 7):
            assert np.array_equal(bits(outs[(1, kv)]), bits(outs[(kernel, kv)])), (kernel, kv)
    group = qheads // kvh
    for i in (0, nq - 1):
        ok, want = oracle.heads(q[i], k.reshape(-1), v.reshape(-1), qheads, kvh, dim, nkeys,
                                mask[i].astype(np.uint8), 2 * group, 7 * group)
        assert ok
        assert_parity(outs[(3, (2, 7))][i], want, dim)


def test_explicit_masks_segments_scale_and_kv_ranges_keep_bits(torch, ctx):
    qheads, kvh, dim, nq, nkeys = 16, 8, 256, 40, 777
    g = np.random.default_rng(99)
    q = g.standard_normal((nq, qheads * dim), dtype=np.float32)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    fq = nkeys - nq
    mask = np.array([[t <= fq + i and fq + i - t < 300 for t in range(nkeys)]
                     for i in range(nq)])
    scale = np.float32(1.0 / 16.0)
    base, err = run_desc(torch, ctx, prescale(q, dim), k, v, qheads, kvh, dim, 1, 1, 300, 0, fq)
    assert err == 0
    for kernel in (1, 2, 3, 4, 6, 7):
        # explicit byte masks equal the descriptor's causal window
        got, err = run_desc(torch, ctx, prescale(q, dim), k, v, qheads, kvh, dim, kernel,
                            mask=mask)
        assert err == 0 and np.array_equal(bits(got), bits(base))
        # the in-kernel q_scale equals the engine's host pre-scale
        got, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, 1, 300, 0, fq,
                            q_scale=float(scale))
        assert err == 0 and np.array_equal(bits(got), bits(base))
        # two KV segments equal one buffer, also across a chunk boundary
        for split in (256, 301):
            got, err = run_desc(torch, ctx, prescale(q, dim), k, v, qheads, kvh, dim, kernel, 1,
                                300, 0, fq, split_at=split)
            assert err == 0 and np.array_equal(bits(got), bits(base))
        # a KV-head range is that slice of the full result
        got, err = run_desc(torch, ctx, prescale(q, dim), k, v, qheads, kvh, dim, kernel, 1,
                            300, 0, fq, kv=(3, 6))
        group = qheads // kvh
        assert err == 0 and np.array_equal(bits(got), bits(base[:, 3 * group * dim:
                                                                6 * group * dim]))


def test_long_launch_combines_agree_across_kernels(torch, ctx, oracle):
    """More than 8 spans of 4096 keys: the split kernels' two-level combine
    and the tiled kernel's in-kernel merges give the same bits."""
    qheads, kvh, dim, nq, nkeys = 16, 8, 256, 64, 36000
    fq = nkeys - nq
    q = gpu_normals(torch, 0x5EED0777, (nq, qheads, dim)) * (1.0 / 16.0)
    k = gpu_normals(torch, 0x5EED0778, (nkeys, kvh, dim))
    v = gpu_normals(torch, 0x5EED0779, (nkeys, kvh, dim))
    outs = {}
    for kernel in (1, 2, 3, 4, 6, 7):
        out = torch.full((nq, qheads, dim), float("nan"), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=nq, k0=k.data_ptr(),
                     v0=v.data_ptr(), n0=nkeys, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0,
                     kh_end=kvh, causal=1, window=0, first_key=0, first_query=fq,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy()
    for kernel in (2, 3, 4, 6, 7):
        assert np.array_equal(bits(outs[1]), bits(outs[kernel])), kernel
    qn, kn, vn = (x.cpu().numpy().reshape(-1) for x in (q, k, v))
    for i in (0, nq - 1):
        m = oracle.encoder_mask(0, nkeys, fq + i, None)
        ok, want = oracle.heads(qn[i * qheads * dim:(i + 1) * qheads * dim], kn, vn, qheads,
                                kvh, dim, nkeys, m)
        assert ok
        assert_parity(outs[1][i], want, dim)


def test_masked_suffix_does_not_change_results(torch, ctx):
    """Decode of position p over keys [0, p] equals the same query inside a
    longer call whose later keys are causally masked (chunk-size
    independence of the engine, docs/architecture.md:34)."""
    qheads, kvh, dim, nkeys = 16, 8, 256, 1500
    g = np.random.default_rng(5)
    q = prescale(g.standard_normal((nkeys, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    full, err = run_desc(torch, ctx, q[1000:1100], k, v, qheads, kvh, dim, 2, 1, 0, 0, 1000)
    assert err == 0
    for p in (1000, 1023, 1024, 1050, 1099):
        one, err = run_desc(torch, ctx, q[p:p + 1], k[:p + 1], v[:p + 1], qheads, kvh, dim, 1,
                            1, 0, 0, p)
        assert err == 0 and np.array_equal(bits(one[0]), bits(full[p - 1000]))


def test_device_error_flags(torch, ctx):
    qheads, kvh, dim, nkeys = 4, 2, 64, 300
    g = np.random.default_rng(8)
    q = g.standard_normal((3, qheads * dim), dtype=np.float32)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    bad_k = k.copy()
    bad_k[10, 1, 5] = np.nan
    bad_v = v.copy()
    bad_v[20, 0, 3] = np.inf
    for kernel in (1, 2, 3, 4, 6, 7):
        _, err = run_desc(torch, ctx, q, bad_k, v, qheads, kvh, dim, kernel)
        assert err & 1
        _, err = run_desc(torch, ctx, q, k, bad_v, qheads, kvh, dim, kernel)
        assert err & 2
        _, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel)
        assert err == 0


@pytest.mark.parametrize("dim", [48, 80, 144, 208, 320, 400])
def test_padded_head_dims_read_only_the_callers_rows(torch, ctx, oracle, dim):
    """Head dims below the kernels' padded size (64, 128, 256, 512): K and V
    end where a NaN-filled tail of their allocation begins, so any read past
    the last key row's last head would turn a score or an output non-finite.
    Every kernel stays finite, error-free and bitwise equal (at 320 and 400
    the head-dim-512 forms: the wave-pair tiled kernel and its fanned last
    round, the four-phase, pipelined and fanned decodes)."""
    qheads, kvh, nq, nkeys = 8, 2, 160, 300
    g = np.random.default_rng(dim)
    q = prescale(g.standard_normal((nq, qheads * dim), dtype=np.float32), dim)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    n = nkeys * kvh * dim
    kbuf = torch.full((n + 4096,), float("nan"), device="cuda:0")
    vbuf = torch.full((n + 4096,), float("nan"), device="cuda:0")
    kbuf[:n] = torch.from_numpy(k.reshape(-1)).to("cuda:0")
    vbuf[:n] = torch.from_numpy(v.reshape(-1)).to("cuda:0")
    tq = torch.from_numpy(q).to("cuda:0")
    outs = {}
    for kernel in (2, 3, 1, 4, 6, 7):
        out = torch.full((nq, qheads * dim), float("nan"), device="cuda:0")
        d = ctx.desc(q=tq.data_ptr(), q_stride=qheads * dim, nq=nq, k0=kbuf.data_ptr(),
                     v0=vbuf.data_ptr(), n0=nkeys, qheads=qheads, kvheads=kvh, dim=dim,
                     kh_first=0, kh_end=kvh, causal=1, window=0, first_key=0,
                     first_query=nkeys - nq, out=out.data_ptr(), o_stride=qheads * dim,
                     kernel=kernel)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0, kernel
        outs[kernel] = out.cpu().numpy()
        assert np.all(np.isfinite(outs[kernel])), kernel
    for kernel in (3, 1, 4, 6, 7):
        assert np.array_equal(bits(outs[2]), bits(outs[kernel])), kernel
    for i in (0, nq - 1):
        m = oracle.encoder_mask(0, nkeys, nkeys - nq + i, None)
        ok, want = oracle.heads(q[i], k, v, qheads, kvh, dim, nkeys, m)
        assert ok
        assert_parity(outs[2][i], want, dim)


# ---- BASELINE.json configs ---------------------------------------------------

def gpu_normals(torch, seed, shape):
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    return torch.randn(shape, generator=gen, device="cuda:0", dtype=torch.float32)


def decode_config(torch, ctx, oracle, qheads, kvh, dim, nkeys, window, seed, unit_k=False):
    q = gpu_normals(torch, seed, (1, qheads, dim)) * float(np.float32(1.0 / math.sqrt(dim)))
    k = gpu_normals(torch, seed + 1, (nkeys, kvh, dim))
    v = gpu_normals(torch, seed + 2, (nkeys, kvh, dim))
    if unit_k:
        k = k / k.norm(dim=-1, keepdim=True)
    outs = {}
    # the automatic choice, then every split-KV kernel: all bitwise equal
    for kernel in (0, 1, 4, 6, 7):
        out = torch.full((1, qheads, dim), float("nan"), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=1, k0=k.data_ptr(),
                     v0=v.data_ptr(), n0=nkeys, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0,
                     kh_end=kvh, causal=1, window=window, first_key=0, first_query=nkeys - 1,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy().reshape(-1)
    for kernel in outs:
        assert np.array_equal(bits(outs[kernel]), bits(outs[0])), kernel
    got = outs[0]
    qn, kn, vn = (x.cpu().numpy().reshape(-1) for x in (q, k, v))
    ok, want = oracle.threaded(qn, 1, kn, vn, qheads, kvh, dim, nkeys, True, 0, nkeys - 1,
                               window, threads=THREADS)
    assert ok
    return assert_parity(got, want, dim)


def test_config1_decode_2048(torch, ctx, oracle):
    decode_config(torch, ctx, oracle, 16, 8, 256, 2048, 0, 0x5EED0001)


def test_config2_sliding_decode_32k_window_1024(torch, ctx, oracle):
    decode_config(torch, ctx, oracle, 16, 8, 256, 32768, 1024, 0x5EED0002)


def test_config2_full_causal_decode_32k(torch, ctx, oracle):
    decode_config(torch, ctx, oracle, 16, 8, 256, 32768, 0, 0x5EED0012)


def test_config3_global_decode_131072_d512(torch, ctx, oracle):
    decode_config(torch, ctx, oracle, 16, 2, 512, 131072, 0, 0x5EED0003, unit_k=True)


@pytest.mark.parametrize("nkeys", [2048, 8192, 32768])
def test_global_layer_decode_below_128k_d512(torch, ctx, oracle, nkeys):
    # config 3's geometry (16/2/512, unit-norm K) at the cache lengths of a
    # conversation before 128K: AUTO fans each chunk item over a workgroup
    decode_config(torch, ctx, oracle, 16, 2, 512, nkeys, 0, 0x5EED0030 + nkeys, unit_k=True)


@pytest.mark.parametrize("label,qheads,kvh,dim,nkeys", [
    ("sliding", 16, 8, 256, 1279), ("global", 16, 2, 512, 3194)])
def test_reference_probe_shapes(pcl, torch, ctx, kernels, oracle, label, qheads, kvh, dim,
                                nkeys):
    # the reference's attention throughput probe (int8/tests.rs:770-809): 8
    # queries (Rng(7) units x 0.1), keys and values (Rng units), every key
    # allowed, through AttentionMulti (attention_multi over host arrays) and
    # through the device entry with every kernel: all bitwise equal, each
    # query within 1e-4 of the exact oracle with the same argmax per head
    nq = 8
    rng = Rng(7)
    queries = [rng.units_c(qheads * dim, 0.1) for _ in range(nq)]
    keys = rng.units_c(nkeys * kvh * dim)
    values = rng.units_c(nkeys * kvh * dim)
    got = kernels.attention_multi(queries, keys, values, kvh, dim, None)
    q = np.stack(queries)
    k = keys.reshape(nkeys, kvh, dim)
    v = values.reshape(nkeys, kvh, dim)
    for kernel in (0, 1, 2, 3, 4, 6, 7):
        out, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel)
        assert err == 0, kernel
        for i in range(nq):
            assert np.array_equal(bits(out[i]), bits(got[i])), (kernel, i)
    for i in range(nq):
        ok, want = oracle.heads(queries[i], keys, values, qheads, kvh, dim, nkeys, None)
        assert ok
        assert_parity(got[i], want, dim)


@pytest.mark.parametrize("window", [1024, 0], ids=["window1024", "global"])
def test_config4_prefill_4096(torch, ctx, oracle, window):
    """Both 4K prefills (sliding window 1024 and global) compared elementwise
    with the exact oracle: every one of the 4096 x 16 rows within 1e-4, the
    same argmax in every row. The oracle runs its bit-identical checker form
    on the host's threads."""
    qheads, kvh, dim, n = 16, 8, 256, 4096
    seed = 0x5EED0004
    q = gpu_normals(torch, seed, (n, qheads, dim)) * float(np.float32(1.0 / 16.0))
    k = gpu_normals(torch, seed + 1, (n, kvh, dim))
    v = gpu_normals(torch, seed + 2, (n, kvh, dim))
    outs = {}
    for kernel in (0, 2, 1):
        out = torch.empty((n, qheads, dim), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=n, k0=k.data_ptr(),
                     v0=v.data_ptr(), n0=n, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0,
                     kh_end=kvh, causal=1, window=window, first_key=0, first_query=0,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy()
    # the whole output: the automatic choice, tiled and split-KV agree bitwise
    assert np.array_equal(bits(outs[0]), bits(outs[2]))
    assert np.array_equal(bits(outs[1]), bits(outs[2]))
    qn, kn, vn = (x.cpu().numpy().reshape(-1) for x in (q, k, v))
    ok, want = oracle.threaded(qn, n, kn, vn, qheads, kvh, dim, n, True, 0, 0, window,
                               threads=THREADS, checker=True)
    assert ok
    assert_parity(outs[0], want, dim)


CANVAS_STEP_GROUPS = [range(0, 12), range(12, 24), range(24, 36), range(36, 48)]


@pytest.mark.parametrize("steps", CANVAS_STEP_GROUPS, ids=lambda r: "steps%d-%d" % (r[0], r[-1]))
def test_config5_canvas_48_denoising_steps(torch, ctx, oracle, steps):
    """The DiffusionGemma canvas: 256 canvas rows attend non-causally to a
    fixed 2048-token prefix and to the step's own canvas K/V (a second
    segment). Every row of every step is compared elementwise with the exact
    oracle (1e-4, same argmax); the 48 steps run as four groups of 12."""
    qheads, kvh, dim, prefix, canvas = 16, 8, 256, 2048, 256
    kp = gpu_normals(torch, 0x5EED0005, (prefix, kvh, dim))
    vp = gpu_normals(torch, 0x5EED0105, (prefix, kvh, dim))
    kpn, vpn = kp.cpu().numpy(), vp.cpu().numpy()
    for step in steps:
        seed = 0x5EED0500 + step
        q = gpu_normals(torch, seed, (canvas, qheads, dim)) * float(np.float32(1.0 / 16.0))
        kc = gpu_normals(torch, seed + 1000, (canvas, kvh, dim))
        vc = gpu_normals(torch, seed + 2000, (canvas, kvh, dim))
        out = torch.empty((canvas, qheads, dim), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=canvas, k0=kp.data_ptr(),
                     v0=vp.data_ptr(), n0=prefix, k1=kc.data_ptr(), v1=vc.data_ptr(), n1=canvas,
                     qheads=qheads, kvheads=kvh, dim=dim, kh_first=0, kh_end=kvh, causal=0,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=0)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        got = out.cpu().numpy()
        kn = np.concatenate([kpn, kc.cpu().numpy()]).reshape(-1)
        vn = np.concatenate([vpn, vc.cpu().numpy()]).reshape(-1)
        qn = q.cpu().numpy().reshape(-1)
        ok, want = oracle.threaded(qn, canvas, kn, vn, qheads, kvh, dim, prefix + canvas, False,
                                   threads=THREADS, checker=True)
        assert ok, step
        assert_parity(got, want, dim)


@pytest.mark.parametrize("window", [0, 1024], ids=["global", "window1024"])
def test_head_dim_512_prefill_4096(torch, ctx, oracle, window):
    """The Gemma-4 / DiffusionGemma global-layer geometry (16 query heads, 2
    KV heads, head dim 512) over a 4096-token prompt, K rows unit-norm: the
    automatic choice (the wave-pair tiled kernel), the chunk-split tiled
    kernel and the split-KV kernel agree bitwise, and every row matches the
    exact oracle within 1e-4 with the same argmax."""
    qheads, kvh, dim, n = 16, 2, 512, 4096
    seed = 0x5EED0D12
    q = gpu_normals(torch, seed, (n, qheads, dim)) * float(np.float32(1.0 / math.sqrt(dim)))
    k = gpu_normals(torch, seed + 1, (n, kvh, dim))
    k = k / k.norm(dim=-1, keepdim=True)
    v = gpu_normals(torch, seed + 2, (n, kvh, dim))
    outs = {}
    for kernel in (0, 2, 3, 1):
        out = torch.empty((n, qheads, dim), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=n, k0=k.data_ptr(),
                     v0=v.data_ptr(), n0=n, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0,
                     kh_end=kvh, causal=1, window=window, first_key=0, first_query=0,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)
        if kernel == 0:
            assert ctx.resolve_kernel(d) == 2
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy()
    for kernel in (2, 3, 1):
        assert np.array_equal(bits(outs[0]), bits(outs[kernel])), kernel
    qn, kn, vn = (x.cpu().numpy().reshape(-1) for x in (q, k, v))
    ok, want = oracle.threaded(qn, n, kn, vn, qheads, kvh, dim, n, True, 0, 0, window,
                               threads=THREADS, checker=True)
    assert ok
    assert_parity(outs[0], want, dim)


def test_head_dim_512_canvas(torch, ctx, oracle):
    """A DiffusionGemma global-layer canvas step: 256 canvas rows over a
    2048-token prefix and the step's own K/V (second segment), non-causal,
    16/2 heads at head dim 512: every kernel bitwise equal, every row within
    1e-4 of the exact oracle with the same argmax."""
    qheads, kvh, dim, prefix, canvas = 16, 2, 512, 2048, 256
    kp = gpu_normals(torch, 0x5EED0D15, (prefix, kvh, dim))
    vp = gpu_normals(torch, 0x5EED0D16, (prefix, kvh, dim))
    q = gpu_normals(torch, 0x5EED0D17, (canvas, qheads, dim)) * float(
        np.float32(1.0 / math.sqrt(dim)))
    kc = gpu_normals(torch, 0x5EED0D18, (canvas, kvh, dim))
    vc = gpu_normals(torch, 0x5EED0D19, (canvas, kvh, dim))
    outs = {}
    for kernel in (0, 2, 3, 4, 1):
        out = torch.empty((canvas, qheads, dim), device="cuda:0")
        d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=canvas, k0=kp.data_ptr(),
                     v0=vp.data_ptr(), n0=prefix, k1=kc.data_ptr(), v1=vc.data_ptr(), n1=canvas,
                     qheads=qheads, kvheads=kvh, dim=dim, kh_first=0, kh_end=kvh, causal=0,
                     out=out.data_ptr(), o_stride=qheads * dim, kernel=kernel)
        if kernel == 0:
            assert ctx.resolve_kernel(d) in (2, 3)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy()
    for kernel in (2, 3, 4, 1):
        assert np.array_equal(bits(outs[0]), bits(outs[kernel])), kernel
    kn = np.concatenate([kp.cpu().numpy(), kc.cpu().numpy()]).reshape(-1)
    vn = np.concatenate([vp.cpu().numpy(), vc.cpu().numpy()]).reshape(-1)
    ok, want = oracle.threaded(q.cpu().numpy().reshape(-1), canvas, kn, vn, qheads, kvh, dim,
                               prefix + canvas, False, threads=THREADS, checker=True)
    assert ok
    assert_parity(outs[0], want, dim)
