"""The device-resident layer cache (pcl_kv_cache_*) against the engine's
LayerCache (src/engine/attention.rs:244-311).

CPU tests pin the oracle's restatement (oracle_cache_*) with the numbers of
the reference's own cache tests (src/engine/attention/tests.rs) and with a
brute-force model of what a cache must retain: all kept rows, then only the
last window-1 of them after a commit. GPU tests drive the device cache and
the oracle through the same operation sequences and compare rows bitwise,
then check that attention through the cache's descriptors equals attention
over the oracle's staged rows with the engine's explicit encoder masks.
"""
import numpy as np
import pytest

from helpers import normals

RESOURCE_LIMIT = 4


def model_rows(kept, window):
    """What a committed cache retains: the last retained_count kept rows."""
    r = len(kept) if window is None else min(len(kept), window - 1)
    return kept[len(kept) - r:]


def rows_of(seed, n, width):
    return normals(seed, n * width).reshape(n, width)


# ---- oracle pinning (CPU) --------------------------------------------------

def test_window_three_keeps_two_and_chunking_agrees(oracle):
    # attention/tests.rs:5-29 (fixture window 3: layer 0 sliding, layer 1
    # global, 4 encoder tokens) and tests.rs:206-225 (5 tokens, chunks 1+2+2)
    width = 8
    for window, tokens, chunks, retained in ((3, 4, (2, 2), 2), (None, 4, (2, 2), 4),
                                            (3, 5, (1, 2, 2), 2)):
        k = rows_of(1, tokens, width)
        v = rows_of(2, tokens, width)
        whole = oracle.OracleCache(2, 4, 64, window, 1 << 20)
        rc, _ = whole.append(k, v, tokens)
        assert rc == 0
        whole.commit()
        assert whole.total == tokens
        assert whole.retained() == retained
        chunked = oracle.OracleCache(2, 4, 64, window, 1 << 20)
        at = 0
        for n in chunks:
            rc, _ = chunked.append(k[at:at + n], v[at:at + n], n)
            assert rc == 0
            chunked.commit()
            at += n
        wk, wv = whole.rows()
        ck, cv = chunked.rows()
        assert np.array_equal(wk, ck) and np.array_equal(wv, cv)
        assert np.array_equal(wk, k[tokens - retained:])
        assert whole.first_position() == tokens - retained


def test_byte_limit_is_one_staged_pair_and_failures_leave_the_cache(oracle):
    # attention/tests.rs:40-47: new_cache(16) holds exactly one K/V token of
    # width 2; two tokens are a ResourceLimit, the total stays 0
    c = oracle.OracleCache(1, 2, 64, 3, 16)
    assert c.status == 0
    rc, _ = c.append(np.ones(4), np.ones(4), 2)
    assert rc == RESOURCE_LIMIT
    assert c.total == 0 and c.retained() == 0
    rc, _ = c.append(np.ones(2), np.ones(2), 1)
    assert rc == 0 and c.total == 1
    # below one token's K+V (attention.rs:487-492; tests.rs:270-276)
    assert oracle.OracleCache(1, 2, 64, 3, 15).status == RESOURCE_LIMIT
    # the position limit (check_stage: total + n <= context)
    c = oracle.OracleCache(1, 2, 3, None, 1 << 20)
    rc, _ = c.append(np.ones(4), np.ones(4), 2)
    assert rc == 0
    rc, _ = c.append(np.ones(4), np.ones(4), 2)
    assert rc == RESOURCE_LIMIT and c.total == 2
    rc, _ = c.append(np.ones(2), np.ones(2), 1)
    assert rc == 0 and c.total == 3
    rc, _ = c.append(np.ones(0), np.ones(0), 0)
    assert rc == 1  # empty input: Error::Shape


def random_steps(seed, steps, max_n):
    """(n, action, tokens) per step: action 0 commit, 1 keep, 2 rollback."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(steps):
        n = int(rng.integers(1, max_n + 1))
        action = int(rng.choice(3, p=[0.6, 0.25, 0.15]))
        out.append((n, action, int(rng.integers(1, n + 1))))
    return out


@pytest.mark.parametrize("window", [None, 1, 2, 5, 17])
def test_oracle_matches_the_retention_model(oracle, window):
    width = 6
    c = oracle.OracleCache(2, 3, 10_000, window, 1 << 24)
    kept = []
    for i, (n, action, tokens) in enumerate(random_steps(7 + (window or 0), 120, 9)):
        k = rows_of(100 + i, n, width)
        v = rows_of(200 + i, n, width)
        before = c.rows()
        rc, pending = c.append(k, v, n)
        assert rc == 0
        ck, _ = c.rows()
        assert np.array_equal(ck, np.concatenate([before[0], k]))
        if action == 2:
            c.rollback(pending)
            assert all(np.array_equal(a, b) for a, b in zip(c.rows(), before))
            continue
        if action == 1:
            c.keep(pending, tokens)
            k, v = k[:tokens], v[:tokens]
        c.commit()
        kept += list(zip(k, v))
        assert c.total == len(kept)
        want = model_rows(kept, window)
        got_k, got_v = c.rows()
        assert c.retained() == len(want)
        assert np.array_equal(got_k, np.array([r[0] for r in want]).reshape(-1, width))
        assert np.array_equal(got_v, np.array([r[1] for r in want]).reshape(-1, width))
        assert c.first_position() == len(kept) - len(want)


def test_keep_beyond_the_step_only_moves_the_position(oracle):
    # keep() truncates only when the kept length is shorter (attention.rs:
    # 286-296): a layer without rows for the step keeps its rows
    c = oracle.OracleCache(1, 2, 100, None, 1 << 20)
    rc, pending = c.append(np.arange(6), np.arange(6), 3)
    assert rc == 0
    c.keep(pending, 5)
    assert c.total == 5 and c.retained() == 3


# ---- the device cache (GPU) -------------------------------------------------

@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


@pytest.fixture(scope="module")
def ctx(pcl, torch):
    c = pcl.Context(0, torch.cuda.current_stream().cuda_stream)
    yield c
    c.close()


def read_rows(cache, width):
    """(keys, values, first_position) of the device cache on the host."""
    _, _, rows, first = cache.view()
    keys, values = cache.read(0, rows)
    return keys.reshape(rows, width), values.reshape(rows, width), first


def to_dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to("cuda:0")


def assert_same_cache(cache, ref, width):
    keys, values, first = read_rows(cache, width)
    want_k, want_v = ref.rows()
    assert cache.total_tokens() == ref.total
    assert cache.retained_tokens() == ref.retained()
    assert first == ref.first_position()
    assert np.array_equal(keys.view(np.uint32), want_k.view(np.uint32))
    assert np.array_equal(values.view(np.uint32), want_v.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("window", [None, 2, 7, 40])
def test_device_cache_follows_the_oracle_through_random_steps(pcl, torch, ctx, oracle, window):
    kvh, dim = 2, 16
    width = kvh * dim
    cache = pcl.LayerCache(ctx, kvh, dim, 4000, window, 1 << 24)
    ref = oracle.OracleCache(kvh, dim, 4000, window, 1 << 24)
    for i, (n, action, tokens) in enumerate(random_steps(31 + (window or 0), 90, 13)):
        k = rows_of(1000 + i, n, width)
        v = rows_of(2000 + i, n, width)
        tk, tv = to_dev(torch, k), to_dev(torch, v)
        pending = cache.append(tk.data_ptr(), tv.data_ptr(), n)
        rc, ref_pending = ref.append(k, v, n)
        assert rc == 0
        assert_same_cache(cache, ref, width)
        if action == 2:
            cache.rollback(pending)
            ref.rollback(ref_pending)
        else:
            if action == 1:
                cache.keep(pending, tokens)
                ref.keep(ref_pending, tokens)
            cache.commit()
            ref.commit()
        assert_same_cache(cache, ref, width)
    cache.close()


@pytest.mark.gpu
def test_device_cache_appends_device_unaligned_and_host_rows(pcl, torch, ctx, oracle):
    # device rows on the cache's device take the one-launch copy (16-byte
    # pieces when aligned, floats when not); host rows take runtime copies:
    # every source lands the same rows
    kvh, dim = 2, 16
    width = kvh * dim
    cache = pcl.LayerCache(ctx, kvh, dim, 4000, None, 1 << 24)
    ref = oracle.OracleCache(kvh, dim, 4000, None, 1 << 24)
    for i, n in enumerate([1, 3, 64, 1, 517]):
        k = rows_of(3000 + i, n, width)
        v = rows_of(4000 + i, n, width)
        kind = i % 3
        if kind == 0:  # aligned device rows
            tk, tv = to_dev(torch, k), to_dev(torch, v)
            pk, pv = tk.data_ptr(), tv.data_ptr()
        elif kind == 1:  # device rows one float past an aligned start
            tk = to_dev(torch, np.concatenate([[np.nan], k.reshape(-1)]))
            tv = to_dev(torch, np.concatenate([[np.nan], v.reshape(-1)]))
            pk, pv = tk.data_ptr() + 4, tv.data_ptr() + 4
        else:  # pageable host rows
            hk = np.ascontiguousarray(k, dtype=np.float32)
            hv = np.ascontiguousarray(v, dtype=np.float32)
            pk, pv = hk.ctypes.data, hv.ctypes.data
        cache.append(pk, pv, n)
        ref.append(k, v, n)
        cache.commit()
        ref.commit()
        torch.cuda.synchronize()
        assert_same_cache(cache, ref, width)
    assert ctx.sync() == 0
    cache.close()


@pytest.mark.gpu
def test_reserved_rows_keep_the_buffers_until_exceeded(pcl, torch, ctx, oracle):
    # room reserved up front: appends within it keep the buffers in place;
    # past it the cache grows as before; the rows follow the oracle's cache
    # throughout, and a reservation past the byte limit is held to it
    kvh, dim = 2, 16
    width = kvh * dim
    token = width * 2 * 4
    cache = pcl.LayerCache(ctx, kvh, dim, 4000, None, 150 * token)
    ref = oracle.OracleCache(kvh, dim, 4000, None, 150 * token)
    with pytest.raises(pcl.AttentionError):
        cache.reserve_rows(-1)
    keep = []  # the appended device rows stay alive until the copies ran

    def append(k, v, n):
        tk, tv = to_dev(torch, k), to_dev(torch, v)
        keep.append((tk, tv))
        cache.append(tk.data_ptr(), tv.data_ptr(), n)
        ref.append(k, v, n)
        cache.commit()
        ref.commit()

    cache.reserve_rows(100)
    k0, v0, _, _ = cache.view()
    for i, n in enumerate([1, 40, 59]):  # 100 rows in all
        append(rows_of(5000 + i, n, width), rows_of(6000 + i, n, width), n)
        assert cache.view()[:2] == (k0, v0)
        assert_same_cache(cache, ref, width)
    cache.reserve_rows(80)  # grow-only: nothing moves
    assert cache.view()[:2] == (k0, v0)
    append(rows_of(7000, 3, width), rows_of(7001, 3, width), 3)
    assert cache.view()[:2] != (k0, v0)
    assert_same_cache(cache, ref, width)
    cache.reserve_rows(10 ** 9)  # held to the 150-row byte limit
    k1, v1, _, _ = cache.view()
    append(rows_of(7002, 47, width), rows_of(7003, 47, width), 47)
    assert cache.view()[:2] == (k1, v1)
    assert_same_cache(cache, ref, width)
    cache.close()


@pytest.mark.gpu
def test_device_cache_limits_match_check_stage(pcl, torch, ctx):
    # attention/tests.rs:40-47 and 270-276 on the device cache: max_bytes
    # bounds the retained plus appended K+V of a step
    token = 16 * 2 * 4
    with pytest.raises(pcl.AttentionError) as e:
        pcl.LayerCache(ctx, 1, 16, 64, 3, token - 1)
    assert e.value.kind == "ResourceLimit"
    rows = to_dev(torch, np.ones((4, 16)))
    cache = pcl.LayerCache(ctx, 1, 16, 64, 3, token)
    with pytest.raises(pcl.AttentionError) as e:
        cache.append(rows.data_ptr(), rows.data_ptr(), 2)
    assert e.value.kind == "ResourceLimit"
    assert cache.total_tokens() == 0 and cache.retained_tokens() == 0
    cache.append(rows.data_ptr(), rows.data_ptr(), 1)
    cache.commit()
    with pytest.raises(pcl.AttentionError) as e:  # 1 retained + 1 new > one token
        cache.append(rows.data_ptr(), rows.data_ptr(), 1)
    assert e.value.kind == "ResourceLimit"
    assert cache.total_tokens() == 1 and cache.retained_tokens() == 1
    with pytest.raises(pcl.AttentionError) as e:
        cache.append(rows.data_ptr(), rows.data_ptr(), 0)
    assert e.value.kind == "InvalidShape"
    cache.close()
    # the position limit: window 3 retains 2, so three tokens always fit
    cache = pcl.LayerCache(ctx, 1, 16, 3, 3, 3 * token)
    for _ in range(3):
        cache.append(rows.data_ptr(), rows.data_ptr(), 1)
        cache.commit()
    assert cache.total_tokens() == 3 and cache.retained_tokens() == 2
    with pytest.raises(pcl.AttentionError) as e:
        cache.append(rows.data_ptr(), rows.data_ptr(), 1)
    assert e.value.kind == "ResourceLimit"
    cache.close()


def direct_attention(torch, ctx, q, keys, values, qheads, kvh, dim, mask):
    """The same keys with an explicit [nq][nkeys] mask (or none)."""
    nq, nkeys = q.shape[0], keys.shape[0]
    tq, tk, tv = to_dev(torch, q), to_dev(torch, keys), to_dev(torch, values)
    out = torch.full((nq, qheads * dim), float("nan"), device="cuda:0")
    kw = dict(q=tq.data_ptr(), q_stride=qheads * dim, nq=nq, k0=tk.data_ptr(),
              v0=tv.data_ptr(), n0=nkeys, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0,
              kh_end=kvh, out=out.data_ptr(), o_stride=qheads * dim)
    keep = [tq, tk, tv]
    if mask is not None:
        tm = torch.from_numpy(np.ascontiguousarray(mask, dtype=np.uint8)).to("cuda:0")
        kw.update(mask=tm.data_ptr(), mask_stride=nkeys)
        keep.append(tm)
    ctx.launch(ctx.desc(**kw))
    assert ctx.sync() == 0
    return out.cpu().numpy()


def cache_attention(torch, ctx, desc_fn, q, qheads, kvh, dim, **extra):
    nq = q.shape[0]
    tq = to_dev(torch, q)
    out = torch.full((nq, qheads * dim), float("nan"), device="cuda:0")
    d = desc_fn(q=tq.data_ptr(), q_stride=qheads * dim, nq=nq, qheads=qheads, kh_first=0,
                kh_end=kvh, out=out.data_ptr(), o_stride=qheads * dim, **extra)
    ctx.launch(d)
    assert ctx.sync() == 0
    return out.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("window,dim", [(None, 256), (5, 256), (300, 128), (9, 512)])
def test_encoder_passes_through_the_cache_equal_the_staged_view(pcl, torch, ctx, oracle,
                                                                 window, dim):
    # encode_in_place's view (attention.rs:956-987): the retained rows plus
    # the step, masks encoder_mask(first_key, count, first_query + i, window)
    qheads, kvh = 8, 2
    width = kvh * dim
    cache = pcl.LayerCache(ctx, kvh, dim, 100_000, window, 1 << 30)
    ref = oracle.OracleCache(kvh, dim, 100_000, window, 1 << 30)
    for step, n in enumerate((37, 1, 300, 4, 1)):
        k = rows_of(3000 + step, n, width) * np.float32(0.5)
        v = rows_of(4000 + step, n, width)
        q = rows_of(5000 + step, n, qheads * dim) * np.float32(1.0 / 16.0)
        tk, tv = to_dev(torch, k), to_dev(torch, v)
        pending = cache.append(tk.data_ptr(), tv.data_ptr(), n)
        rc, _ = ref.append(k, v, n)
        assert rc == 0
        got = cache_attention(torch, ctx, lambda **kw: cache.encoder_desc(pending, **kw), q,
                              qheads, kvh, dim)
        keys, values = ref.rows()
        first_key = ref.total - n - (ref.retained() - n)
        mask = np.stack([oracle.encoder_mask(first_key, keys.shape[0], ref.total - n + i,
                                             window) for i in range(n)])
        want = direct_attention(torch, ctx, q, keys, values, qheads, kvh, dim, mask)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        ok, exact = oracle.threaded(q, n, keys, values, qheads, kvh, dim, keys.shape[0], 1,
                                    first_key, ref.total - n, window or 0, threads=8)
        assert ok
        assert float(np.max(np.abs(got.reshape(-1) - exact))) <= 1e-4
        cache.commit()
        ref.commit()
    cache.close()


@pytest.mark.gpu
def test_decoder_canvas_over_the_cache_is_bidirectional_and_read_only(pcl, torch, ctx, oracle):
    # decode_routed (attention.rs:1156-1163): retained rows then the canvas
    # K/V, no mask; actual_diffusiongemma_local_complete_block (tests.rs:
    # 204-264): the cache is unchanged and a repeat gives the same output
    qheads, kvh, dim, window = 8, 1, 256, 3
    width = kvh * dim
    cache = pcl.LayerCache(ctx, kvh, dim, 1000, window, 1 << 26)
    ref = oracle.OracleCache(kvh, dim, 1000, window, 1 << 26)
    k, v = rows_of(1, 5, width), rows_of(2, 5, width)
    tk, tv = to_dev(torch, k), to_dev(torch, v)
    cache.append(tk.data_ptr(), tv.data_ptr(), 5)
    ref.append(k, v, 5)
    cache.commit()
    ref.commit()
    assert cache.retained_tokens() == 2 and cache.total_tokens() == 5
    ck, cv = rows_of(3, 2, width), rows_of(4, 2, width)
    q = rows_of(5, 2, qheads * dim) * np.float32(1.0 / 16.0)
    tck, tcv = to_dev(torch, ck), to_dev(torch, cv)
    before = read_rows(cache, width)
    got = cache_attention(torch, ctx, lambda **kw: cache.decoder_desc(tck.data_ptr(),
                                                                      tcv.data_ptr(), 2, **kw),
                          q, qheads, kvh, dim)
    again = cache_attention(torch, ctx, lambda **kw: cache.decoder_desc(tck.data_ptr(),
                                                                        tcv.data_ptr(), 2, **kw),
                            q, qheads, kvh, dim)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    after = read_rows(cache, width)
    assert all(np.array_equal(a, b) for a, b in zip(before[:2], after[:2]))
    assert before[2] == after[2] and cache.total_tokens() == 5
    keys, values = ref.rows()
    keys = np.concatenate([keys, ck])
    values = np.concatenate([values, cv])
    want = direct_attention(torch, ctx, q, keys, values, qheads, kvh, dim, None)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # query 0 sees the second canvas key (no causal mask): masking it changes
    # the output, as the reference test asserts
    causal = direct_attention(torch, ctx, q[:1], keys, values, qheads, kvh, dim,
                              np.array([[1, 1, 1, 0]]))
    assert np.any(np.abs(causal[0] - got[0]) > 1e-6)
    cache.close()


@pytest.mark.gpu
def test_shared_kv_layer_attends_over_its_source_step(pcl, torch, ctx, oracle):
    # encode_shared_in_place (attention.rs:1086-1145): queries at this
    # cache's positions over the source's rows of the same step, this
    # layer's window; only the position advances
    qheads, kvh, dim = 8, 2, 128
    width = kvh * dim
    source = pcl.LayerCache(ctx, kvh, dim, 1000, None, 1 << 26)
    shared = pcl.LayerCache(ctx, kvh, dim, 1000, 4, 1 << 26)
    first = rows_of(9, 6, width)
    t0 = to_dev(torch, first)
    source.append(t0.data_ptr(), t0.data_ptr(), 6)
    source.commit()
    shared.advance(6)
    shared.commit()
    k, v = rows_of(10, 3, width), rows_of(11, 3, width)
    tk, tv = to_dev(torch, k), to_dev(torch, v)
    sp = source.append(tk.data_ptr(), tv.data_ptr(), 3)
    q = rows_of(12, 3, qheads * dim) * np.float32(1.0 / 16.0)
    got = cache_attention(torch, ctx, lambda **kw: shared.shared_desc(source, sp, 3, **kw), q,
                          qheads, kvh, dim)
    keys = np.concatenate([first, k])
    values = np.concatenate([first, v])
    mask = np.stack([oracle.encoder_mask(0, 9, 6 + i, 4) for i in range(3)])
    want = direct_attention(torch, ctx, q, keys, values, qheads, kvh, dim, mask)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    pending = shared.advance(3)
    assert shared.total_tokens() == 9 and shared.retained_tokens() == 0
    with pytest.raises(pcl.AttentionError):
        shared.shared_desc(source, sp, 3)  # the shared total has moved on
    shared.keep(pending, 2)
    source.keep(sp, 2)
    assert shared.total_tokens() == 8 and source.total_tokens() == 8
    shared.close()
    source.close()


@pytest.mark.gpu
@pytest.mark.parametrize("nq,window", [(8, 0), (5, 0), (16, 1024), (2, 0)])
def test_speculative_verify_over_a_long_cache(pcl, torch, ctx, oracle, nq, window):
    # encode_speculative (text.rs:709-797): the previous token and its drafts
    # appended to a 32K cache, causal attention of those positions over the
    # cache and themselves, then keep(accepted) and commit; every kernel gives
    # the same bits, within 1e-4 of the exact oracle
    qheads, kvh, dim, cached = 16, 8, 256, 32760
    width = kvh * dim
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x5EED0900 + nq)
    k = torch.randn((cached + nq, width), generator=g, device="cuda:0")
    v = torch.randn((cached + nq, width), generator=g, device="cuda:0")
    q = torch.randn((nq, qheads * dim), generator=g, device="cuda:0") * (1.0 / 16.0)
    cache = pcl.LayerCache(ctx, kvh, dim, 40000, window or None, 1 << 32)
    cache.append(k.data_ptr(), v.data_ptr(), cached)
    cache.commit()
    pending = cache.append(k[cached:].data_ptr(), v[cached:].data_ptr(), nq)
    outs = {}
    for kernel in (0, 1, 2, 4, 6, 7):
        out = torch.full((nq, qheads * dim), float("nan"), device="cuda:0")
        d = cache.encoder_desc(pending, q=q.data_ptr(), q_stride=qheads * dim, nq=nq,
                               qheads=qheads, kh_first=0, kh_end=kvh, out=out.data_ptr(),
                               o_stride=qheads * dim, kernel=kernel)
        if kernel == 0:
            assert ctx.resolve_kernel(d) in (pcl.KERNEL_SPLIT_KV, pcl.KERNEL_PIPE_KV,
                                             pcl.KERNEL_SPREAD_KV)
        ctx.reserve(ctx.workspace_bytes(d))
        ctx.launch(d)
        assert ctx.sync() == 0
        outs[kernel] = out.cpu().numpy()
    for kernel in outs:
        assert np.array_equal(outs[kernel].view(np.uint32), outs[0].view(np.uint32)), kernel
    _, _, rows, first = cache.view()
    kn, vn = k[cached + nq - rows:].cpu().numpy(), v[cached + nq - rows:].cpu().numpy()
    ok, want = oracle.threaded(q.cpu().numpy(), nq, kn, vn, qheads, kvh, dim, rows, True, first,
                               cached, window, threads=8)
    assert ok
    got = outs[0].reshape(-1)
    assert float(np.max(np.abs(got - want))) <= 1e-4
    # accept the first half of the drafts: later positions are gone
    accepted = max(1, nq // 2)
    cache.keep(pending, accepted)
    cache.commit()
    assert cache.total_tokens() == cached + accepted
    keys, _, first = read_rows(cache, width)
    assert first == cache.total_tokens() - keys.shape[0]
    assert np.array_equal(keys[-1], k[cached + accepted - 1].cpu().numpy())
    cache.close()
