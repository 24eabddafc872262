"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Checks come from the reference's own known-answer tests (numbers copied),
the reference's independent NumPy oracle equation, closed forms and
invariants chosen so that a wrong head mapping, stride, sign, mask or
rounding point fails at least one of them.
"""
import math
import os

import numpy as np
import pytest

from helpers import Rng, softmax_attention_f64

E = math.e


def test_grouped_attention_is_token_major_contiguous_heads_and_scale_one(oracle):
    # src/kernels/reference/tests.rs:115-135
    query = [1.0, 0.0, 2.0, 0.0, 0.0, 1.0, 0.0, 2.0]
    keys = [1.0, 0.0, 0.0, 1.0, -1.0, 0.0, 0.0, -1.0]
    values = [10.0, 11.0, 20.0, 21.0, 30.0, 31.0, 40.0, 41.0]
    rc, y = oracle.attention_heads_checked(query, keys, values, 2, 2)
    assert rc == 0
    for h in range(4):
        score = 1.0 if h % 2 == 0 else 2.0
        p = math.exp(score) / (math.exp(score) + math.exp(-score))
        kh = h // 2
        for d in range(2):
            expected = p * values[kh * 2 + d] + (1.0 - p) * values[4 + kh * 2 + d]
            assert abs(float(y[h * 2 + d]) - expected) < 3e-6
    rc, y = oracle.attention_heads_checked(query, keys, values, 2, 2, [False, True])
    assert rc == 0
    assert y.tolist() == [30.0, 31.0, 30.0, 31.0, 40.0, 41.0, 40.0, 41.0]


def _patterned():
    f = np.float32
    query = np.array([f(i % 11) / f(7.0) - f(0.5) for i in range(24)], np.float32)
    keys = np.array([f(i % 17) / f(13.0) - f(0.5) for i in range(60)], np.float32)
    values = np.array([f(i % 19) / f(3.0) - f(2.0) for i in range(60)], np.float32)
    return query, keys, values


def test_attention_matches_independent_nontrivial_masked_equations(oracle):
    # src/kernels/reference/tests.rs:137-170
    query, keys, values = _patterned()
    mask = [True, False, True, True, False]
    rc, actual = oracle.attention_heads_checked(query, keys, values, 2, 6, mask)
    assert rc == 0
    for h in range(4):
        kh = h // 2
        scores = []
        for t in range(5):
            if not mask[t]:
                scores.append(-np.inf)
                continue
            s = sum(float(query[h * 6 + d]) * float(keys[t * 12 + kh * 6 + d]) for d in range(6))
            scores.append(float(np.float32(s)))
        mx = max(scores)
        exps = [math.exp(s - mx) for s in scores]
        total = sum(exps)
        probs = [float(np.float32(e / total)) for e in exps]
        for d in range(6):
            expected = float(np.float32(sum(probs[t] * float(values[t * 12 + kh * 6 + d])
                                            for t in range(5))))
            assert abs(float(actual[h * 6 + d]) - expected) < 1e-6


def test_attention_rejects_invalid_shapes_masks_and_overflow(oracle):
    # src/kernels/reference/tests.rs:180-186; status 1 InvalidShape,
    # 2 InvalidParameter, 3 NonFiniteValue (src/kernels/reference.rs:6-11).
    one = [1.0, 1.0]
    assert oracle.attention_heads_checked(one, one, one, 0, 2)[0] == 1
    assert oracle.attention_heads_checked(one, one, one, 1, 0)[0] == 1
    assert oracle.attention_heads_checked(one, one, one, 1, 2, [False])[0] == 2
    assert oracle.attention_heads_checked(one, one, one, 1, 2, [])[0] == 1
    assert oracle.attention_heads_checked([1.0] * 3, [1.0] * 4, [1.0] * 4, 2, 1)[0] == 1
    assert oracle.attention_heads_checked(one, one, [1.0], 1, 2)[0] == 1
    big = [np.finfo(np.float32).max] * 2
    assert oracle.attention_heads_checked(big, big, one, 1, 2)[0] == 3


def test_encoder_window_and_cache_retention_have_distinct_boundaries(oracle):
    # src/engine/attention/tests.rs:130-149
    T, F = True, False
    assert oracle.encoder_mask(7, 6, 10).tolist() == [T, T, T, T, F, F]
    assert oracle.encoder_mask(7, 6, 10, 3).tolist() == [F, T, T, T, F, F]
    assert oracle.encoder_mask(7, 6, 10, 1).tolist() == [F, F, F, T, F, F]
    assert oracle.retained_count(10, 3) == 2
    assert oracle.retained_count(10, 1) == 0
    assert oracle.retained_count(10) == 10
    assert oracle.encoder_mask(2**64 - 1, 2, 0) is None
    assert oracle.encoder_mask(0, 1, 0, 0) is None


TWIN_GEOMETRIES = [
    # src/kernels/quantized/int8/tests.rs:405-423
    (16, 8, 256, 37), (16, 2, 512, 5), (4, 4, 16, 1), (2, 1, 32, 64), (6, 3, 48, 6),
    (4, 2, 80, 7), (8, 2, 144, 3), (2, 1, 320, 130), (6, 2, 16, 9), (9, 3, 32, 2),
    (10, 2, 48, 11), (8, 1, 16, 1), (4, 1, 96, 3), (16, 2, 512, 130),
]


def twin_inputs():
    """The twin test's inputs, in its generator order (int8/tests.rs:403-429)."""
    rng = Rng(0xa77e)
    for qheads, kvh, dim, nkeys in TWIN_GEOMETRIES:
        query = rng.units(qheads * dim, 0.5)
        keys = rng.units(nkeys * kvh * dim, 0.5)
        values = rng.units(nkeys * kvh * dim)
        mask = np.array([t % 3 != 1 or nkeys == 1 for t in range(nkeys)])
        yield qheads, kvh, dim, nkeys, query, keys, values, mask


@pytest.fixture(scope="module")
def twin_cases():
    return list(twin_inputs())


def test_binary32_is_close_to_exact_on_the_twin_geometries(oracle, twin_cases):
    # int8/tests.rs:459-461: |binary32 - exact| <= 2e-5 (1 + |exact|)
    for qheads, kvh, dim, nkeys, query, keys, values, mask in twin_cases:
        for allowed in (None, mask):
            ok_a, a = oracle.heads(query, keys, values, qheads, kvh, dim, nkeys, allowed,
                                   binary32=True)
            ok_e, e = oracle.heads(query, keys, values, qheads, kvh, dim, nkeys, allowed)
            assert ok_a and ok_e
            assert np.all(np.abs(a - e) <= 2e-5 * (1.0 + np.abs(e)))


def test_exact_matches_the_reference_numpy_equation(oracle, twin_cases):
    # tools/oracle/reference.py:125-137 restated independently in f64; the
    # exact path rounds scores and probabilities to f32, so they agree to
    # a few f32 ulps of the result.
    for qheads, kvh, dim, nkeys, query, keys, values, mask in twin_cases:
        for allowed in (None, mask):
            ok, e = oracle.heads(query, keys, values, qheads, kvh, dim, nkeys, allowed)
            assert ok
            ref = softmax_attention_f64(query, keys, values, qheads, kvh, dim, allowed)
            assert np.max(np.abs(e - ref)) < 2e-6


def test_closed_forms_pin_mask_mapping_and_weights(oracle):
    rng = np.random.default_rng(11)
    qheads, kvh, dim, nkeys = 8, 2, 32, 19
    q = rng.standard_normal(qheads * dim).astype(np.float32)
    k = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    v = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    vv = v.reshape(nkeys, kvh, dim)
    # one allowed key: the output is exactly that key's value row of the
    # head's KV head (pins the GQA mapping h // group and the V stride)
    for t in (0, 7, 18):
        mask = np.zeros(nkeys, bool)
        mask[t] = True
        ok, out = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask)
        assert ok
        for h in range(qheads):
            assert np.array_equal(out[h * dim:(h + 1) * dim], vv[t, h // (qheads // kvh)])
    # q = 0: uniform weights, the output is the mean of the allowed values
    mask = np.arange(nkeys) % 4 != 2
    ok, out = oracle.heads(np.zeros_like(q), k, v, qheads, kvh, dim, nkeys, mask)
    assert ok
    for h in range(qheads):
        mean = vv[mask, h // (qheads // kvh)].astype(np.float64).mean(0)
        assert np.max(np.abs(out[h * dim:(h + 1) * dim] - mean)) < 1e-6
    # two keys: p = sigmoid(s0 - s1) exactly as the two-key closed form
    ok, out = oracle.heads(q, k[:2 * kvh * dim], v[:2 * kvh * dim], qheads, kvh, dim, 2)
    kk = k.reshape(nkeys, kvh, dim)
    for h in range(qheads):
        kh = h // (qheads // kvh)
        s0 = float(np.float32(np.dot(q[h * dim:(h + 1) * dim].astype(np.float64),
                                     kk[0, kh].astype(np.float64))))
        s1 = float(np.float32(np.dot(q[h * dim:(h + 1) * dim].astype(np.float64),
                                     kk[1, kh].astype(np.float64))))
        p0 = 1.0 / (1.0 + math.exp(s1 - s0))
        want = p0 * vv[0, kh].astype(np.float64) + (1.0 - p0) * vv[1, kh].astype(np.float64)
        assert np.max(np.abs(out[h * dim:(h + 1) * dim] - want)) < 2e-6


def test_invariants_permutation_and_linearity(oracle):
    rng = np.random.default_rng(12)
    qheads, kvh, dim, nkeys = 4, 2, 16, 23
    q = rng.standard_normal(qheads * dim).astype(np.float32)
    k = rng.standard_normal((nkeys, kvh, dim)).astype(np.float32)
    v = rng.standard_normal((nkeys, kvh, dim)).astype(np.float32)
    mask = rng.random(nkeys) < 0.7
    mask[3] = True
    ok, base = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask)
    assert ok
    perm = rng.permutation(nkeys)
    ok, permuted = oracle.heads(q, k[perm], v[perm], qheads, kvh, dim, nkeys, mask[perm])
    assert ok
    assert np.max(np.abs(permuted - base)) < 1e-6
    # linear in V: out(2V + 1) = 2 out(V) + 1 (weights sum to one)
    ok, lin = oracle.heads(q, k, (2 * v + 1).astype(np.float32), qheads, kvh, dim, nkeys, mask)
    assert ok
    assert np.max(np.abs(lin - (2 * base + 1))) < 1e-5
    # masked keys never matter: replacing them changes nothing, bitwise
    k2, v2 = k.copy(), v.copy()
    k2[~mask] = 123.0
    v2[~mask] = -7.0
    ok, same = oracle.heads(q, k2, v2, qheads, kvh, dim, nkeys, mask)
    assert ok and np.array_equal(same, base)


def test_head_ranges_and_threads_do_not_change_results(oracle):
    # int8/tests.rs:594-659 (head ranges) and docs/architecture.md:34 (worker
    # count) for the exact and binary32 paths of the oracle.
    rng = Rng(0x7f4a7c159e3779b9)
    for qheads, kvh, dim, nkeys in [(16, 8, 32, 7), (8, 1, 64, 33), (4, 2, 16, 1),
                                    (6, 2, 48, 5), (9, 3, 16, 2)]:
        q = rng.units(qheads * dim)
        k = rng.units(nkeys * kvh * dim)
        v = rng.units(nkeys * kvh * dim)
        mask = np.array([t % 3 != 1 or t == 0 for t in range(nkeys)])
        for binary32 in (False, True):
            for allowed in (None, mask):
                ok, full = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed,
                                        binary32=binary32)
                assert ok
                for a in range(qheads):
                    for b in range(a, qheads + 1):
                        ok, part = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, a, b,
                                                binary32=binary32)
                        assert ok and np.array_equal(part, full[a * dim:b * dim])
                ok, _ = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, 0, qheads + 1,
                                     binary32=binary32)
                assert not ok
    rng = np.random.default_rng(5)
    qheads, kvh, dim, nkeys, nq = 8, 2, 32, 40, 12
    q = rng.standard_normal(nq * qheads * dim).astype(np.float32)
    k = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    v = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    for binary32 in (False, True):
        outs = [oracle.threaded(q, nq, k, v, qheads, kvh, dim, nkeys, True, 0, nkeys - nq, 9,
                                threads=t, binary32=binary32)[1] for t in (1, 3, 16)]
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
        ok, one = oracle.threaded(q[:qheads * dim], 1, k, v, qheads, kvh, dim, nkeys, True, 0,
                                  nkeys - nq, 9, threads=5, binary32=binary32)
        assert ok and np.array_equal(one, outs[0][:qheads * dim])


def bits32(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def test_checker_form_equals_the_exact_oracle_bit_for_bit(oracle):
    # the fast form used to check full-size GPU outputs gives the exact
    # oracle's bits: random geometries and scales, sparse and dense masks,
    # head ranges, key counts that are not multiples of its four-key step,
    # non-finite scores rejected the same way
    g = np.random.default_rng(0xC4EC)
    for case in range(60):
        kvh = int(g.choice([1, 2, 3, 8]))
        group = int(g.choice([1, 2, 4]))
        qheads = kvh * group
        dim = int(g.choice([16, 48, 64, 256, 512]))
        nkeys = int(g.integers(1, 90))
        scale = float(g.choice([0.05, 1.0, 6.0]))
        q = (g.standard_normal(qheads * dim) * scale).astype(np.float32)
        k = g.standard_normal(nkeys * kvh * dim).astype(np.float32)
        v = g.standard_normal(nkeys * kvh * dim).astype(np.float32)
        density = float(g.choice([0.05, 0.5, 1.0]))
        mask = g.random(nkeys) < density
        mask[int(g.integers(nkeys))] = True
        a = int(g.integers(qheads))
        b = int(g.integers(a, qheads + 1))
        for allowed in (None, mask):
            ok1, want = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, a, b)
            ok2, got = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, a, b,
                                    checker=True)
            assert ok1 and ok2
            assert np.array_equal(bits32(got), bits32(want)), case
    q = np.ones(32, np.float32)
    big = np.full(32, np.finfo(np.float32).max, np.float32)
    assert not oracle.heads(big, big, q, 1, 1, 32, 1, checker=True)[0]
    # threaded prefill with a window: the checker form equals the timed form
    qheads, kvh, dim, n = 8, 2, 64, 150
    q = (g.standard_normal(n * qheads * dim) / 8).astype(np.float32)
    k = g.standard_normal(n * kvh * dim).astype(np.float32)
    v = g.standard_normal(n * kvh * dim).astype(np.float32)
    for window in (0, 37):
        ok1, want = oracle.threaded(q, n, k, v, qheads, kvh, dim, n, True, 0, 0, window,
                                    threads=4)
        ok2, got = oracle.threaded(q, n, k, v, qheads, kvh, dim, n, True, 0, 0, window,
                                   threads=3, checker=True)
        assert ok1 and ok2 and np.array_equal(bits32(got), bits32(want))


def test_sampled_prefill_rows_equal_the_whole_prompts_rows(oracle):
    # the CPU baseline's prefill sample: every step-th query of a prompt, each
    # with its own position's causal (and window) mask
    g = np.random.default_rng(0x5A3)
    qheads, kvh, dim, n, step = 8, 2, 32, 97, 16
    q = (g.standard_normal((n, qheads * dim)) / 6).astype(np.float32)
    k = g.standard_normal(n * kvh * dim).astype(np.float32)
    v = g.standard_normal(n * kvh * dim).astype(np.float32)
    for window in (0, 20):
        ok, full = oracle.threaded(q.reshape(-1), n, k, v, qheads, kvh, dim, n, True, 0, 0,
                                   window, threads=3)
        assert ok
        rows = q[::step]
        ok, part = oracle.threaded(rows.reshape(-1), len(rows), k, v, qheads, kvh, dim, n, True,
                                   0, 0, window, threads=4, query_step=step)
        assert ok
        assert np.array_equal(part.reshape(len(rows), -1), full.reshape(n, -1)[::step])


def test_multi_query_contract_equals_single_queries(oracle):
    # int8/tests.rs:661-768: every multi row equals its single-query call
    rng = Rng(0x7a11ed)
    for qheads, kvh, dim, nkeys, nq, window in [(16, 2, 512, 150, 6, 40), (4, 2, 16, 37, 9, 5)]:
        queries = [rng.units(qheads * dim) for _ in range(nq)]
        k = rng.units(nkeys * kvh * dim)
        v = rng.units(nkeys * kvh * dim)
        masks = np.array([[t <= nkeys - nq + i and t + window > nkeys - nq + i
                           for t in range(nkeys)] for i in range(nq)])
        group = qheads // kvh
        flat = np.concatenate(queries)
        for binary32 in (False, True):
            singles = [oracle.heads(q, k, v, qheads, kvh, dim, nkeys, masks[i],
                                    binary32=binary32)[1] for i, q in enumerate(queries)]
            for k0, k1 in [(0, kvh), (0, 1), (kvh - 1, kvh)]:
                olen = (k1 - k0) * group * dim
                ok, part = oracle.multi_kv(flat, nq, qheads * dim, k, v, qheads, kvh, dim, nkeys,
                                           masks, nkeys, olen, k0, k1, binary32=binary32)
                assert ok
                for i in range(nq):
                    want = singles[i][k0 * group * dim:k1 * group * dim]
                    assert np.array_equal(part[i * olen:(i + 1) * olen], want)


def test_non_finite_inputs_are_errors(oracle):
    # int8/tests.rs:443-457 and reference.rs:450-452
    rng = np.random.default_rng(3)
    qheads, kvh, dim, nkeys = 4, 2, 16, 5
    q = rng.standard_normal(qheads * dim).astype(np.float32)
    k = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    v = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    bad_v = v.copy()
    bad_v[(nkeys - 1) * kvh * dim + dim - 1] = np.inf
    bad_k = k.copy()
    bad_k[dim - 1] = np.nan
    assert oracle.attention_heads_checked(q, k, bad_v, kvh, dim)[0] == 3
    assert oracle.attention_heads_checked(q, bad_k, v, kvh, dim)[0] == 3
    assert not oracle.heads(q, k, bad_v, qheads, kvh, dim, nkeys, binary32=True)[0]
    assert not oracle.heads(q, bad_k, v, qheads, kvh, dim, nkeys, binary32=True)[0]


def test_softcap_oracle_reduces_to_the_exact_path_for_a_huge_cap(oracle):
    # cap * tanh(s / cap) = s to far below an f32 ulp when s / cap is tiny, so
    # a cap of 1e30 must leave every bit of the exact path (a misplaced cap,
    # s * cap inside tanh, or a cap applied after the softmax all fail)
    rng = np.random.default_rng(41)
    qheads, kvh, dim, nkeys = 8, 2, 64, 300
    q = (rng.standard_normal(qheads * dim) * 0.5).astype(np.float32)
    k = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    v = rng.standard_normal(nkeys * kvh * dim).astype(np.float32)
    mask = oracle.encoder_mask(0, nkeys, 250, 100)
    ok, plain = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask)
    ok2, capped = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask, softcap=1e30)
    assert ok and ok2
    assert np.array_equal(plain.view(np.uint32), capped.view(np.uint32))
    # and a moderate cap changes results
    ok3, cap4 = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask, softcap=4.0)
    assert ok3 and not np.array_equal(plain, cap4)


def test_softcap_oracle_two_key_sigmoid_closed_form(oracle):
    # two keys with scores +a and -a: the output is sigma(c1 - c2) v1 +
    # sigma(c2 - c1) v2 with c = cap tanh(s / cap), a different formula from
    # the oracle's softmax; capped and uncapped weights differ visibly
    dim = 16
    for a, cap in ((3.0, 2.0), (0.5, 30.0), (7.0, 0.75)):
        q = np.zeros(dim, np.float32)
        q[0] = a
        k = np.zeros((2, dim), np.float32)
        k[0, 0], k[1, 0] = 1.0, -1.0
        v = np.zeros((2, dim), np.float32)
        v[0, 1], v[1, 1] = 5.0, -3.0
        v[0, 2] = 1.0
        ok, y = oracle.heads(q, k, v, 1, 1, dim, 2, softcap=cap)
        assert ok
        c1 = cap * math.tanh(a / cap)
        w1 = 1.0 / (1.0 + math.exp(-2.0 * c1))
        assert abs(float(y[1]) - (5.0 * w1 - 3.0 * (1.0 - w1))) < 2e-6
        assert abs(float(y[2]) - w1) < 1e-6
        assert y[0] == 0.0


def test_softcap_oracle_saturates_to_the_mean_of_values(oracle):
    # a tiny cap maps every score of 10 caps or more to the same f32 value, so
    # the weights are exactly uniform: the output is the mean of the values
    rng = np.random.default_rng(5)
    dim, nkeys, cap = 32, 37, 0.01
    k = np.abs(rng.standard_normal((nkeys, dim))).astype(np.float32) + 0.5
    q = np.full(dim, 1.0, np.float32)  # every score >= 16 >> 10 caps
    v = rng.standard_normal((nkeys, dim)).astype(np.float32)
    ok, y = oracle.heads(q, k, v, 1, 1, dim, nkeys, softcap=cap)
    assert ok
    assert np.max(np.abs(y - v.astype(np.float64).mean(axis=0))) < 1e-6
    assert not oracle.heads(q, k, v, 1, 1, dim, nkeys, softcap=-1.0)[0]


def test_c_xorshift_stream_equals_the_python_generator(oracle):
    # The reference tests' generator (int8/tests.rs:15-33), whose Python form
    # follows it line by line; the C form feeds the large GPU cases.
    for seed, scale in [(7, 1.0), (7, 0.1), (0xa77e, 1.0), (0x7f4a7c159e3779b9, 0.1)]:
        a, b = Rng(seed), Rng(seed)
        for n in (1, 3000, 17):
            want = a.units(n, scale)
            got = b.units_c(n, scale)
            assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), (seed, scale, n)
            assert a.state == b.state
    # a known point of the stream: xorshift64 of 1 is 0x40822041
    r = Rng(1)
    r.units_c(1)
    assert r.state == 0x40822041


def test_binary32_twin_expf_matches_the_reference_libm_digest(oracle):
    # the twin's softmax exponential gives the reference's bits on every 61st
    # binary32 pattern (src/libm/tests.rs:20-22, 70, 80-84): glibc 2.28's
    # POWER8 expf, which the reference's libm ports
    assert oracle.libm_digest(2) == 0xFE568FD438D7D408


def test_oracle_self_check_under_address_and_undefined_behaviour_sanitizers():
    # make -C oracle sanitize: the oracle and its self-check built with
    # -fsanitize=address,undefined (host code only) and run
    import shutil
    import subprocess
    if shutil.which("make") is None or shutil.which("gcc") is None:
        pytest.skip("no host C toolchain")
    odir = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")
    res = subprocess.run(["make", "-s", "-B", "-C", odir, "sanitize"], capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "oracle selftest: ok" in res.stdout
