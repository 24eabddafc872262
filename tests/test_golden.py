"""Golden vectors (tests/golden/): the oracle reproduces them bit for bit on
the CPU, and the GPU path matches them within 1e-4 with the same argmax."""
import os

import numpy as np
import pytest

from helpers import row_argmax_agree

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def twin_cases():
    import sys
    sys.path.insert(0, GOLDEN)
    import make_golden
    return list(make_golden.twin_cases()), make_golden.checksum


def test_twin_fixtures_regenerate_and_the_oracle_reproduces_them(oracle):
    data = load("twin_outputs.npz")
    cases, checksum = twin_cases()
    for i, (geom, q, k, v, mask) in enumerate(cases):
        assert tuple(data["twin%d_geometry" % i]) == geom
        sums = data["twin%d_input_checksums" % i]
        assert [checksum(q), checksum(k), checksum(v)] == list(sums)
        qheads, kvh, dim, nkeys = geom
        for tag, allowed in (("all", None), ("mask", mask)):
            ok, exact = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed)
            assert ok and np.array_equal(exact, data["twin%d_%s_exact" % (i, tag)])
            ok, b32 = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, binary32=True)
            assert ok and np.array_equal(b32, data["twin%d_%s_binary32" % (i, tag)])


def small_cases():
    data = load("small_cases.npz")
    n = len([k for k in data if k.endswith("_geometry")])
    for i in range(n):
        geom = tuple(int(x) for x in data["small%d_geometry" % i])
        mask = data["small%d_mask" % i] if bool(data["small%d_has_mask" % i]) else None
        yield (geom, data["small%d_query" % i], data["small%d_keys" % i],
               data["small%d_values" % i], mask, data["small%d_exact" % i])


def test_small_fixtures_reproduce_bitwise(oracle):
    for (qheads, kvh, dim, nkeys), q, k, v, mask, exact in small_cases():
        ok, got = oracle.heads(q, k, v, qheads, kvh, dim, nkeys, mask)
        assert ok and np.array_equal(got, exact)


@pytest.mark.gpu
def test_gpu_matches_golden_vectors(pcl):
    kernels = pcl.HipKernels()
    data = load("twin_outputs.npz")
    cases, _ = twin_cases()
    for i, (geom, q, k, v, mask) in enumerate(cases):
        qheads, kvh, dim, nkeys = geom
        for tag, allowed in (("all", None), ("mask", mask)):
            want = data["twin%d_%s_exact" % (i, tag)]
            got = kernels.attention(q, k, v, kvh, dim, allowed)
            assert np.max(np.abs(got - want)) <= 1e-4
            assert row_argmax_agree(got, want, dim)[0]
    for (qheads, kvh, dim, nkeys), q, k, v, mask, exact in small_cases():
        got = kernels.attention(q, k, v, kvh, dim, mask)
        assert np.max(np.abs(got - exact)) <= 1e-4
        assert row_argmax_agree(got, exact, dim)[0]
