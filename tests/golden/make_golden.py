"""Writes the golden attention vectors under tests/golden/.

Inputs follow the reference tests' generators (the xorshift Rng and seeds of
src/kernels/quantized/int8/tests.rs:15-33, 399-476, 594-659). Expected
outputs come from this repository's CPU oracle (oracle/), whose exact path
restates p9_ref_attention_heads (src/kernels/portable/reference.rs:320-393);
the reference holds no stored attention vectors of its own
(fixtures/README.md:5-11). Before writing, every exact output is checked
against an independent f64 NumPy restatement (tools/oracle/reference.py:
125-137 equation) so a fixture never records an oracle error.

python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from helpers import Rng, softmax_attention_f64  # noqa: E402
from oracle import binding as orc  # noqa: E402

TWIN = [(16, 8, 256, 37), (16, 2, 512, 5), (4, 4, 16, 1), (2, 1, 32, 64), (6, 3, 48, 6),
        (4, 2, 80, 7), (8, 2, 144, 3), (2, 1, 320, 130), (6, 2, 16, 9), (9, 3, 32, 2),
        (10, 2, 48, 11), (8, 1, 16, 1), (4, 1, 96, 3), (16, 2, 512, 130)]


def twin_cases():
    rng = Rng(0xa77e)
    for qheads, kvh, dim, nkeys in TWIN:
        query = rng.units(qheads * dim, 0.5)
        keys = rng.units(nkeys * kvh * dim, 0.5)
        values = rng.units(nkeys * kvh * dim)
        mask = np.array([t % 3 != 1 or nkeys == 1 for t in range(nkeys)])
        yield (qheads, kvh, dim, nkeys), query, keys, values, mask


def checksum(x):
    return np.uint64(int(np.asarray(x, np.float32).view(np.uint32).astype(np.uint64).sum()))


def main():
    out = {}
    for i, (geom, q, k, v, mask) in enumerate(twin_cases()):
        qheads, kvh, dim, nkeys = geom
        out["twin%d_geometry" % i] = np.array(geom, np.int64)
        out["twin%d_input_checksums" % i] = np.array([checksum(q), checksum(k), checksum(v)],
                                                     np.uint64)
        for tag, allowed in (("all", None), ("mask", mask)):
            ok, exact = orc.heads(q, k, v, qheads, kvh, dim, nkeys, allowed)
            ok2, b32 = orc.heads(q, k, v, qheads, kvh, dim, nkeys, allowed, binary32=True)
            assert ok and ok2
            ref = softmax_attention_f64(q, k, v, qheads, kvh, dim, allowed)
            assert np.max(np.abs(exact - ref)) < 2e-6
            out["twin%d_%s_exact" % (i, tag)] = exact
            out["twin%d_%s_binary32" % (i, tag)] = b32
    np.savez_compressed(os.path.join(HERE, "twin_outputs.npz"), **out)

    # Small cases stored with their inputs: GQA groups, masks with holes,
    # a causal window, one allowed key.
    rng = Rng(0x5eed)
    small = {}
    specs = [(4, 2, 16, 9, "window"), (6, 3, 32, 17, "holes"), (8, 1, 64, 5, "one"),
             (2, 2, 16, 33, "all")]
    for i, (qheads, kvh, dim, nkeys, kind) in enumerate(specs):
        q = rng.units(qheads * dim)
        k = rng.units(nkeys * kvh * dim)
        v = rng.units(nkeys * kvh * dim)
        if kind == "window":
            mask = orc.encoder_mask(0, nkeys, nkeys - 2, 4)
        elif kind == "holes":
            mask = np.array([t % 4 in (0, 3) for t in range(nkeys)])
        elif kind == "one":
            mask = np.arange(nkeys) == 3
        else:
            mask = None
        ok, exact = orc.heads(q, k, v, qheads, kvh, dim, nkeys, mask)
        assert ok
        ref = softmax_attention_f64(q, k, v, qheads, kvh, dim, mask)
        assert np.max(np.abs(exact - ref)) < 2e-6
        small["small%d_geometry" % i] = np.array([qheads, kvh, dim, nkeys], np.int64)
        small["small%d_query" % i] = q
        small["small%d_keys" % i] = k
        small["small%d_values" % i] = v
        small["small%d_mask" % i] = (np.ones(nkeys, bool) if mask is None else mask)
        small["small%d_has_mask" % i] = np.array(mask is not None)
        small["small%d_exact" % i] = exact
    np.savez_compressed(os.path.join(HERE, "small_cases.npz"), **small)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
