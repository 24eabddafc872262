"""Test data and independent checks shared by the test modules."""
import numpy as np


class Rng:
    """The reference tests' xorshift64 generator
    (src/kernels/quantized/int8/tests.rs:15-33)."""

    MASK = (1 << 64) - 1

    def __init__(self, seed):
        self.state = seed & self.MASK

    def next(self):
        x = self.state
        x ^= (x << 13) & self.MASK
        x ^= x >> 7
        x ^= (x << 17) & self.MASK
        self.state = x
        return x

    def unit(self):
        """(next % 20001) as f32 / 10000 - 1, in binary32 arithmetic."""
        return np.float32(np.float32(self.next() % 20001) / np.float32(10000.0)) - np.float32(1.0)

    def units(self, n, scale=1.0):
        out = np.empty(n, np.float32)
        for i in range(n):
            out[i] = self.unit()
        if scale != 1.0:
            out = (out * np.float32(scale)).astype(np.float32)
        return out

    def units_c(self, n, scale=1.0):
        """units() through the oracle's C generator (for inputs of millions of
        values); the same values and state, which a CPU test checks."""
        from oracle import binding
        out, self.state = binding.xorshift_units(self.state, n, scale)
        return out


def normals(seed, n):
    """Seeded i.i.d. N(0,1) f32 (numpy PCG64, deterministic across hosts)."""
    return np.random.default_rng(seed).standard_normal(n, dtype=np.float32)


def prescale(q, dim):
    """The engine's query pre-scale: f32(q * f32(1/sqrt(d)))
    (src/engine/nemotron/forward.rs:336-346)."""
    s = np.float32(1.0 / np.sqrt(np.float64(dim)))
    return (np.asarray(q, np.float32) * s).astype(np.float32)


def softmax_attention_f64(query, keys, values, qheads, kvheads, dim, allowed=None):
    """Independent restatement of the reference's NumPy oracle equation
    (tools/oracle/reference.py:125-137): scores = K q, softmax over
    np.where(allowed, scores, -inf) in f64, w @ V. One query position."""
    q = np.asarray(query, np.float64).reshape(qheads, dim)
    k = np.asarray(keys, np.float64).reshape(-1, kvheads, dim)
    v = np.asarray(values, np.float64).reshape(-1, kvheads, dim)
    rep = qheads // kvheads
    out = np.empty((qheads, dim))
    for head in range(qheads):
        kv = head // rep
        scores = k[:, kv, :] @ q[head]
        if allowed is not None:
            scores = np.where(np.asarray(allowed, bool), scores, -np.inf)
        w = np.exp(scores - scores.max())
        w /= w.sum()
        out[head] = w @ v[:, kv, :]
    return out.reshape(-1)


def row_argmax_agree(got, want, dim):
    """Per (query, head) row of dim values: the same argmax. Any mismatch
    fails, near-ties included: the reference's comparator reports a near-tie
    as an explanation, never as a pass (tools/compare-full-canvas.py:14-17).
    Returns (ok, mismatches) with one (row, expected top-1 minus top-2
    margin) per mismatching row, for the failure report."""
    g = np.asarray(got).reshape(-1, dim)
    w = np.asarray(want).reshape(-1, dim)
    bad = np.nonzero(g.argmax(1) != w.argmax(1))[0]
    mismatches = []
    for r in bad:
        s = np.sort(w[r])
        mismatches.append((int(r), float(s[-1] - s[-2])))
    return not mismatches, mismatches
