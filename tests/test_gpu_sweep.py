"""Seeded sweep of random attention geometries on the GPU.

Each case draws a geometry (GQA group, head dim 16-512, query count, key
count, causal / sliding / explicit masks, one or two K/V segments, a KV-head
sub-range, the Q pre-scale) and runs it through every kernel choice of the
device-resident entry. All kernels must return the same bits (the canonical
arithmetic of csrc/attention_device.hpp), and sampled rows must match the
exact oracle (p9_ref_attention_heads, src/kernels/portable/reference.rs:
320-393) within 1e-4 with the same argmax, as the fixed cases of
test_gpu_parity.py require. The cases are fixed by their seeds.
"""
import numpy as np
import pytest

from test_gpu_parity import assert_parity, bits, run_desc

pytestmark = pytest.mark.gpu

DIMS = [16, 32, 48, 64, 80, 128, 144, 256, 320, 512]
GROUPS = [1, 2, 4, 8]
KERNELS = (1, 2, 3, 4, 6, 7)


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


def draw(seed):
    """One geometry; every query row keeps at least its own position."""
    g = np.random.default_rng(0x5EED5000 + seed)
    dim = int(g.choice(DIMS))
    group = int(g.choice(GROUPS))
    kvh = int(g.choice([1, 2, 4, 8] if dim <= 256 else [1, 2]))
    qheads = kvh * group
    nkeys = int(g.choice([1, 17, 256, 300, 1000, 2049, 4100, 6000]))
    nq = int(min(nkeys, g.choice([1, 1, 3, 8, 33, 64, 300])))
    mode = g.choice(["causal", "window", "mask", "none"])
    window = int(g.integers(1, nkeys + 1)) if mode == "window" else 0
    first_query = int(g.integers(nq - 1, nkeys)) - (nq - 1)  # last query <= nkeys - 1
    split_at = int(g.integers(1, nkeys)) if nkeys > 1 and g.random() < 0.4 else None
    kv = (0, kvh)
    if kvh > 1 and g.random() < 0.4:
        a = int(g.integers(0, kvh))
        kv = (a, int(g.integers(a + 1, kvh + 1)))
    q_scale = float(np.float32(1.0 / np.sqrt(dim))) if g.random() < 0.5 else 1.0
    return dict(dim=dim, kvh=kvh, qheads=qheads, nkeys=nkeys, nq=nq, mode=str(mode),
                window=window, first_query=first_query, split_at=split_at, kv=kv,
                q_scale=q_scale, seed=seed)


def masks_of(c):
    """Per-query allowed keys (the engine's encoder_mask form, attention.rs:
    1166-1182), or a random explicit mask that keeps each query's own key."""
    nq, nkeys, fq = c["nq"], c["nkeys"], c["first_query"]
    t = np.arange(nkeys)[None, :]
    qp = fq + np.arange(nq)[:, None]
    if c["mode"] == "none":
        return np.ones((nq, nkeys), bool)
    if c["mode"] == "mask":
        g = np.random.default_rng(0x5EED6000 + c["seed"])
        m = g.random((nq, nkeys)) < 0.6
        m[np.arange(nq), fq + np.arange(nq)] = True
        return m
    m = t <= qp
    if c["window"]:
        m &= qp - t < c["window"]
    return m


@pytest.mark.parametrize("seed", range(160))
def test_random_geometry_every_kernel_same_bits_and_oracle(torch, ctx, oracle, seed):
    c = draw(seed)
    g = np.random.default_rng(0x5EED7000 + seed)
    dim, kvh, qheads, nq, nkeys = c["dim"], c["kvh"], c["qheads"], c["nq"], c["nkeys"]
    q = g.standard_normal((nq, qheads * dim), dtype=np.float32)
    k = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    v = g.standard_normal((nkeys, kvh, dim), dtype=np.float32)
    allowed = masks_of(c)
    causal = 1 if c["mode"] in ("causal", "window") else 0
    mask = allowed if c["mode"] == "mask" else None
    outs = {}
    for kernel in KERNELS:
        out, err = run_desc(torch, ctx, q, k, v, qheads, kvh, dim, kernel, causal=causal,
                            window=c["window"], first_query=c["first_query"], mask=mask,
                            split_at=c["split_at"], kv=c["kv"], q_scale=c["q_scale"])
        assert err == 0, (c, kernel)
        outs[kernel] = out
    for kernel in KERNELS[1:]:
        assert np.array_equal(bits(outs[KERNELS[0]]), bits(outs[kernel])), (c, kernel)
    group = qheads // kvh
    h0, h1 = c["kv"][0] * group, c["kv"][1] * group
    # the engine pre-scales Q in f32 before the call (nemotron/forward.rs:336-346)
    qs = (q * np.float32(c["q_scale"])).astype(np.float32)
    for i in sorted({0, nq // 2, nq - 1}):
        ok, want = oracle.heads(qs[i], k.reshape(-1), v.reshape(-1), qheads, kvh, dim, nkeys,
                                allowed[i].astype(np.uint8), h0, h1)
        assert ok, c
        assert_parity(outs[KERNELS[0]][i], want, dim)
