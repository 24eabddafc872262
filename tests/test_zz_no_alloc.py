"""pcl_attention_launch_noalloc (include/pcl_attention.h) against
pcl_attention_launch, through the C ABI: the same kernels with the partials
in the GPU's fixed scratch array instead of the context's workspace, so the
outputs must be equal bit for bit; two calls in a row, the second smaller
(the array keeps the first call's contents), and the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 64 << 20  # PCL_NOALLOC_SCRATCH_BYTES


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


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def normals(torch, seed, shape):
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    return torch.randn(shape, generator=gen, device="cuda:0", dtype=torch.float32)


def both(torch, ctx, qheads, kvh, dim, nq, prefix, canvas, causal, window, seed, kernel=0):
    """One descriptor launched through both entries; (noalloc out, launch
    out, workspace bytes)."""
    nkeys = prefix + canvas
    q = normals(torch, seed, (nq, qheads, dim)) * float(np.float32(1.0 / np.sqrt(dim)))
    k = normals(torch, seed + 1, (nkeys, kvh, dim))
    v = normals(torch, seed + 2, (nkeys, kvh, dim))
    kw = dict(q=q.data_ptr(), q_stride=qheads * dim, nq=nq, qheads=qheads, kvheads=kvh, dim=dim,
              kh_first=0, kh_end=kvh, causal=causal, window=window, first_key=0,
              first_query=nkeys - nq if causal else prefix, o_stride=qheads * dim,
              kernel=kernel)
    if canvas:
        kc, vc = k[prefix:].contiguous(), v[prefix:].contiguous()
        kp, vp = k[:prefix].contiguous(), v[:prefix].contiguous()
        kw.update(k0=kp.data_ptr(), v0=vp.data_ptr(), n0=prefix, k1=kc.data_ptr(),
                  v1=vc.data_ptr(), n1=canvas)
        keep = (kc, vc, kp, vp)
    else:
        kw.update(k0=k.data_ptr(), v0=v.data_ptr(), n0=nkeys)
        keep = ()
    outs = []
    for noalloc in (True, False):
        out = torch.full((nq, qheads, dim), float("nan"), device="cuda:0")
        d = ctx.desc(out=out.data_ptr(), **kw)
        if noalloc:
            ws = ctx.workspace_bytes(d)
            assert 0 < ws <= NOALLOC_BYTES, ws
            ctx.launch_noalloc(d)
        else:
            ctx.reserve(ctx.workspace_bytes(d))
            ctx.launch(d)
        assert ctx.sync() == 0
        outs.append(out.cpu().numpy())
    del keep
    return outs[0], outs[1], ws


@pytest.mark.parametrize("first,second", [
    # 32K decode (128 chunk partials, 8 spans), then a 2K decode (which
    # merges its own partials)
    ((16, 8, 256, 1, 32768, 0, 1, 0, 0x5EED0A01), (16, 8, 256, 1, 2048, 0, 1, 0, 0x5EED0A02)),
    # the same 32K decode through the four-phase kernel (chunk partials in
    # the scratch body, then the combine kernel), then a 2K decode
    ((16, 8, 256, 1, 32768, 0, 1, 0, 0x5EED0A07, 1), (16, 8, 256, 1, 2048, 0, 1, 0, 0x5EED0A08)),
    # 128K decode at head dim 512, then a sliding 1024-key window over 4K
    ((16, 2, 512, 1, 131072, 0, 1, 0, 0x5EED0A03), (16, 8, 256, 1, 4096, 0, 1, 1024, 0x5EED0A04)),
    # the 256 x 2304 canvas (chunk-split prefill, pipelined tail, combine),
    # then a smaller canvas
    ((16, 8, 256, 256, 2048, 256, 0, 0, 0x5EED0A05), (16, 8, 256, 64, 700, 64, 0, 0, 0x5EED0A06)),
], ids=["decode32k-then-2k", "decode32k-four-phase-then-2k", "decode128k-d512-then-window",
        "canvas-then-smaller"])
def test_noalloc_equals_launch_bitwise_on_two_calls(pcl, torch, ctx, first, second):
    # the second call's input is smaller, and so is its workspace (or equal,
    # for two launches that each need only the published-word region)
    sizes = []
    for case in (first, second):
        qheads, kvh, dim, nq, prefix, canvas, causal, window, seed = case[:9]
        kernel = case[9] if len(case) > 9 else 0
        got, want, ws = both(torch, ctx, qheads, kvh, dim, nq, prefix, canvas, causal, window,
                             seed, kernel)
        assert np.all(np.isfinite(got))
        assert np.array_equal(bits(got), bits(want))
        sizes.append(ws)
    assert sizes[1] <= sizes[0]


def test_noalloc_rejects_a_launch_beyond_its_scratch(pcl, torch, ctx):
    # an 8K-token prefill runs the tiled kernel with running totals across
    # two 4096-key spans: 8 KV heads x 16384 rows x 256 floats = 128 MiB of
    # workspace, beyond the 64 MiB array; refused before any launch, the
    # output untouched, and the context still works afterwards
    qheads, kvh, dim, n = 16, 8, 256, 8192
    q = torch.zeros((n, qheads, dim), device="cuda:0")
    k = torch.zeros((n, kvh, dim), device="cuda:0")
    v = torch.zeros((n, kvh, dim), device="cuda:0")
    out = torch.full((n, qheads, dim), 7.0, device="cuda:0")
    d = ctx.desc(q=q.data_ptr(), q_stride=qheads * dim, nq=n, k0=k.data_ptr(), v0=v.data_ptr(),
                 n0=n, qheads=qheads, kvheads=kvh, dim=dim, kh_first=0, kh_end=kvh, causal=1,
                 window=0, first_key=0, first_query=0, out=out.data_ptr(), o_stride=qheads * dim,
                 kernel=0)
    assert ctx.workspace_bytes(d) > NOALLOC_BYTES
    with pytest.raises(pcl.AttentionError) as e:
        ctx.launch_noalloc(d)
    assert e.value.kind == "ResourceLimit"
    assert ctx.sync() == 0
    assert bool(torch.all(out == 7.0))
    got, want, _ = both(torch, ctx, 16, 8, 256, 1, 2048, 0, 1, 0, 0x5EED0A07)
    assert np.array_equal(bits(got), bits(want))
