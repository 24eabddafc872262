"""Device-resident launches captured into a HIP graph (GPU).

A caller that replays a decode step as a graph (torch.cuda.CUDAGraph on the
context's stream) gets, on every replay, the bits the same launch gives
eagerly, with new inputs copied into the captured buffers between replays.
While a stream is capturing, AUTO never picks the spread decode (its
workgroups accept a published word by the launch's epoch, a kernel argument
every replay would repeat): it takes the pipelined kernel, whose bits are the
same, and an explicit spread request is refused. Both the allocating entry
(workspace reserved before the capture) and the allocation-free entry are
captured. Replays are checked against eager launches of the same inputs, with
eager work and synchronisations between the replays.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


class Step:
    """Device buffers of one decode (Q, K, V, out) and its descriptor."""

    def __init__(self, torch, ctx, qheads, kvh, dim, nkeys, kernel=0):
        dev = torch.device("cuda:0")
        self.q = torch.empty((1, qheads * dim), device=dev)
        self.k = torch.empty((nkeys, kvh, dim), device=dev)
        self.v = torch.empty((nkeys, kvh, dim), device=dev)
        self.out = torch.full((1, qheads * dim), float("nan"), device=dev)
        self.desc = ctx.desc(q=self.q.data_ptr(), q_stride=qheads * dim, nq=1, qheads=qheads,
                             kvheads=kvh, dim=dim, kh_first=0, kh_end=kvh, causal=1,
                             first_query=nkeys - 1, k0=self.k.data_ptr(), v0=self.v.data_ptr(),
                             n0=nkeys, out=self.out.data_ptr(), o_stride=qheads * dim,
                             kernel=kernel, q_scale=float(np.float32(1.0 / np.sqrt(dim))))

    def fill(self, torch, seed):
        g = torch.Generator(device="cuda:0")
        g.manual_seed(seed)
        for t in (self.q, self.k, self.v):
            t.copy_(torch.randn(t.shape, generator=g, device="cuda:0"))


def eager(torch, pcl, step, kernel=0):
    """The same inputs through an eager launch on torch's current stream."""
    ctx = pcl.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        out = torch.full_like(step.out, float("nan"))
        d = ctx.desc(**{f: getattr(step.desc, f) for f, _ in step.desc._fields_})
        d.out = out.data_ptr()
        d.kernel = kernel
        ctx.launch(d)
        assert ctx.sync() == 0
        return out.cpu().numpy()
    finally:
        ctx.close()


# a 2K decode (AUTO picks the spread decode eagerly) and a 32K one (the
# pipelined decode and its combine)
GRAPH_CASES = [(16, 8, 256, 2048), (16, 8, 256, 32768)]


@pytest.mark.parametrize("noalloc", [False, True], ids=["launch", "noalloc"])
@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: "x".join(map(str, c)))
def test_graph_replays_give_the_eager_bits(pcl, torch, case, noalloc):
    qheads, kvh, dim, nkeys = case
    stream = torch.cuda.Stream()
    ctx = pcl.Context(0, stream.cuda_stream)
    try:
        step = Step(torch, ctx, qheads, kvh, dim, nkeys)
        step.fill(torch, 0x6A0)
        launch = ctx.launch_noalloc if noalloc else ctx.launch
        torch.cuda.synchronize()
        if not noalloc:
            ctx.reserve(ctx.workspace_bytes(step.desc))
        with torch.cuda.stream(stream):
            launch(step.desc)  # eager on the capture stream first
        stream.synchronize()
        assert ctx.sync() == 0
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            launch(step.desc)
        for rep in range(4):
            step.fill(torch, 0x6A1 + rep)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = step.out.cpu().numpy()
            assert ctx.sync() == 0
            want = eager(torch, pcl, step)
            assert np.array_equal(bits(got), bits(want)), rep
        graph.reset()
    finally:
        ctx.close()


def test_capture_refuses_an_explicit_spread_request(pcl, torch):
    stream = torch.cuda.Stream()
    ctx = pcl.Context(0, stream.cuda_stream)
    try:
        step = Step(torch, ctx, 16, 8, 256, 2048, kernel=pcl.KERNEL_SPREAD_KV)
        step.fill(torch, 0x6B0)
        ctx.reserve(ctx.workspace_bytes(step.desc))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(pcl.AttentionError) as e:
            with torch.cuda.graph(graph, stream=stream):
                step.out.mul_(1.0)  # the capture holds one node either way
                ctx.launch(step.desc)
        assert e.value.kind == "InvalidParameter"
        torch.cuda.synchronize()
        # outside a capture the same request runs, with the pipelined bits
        with torch.cuda.stream(stream):
            ctx.launch(step.desc)
        stream.synchronize()
        assert ctx.sync() == 0
        got = step.out.cpu().numpy()
        want = eager(torch, pcl, step, kernel=pcl.KERNEL_PIPE_KV)
        assert np.array_equal(bits(got), bits(want))
    finally:
        ctx.close()
