"""The attention output block (pcl_attention_output): projection, post-norm
and residual, src/engine/attention.rs:866-884.

CPU tests pin the oracle's p9_ref_matvec and p9_ref_add restatements with the
reference's known answers (src/kernels/reference/tests.rs:14-19, 67-73) and
with the f64-accumulation property the reference tests for its projections
(tests.rs:21-47: 2^24 + 1 - 2^24 keeps the 1). GPU tests compare both
projection kernels (few tokens: row streaming; many tokens: f64 MFMA tiles)
and the fused post-norm with the oracle.
"""
import numpy as np
import pytest

from helpers import normals


# ---- oracle pinning (CPU) --------------------------------------------------

def test_matrix_orientation_is_output_rows_by_input_columns(oracle):
    # src/kernels/reference/tests.rs:14-19
    y = oracle.matvec([1.0, 2.0, 3.0, -1.0, 0.0, 2.0], [1.0, 2.0, 4.0], 2, 3)
    assert y.tolist() == [17.0, 7.0]


def test_projection_accumulates_in_f64(oracle):
    # the property of tests.rs:21-47: an f32 sum would lose the 1
    y = oracle.matvec([16777216.0, 1.0, -16777216.0], [1.0, 1.0, 1.0], 1, 3)
    assert y.tolist() == [1.0]


def test_add_and_block_composition(oracle):
    # tests.rs:67-73, then the block: residual + rms_norm(W x) (attention.rs:
    # 866-884) against an independent f64 restatement
    assert oracle.add([2.0], [3.0]).tolist() == [5.0]
    rows, cols = 48, 64
    w = normals(1, rows * cols) * np.float32(0.1)
    x = normals(2, cols)
    scale = normals(3, rows)
    res = normals(4, rows)
    proj, out = oracle.attention_output(x, w, scale, 1e-6, res, rows, cols)
    want_p = (w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(proj, want_p)
    p64 = proj.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(p64 * p64) + 1e-6)
    want = (res + (p64 * inv).astype(np.float32) * scale).astype(np.float32)
    assert np.max(np.abs(out - want)) <= 1e-6


# ---- the device output block (GPU) -----------------------------------------

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


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to("cuda:0")


def run_block(torch, ctx, x, w, scale, res, eps=1e-6, in_place=False):
    n, cols = x.shape
    rows = w.shape[0]
    tx, tw, ts, tr = dev(torch, x), dev(torch, w), dev(torch, scale), dev(torch, res)
    proj = torch.full((n, rows), float("nan"), device="cuda:0")
    out = tr if in_place else torch.full((n, rows), float("nan"), device="cuda:0")
    ctx.attention_output(tx.data_ptr(), n, cols, tw.data_ptr(), rows, ts.data_ptr(), eps,
                         tr.data_ptr(), proj.data_ptr(), out.data_ptr())
    err = ctx.sync()
    return proj.cpu().numpy(), out.cpu().numpy(), err


# n = 1, 5, 16, 32: row streaming; 33, 200, 300: f64 MFMA tiles. One token
# with input rows of at most 16384 columns (a multiple of 4) is projected
# with the input row staged in LDS: rows of 1000 (fewer than 4096 columns),
# 5000 (4096 and a partial step), 4000 (one 4096-column step taken by some
# lanes only) and 4096 columns, the last token of 17; 16388 and 1001
# columns take the plain one-token kernel.
BLOCK_CASES = [(1, 4096, 2816), (5, 4096, 2816), (16, 8192, 2816), (32, 4096, 1536),
               (33, 4096, 2816), (200, 4096, 300), (300, 1000, 130), (7, 1001, 77),
               (1, 1000, 77), (1, 5000, 300), (1, 4000, 300), (17, 4096, 300),
               (1, 16388, 64), (1, 1001, 77)]


@pytest.mark.gpu
@pytest.mark.parametrize("case", BLOCK_CASES, ids=lambda c: "x".join(map(str, c)))
def test_output_block_matches_the_oracle(torch, ctx, oracle, case):
    n, cols, rows = case
    g = np.random.default_rng(sum(case))
    x = g.standard_normal((n, cols)).astype(np.float32)
    w = (g.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    scale = (1 + 0.1 * g.standard_normal(rows)).astype(np.float32)
    res = g.standard_normal((n, rows)).astype(np.float32)
    proj, out, err = run_block(torch, ctx, x, w, scale, res)
    assert err == 0
    same = 0
    for t in range(n):
        want_p, want = oracle.attention_output(x[t], w, scale, 1e-6, res[t], rows, cols)
        # f64 sums in another order: equal unless an f32 rounding boundary
        # falls between the two f64 sums (relative 1e-15 apart)
        assert np.max(np.abs(proj[t] - want_p) / (1e-30 + np.abs(want_p))) <= 2 ** -23
        assert np.max(np.abs(out[t] - want)) <= 1e-5
        same += int(np.sum(proj[t].view(np.uint32) == want_p.view(np.uint32)))
    assert same >= 0.999 * n * rows


@pytest.mark.gpu
@pytest.mark.parametrize("cols", [1000, 3848, 4000, 4092, 4096, 5000, 16384])
def test_one_token_projection_equals_the_multi_token_one_bitwise(torch, ctx, cols):
    # the one-token kernel (input row staged in LDS) sums each row's f64
    # products in the order of the multi-token row kernel
    rows = 300
    g = np.random.default_rng(cols)
    x = g.standard_normal((2, cols)).astype(np.float32)
    w = (g.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    scale = (1 + 0.1 * g.standard_normal(rows)).astype(np.float32)
    res = g.standard_normal((2, rows)).astype(np.float32)
    proj2, out2, err2 = run_block(torch, ctx, x, w, scale, res)
    proj1, out1, err1 = run_block(torch, ctx, x[1:], w, scale, res[1:])
    assert err1 == 0 and err2 == 0
    assert np.array_equal(proj1[0].view(np.uint32), proj2[1].view(np.uint32))
    assert np.array_equal(out1[0].view(np.uint32), out2[1].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 40])
def test_output_block_keeps_f64_cancellation_and_runs_in_place(torch, ctx, oracle, n):
    cols, rows = 96, 40
    x = np.ones((n, cols), np.float32)
    w = np.zeros((rows, cols), np.float32)
    w[:, 0], w[:, 1], w[:, 2] = 16777216.0, 1.0, -16777216.0
    w[:, 3:] = np.float32(1e-3)
    scale = np.ones(rows, np.float32)
    res = normals(5, n * rows).reshape(n, rows)
    proj, out, err = run_block(torch, ctx, x, w, scale, res.copy(), in_place=True)
    assert err == 0
    want_p, want = oracle.attention_output(x[0], w, scale, 1e-6, res[0], rows, cols)
    # the 1 survives (1 + 93e-3, where an f32 sum gives 93e-3); the small
    # terms the MFMA path adds while its partial sum is at 2^24 may move the
    # f32 result by an ulp
    assert np.all(np.abs(proj - 1.093) < 1e-3)
    assert np.max(np.abs(proj - want_p[None, :])) <= 2 ** -23 * 1.1
    assert np.max(np.abs(out - want[None, :] + res[0][None, :] - res)) <= 1e-6


@pytest.mark.gpu
def test_output_block_rejects_bad_arguments_and_flags_non_finite(pcl, torch, ctx):
    x = torch.ones((2, 64), device="cuda:0")
    w = torch.ones((8, 64), device="cuda:0")
    s = torch.ones(8, device="cuda:0")
    r = torch.ones((2, 8), device="cuda:0")
    out = torch.empty((2, 8), device="cuda:0")
    with pytest.raises(pcl.AttentionError) as e:
        ctx.attention_output(x.data_ptr(), 0, 64, w.data_ptr(), 8, s.data_ptr(), 1e-6,
                             r.data_ptr(), out.data_ptr(), out.data_ptr())
    assert e.value.kind == "InvalidShape"
    with pytest.raises(pcl.AttentionError) as e:
        ctx.attention_output(x.data_ptr(), 2, 64, w.data_ptr(), 8, s.data_ptr(), 0.0,
                             r.data_ptr(), out.data_ptr(), out.data_ptr())
    assert e.value.kind == "InvalidParameter"
    x[1, 3] = float("inf")
    proj = torch.empty((2, 8), device="cuda:0")
    ctx.attention_output(x.data_ptr(), 2, 64, w.data_ptr(), 8, s.data_ptr(), 1e-6,
                         r.data_ptr(), proj.data_ptr(), out.data_ptr())
    assert ctx.sync() == 8
