"""The head-transform prologue (pcl_head_transform_*) against the engine's
HeadTransform (src/engine/attention.rs:51-243).

CPU tests pin the oracle's restatement of p9_ref_rms_norm and p9_ref_rope
(src/kernels/portable/reference.rs:11-33, 277-318) with the reference's own
known answers (src/kernels/reference/tests.rs:4-11, 79-113), its libm digests
for powf and sincosf (src/libm/tests.rs:20-92, 136), closed forms (the RMS of a
normalised row, the rotation's invariant pair norms, f64 angles) and the
prepare() structure (V unscaled and not rotated, K as V for global layers).
GPU tests compare the device transform with the oracle, alone, fused into
the cache append, and end to end through attention: V rows bit for bit, the
rotated Q and K rows within the bound the rotation table's one-ulp agreement
with the reference's sincosf allows.
"""
import math
import os
import subprocess

import numpy as np
import pytest

from helpers import normals

POWF_DIGEST = 0xE03CB0D507CDCB95  # src/libm/tests.rs:77
SINCOSF_DIGEST = 0x684C340564E05BFC  # src/libm/tests.rs:71
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---- oracle pinning (CPU) --------------------------------------------------

def test_powf_matches_the_reference_libm_digest(oracle):
    # the rotary frequencies' powf gives the reference's bits on all 2^22
    # digest inputs (src/libm/tests.rs:53-62, 134-137)
    assert oracle.libm_digest(0) == POWF_DIGEST


def test_sincosf_matches_the_reference_libm_digest(oracle):
    # the rotation's (sin, cos) give the reference's bits on every 61st
    # binary32 pattern (src/libm/tests.rs:20-22, 86-92): glibc 2.28's sincosf, which
    # the reference's libm ports (the newer C library here differs)
    assert oracle.libm_digest(1) == SINCOSF_DIGEST


ROTATION_COMPARE_MAIN = r"""
#include "rotation.hpp"
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
extern "C" void oracle_sincosf(float x, float *s, float *c);
// position of a float on the number line in ulps (+0 and -0 both 0)
static int64_t ulps(float f) {
    int32_t i; std::memcpy(&i, &f, 4);
    return i < 0 ? -(int64_t)(i & 0x7fffffff) : (int64_t)i;
}
int main() {
    unsigned long long n = 0, differ = 0;
    long long worst = 0;
    for (uint64_t k = 0; k <= 0xffffffffULL / 61; ++k) {
        const uint32_t u = (uint32_t)(k * 61);
        float x; std::memcpy(&x, &u, 4);
        if (!std::isfinite(x)) continue;
        float s, c, rs, rc;
        pcl::rotation_sincos(x, &s, &c);
        oracle_sincosf(x, &rs, &rc);
        const long long ds = llabs(ulps(s) - ulps(rs)), dc = llabs(ulps(c) - ulps(rc));
        ++n;
        differ += (ds || dc);
        if (ds > worst) worst = ds;
        if (dc > worst) worst = dc;
    }
    std::printf("%llu %llu %lld\n", n, differ, worst);
}
"""


def test_product_rotation_table_is_within_an_ulp_of_the_reference_sincosf(tmp_path, oracle):
    # the product's table entries (rotation.hpp, compiled on its own with the
    # library's no-contraction flag) against the oracle's glibc 2.28 sincosf,
    # which reproduces the reference's SINCOSF digest (test above), on the
    # digest's inputs: every 61st binary32 pattern, the finite ones
    src = tmp_path / "rotation.cpp"
    src.write_text(ROTATION_COMPARE_MAIN)
    exe = tmp_path / "rotation"
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "power-cpu-llm_amd", "csrc"), str(src),
                    "-L", odir, "-loracle_attention", "-Wl,-rpath," + odir, "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    n, differ, worst = (int(x) for x in out.split())
    assert n > 69_000_000
    assert worst <= 1, worst
    assert differ / n < 0.005, differ / n


def test_direct_rms_scale_and_unscaled_normalization(oracle):
    # src/kernels/reference/tests.rs:4-11
    y = oracle.rms_norm([3.0, 4.0], None, 0.5)
    assert abs(float(y[0]) - 3.0 / float(np.sqrt(np.float32(13.0)))) < 1e-6
    scaled = oracle.rms_norm([3.0, 4.0], [2.0, 0.0], 0.5)
    assert scaled[0] == np.float32(2.0) * y[0]
    assert scaled[1] == 0.0  # the scale is direct, not (1 + scale)
    assert oracle.rms_norm([0.0, 0.0], None, 1e-6).tolist() == [0.0, 0.0]


@pytest.mark.parametrize("dim", [64, 256, 512])
def test_rms_norm_closed_form(oracle, dim):
    # mean(y^2) = ms / (ms + eps) for y = x / sqrt(ms + eps)
    for seed in range(4):
        x = normals(seed, dim) * np.float32(3.0 ** seed)
        eps = 1e-6
        y = oracle.rms_norm(x, None, eps).astype(np.float64)
        ms = float(np.mean(x.astype(np.float64) ** 2))
        assert abs(float(np.mean(y * y)) - ms / (ms + eps)) < 1e-6
        s = normals(100 + seed, dim)
        ys = oracle.rms_norm(x, s, eps)
        assert np.array_equal(ys, (oracle.rms_norm(x, None, eps) * s).astype(np.float32))


def test_rope_pairs_split_halves_and_uses_frequency_divisors(oracle):
    # src/kernels/reference/tests.rs:79-95
    x = np.array([1.0, 2.0, 3.0, 4.0, -1.0, -2.0, -3.0, -4.0], np.float32)
    ok, y = oracle.rope(x, 4, 0, 10000.0)
    assert ok and np.array_equal(y, x)
    ok, out = oracle.rope(x, 4, 3, 10000.0, [2.0, 1e30])
    assert ok
    s, c = math.sin(1.5), math.cos(1.5)
    for raw, o in zip(x.reshape(2, 4), out.reshape(2, 4)):
        assert abs(float(o[0]) - (float(raw[0]) * c - float(raw[2]) * s)) < 1e-6
        assert abs(float(o[2]) - (float(raw[2]) * c + float(raw[0]) * s)) < 1e-6
        assert o[1] == raw[1] and o[3] == raw[3]


def test_proportional_rope_at_large_position(oracle):
    # src/kernels/reference/tests.rs:97-113: pairs (i, i+256), zero
    # frequencies after pair 63, position 262143, base 1e6
    x = np.array([(i % 13) - 6.0 for i in range(512)], np.float32)
    factors = np.array([1.0 if i < 64 else 1e30 for i in range(256)], np.float32)
    ok, y = oracle.rope(x, 512, 262143, 1e6, factors)
    assert ok
    for i in range(256):
        if i < 64:
            inv = np.float32(1.0) / np.float32(math.pow(1e6, float(np.float32(2 * i) /
                                                                   np.float32(512))))
            angle = float(np.float32(262143.0) * inv)
        else:
            angle = 0.0
        s, c = math.sin(angle), math.cos(angle)
        assert abs(float(y[i]) - (x[i] * c - x[i + 256] * s)) < 2e-6
        assert abs(float(y[i + 256]) - (x[i + 256] * c + x[i] * s)) < 2e-6


def test_rope_is_a_rotation_by_the_f32_angles(oracle):
    dim, heads = 128, 3
    x = normals(7, heads * dim)
    for position in (1, 17, 4095, 131071):
        ok, y = oracle.rope(x, dim, position, 10000.0)
        assert ok
        xr, yr = x.reshape(heads, dim).astype(np.float64), y.reshape(heads, dim).astype(np.float64)
        half = dim // 2
        # pair norms are kept
        assert np.allclose(xr[:, :half] ** 2 + xr[:, half:] ** 2,
                           yr[:, :half] ** 2 + yr[:, half:] ** 2, rtol=1e-5, atol=1e-6)
        # the angle of each pair, in f64 from the f32 frequencies
        # powf as the correctly rounded f64 power rounded to f32
        inv = np.array([np.float32(1.0) / np.float32(math.pow(10000.0, float(
            np.float32(2 * i) / np.float32(dim)))) for i in range(half)], np.float32)
        ang = (np.float32(position) * inv).astype(np.float64)
        want_a = xr[:, :half] * np.cos(ang) - xr[:, half:] * np.sin(ang)
        assert float(np.max(np.abs(yr[:, :half] - want_a))) < 1e-5


def test_rope_rejects_a_non_finite_angle(oracle):
    ok, _ = oracle.rope(np.ones(4, np.float32), 4, 10, 10000.0, [1e-45, 1.0])
    assert not ok


def test_prepare_keeps_v_unscaled_and_unrotated(oracle):
    # attention.rs:121-155: K as V for a global layer, V normalised without
    # the learned scale and not rotated; at position 0 Q and K are only
    # normalised and scaled
    qh, kvh, dim = 4, 2, 64
    rq, rk = normals(1, qh * dim), normals(2, kvh * dim)
    qs, ks = normals(3, dim), normals(4, dim)
    ok, q, k, v = oracle.head_transform(rq, rk, None, qh, kvh, dim, 0, qs, ks, 1e-6, 10000.0)
    assert ok
    assert np.array_equal(v, np.concatenate([oracle.rms_norm(h, None, 1e-6)
                                             for h in rk.reshape(kvh, dim)]))
    assert np.array_equal(q, np.concatenate([oracle.rms_norm(h, qs, 1e-6)
                                             for h in rq.reshape(qh, dim)]))
    ok, q5, k5, v5 = oracle.head_transform(rq, rk, None, qh, kvh, dim, 5, qs, ks, 1e-6, 10000.0)
    assert np.array_equal(v5, v) and not np.array_equal(q5, q)


# ---- the device transform (GPU) --------------------------------------------

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


def oracle_tokens(oracle, rq, rk, rv, n, qh, kvh, dim, position, qs, ks, eps, base, factors):
    qs_out, ks_out, vs_out = [], [], []
    for i in range(n):
        ok, q, k, v = oracle.head_transform(rq[i], rk[i], None if rv is None else rv[i], qh, kvh,
                                            dim, position + i, qs, ks, eps, base, factors)
        assert ok
        qs_out.append(q)
        ks_out.append(k)
        vs_out.append(v)
    return np.stack(qs_out), np.stack(ks_out), np.stack(vs_out)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def assert_rotated_close(got, want, dim):
    """Rotated Q or K rows against the oracle's. The product's rotation table
    is within an f32 ulp of the reference's sincosf (CPU test above), so each
    value of pair (j, j + dim/2) is within 2^-20 (|w_j| + |w_{j+dim/2}|) of
    the oracle's w: one ulp of a table entry moves a product by at most
    2^-24 of the other factor, and the two products and their difference
    round at most once more each. A wrong sign, a swapped sine and cosine or
    a wrong angle moves values by the pair's own size."""
    g = np.asarray(got, np.float32).reshape(-1, dim).astype(np.float64)
    w = np.asarray(want, np.float32).reshape(-1, dim).astype(np.float64)
    half = dim // 2
    pair = np.abs(w[:, :half]) + np.abs(w[:, half:])
    bound = np.concatenate([pair, pair], axis=1) * 2.0 ** -20
    assert np.all(np.abs(g - w) <= bound), float(np.max(np.abs(g - w) - bound))


TRANSFORM_CASES = [
    # qheads, kvh, dim, n, position, K-as-V, proportional factors
    (16, 8, 256, 1, 32767, False, False),
    (16, 8, 256, 37, 0, False, False),
    (16, 2, 512, 3, 131069, True, True),
    (8, 2, 128, 70, 1000, False, False),
    (4, 4, 64, 5, 262143, True, False),
    (6, 3, 16, 9, 7, False, True),
    # enough tokens for the packed workgroups (16 heads at 256, 8 at 512, a
    # token's 8 heads of three kinds in one pass at 32)
    (16, 8, 256, 160, 5000, False, False),
    (16, 2, 512, 100, 77, True, False),
    (4, 2, 32, 300, 3, False, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", TRANSFORM_CASES, ids=lambda c: "x".join(map(str, c)))
def test_device_transform_matches_the_oracle(pcl, torch, ctx, oracle, case):
    qh, kvh, dim, n, position, k_as_v, proportional = case
    g = np.random.default_rng(sum(case[:5]))
    rq = (g.standard_normal((n, qh * dim)) * 3).astype(np.float32)
    rk = (g.standard_normal((n, kvh * dim)) * 0.2).astype(np.float32)
    rv = None if k_as_v else g.standard_normal((n, kvh * dim)).astype(np.float32)
    qs = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    ks = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    factors = (np.array([1.0 if i < dim // 8 else 1e30 for i in range(dim // 2)], np.float32)
               if proportional else None)
    eps, base = 1e-6, (1e6 if proportional else 10000.0)
    t = pcl.HeadTransform(ctx, qh, kvh, dim, qs, ks, eps, base, factors)
    tq, tk = dev(torch, rq), dev(torch, rk)
    tv = dev(torch, rv) if rv is not None else None
    oq = torch.full((n, qh * dim), float("nan"), device="cuda:0")
    ok_ = torch.full((n, kvh * dim), float("nan"), device="cuda:0")
    ov = torch.full((n, kvh * dim), float("nan"), device="cuda:0")
    t.prepare(tq.data_ptr(), tk.data_ptr(), tv.data_ptr() if tv is not None else 0, n, position,
              oq.data_ptr(), ok_.data_ptr(), ov.data_ptr())
    assert ctx.sync() == 0
    wq, wk, wv = oracle_tokens(oracle, rq, rk, rv, n, qh, kvh, dim, position, qs, ks, eps, base,
                               factors)
    assert_rotated_close(oq.cpu().numpy(), wq, dim)
    assert_rotated_close(ok_.cpu().numpy(), wk, dim)
    assert np.array_equal(bits(ov.cpu().numpy()), bits(wv))
    # the query half alone (prepare_query) gives the same queries, bitwise
    oq2 = torch.full((n, qh * dim), float("nan"), device="cuda:0")
    t.query(tq.data_ptr(), n, position, oq2.data_ptr())
    assert ctx.sync() == 0
    assert np.array_equal(bits(oq2.cpu().numpy()), bits(oq.cpu().numpy()))
    t.close()


@pytest.mark.gpu
def test_transform_rejects_bad_geometry_parameters_and_inputs(pcl, torch, ctx):
    ones = np.ones(64, np.float32)
    with pytest.raises(pcl.AttentionError) as e:
        pcl.HeadTransform(ctx, 4, 3, 64, ones, ones, 1e-6, 1e4)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(pcl.AttentionError) as e:
        pcl.HeadTransform(ctx, 4, 2, 64, ones, ones, 0.0, 1e4)
    assert e.value.kind == "InvalidParameter"
    with pytest.raises(pcl.AttentionError) as e:
        pcl.HeadTransform(ctx, 4, 2, 64, ones, ones, 1e-6, 1e4, factors=-ones[:32])
    assert e.value.kind == "InvalidParameter"
    bad = ones.copy()
    bad[3] = np.inf
    with pytest.raises(pcl.AttentionError) as e:
        pcl.HeadTransform(ctx, 4, 2, 64, bad, ones, 1e-6, 1e4)
    assert e.value.kind == "InvalidParameter"
    # a sliding layer needs V
    t = pcl.HeadTransform(ctx, 4, 2, 64, ones, ones, 1e-6, 1e4, sliding=True)
    x = torch.ones((1, 4 * 64), device="cuda:0")
    out = torch.empty((1, 4 * 64), device="cuda:0")
    with pytest.raises(pcl.AttentionError) as e:
        t.prepare(x.data_ptr(), x.data_ptr(), 0, 1, 0, out.data_ptr(), out.data_ptr(),
                  out.data_ptr())
    assert e.value.kind == "InvalidShape"
    # a non-finite raw value sets the transform's device error bit
    xq = torch.ones((1, 4 * 64), device="cuda:0")
    xq[0, 5] = float("nan")
    t.query(xq.data_ptr(), 1, 0, out.data_ptr())
    assert ctx.sync() == 4
    assert ctx.sync() == 0
    t.close()


@pytest.mark.gpu
@pytest.mark.parametrize("window,k_as_v", [(None, False), (5, False), (None, True)])
def test_fused_append_writes_prepared_rows_into_the_cache(pcl, torch, ctx, oracle, window,
                                                          k_as_v):
    # encode_in_place with project_tokens (attention.rs:949-987): each step's
    # prepared K/V land in the cache at positions total.., the queries attend
    # through the cache's encoder descriptor; within 1e-4 of the exact oracle
    qh, kvh, dim = 16, 8, 256
    width = kvh * dim
    g = np.random.default_rng(11 + (window or 0) + k_as_v)
    qs = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    ks = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    t = pcl.HeadTransform(ctx, qh, kvh, dim, qs, ks, 1e-6, 10000.0)
    cache = pcl.LayerCache(ctx, kvh, dim, 10_000, window, 1 << 30)
    ref = oracle.OracleCache(kvh, dim, 10_000, window, 1 << 30)
    # 160 tokens take the packed workgroups (16 heads each) writing into the
    # cache's rows; 40 take four heads a workgroup, one token one head
    for step, n in enumerate((40, 1, 160, 1, 9)):
        rq = g.standard_normal((n, qh * dim)).astype(np.float32)
        rk = g.standard_normal((n, width)).astype(np.float32)
        rv = None if k_as_v else g.standard_normal((n, width)).astype(np.float32)
        position = cache.total_tokens()
        wq, wk, wv = oracle_tokens(oracle, rq, rk, rv, n, qh, kvh, dim, position, qs, ks, 1e-6,
                                   10000.0, None)
        tq, tk = dev(torch, rq), dev(torch, rk)
        tv = dev(torch, rv) if rv is not None else None
        q_out = torch.full((n, qh * dim), float("nan"), device="cuda:0")
        pending = cache.append_transformed(t, tq.data_ptr(), tk.data_ptr(),
                                           tv.data_ptr() if tv is not None else 0, n,
                                           q_out.data_ptr())
        rc, _ = ref.append(wk, wv, n)
        assert rc == 0
        assert_rotated_close(q_out.cpu().numpy(), wq, dim)
        rows = cache.retained_tokens()
        keys, values = (x.reshape(rows, width) for x in cache.read(0, rows))
        want_k, want_v = ref.rows()
        assert_rotated_close(keys, want_k, dim)
        assert np.array_equal(bits(values), bits(want_v))
        out = torch.full((n, qh * dim), float("nan"), device="cuda:0")
        d = cache.encoder_desc(pending, q=q_out.data_ptr(), q_stride=qh * dim, nq=n, qheads=qh,
                               kh_first=0, kh_end=kvh, out=out.data_ptr(), o_stride=qh * dim)
        ctx.launch(d)
        assert ctx.sync() == 0
        first_key = ref.first_position()
        ok, want = oracle.threaded(wq, n, want_k, want_v, qh, kvh, dim, rows, True, first_key,
                                   position, window or 0, threads=8)
        assert ok
        assert float(np.max(np.abs(out.cpu().numpy().reshape(-1) - want))) <= 1e-4
        cache.commit()
        ref.commit()
    cache.close()
    t.close()


STEP_CASES = [
    # qheads, kvh, dim, keys with the new token, window, K-as-V
    (16, 8, 256, 16500, None, False),  # narrow pipelined layout (>= 512 items), chunk partials
    (16, 8, 256, 3000, 1024, False),   # wide layout at head dim 256, sliding window
    (16, 2, 512, 5000, None, True),    # two score waves, K as V
    (8, 4, 64, 700, None, False),      # head dim 64 (narrow)
    (8, 2, 128, 1500, None, False),    # head dim 128 (wide)
    (16, 8, 256, 2049, None, False),   # the new key alone in its chunk
    (16, 8, 256, 200, None, False),    # one chunk: direct output
    # the new key among the first keys of its chunk, which the chunk's
    # first requests would read: those wait for its row
    (16, 8, 256, 16425, None, False),  # narrow layout, key 40 of its chunk
    (16, 2, 512, 4865, None, True),    # two score waves, key 0 of its chunk
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", STEP_CASES, ids=lambda c: "x".join(map(str, c)))
def test_attend_token_folds_the_transform_into_the_decode(pcl, torch, ctx, oracle, case):
    # one decode token of encode_in_place (attention.rs:949-1080): prepare
    # (102-156), the cache append, the attention pass. Through the pipelined
    # decode the transform runs inside the attention launch; its prepared
    # queries, new K/V row and output equal the two-launch path bit for
    # bit, whatever kernel AUTO picks, and the exact oracle within 1e-4
    qh, kvh, dim, nkeys, window, k_as_v = case
    width = kvh * dim
    g = np.random.default_rng(nkeys + dim)
    qs = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    ks = (1 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    t = pcl.HeadTransform(ctx, qh, kvh, dim, qs, ks, 1e-6, 10000.0, sliding=not k_as_v)
    cache = pcl.LayerCache(ctx, kvh, dim, nkeys + 8, window, 1 << 40)
    cache.reserve_rows(nkeys + 1)
    k0 = dev(torch, g.standard_normal((nkeys - 1, width), dtype=np.float32))
    v0 = dev(torch, g.standard_normal((nkeys - 1, width), dtype=np.float32))
    cache.append(k0.data_ptr(), v0.data_ptr(), nkeys - 1)
    cache.commit()
    position = cache.total_tokens()
    rq = (g.standard_normal(qh * dim) * 3).astype(np.float32)
    rk = g.standard_normal(width).astype(np.float32)
    rv = None if k_as_v else g.standard_normal(width).astype(np.float32)
    tq, tk = dev(torch, rq), dev(torch, rk)
    tv = dev(torch, rv) if rv is not None else None
    scale = np.float32(1.0 / np.sqrt(np.float64(dim)))

    def run(mode, kernel):
        q_out = torch.full((qh * dim,), float("nan"), device="cuda:0")
        out = torch.full((qh * dim,), float("nan"), device="cuda:0")
        if mode == "fused":
            pending = cache.attend_token(t, tq.data_ptr(), tk.data_ptr(),
                                         tv.data_ptr() if tv is not None else 0,
                                         q_out.data_ptr(), out.data_ptr(), q_scale=float(scale),
                                         kernel=kernel)
        else:
            pending = cache.append_transformed(t, tq.data_ptr(), tk.data_ptr(),
                                               tv.data_ptr() if tv is not None else 0, 1,
                                               q_out.data_ptr())
            d = cache.encoder_desc(pending, q=q_out.data_ptr(), q_stride=qh * dim, nq=1,
                                   qheads=qh, kh_first=0, kh_end=kvh, out=out.data_ptr(),
                                   o_stride=qh * dim, q_scale=float(scale), kernel=kernel)
            ctx.launch(d)
        assert ctx.sync() == 0, (mode, kernel)
        rows = cache.retained_tokens()
        assert cache.total_tokens() == position + 1
        new_k, new_v = cache.read(rows - 1, 1)
        got = [q_out.cpu().numpy(), out.cpu().numpy(), new_k, new_v]
        if mode == "fused" and kernel == pcl.KERNEL_PIPE_KV:
            got.append(cache.read(0, rows))
        cache.rollback(pending)
        return got, rows

    fused, rows = run("fused", pcl.KERNEL_PIPE_KV)
    for mode, kernel in (("separate", pcl.KERNEL_PIPE_KV), ("fused", pcl.KERNEL_AUTO)):
        other, _ = run(mode, kernel)
        for a, b in zip(fused[:4], other):
            assert np.array_equal(bits(a), bits(b)), (mode, kernel)
    q_out, out, new_k, new_v, (keys, values) = fused
    wq, wk, wv = oracle_tokens(oracle, rq[None], rk[None], None if rv is None else rv[None], 1,
                               qh, kvh, dim, position, qs, ks, 1e-6, 10000.0, None)
    assert_rotated_close(q_out, wq, dim)
    assert_rotated_close(new_k, wk, dim)
    assert np.array_equal(bits(new_v), bits(wv.reshape(-1)))
    # the attention over the cache's rows with the prepared new row, from
    # the device's prepared query pre-scaled in f32 as the kernels scale it
    qsc = (q_out * scale).astype(np.float32)
    ok, want = oracle.threaded(qsc, 1, keys, values, qh, kvh, dim, rows, True,
                               position + 1 - rows, position, window or 0, threads=8)
    assert ok
    assert float(np.max(np.abs(out - want))) <= 1e-4
    assert np.array_equal(out.reshape(qh, dim).argmax(1), want.reshape(qh, dim).argmax(1))
    # a non-finite raw value sets the transform's error bit through the fold
    bad_q = tq.clone()
    bad_q[7] = float("nan")
    q_out = torch.empty((qh * dim,), device="cuda:0")
    out = torch.empty((qh * dim,), device="cuda:0")
    pending = cache.attend_token(t, bad_q.data_ptr(), tk.data_ptr(),
                                 tv.data_ptr() if tv is not None else 0, q_out.data_ptr(),
                                 out.data_ptr(), q_scale=float(scale),
                                 kernel=pcl.KERNEL_PIPE_KV)
    assert ctx.sync() & 4
    assert ctx.sync() == 0
    cache.rollback(pending)
    cache.close()
    t.close()


@pytest.mark.gpu
def test_attend_token_rejects_bad_arguments_and_leaves_the_cache(pcl, torch, ctx):
    # the fused entry's errors are append_transformed's and the launch's; a
    # refused call launches nothing and leaves the cache's counts unchanged
    qh, kvh, dim = 8, 2, 128
    ones = np.ones(dim, np.float32)
    t = pcl.HeadTransform(ctx, qh, kvh, dim, ones, ones, 1e-6, 1e4, sliding=True)
    other = pcl.HeadTransform(ctx, qh, kvh, 64, ones[:64], ones[:64], 1e-6, 1e4)
    cache = pcl.LayerCache(ctx, kvh, dim, 100, None, 1 << 30)
    rq = torch.ones(qh * dim, device="cuda:0")
    rk = torch.ones(kvh * dim, device="cuda:0")
    q_out = torch.empty(qh * dim, device="cuda:0")
    out = torch.empty(qh * dim, device="cuda:0")
    cases = [
        (other, rk, rk, q_out, out, 0, "InvalidShape"),  # transform of another head dim
        (t, rk, None, q_out, out, 0, "InvalidShape"),    # a sliding layer needs V
        (t, rk, rk, None, out, 0, "InvalidShape"),       # no query output
        (t, rk, rk, q_out, None, 0, "InvalidShape"),     # no attention output
        (t, rk, rk, q_out, out, 5, "InvalidParameter"),  # the retired kernel choice
    ]
    for tr, k_, v_, qo, o, kernel, kind in cases:
        with pytest.raises(pcl.AttentionError) as e:
            cache.attend_token(tr, rq.data_ptr(), k_.data_ptr(), v_.data_ptr() if v_ is not None
                               else 0, qo.data_ptr() if qo is not None else 0,
                               o.data_ptr() if o is not None else 0, kernel=kernel)
        assert e.value.kind == kind
        assert cache.total_tokens() == 0 and cache.retained_tokens() == 0
    assert ctx.sync() == 0
    # a good call then counts its token
    pending = cache.attend_token(t, rq.data_ptr(), rk.data_ptr(), rk.data_ptr(),
                                 q_out.data_ptr(), out.data_ptr())
    assert ctx.sync() == 0
    assert cache.total_tokens() == 1 and cache.retained_tokens() == 1
    cache.rollback(pending)
    assert cache.total_tokens() == 0
    cache.close()
    other.close()
    t.close()
