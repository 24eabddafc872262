// Head normalisation and rotary transform of projected Q/K/V rows on gfx950:
// the engine's HeadTransform (src/engine/attention.rs:51-243), applied to n
// tokens at once on the device, with K and V optionally written straight
// into a layer cache's rows (no staging copy).
//
// Per head (p9_ref_rms_norm, src/kernels/portable/reference.rs:11-33; the
// arithmetic of step_prologue.hpp, which a decode kernel also runs when a
// one-token step's transform is folded into its launch):
//   sum = sequential f64 sum of f64(x_j)^2, j ascending;
//   inv = 1 / sqrt(sum / dim + f64(eps))            (f64, correctly rounded);
//   y_j = f32(f64(x_j) * inv), times scale_j in f32 for Q and K.
// Q and K then rotate pairs (j, j + dim/2) (p9_ref_rope, reference.rs:277-318):
//   y_j' = y_j*c - y_{j+h}*s,  y_{j+h}' = y_{j+h}*c + y_j*s   (f32, unfused),
// with (s, c) = sin, cos of the f32 angle position * f32(1 / powf(base,
// 2j/dim)) / factor_j from a host-built table (the C library's powf; the C
// library's double sin and cos of the angle rounded once to f32, within an
// f32 ulp of the engine's sincosf, rotation.hpp). V is normalised
// without scale and not rotated; a global layer without a V projection uses
// the raw K as V (attention.rs:121-129).
//
// One 64-lane workgroup takes up to kItems heads of one token: it loads the
// token's rotation factors and the scales once per lane, issues the loads of
// all its rows at once (16-byte, coalesced) and stages them in LDS, each lane
// sums one row in order, and the outputs are written back coalesced. Launches
// of a few tokens take 4 or 1 heads per workgroup instead, so that a decode
// step's heads run on many CUs at once.
#include "attention_device.hpp"
#include "context.hpp"
#include "pcl_attention.h"
#include "rotation.hpp"
#include "step_prologue.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

namespace pcl {

struct TransformParams {
    const float *rq, *rk, *rv; // raw rows [n][heads*dim]; rv null: V = raw K
    float *oq, *ok, *ov;       // outputs; ok null: query heads only
    int64_t o_kv_stride;       // floats between K/V output rows
    const float *qs, *ks;      // learned scales [dim]
    const float *tab;          // (sin, cos) pairs [position][dim/2][2]
    int64_t pos0;
    int n, qheads, kvh, dim, slots;
    float eps;
    int *err;
};

// Heads per workgroup: about 16 KiB of staged rows, so that several
// workgroups share a CU and one's loads overlap another's sums and stores.
template <int DK>
constexpr int transform_items()
{
    return 4096 / DK < 64 ? 4096 / DK : 64;
}

// Workgroup (token t, slot group y): heads y*ITEMS.. of token t.
template <int DK, int ITEMS>
__global__ __launch_bounds__(64) void head_transform_kernel(TransformParams p)
{
    constexpr int kItems = ITEMS;
    constexpr int kStride = DK + 4; // 16-byte aligned rows
    constexpr int kHalf = DK / 2;
    constexpr int kVec = DK / 4;                          // float4 per row
    constexpr int kLoads = (kItems * kVec + 63) / 64;     // float4 per lane
    __shared__ __attribute__((aligned(16))) float rows[kItems * kStride];
    __shared__ double inv[kItems];
    const int lane = threadIdx.x;
    const int64_t t = blockIdx.x;
    const int s0 = blockIdx.y * kItems;
    const int count = p.slots - s0 < kItems ? p.slots - s0 : kItems;

    // this lane's pairs j0..j0+3 of every row it writes: (sin, cos) of the
    // token's position and the learned scales of both halves
    constexpr int kRowLanes = kHalf / 4;
    constexpr int kPassRows = 64 / kRowLanes;
    const int j0 = 4 * (lane % kRowLanes);
    const float *tab = p.tab + (p.pos0 + t) * DK;
    const f4 sc0 = ldg4(tab + 2 * j0), sc1 = ldg4(tab + 2 * j0 + 4);
    const f4 qa4 = ldg4(p.qs + j0), qb4 = ldg4(p.qs + j0 + kHalf);
    const f4 ka4 = ldg4(p.ks + j0), kb4 = ldg4(p.ks + j0 + kHalf);

    // slot s of the token: Q heads, then K heads, then V heads
    auto source = [&](int s) -> const float * {
        if (s < p.qheads)
            return p.rq + (t * p.qheads + s) * DK;
        if (s < p.qheads + p.kvh)
            return p.rk + (t * p.kvh + (s - p.qheads)) * DK;
        const float *v = p.rv ? p.rv : p.rk;
        return v + (t * p.kvh + (s - p.qheads - p.kvh)) * DK;
    };

    // every row's loads in flight at once, then the LDS stores
    f4 staged[kLoads];
    bool bad = false;
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
        const int idx = lane + 64 * k;
        const int r = idx / kVec, c = idx % kVec;
        if (r < count)
            staged[k] = ldg4(source(s0 + r) + 4 * c);
    }
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
        const int idx = lane + 64 * k;
        const int r = idx / kVec, c = idx % kVec;
        if (r < count) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                bad |= !is_finite(staged[k][e]);
            *(f4 *)(rows + r * kStride + 4 * c) = staged[k];
        }
    }
    __syncthreads();
    if (lane < count)
        inv[lane] = norm_inverse<DK>(rows + lane * kStride, p.eps);
    __syncthreads();
    // the outputs: kHalf / 4 lanes per row, four consecutive pairs j0..j0+3
    // each (a 16-byte store into either half), 256 / kHalf rows per pass
    for (int r = lane / kRowLanes; r < count; r += kPassRows) {
        const int s = s0 + r;
        const int kind = s < p.qheads ? 0 : s < p.qheads + p.kvh ? 1 : 2;
        float *out = kind == 0   ? p.oq + (t * p.qheads + s) * DK
                     : kind == 1 ? p.ok + t * p.o_kv_stride + (int64_t)(s - p.qheads) * DK
                                 : p.ov + t * p.o_kv_stride + (int64_t)(s - p.qheads - p.kvh) * DK;
        const double iv = inv[r];
        const f4 xa = *(const f4 *)(rows + r * kStride + j0);
        const f4 xb = *(const f4 *)(rows + r * kStride + j0 + kHalf);
        const float sn[4] = {sc0[0], sc0[2], sc1[0], sc1[2]};
        const float cs[4] = {sc0[1], sc0[3], sc1[1], sc1[3]};
        f4 ya, yb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float a, b;
            if (kind == 2)
                transform_pair<false>(xa[e], xb[e], iv, 0.f, 0.f, 0.f, 0.f, &a, &b);
            else
                transform_pair<true>(xa[e], xb[e], iv, kind == 0 ? qa4[e] : ka4[e],
                                     kind == 0 ? qb4[e] : kb4[e], sn[e], cs[e], &a, &b);
            bad |= !is_finite(a) || !is_finite(b);
            ya[e] = a;
            yb[e] = b;
        }
        stg4(out + j0, ya);
        stg4(out + j0 + kHalf, yb);
    }
    if (bad)
        atomicOr(p.err, kErrTransform);
}

// Workgroups a launch should at least fill before its heads are packed
// kItems to a workgroup: a decode step (one or a few tokens) is a chain of
// one load round trip, one lane's sequential sum and the row stores per
// workgroup, so fewer heads per workgroup spread it over more CUs.
constexpr int64_t kTransformSpreadGroups = 256;

template <int DK> static hipError_t launch_dk(const TransformParams &p, hipStream_t stream)
{
    auto go = [&](auto kernel, int per) {
        const dim3 grid((unsigned)p.n, (unsigned)((p.slots + per - 1) / per));
        hipLaunchKernelGGL(kernel, grid, dim3(64), 0, stream, p);
        return hipGetLastError();
    };
    constexpr int full = transform_items<DK>();
    auto groups = [&](int per) { return (int64_t)p.n * ((p.slots + per - 1) / per); };
    if (groups(full) >= kTransformSpreadGroups || full <= 4)
        return go(head_transform_kernel<DK, full>, full);
    if (groups(4) >= kTransformSpreadGroups)
        return go(head_transform_kernel<DK, 4>, 4);
    return go(head_transform_kernel<DK, 1>, 1);
}

hipError_t launch_head_transform(const TransformParams &p, hipStream_t stream)
{
    switch (p.dim) {
    case 16: return launch_dk<16>(p, stream);
    case 32: return launch_dk<32>(p, stream);
    case 64: return launch_dk<64>(p, stream);
    case 128: return launch_dk<128>(p, stream);
    case 256: return launch_dk<256>(p, stream);
    case 512: return launch_dk<512>(p, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl

struct pcl_head_transform {
    pcl_context *ctx = nullptr;
    int64_t qheads = 0, kvheads = 0, dim = 0;
    int sliding = 0;
    float eps = 0.0f, base = 0.0f;
    std::vector<float> factors; // empty: none
    float *scales = nullptr;    // device [2][dim]: query, key
    float *tab = nullptr;       // device (sin, cos) pairs [rows][dim/2][2]
    int64_t tab_rows = 0;
};

namespace {

using pcl::TransformParams;

// Positions are converted to f32 for the angles (exact below 2^24).
constexpr int64_t kMaxPositions = (int64_t)1 << 24;

void report(const char *what, hipError_t e)
{
    std::fprintf(stderr, "pcl_head_transform: %s: %s\n", what, hipGetErrorString(e));
}

bool finite_all(const float *x, int64_t n)
{
    for (int64_t i = 0; i < n; ++i)
        if (!std::isfinite(x[i]))
            return false;
    return true;
}

// (sin, cos) of every pair of positions [from, to): p9_ref_rope's
// frequencies and angles in f32 (reference.rs:294-305), the C library's
// powf (equal to the reference's libm powf on its digest inputs) and the
// table's sine and cosine of rotation.hpp. False on a non-finite angle.
bool rope_rows(const pcl_head_transform *t, int64_t from, int64_t to, float *out)
{
    const int64_t half = t->dim / 2;
    std::vector<float> inv(half);
    for (int64_t i = 0; i < half; ++i) {
        float f = 1.0f / powf(t->base, (2.0f * (float)i) / (float)t->dim);
        if (!t->factors.empty())
            f = f / t->factors[i];
        inv[i] = f;
    }
    for (int64_t p = from; p < to; ++p) {
        for (int64_t i = 0; i < half; ++i) {
            const float angle = (float)p * inv[i];
            if (!std::isfinite(angle))
                return false;
            float s, c;
            pcl::rotation_sincos(angle, &s, &c);
            out[2 * ((p - from) * half + i)] = s;
            out[2 * ((p - from) * half + i) + 1] = c;
        }
    }
    return true;
}

// Table rows for positions [0, end): grown by doubling, built on the host.
int ensure_table(pcl_head_transform *t, int64_t end)
{
    if (end <= t->tab_rows)
        return PCL_OK;
    const int64_t half = t->dim / 2;
    const int64_t rows = std::min<int64_t>(
        kMaxPositions, std::max<int64_t>(end, std::max<int64_t>(2 * t->tab_rows, 256)));
    std::vector<float> host;
    try {
        host.resize((size_t)(rows - t->tab_rows) * half * 2);
    } catch (const std::bad_alloc &) {
        return PCL_RESOURCE_LIMIT;
    }
    if (!rope_rows(t, t->tab_rows, rows, host.data()))
        return PCL_NON_FINITE_VALUE;
    float *tab = nullptr;
    hipError_t e = hipMalloc(&tab, (size_t)rows * half * 2 * sizeof(float));
    if (e == hipSuccess && t->tab_rows)
        e = hipMemcpyAsync(tab, t->tab, (size_t)t->tab_rows * half * 2 * sizeof(float),
                           hipMemcpyDeviceToDevice, t->ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(tab + t->tab_rows * half * 2, host.data(),
                           host.size() * sizeof(float), hipMemcpyHostToDevice, t->ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(t->ctx->stream); // the old table and host rows are read
    if (e != hipSuccess) {
        report("growing the rotary table", e);
        if (tab)
            (void)hipFree(tab);
        return PCL_RESOURCE_LIMIT;
    }
    if (t->tab)
        (void)hipFree(t->tab);
    t->tab = tab;
    t->tab_rows = rows;
    return PCL_OK;
}

int run(pcl_head_transform *t, const float *rq, const float *rk, const float *rv, int64_t n,
        int64_t position, float *oq, float *ok, float *ov, int64_t kv_stride)
{
    if (n <= 0 || position < 0 || position > kMaxPositions - n)
        return PCL_RESOURCE_LIMIT;
    if (!rq || !oq || (ok && (!rk || !ov)))
        return PCL_INVALID_SHAPE;
    if (ok && !rv && t->sliding)
        return PCL_INVALID_SHAPE; // "sliding attention needs V"
    const int64_t slots = t->qheads + (ok ? 2 * t->kvheads : 0);
    if (n > ((int64_t)1 << 31) / slots)
        return PCL_INVALID_SHAPE;
    (void)hipSetDevice(t->ctx->device);
    const int rc = ensure_table(t, position + n);
    if (rc != PCL_OK)
        return rc;
    TransformParams p{};
    p.rq = rq;
    p.rk = rk;
    p.rv = rv;
    p.oq = oq;
    p.ok = ok;
    p.ov = ov;
    p.o_kv_stride = kv_stride;
    p.qs = t->scales;
    p.ks = t->scales + t->dim;
    p.tab = t->tab;
    p.pos0 = position;
    p.n = (int)n;
    p.qheads = (int)t->qheads;
    p.kvh = (int)t->kvheads;
    p.dim = (int)t->dim;
    p.slots = (int)slots;
    p.eps = t->eps;
    p.err = t->ctx->err;
    const hipError_t e = pcl::launch_head_transform(p, t->ctx->stream);
    if (e != hipSuccess) {
        report("launch", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

} // namespace

extern "C" {

int pcl_head_transform_create(pcl_context *ctx, int64_t qheads, int64_t kvheads, int64_t dim,
                              int sliding, const float *query_scale, const float *key_scale,
                              float epsilon, float base, const float *factors,
                              pcl_head_transform **out)
{
    if (!out)
        return PCL_INVALID_SHAPE;
    *out = nullptr;
    // widths (attention.rs:12-32) and this backend's head dims
    if (!ctx || qheads <= 0 || kvheads <= 0 || qheads % kvheads != 0 || qheads > 4096 ||
        !query_scale || !key_scale)
        return PCL_INVALID_SHAPE;
    if (dim != 16 && dim != 32 && dim != 64 && dim != 128 && dim != 256 && dim != 512)
        return PCL_INVALID_SHAPE;
    // HeadTransform::new's parameter checks (attention.rs:74-97)
    if (!std::isfinite(epsilon) || epsilon <= 0.0f || !std::isfinite(base) || base <= 0.0f ||
        !finite_all(query_scale, dim) || !finite_all(key_scale, dim))
        return PCL_INVALID_PARAMETER;
    if (factors) {
        for (int64_t i = 0; i < dim / 2; ++i)
            if (!std::isfinite(factors[i]) || factors[i] <= 0.0f)
                return PCL_INVALID_PARAMETER;
    }
    auto *t = new pcl_head_transform;
    t->ctx = ctx;
    t->qheads = qheads;
    t->kvheads = kvheads;
    t->dim = dim;
    t->sliding = sliding != 0;
    t->eps = epsilon;
    t->base = base;
    if (factors)
        t->factors.assign(factors, factors + dim / 2);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(&t->scales, 2 * dim * sizeof(float));
    if (e == hipSuccess)
        e = hipMemcpy(t->scales, query_scale, dim * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(t->scales + dim, key_scale, dim * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        report("create", e);
        if (t->scales)
            (void)hipFree(t->scales);
        delete t;
        return PCL_RESOURCE_LIMIT;
    }
    *out = t;
    return PCL_OK;
}

void pcl_head_transform_destroy(pcl_head_transform *t)
{
    if (!t)
        return;
    (void)hipSetDevice(t->ctx->device);
    (void)hipStreamSynchronize(t->ctx->stream);
    if (t->scales)
        (void)hipFree(t->scales);
    if (t->tab)
        (void)hipFree(t->tab);
    delete t;
}

int pcl_head_transform_prepare(pcl_head_transform *t, const float *raw_q, const float *raw_k,
                               const float *raw_v, int64_t n, int64_t position, float *q_out,
                               float *k_out, float *v_out)
{
    if (!t || !k_out)
        return PCL_INVALID_SHAPE;
    return run(t, raw_q, raw_k, raw_v, n, position, q_out, k_out, v_out, t->kvheads * t->dim);
}

int pcl_head_transform_query(pcl_head_transform *t, const float *raw_q, int64_t n,
                             int64_t position, float *q_out)
{
    if (!t)
        return PCL_INVALID_SHAPE;
    return run(t, raw_q, nullptr, nullptr, n, position, q_out, nullptr, nullptr, 0);
}

int pcl_kv_cache_append_transformed(pcl_kv_cache *c, pcl_head_transform *t, const float *raw_q,
                                    const float *raw_k, const float *raw_v, int64_t n,
                                    float *q_out, pcl_kv_pending *pending)
{
    if (!c || !t || !pending || n <= 0 || !raw_q || !raw_k || !q_out)
        return PCL_INVALID_SHAPE;
    if (t->ctx != c->ctx || t->kvheads != c->kvheads || t->dim != c->dim)
        return PCL_INVALID_SHAPE; // "cache owner/layer/geometry mismatch"
    if (!raw_v && t->sliding)
        return PCL_INVALID_SHAPE;
    int rc = pcl::kv_cache_reserve(c, n);
    if (rc != PCL_OK)
        return rc;
    rc = run(t, raw_q, raw_k, raw_v, n, c->total, q_out, c->k + c->len * c->width,
             c->v + c->len * c->width, c->width);
    if (rc != PCL_OK)
        return rc;
    pcl::kv_cache_advance_rows(c, n, pending);
    return PCL_OK;
}

int pcl_kv_cache_attend_token(pcl_kv_cache *c, pcl_head_transform *t, const float *raw_q,
                              const float *raw_k, const float *raw_v, float q_scale, int kernel,
                              float *q_out, float *out, pcl_kv_pending *pending)
{
    if (!c || !t || !pending || !raw_q || !raw_k || !q_out || !out)
        return PCL_INVALID_SHAPE;
    if (t->ctx != c->ctx || t->kvheads != c->kvheads || t->dim != c->dim)
        return PCL_INVALID_SHAPE; // "cache owner/layer/geometry mismatch"
    if (!raw_v && t->sliding)
        return PCL_INVALID_SHAPE;
    if (c->total > kMaxPositions - 1)
        return PCL_RESOURCE_LIMIT;
    int rc = pcl::kv_cache_reserve(c, 1);
    if (rc != PCL_OK)
        return rc;
    (void)hipSetDevice(t->ctx->device);
    rc = ensure_table(t, c->total + 1);
    if (rc != PCL_OK)
        return rc;
    // the encoder descriptor of the step, its row counted (encoder_desc
    // after the append)
    const int64_t width = c->width, retained = c->len - c->start + 1;
    float *nk = c->k + c->len * width, *nv = c->v + c->len * width;
    pcl_attention_desc d;
    std::memset(&d, 0, sizeof d);
    d.q = q_out;
    d.q_stride = t->qheads * t->dim;
    d.nq = 1;
    d.k0 = c->k + c->start * width;
    d.v0 = c->v + c->start * width;
    d.n0 = retained;
    d.qheads = t->qheads;
    d.kvheads = c->kvheads;
    d.dim = c->dim;
    d.kh_first = 0;
    d.kh_end = c->kvheads;
    d.causal = 1;
    d.window = c->window;
    d.first_key = c->total + 1 - retained;
    d.first_query = c->total;
    d.q_scale = q_scale;
    d.out = out;
    d.o_stride = t->qheads * t->dim;
    d.kernel = kernel;
    const pcl::StepFold fold{raw_q, raw_k, raw_v, t->scales, t->scales + t->dim,
                             t->tab + c->total * t->dim, nk, nv, q_out, t->eps};
    const int64_t position = c->total;
    rc = pcl::launch_step(c->ctx, d, fold, [&] {
        return run(t, raw_q, raw_k, raw_v, 1, position, q_out, nk, nv, width);
    });
    if (rc != PCL_OK)
        return rc;
    pcl::kv_cache_advance_rows(c, 1, pending);
    return PCL_OK;
}

} // extern "C"
