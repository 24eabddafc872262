// Split-KV flash decode for gfx950.
//
// One workgroup computes one 256-key chunk for one 16-row unit (up to 16
// (query, head) rows of one KV head) with DK/64 waves:
//   phase 1  each wave computes the scores of its tiles, one 16-key block at
//            a time: the block's K is requested in one batch (straight from
//            HBM into MFMA A operands, addresses clamped instead of branched
//            so the loads issue back to back) and the first block is
//            requested before the workgroup stages Q^T in LDS;
//   phase 2  each wave turns its tiles into probabilities with the running
//            maxima of the tiles before them, and leaves P, alpha and the row
//            sums in LDS;
//   phase 3  wave w streams V for dims [64w, 64w+64) through the MFMA P.V
//            chain over the chunk's tiles in order, VD tiles of V in flight.
// With more than one chunk the workgroup writes its chunk partial (m, l, O)
// and counts itself in; the last workgroup of a span merges the span's
// chunks, and the last span of a unit merges the spans and writes the output,
// both in ascending order (the ordered merges of attention_device.hpp). The
// counters reset themselves, so the workspace needs no clearing between
// launches. A launch of a single chunk writes the output directly.
#include "attention_device.hpp"

namespace pcl {

__device__ __forceinline__ f4 ld4(const float *p)
{
    return ldg4(p);
}

__device__ __forceinline__ f4 zero4()
{
    return f4{0.f, 0.f, 0.f, 0.f};
}

// Occupancy (waves per SIMD) and V tiles in flight per head-dim class.
template <int DK> struct SplitCfg {
    static constexpr int waves_per_eu = DK >= 512 ? 2 : 4;
    static constexpr int vdepth = DK >= 512 ? 4 : 2;
};

// Running merge state of one (row, dim) element.
struct Merged {
    float M, L, acc;
};

__device__ __forceinline__ void merge_into(Merged &s, float m, float l, float o)
{
    if (m == kNegInf)
        return; // a part with nothing allowed merges as a no-op
    const MergeFactors f = merge_factors(s.M, m);
    s.L = merge_value(s.L, l, f);
    s.acc = merge_value(s.acc, o, f);
    s.M = f.m;
}

template <bool DEV> __device__ __forceinline__ float ld_part(const float *p)
{
    return DEV ? ld_dev(p) : ldg(p);
}

template <bool DEV> __device__ __forceinline__ void st_part(float *p, float v)
{
    if (DEV)
        st_dev(p, v);
    else
        stg(p, v);
}

// Chunks [c0, c1) (launch-local indices) of one element, in order. DEV: the
// partials were written by other workgroups of this launch.
template <bool DEV>
__device__ __forceinline__ Merged merge_span_chunks(const float *ml, const float *o, int dk,
                                                    int c0, int c1)
{
    float mv[kSpanChunks], lv[kSpanChunks], ov[kSpanChunks];
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i) {
        const int cc = c0 + i < c1 ? c0 + i : c0;
        mv[i] = ld_part<DEV>(ml + 2 * cc);
        lv[i] = ld_part<DEV>(ml + 2 * cc + 1);
        ov[i] = ld_part<DEV>(o + (int64_t)cc * dk);
    }
    Merged s = {kNegInf, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i)
        if (c0 + i < c1)
            merge_into(s, mv[i], lv[i], ov[i]);
    return s;
}

// Spans [0, nspan) of one element, in order.
template <bool DEV>
__device__ __forceinline__ Merged merge_spans(const float *ml, const float *o, int dk, int nspan)
{
    Merged s = {kNegInf, 0.f, 0.f};
    constexpr int B = 8; // spans requested per batch
    for (int s0 = 0; s0 < nspan; s0 += B) {
        float mv[B], lv[B], ov[B];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int ss = s0 + i < nspan ? s0 + i : s0;
            mv[i] = ld_part<DEV>(ml + 2 * ss);
            lv[i] = ld_part<DEV>(ml + 2 * ss + 1);
            ov[i] = ld_part<DEV>(o + (int64_t)ss * dk);
        }
#pragma unroll
        for (int i = 0; i < B; ++i)
            if (s0 + i < nspan)
                merge_into(s, mv[i], lv[i], ov[i]);
    }
    return s;
}

// Launch-local chunk range of span `sl`.
__device__ __forceinline__ void span_chunks(const Params &p, int sl, int *c0, int *c1)
{
    const int span = p.s_lo + sl;
    *c0 = max(span * kSpanChunks, p.c_lo) - p.c_lo;
    *c1 = min((span + 1) * kSpanChunks, p.c_lo + p.nch) - p.c_lo;
}

__device__ __forceinline__ float *out_ptr(const Params &p, int kh, int row)
{
    const int query = row / p.group;
    const int h = kh * p.group + row % p.group;
    if (h < p.h_lo || h >= p.h_hi)
        return nullptr;
    return p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
}

// Final value of a merged element: merged into the empty total when there is
// only one span (exact), then normalised.
__device__ __forceinline__ float finish(const Merged &s, bool single_span)
{
    if (single_span) {
        const MergeFactors f = merge_factors(kNegInf, s.M);
        return merge_value(0.f, s.acc, f) / merge_value(0.f, s.L, f);
    }
    return s.acc / s.L;
}

template <int DK>
__global__ __launch_bounds__(DK, SplitCfg<DK>::waves_per_eu) void split_kv_kernel(Params p)
{
    constexpr int NW = DK / 64;
    constexpr int TPW = kTilesPerChunk / NW;
    constexpr int NU = DK / 32;   // score chain steps
    constexpr int QLD = DK + 4;   // padded LDS row stride of Q
    constexpr int VD = SplitCfg<DK>::vdepth;
    __shared__ float q_lds[kRows * QLD];
    __shared__ float tmax_lds[kTilesPerChunk][kRows];
    __shared__ float alpha_lds[kTilesPerChunk][kRows];
    __shared__ float rs_lds[kTilesPerChunk][kRows];
    __shared__ float p_lds[kTilesPerChunk][8][64];
    __shared__ int any_lds[kTilesPerChunk];
    __shared__ int last_lds;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int c = p.c_lo + blockIdx.x;
    const int unit = blockIdx.y % p.units;
    const int kvl = blockIdx.y / p.units;
    const int kh = p.kh_first + kvl;
    const int row0 = unit * kRows;
    const int row = row0 + col; // this lane's row (MFMA column)
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;

    // Masks of this wave's tiles.
    bool ok[TPW][2][4];
    bool wave_any[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int64_t kbase = cbase + (w * TPW + i) * kTile;
        bool any = false;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ok[i][b][r] = allowed(p, row, kbase + 16 * b + 4 * g + r);
                any |= ok[i][b][r];
            }
        wave_any[i] = __any(any);
    }

    // K A operands of one 16-key block: kb[u][h] = K[key][32u + 8g + 4h ..].
    f4 kb[NU][2];
    auto load_kblock = [&](int i, int b) {
        const int64_t key = cbase + (w * TPW + i) * kTile + 16 * b + col;
        const float *kp = key_row(p, key < klast ? key : klast) + (int64_t)kh * p.dim;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int d = 32 * u + 8 * g + 4 * h;
                const f4 x = ld4(kp + (d < p.dim ? d : 0));
                kb[u][h] = d < p.dim ? x : zero4();
            }
    };
    if (wave_any[0])
        load_kblock(0, 0);

    // Q^T of the unit's rows into LDS, scaled; padding rows and dims are 0.
    for (int i = tid; i < kRows * (DK / 4); i += DK) {
        const int r = i / (DK / 4);
        const int d = (i % (DK / 4)) * 4;
        const int f = row0 + r;
        f4 v = zero4();
        if (f < p.nrows && d < p.dim) {
            const int query = f / p.group;
            const int h = kh * p.group + f % p.group;
            v = ld4(p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim + d) * p.q_scale;
        }
        *(f4 *)(q_lds + r * QLD + d) = v;
    }
    __syncthreads();

    // V of this wave's dims, VD tiles in flight (tile t in vbuf[t % VD]).
    const int dv = 64 * w + 4 * col;
    const bool dv_in = dv < p.dim;
    const int dvc = dv_in ? dv : 0;
    f4 vbuf[VD][8];
    auto load_v = [&](f4 (&dst)[8], int t) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = cbase + t * kTile + 16 * b + 4 * g + r;
                const int64_t kc = key < klast ? key : klast;
                dst[4 * b + r] = ld4(value_row(p, kc) + (int64_t)kh * p.dim + dvc);
            }
    };

    // ---- phase 1: scores and tile maxima --------------------------------
    float s[TPW][2][4];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int t = w * TPW + i;
        float tm = kNegInf;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s[i][b][r] = 0.f;
        if (wave_any[i]) {
            f4 acc[2] = {zero4(), zero4()};
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                if (i != 0 || b != 0)
                    load_kblock(i, b);
                // the whole block is requested before the first MFMA needs it
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    const int d = 32 * u + 8 * g;
                    const f4 qa0 = *(const f4 *)(q_lds + col * QLD + d);
                    const f4 qa1 = *(const f4 *)(q_lds + col * QLD + d + 4);
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const float qv = jj < 4 ? qa0[jj] : qa1[jj - 4];
                        acc[b] = mfma(kb[u][jj >> 2][jj & 3], qv, acc[b]);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[i][b][r] = acc[b][r];
            tm = tile_max(s[i], ok[i]);
            bad |= bad_scores(s[i], ok[i]);
        }
        if (g == 0)
            tmax_lds[t][col] = tm;
        if (lane == 0)
            any_lds[t] = wave_any[i];
    }
#pragma unroll
    for (int i = 0; i < VD; ++i)
        load_v(vbuf[i], i);
    if (bad)
        atomicOr(p.err, kErrScore);
    __syncthreads();

    // ---- phase 2: probabilities with the running maxima -----------------
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int t = w * TPW + i;
        float mprev = kNegInf;
        for (int tt = 0; tt < t; ++tt)
            mprev = fmaxf(mprev, tmax_lds[tt][col]);
        const float mn = fmaxf(mprev, tmax_lds[t][col]);
        const float ms = safe_max(mn);
        const float alpha = fexp(mprev - ms);
        float pr[2][4];
        const float rs = tile_probs(s[i], ok[i], ms, pr);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                p_lds[t][4 * b + r][lane] = pr[b][r];
        if (g == 0) {
            alpha_lds[t][col] = alpha;
            rs_lds[t][col] = rs;
        }
    }
    __syncthreads();

    // ---- phase 3: P.V for dims [64w, 64w+64) ----------------------------
    float l = 0.f;
    float m = kNegInf;
    f4 O[4] = {zero4(), zero4(), zero4(), zero4()};
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        const float a = alpha_lds[t][col];
        l = __builtin_fmaf(l, a, rs_lds[t][col]);
        m = fmaxf(m, tmax_lds[t][col]);
        if (any_lds[t]) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                O[j] = O[j] * a;
#pragma unroll
            for (int br = 0; br < 8; ++br) {
                const float pb = p_lds[t][br][lane];
                const f4 v = dv_in ? vbuf[t % VD][br] : zero4();
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[j] = mfma(v[j], pb, O[j]);
            }
        }
        if (t + VD < kTilesPerChunk)
            load_v(vbuf[t % VD], t + VD);
        __builtin_amdgcn_sched_barrier(0);
    }

    // O[j][i] is dim 64w + 16g + 4i + j of row `row`.
    if (p.ws_o == nullptr) { // the launch's only chunk: final output
        float *o = row < p.nrows ? out_ptr(p, kh, row) : nullptr;
        if (!o)
            return;
        bool nonfinite = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 64 * w + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = O[j][i] / l;
                nonfinite |= !is_finite(v[j]);
            }
            stg4(o + d, v);
        }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }
    const bool fused = p.cnt != nullptr; // merged in this kernel, not by the combine kernels
    if (row < p.nrows) {
        const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + blockIdx.x;
        float *wo = p.ws_o + slot * p.dk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 64 * w + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (fused)
                    st_dev(wo + d + j, O[j][i]);
                else
                    stg(wo + d + j, O[j][i]);
            }
        }
        if (w == 0 && g == 0) {
            if (fused) {
                st_dev(p.ws_ml + 2 * slot, m);
                st_dev(p.ws_ml + 2 * slot + 1, l);
            } else {
                stg(p.ws_ml + 2 * slot, m);
                stg(p.ws_ml + 2 * slot + 1, l);
            }
        }
    }
    if (!fused)
        return; // the combine kernels merge the partials

    // ---- the last workgroup of a span merges it -------------------------
    const int sl = (c / kSpanChunks) - p.s_lo;
    int c0, c1;
    span_chunks(p, sl, &c0, &c1);
    // this workgroup's device-scope stores are complete before it counts in
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (tid == 0) {
        int *cs = p.cnt + ((int64_t)kvl * p.units + unit) * p.nspan + sl;
        const int old = atomicAdd(cs, 1);
        last_lds = old == c1 - c0 - 1;
        if (last_lds)
            atomicExch(cs, 0);
    }
    __syncthreads();
    if (!last_lds)
        return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int nreal = min(kRows, p.nrows - row0);
    const bool single = p.nspan == 1;
    bool nonfinite = false;
    for (int e = tid; e < nreal * p.dim; e += DK) {
        const int r = row0 + e / p.dim;
        const int d = e % p.dim;
        const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + r) * p.nch;
        const Merged sm = merge_span_chunks<true>(p.ws_ml + 2 * slot0,
                                                  p.ws_o + slot0 * p.dk + d, p.dk, c0, c1);
        if (single) {
            float *o = out_ptr(p, kh, r);
            if (o) {
                const float v = finish(sm, true);
                stg(o + d, v);
                nonfinite |= !is_finite(v);
            }
        } else {
            const int64_t s2 = ((int64_t)kvl * p.nrows_pad + r) * p.nspan + sl;
            st_dev(p.ws2_o + s2 * p.dk + d, sm.acc);
            if (d == 0) {
                st_dev(p.ws2_ml + 2 * s2, sm.M);
                st_dev(p.ws2_ml + 2 * s2 + 1, sm.L);
            }
        }
    }
    if (single) {
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }

    // ---- the last span of the unit merges the spans -----------------------
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (tid == 0) {
        int *ct = p.cnt + (int64_t)p.nkv * p.units * p.nspan + (int64_t)kvl * p.units + unit;
        const int old = atomicAdd(ct, 1);
        last_lds = old == p.nspan - 1;
        if (last_lds)
            atomicExch(ct, 0);
    }
    __syncthreads();
    if (!last_lds)
        return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    for (int e = tid; e < nreal * p.dim; e += DK) {
        const int r = row0 + e / p.dim;
        const int d = e % p.dim;
        float *o = out_ptr(p, kh, r);
        if (!o)
            continue;
        const int64_t s0 = ((int64_t)kvl * p.nrows_pad + r) * p.nspan;
        const Merged st =
            merge_spans<true>(p.ws2_ml + 2 * s0, p.ws2_o + s0 * p.dk + d, p.dk, p.nspan);
        const float v = finish(st, false);
        stg(o + d, v);
        nonfinite |= !is_finite(v);
    }
    if (nonfinite)
        atomicOr(p.err, kErrOutput);
}

// Level 1 of the combine: the chunks of one span, for one (row, dim) per
// thread. With a single span the result is final.
__global__ __launch_bounds__(256) void combine_span_kernel(Params p)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.nrows * p.dim)
        return;
    const int kvl = blockIdx.z;
    const int sl = blockIdx.y;
    const int row = (int)(idx / p.dim);
    const int d = (int)(idx % p.dim);
    float *o = out_ptr(p, p.kh_first + kvl, row);
    if (!o)
        return;
    int c0, c1;
    span_chunks(p, sl, &c0, &c1);
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
    const Merged sm =
        merge_span_chunks<false>(p.ws_ml + 2 * slot0, p.ws_o + slot0 * p.dk + d, p.dk, c0, c1);
    if (p.nspan == 1) {
        const float v = finish(sm, true);
        stg(o + d, v);
        if (!is_finite(v))
            atomicOr(p.err, kErrOutput);
        return;
    }
    const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nspan + sl;
    stg(p.ws2_o + slot * p.dk + d, sm.acc);
    if (d == 0) {
        stg(p.ws2_ml + 2 * slot, sm.M);
        stg(p.ws2_ml + 2 * slot + 1, sm.L);
    }
}

// Level 2 of the combine: the spans, in ascending order.
__global__ __launch_bounds__(256) void combine_final_kernel(Params p)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.nrows * p.dim)
        return;
    const int kvl = blockIdx.z;
    const int row = (int)(idx / p.dim);
    const int d = (int)(idx % p.dim);
    float *o = out_ptr(p, p.kh_first + kvl, row);
    if (!o)
        return;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nspan;
    const Merged st =
        merge_spans<false>(p.ws2_ml + 2 * slot0, p.ws2_o + slot0 * p.dk + d, p.dk, p.nspan);
    const float v = finish(st, false);
    stg(o + d, v);
    if (!is_finite(v))
        atomicOr(p.err, kErrOutput);
}

hipError_t launch_split_kv(const Params &p, hipStream_t stream)
{
    const dim3 grid(p.nch, p.nkv * p.units);
    switch (p.dk) {
    case 64: split_kv_kernel<64><<<grid, 64, 0, stream>>>(p); break;
    case 128: split_kv_kernel<128><<<grid, 128, 0, stream>>>(p); break;
    case 256: split_kv_kernel<256><<<grid, 256, 0, stream>>>(p); break;
    case 512: split_kv_kernel<512><<<grid, 512, 0, stream>>>(p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_combine(const Params &p, hipStream_t stream)
{
    const int64_t n = (int64_t)p.nrows * p.dim;
    const unsigned bx = (unsigned)((n + 255) / 256);
    combine_span_kernel<<<dim3(bx, p.nspan, p.nkv), 256, 0, stream>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.nspan == 1)
        return e;
    combine_final_kernel<<<dim3(bx, 1, p.nkv), 256, 0, stream>>>(p);
    return hipGetLastError();
}

} // namespace pcl
