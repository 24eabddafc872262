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
// for the combine kernel; a launch of a single chunk writes the output
// directly.
//
// The combine (also used by the pipelined and tiled split kernels) runs both
// levels of the ordered merge of attention_device.hpp in one launch up to 32
// spans (128K keys): span lanes merge the chunks of their spans, one batch of
// loads per span, and the span partials are folded in ascending order from
// registers of the same wave (one span) or from LDS (2 to 32 spans).
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
    const ChunkKeys ck = chunk_keys(p, row, cbase);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const bool any = tile_keys(ck, w * TPW + i, g, ok[i]);
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
                const f4 x = ldg4_stream(kp + (d < p.dim ? d : 0));
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
                dst[4 * b + r] = ldg4_stream(value_row(p, kc) + (int64_t)kh * p.dim + dvc);
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
            cap_scores(p, s[i]);
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
    if (row < p.nrows) {
        const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + blockIdx.x;
        float *wo = p.ws_o + slot * p.dk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 64 * w + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[j] = O[j][i];
            stg4(wo + d, v);
        }
        if (w == 0 && g == 0) {
            stg(p.ws_ml + 2 * slot, m);
            stg(p.ws_ml + 2 * slot + 1, l);
        }
    }
}

// Level 1 of the ordered merge for four dims [d, d+4) of one row: span sl's
// chunk partials merged in ascending order from (-inf, 0, 0), all of the
// span's loads in one batch (a wave's loads are a contiguous KiB of one
// partial). slot0: the row's first chunk slot.
__device__ __forceinline__ Merged4 merge_span_chunks(const Params &p, int64_t slot0, int sl,
                                                     int d, bool din)
{
    int c0, c1;
    span_chunks(p, sl, &c0, &c1);
    float mv[kSpanChunks], lv[kSpanChunks];
    f4 ov[kSpanChunks];
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i) {
        const int64_t cc = slot0 + (c0 + i < c1 ? c0 + i : c0);
        mv[i] = ldg(p.ws_ml + 2 * cc);
        lv[i] = ldg(p.ws_ml + 2 * cc + 1);
        ov[i] = ldg4(p.ws_o + cc * p.dk + (din ? d : 0));
    }
    Merged4 s = {kNegInf, 0.f, zero4()};
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i) {
        // chunks past the span merge as empty parts (no-ops)
        const bool in = c0 + i < c1;
        merge_into4(s, in ? mv[i] : kNegInf, in ? lv[i] : 0.f, in ? ov[i] : zero4());
    }
    return s;
}

// Two-level combine for launches of many spans, one wave per 256 output dims
// of one row, so every load is a contiguous KiB of one partial.
// Level 1: wave ((kv, row), span, piece) merges the span's chunks in order;
// with a single span it writes the output, else the span partial.
__global__ __launch_bounds__(64) void combine_level1_kernel(Params p)
{
    const int lane = threadIdx.x;
    const int piece = blockIdx.z;
    const int sl = blockIdx.y;
    const int kvl = blockIdx.x / p.nrows;
    const int row = blockIdx.x % p.nrows;
    const int d = 256 * piece + 4 * lane;
    const bool din = d < p.dim;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
    const Merged4 s = merge_span_chunks(p, slot0, sl, d, din);
    if (p.nspan == 1) {
        float *o = out_ptr(p, p.kh_first + kvl, row);
        if (!o || !din)
            return;
        // one span: merged into the empty total (exact), then normalised
        const MergeFactors f = merge_factors(kNegInf, s.M);
        const float L = merge_value(0.f, s.L, f);
        f4 v;
        bool nonfinite = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = merge_value(0.f, s.acc[j], f) / L;
            nonfinite |= !is_finite(v[j]);
        }
        stg4(o + d, v);
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }
    const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nspan + sl;
    if (din)
        stg4(p.ws2_o + slot * p.dk + d, s.acc);
    if (lane == 0 && piece == 0) {
        stg(p.ws2_ml + 2 * slot, s.M);
        stg(p.ws2_ml + 2 * slot + 1, s.L);
    }
}

// Level 2: wave ((kv, row), piece) merges the span partials in order.
__global__ __launch_bounds__(64) void combine_level2_kernel(Params p)
{
    const int lane = threadIdx.x;
    const int piece = blockIdx.z;
    const int kvl = blockIdx.x / p.nrows;
    const int row = blockIdx.x % p.nrows;
    const int d = 256 * piece + 4 * lane;
    const bool din = d < p.dim;
    float *o = out_ptr(p, p.kh_first + kvl, row);
    if (!o || !din)
        return;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nspan;
    Merged4 s = {kNegInf, 0.f, zero4()};
    constexpr int B = 32; // spans requested per batch
    for (int s0 = 0; s0 < p.nspan; s0 += B) {
        float mv[B], lv[B];
        f4 ov[B];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int64_t ss = slot0 + (s0 + i < p.nspan ? s0 + i : s0);
            mv[i] = ldg(p.ws2_ml + 2 * ss);
            lv[i] = ldg(p.ws2_ml + 2 * ss + 1);
            ov[i] = ldg4(p.ws2_o + ss * p.dk + d);
        }
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const bool in = s0 + i < p.nspan;
            merge_into4(s, in ? mv[i] : kNegInf, in ? lv[i] : 0.f, in ? ov[i] : zero4());
        }
    }
    f4 v;
    bool nonfinite = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = s.acc[j] / s.L;
        nonfinite |= !is_finite(v[j]);
    }
    stg4(o + d, v);
    if (nonfinite)
        atomicOr(p.err, kErrOutput);
}

// Both levels in one launch for 2 to kCombineLdsSpans spans: a workgroup
// per ((kv, row), slab of 4 * kCombineSpanLanes dims) with a group of
// kCombineSpanLanes lanes per span (the workgroup sized to the spans, at
// least one wave); each group merges its span's chunks exactly as level 1
// (one batch of loads, contiguous bytes of a partial per group) and leaves
// the span partial in LDS, then the first group folds the spans in
// ascending order exactly as level 2. Saves level 2's launch and its
// workspace round trip, and reads whole slabs where the span-lane kernel
// above scatters (3 % faster for an 8-position verification over 32K).
constexpr int kCombineSpanLanes = 8;
constexpr int kCombineLdsSpans = 32;
constexpr int kCombineSpanThreads = kCombineLdsSpans * kCombineSpanLanes;

__global__ __launch_bounds__(kCombineSpanThreads) void combine_spans_kernel(Params p)
{
    constexpr int L = kCombineSpanLanes;
    __shared__ f4 so[kCombineLdsSpans][L];
    __shared__ float sm[kCombineLdsSpans], sls[kCombineLdsSpans];
    const int sl = threadIdx.x / L; // this lane group's span (blockDim >= nspan * L)
    const int q = threadIdx.x % L;
    const int kvl = blockIdx.x / p.nrows;
    const int row = blockIdx.x % p.nrows;
    const int d = 4 * L * blockIdx.z + 4 * q;
    const bool din = d < p.dim;
    float *o = out_ptr(p, p.kh_first + kvl, row);
    if (!o) // the whole workgroup's row is not written
        return;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
    if (sl < p.nspan) {
        const Merged4 s = merge_span_chunks(p, slot0, sl, d, din);
        so[sl][q] = s.acc;
        if (q == 0) {
            sm[sl] = s.M;
            sls[sl] = s.L;
        }
    }
    __syncthreads();
    if (threadIdx.x >= L || !din)
        return;
    Merged4 t = {kNegInf, 0.f, zero4()};
    for (int i = 0; i < p.nspan; ++i)
        merge_into4(t, sm[i], sls[i], so[i][q]);
    f4 v;
    bool nonfinite = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = t.acc[j] / t.L;
        nonfinite |= !is_finite(v[j]);
    }
    stg4(o + d, v);
    if (nonfinite)
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

// Both levels of the combine in one launch, one wave per workgroup (small
// workgroups spread the partial loads over many CUs). The wave holds
// G = 64 / SP element groups (four consecutive dims of one row) x SP span
// lanes: span lane s merges the chunks of span s for its element group (one
// batch of loads), then every lane folds the group's span partials, gathered
// by cross-lane reads, in ascending order. The values are those of the
// two-level kernels above. It serves launches of a single span (one lane per
// element group, G = 64 groups per wave); with more spans a wave's loads
// scatter over span lanes, and the slab kernel above (spans in LDS) is faster.
constexpr int kCombineMaxSpans = 1;

__global__ __launch_bounds__(64) void combine_kernel(Params p, int span_lanes)
{
    const int lane = threadIdx.x;
    const int G = 64 / span_lanes;
    const int gi = lane / span_lanes;
    const int sl = lane % span_lanes;
    const int q4 = p.dim / 4;
    const int e = blockIdx.x * G + gi; // element group within the KV head
    const int kvl = blockIdx.y;
    const bool valid = e < p.nrows * q4;
    const int row = valid ? e / q4 : 0;
    const int d = valid ? 4 * (e % q4) : 0;
    float *o = valid ? out_ptr(p, p.kh_first + kvl, row) : nullptr;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
    bool nonfinite = false;
    f4 v;
    if (p.nspan == 1) {
        // one span: merged into the empty total (exact), then normalised
        if (!o)
            return;
        const Merged4 s = merge_chunks4(p, slot0, d, 0, p.nch);
        const MergeFactors f = merge_factors(kNegInf, s.M);
        const float L = merge_value(0.f, s.L, f);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = merge_value(0.f, s.acc[j], f) / L;
    } else {
        Merged4 s = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
        if (o && sl < p.nspan) {
            int c0, c1;
            span_chunks(p, sl, &c0, &c1);
            s = merge_chunks4(p, slot0, d, c0, c1);
        }
        Merged4 st = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
        const int base = gi * span_lanes;
#pragma unroll 8
        for (int t = 0; t < p.nspan; ++t) {
            f4 acc;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j] = __shfl(s.acc[j], base + t);
            merge_into4(st, __shfl(s.M, base + t), __shfl(s.L, base + t), acc);
        }
        if (!o || sl != 0)
            return;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = st.acc[j] / st.L;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        nonfinite |= !is_finite(v[j]);
    stg4(o + d, v);
    if (nonfinite)
        atomicOr(p.err, kErrOutput);
}

hipError_t launch_combine(const Params &p, hipStream_t stream)
{
    if (p.nspan <= kCombineMaxSpans && (int64_t)p.nrows * (p.dim / 4) < ((int64_t)1 << 31)) {
        int lanes = 1;
        while (lanes < p.nspan)
            lanes *= 2;
        const int G = 64 / lanes;
        const int64_t groups = (int64_t)p.nrows * (p.dim / 4);
        const unsigned bx = (unsigned)((groups + G - 1) / G);
        combine_kernel<<<dim3(bx, p.nkv), 64, 0, stream>>>(p, lanes);
        return hipGetLastError();
    }
    const unsigned pieces = (unsigned)((p.dim + 255) / 256);
    const unsigned rows = (unsigned)(p.nkv * p.nrows);
    if (p.nspan <= kCombineLdsSpans) {
        const unsigned slabs = (unsigned)((p.dim + 4 * kCombineSpanLanes - 1) /
                                          (4 * kCombineSpanLanes));
        const int threads = ((p.nspan * kCombineSpanLanes + 63) / 64) * 64;
        combine_spans_kernel<<<dim3(rows, 1, slabs), threads, 0, stream>>>(p);
        return hipGetLastError();
    }
    // more spans: span partials through the workspace, two launches
    combine_level1_kernel<<<dim3(rows, p.nspan, pieces), 64, 0, stream>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.nspan == 1)
        return e;
    combine_level2_kernel<<<dim3(rows, 1, pieces), 64, 0, stream>>>(p);
    return hipGetLastError();
}

} // namespace pcl
