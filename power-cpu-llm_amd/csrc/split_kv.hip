// Split-KV flash decode for gfx950.
//
// One workgroup computes one 256-key chunk for one 16-row unit (up to 16
// (query, head) rows of one KV head) with DK/64 waves:
//   phase 1  each wave computes the scores of its tiles (K straight from HBM
//            as MFMA A operands, Q^T from LDS) and the per-tile row maxima;
//   phase 2  each wave turns its tiles into probabilities with the running
//            maxima of the tiles before them, and leaves P, alpha and the row
//            sums in LDS;
//   phase 3  wave w streams V for dims [64w, 64w+64) through the MFMA P.V
//            chain over the chunk's tiles in order.
// The chunk's (m, l, O) goes to the workspace, and combine_kernel merges the
// chunks of each row in ascending order. A launch of a single chunk writes the
// output directly (the merge from the empty state is exact).
#include "attention_device.hpp"

namespace pcl {

template <int DK>
__global__ __launch_bounds__(DK) void split_kv_kernel(Params p)
{
    constexpr int NW = DK / 64;
    constexpr int TPW = kTilesPerChunk / NW;
    constexpr int QLD = DK + 4; // padded LDS row stride of Q (conflict-free B reads)
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

    // Q^T of the unit's rows into LDS, scaled; padding rows and dims are 0.
    for (int i = tid; i < kRows * (DK / 4); i += DK) {
        const int r = i / (DK / 4);
        const int d = (i % (DK / 4)) * 4;
        const int f = row0 + r;
        f4 v = {0.f, 0.f, 0.f, 0.f};
        if (f < p.nrows && d < p.dim) {
            const int query = f / p.group;
            const int h = kh * p.group + f % p.group;
            v = *(const f4 *)(p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim + d);
            v = v * p.q_scale;
        }
        *(f4 *)(q_lds + r * QLD + d) = v;
    }
    __syncthreads();

    // ---- phase 1: scores and tile maxima --------------------------------
    float s[TPW][2][4];
    bool ok[TPW][2][4];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int t = w * TPW + i;
        const int64_t kbase = (int64_t)c * kChunk + t * kTile;
        bool any = false;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ok[i][b][r] = allowed(p, row, kbase + 16 * b + 4 * g + r);
                any |= ok[i][b][r];
            }
        const bool wave_any = __any(any);
        float tm = kNegInf;
        if (wave_any) {
            f4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            const float *kp[2];
            bool kin[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int64_t key = kbase + 16 * b + col;
                kin[b] = key < p.nkeys;
                kp[b] = key_row(p, kin[b] ? key : 0) + (int64_t)kh * p.dim;
            }
#pragma unroll
            for (int u = 0; u < DK / 32; ++u) {
                const int d = 32 * u + 8 * g;
                f4 ka[2][2];
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        ka[b][h] = (kin[b] && d + 4 * h < p.dim)
                                       ? *(const f4 *)(kp[b] + d + 4 * h)
                                       : f4{0.f, 0.f, 0.f, 0.f};
                const f4 qa0 = *(const f4 *)(q_lds + col * QLD + d);
                const f4 qa1 = *(const f4 *)(q_lds + col * QLD + d + 4);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const float qv = jj < 4 ? qa0[jj] : qa1[jj - 4];
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        acc[b] = mfma(ka[b][jj >> 2][jj & 3], qv, acc[b]);
                }
            }
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[i][b][r] = acc[b][r];
            tm = tile_max(s[i], ok[i]);
            bad |= bad_scores(s[i], ok[i]);
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[i][b][r] = 0.f;
        }
        if (g == 0)
            tmax_lds[t][col] = tm;
        if (lane == 0)
            any_lds[t] = wave_any;
    }
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
    f4 O[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f},
               {0.f, 0.f, 0.f, 0.f}};
    const int dv = 64 * w + 4 * col; // this lane's V dims (A-operand row)
    for (int t = 0; t < kTilesPerChunk; ++t) {
        const float a = alpha_lds[t][col];
        l = __builtin_fmaf(l, a, rs_lds[t][col]);
        m = fmaxf(m, tmax_lds[t][col]);
        if (!any_lds[t])
            continue;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            O[j] = O[j] * a;
        const int64_t kbase = (int64_t)c * kChunk + t * kTile;
        f4 vv[2][4];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = kbase + 16 * b + 4 * g + r;
                vv[b][r] = (key < p.nkeys && dv < p.dim)
                               ? *(const f4 *)(value_row(p, key) + (int64_t)kh * p.dim + dv)
                               : f4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pb = p_lds[t][4 * b + r][lane];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[j] = mfma(vv[b][r][j], pb, O[j]);
            }
    }

    // O[j][i] is dim 64w + 16g + 4i + j of row `row`.
    if (row >= p.nrows)
        return;
    if (p.nch == 1 && p.ws_o == nullptr) {
        const int query = row / p.group;
        const int h = kh * p.group + row % p.group;
        if (h < p.h_lo || h >= p.h_hi)
            return;
        float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
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
            *(f4 *)(o + d) = v;
        }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }
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
        *(f4 *)(wo + d) = v;
    }
    if (w == 0 && g == 0) {
        p.ws_ml[2 * slot] = m;
        p.ws_ml[2 * slot + 1] = l;
    }
}

// Ordered merge of the chunk partials: one thread per (row, dim).
__global__ __launch_bounds__(256) void combine_kernel(Params p)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_kv = (int64_t)p.nrows * p.dim;
    if (idx >= per_kv * p.nkv)
        return;
    const int kvl = (int)(idx / per_kv);
    const int64_t rem = idx % per_kv;
    const int row = (int)(rem / p.dim);
    const int d = (int)(rem % p.dim);
    const int kh = p.kh_first + kvl;
    const int query = row / p.group;
    const int h = kh * p.group + row % p.group;
    if (h < p.h_lo || h >= p.h_hi)
        return;
    const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
    const float *ml = p.ws_ml + 2 * slot0;
    const float *wo = p.ws_o + slot0 * p.dk + d;
    float M = kNegInf, L = 0.f, acc = 0.f;
    for (int c = 0; c < p.nch; ++c) {
        const float m = ml[2 * c];
        if (m == kNegInf)
            continue; // a chunk with nothing allowed merges as a no-op
        const float l = ml[2 * c + 1];
        const float o = wo[(int64_t)c * p.dk];
        const MergeFactors f = merge_factors(M, m);
        L = merge_value(L, l, f);
        acc = merge_value(acc, o, f);
        M = f.m;
    }
    const float v = acc / L;
    p.out[(int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim + d] = v;
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
    const int64_t n = (int64_t)p.nkv * p.nrows * p.dim;
    combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(p);
    return hipGetLastError();
}

} // namespace pcl
