// LDS-tiled prefill / canvas attention for gfx950.
//
// One workgroup of NWV waves owns 16*NWV flat (query, head) rows of one KV
// head, 16 rows per wave; Q^T stays in registers as MFMA B operands (NWV = 4
// at head dim 256, one wave per SIMD with the whole register file; 8 below). The K and V
// tiles of 32 keys are staged once per workgroup in double-buffered LDS and
// read by all 8 waves (K rows padded by 16 bytes so the 16 rows of an A
// operand fall in distinct banks). Per tile each wave runs the score chain,
// the online softmax and the P.V chain of the canonical arithmetic
// (attention_device.hpp); at each 256-key chunk boundary it merges the chunk
// into its running (M, L, Acc). Tiles wholly masked for the workgroup are
// never loaded; tiles wholly masked for a wave are skipped by that wave.
//
// split != 0: the workgroup computes the single chunk c_lo + blockIdx.z and
// writes its partial for combine_kernel (used when one pass over the keys
// leaves too few workgroups to fill the chip).
#include "attention_device.hpp"

namespace pcl {

template <int DK> struct TiledShape {
    static constexpr int waves = DK > 128 ? 4 : 8;
    static constexpr int threads = 64 * waves;
    static constexpr int rows = kRows * waves;
};

template <int DK> struct TiledLds {
    static constexpr int KLD = DK + 4;
    static constexpr int kFloats = kTile * KLD;
    static constexpr int vFloats = kTile * DK;
    static constexpr int stage = kFloats + vFloats;
    static constexpr size_t bytes = 2 * stage * sizeof(float);
};

template <int DK>
__global__ __launch_bounds__(TiledShape<DK>::threads) void tiled_kernel(Params p, int split)
{
    using L = TiledLds<DK>;
    constexpr int NT = TiledShape<DK>::threads;
    constexpr int kTiledRows = TiledShape<DK>::rows;
    constexpr int KLD = L::KLD;
    constexpr int NU = DK / 32; // score chain steps
    constexpr int NQ = DK / 64; // 64-dim output groups
    constexpr int NL = kTile * (DK / 4) / NT; // float4 per thread per tile
    extern __shared__ float lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int qb = gridDim.x - 1 - blockIdx.x; // longest causal blocks first
    const int kvl = blockIdx.y;
    const int kh = p.kh_first + kvl;
    const int fa = qb * kTiledRows;
    const int row = fa + w * kRows + col;

    // Key range the workgroup can see.
    int64_t k_lo = 0, k_hi = p.nkeys;
    if (!p.mask && p.causal) {
        const int fb = min(fa + kTiledRows, p.nrows) - 1;
        const int64_t qa = p.first_query + fa / p.group;
        const int64_t qz = p.first_query + fb / p.group;
        k_hi = min(max(qz - p.first_key + 1, (int64_t)0), p.nkeys);
        if (p.window)
            k_lo = min(max(qa - p.window + 1 - p.first_key, (int64_t)0), p.nkeys);
    }
    int t_lo = (int)(k_lo / kTile);
    int t_hi = (int)((k_hi + kTile - 1) / kTile);
    if (split) {
        const int c = p.c_lo + blockIdx.z;
        t_lo = max(t_lo, c * kTilesPerChunk);
        t_hi = min(t_hi, (c + 1) * kTilesPerChunk);
    }

    // Q^T B operands: q[u][jj] = Q[row][32u + 8g + jj] * q_scale.
    float q[NU][8];
    {
        const bool rin = row < p.nrows;
        const int query = rin ? row / p.group : 0;
        const int h = kh * p.group + (rin ? row % p.group : 0);
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int d = 32 * u + 8 * g + 4 * hh;
                f4 v = {0.f, 0.f, 0.f, 0.f};
                if (rin && d < p.dim)
                    v = *(const f4 *)(qp + d) * p.q_scale;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[u][4 * hh + j] = v[j];
            }
    }

    float m = kNegInf, l = 0.f;
    float M = kNegInf, Lsum = 0.f;
    f4 O[NQ][4], Acc[NQ][4];
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
            Acc[a][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
    bool processed = false;
    bool bad = false;

    f4 kr[NL], vr[NL];
    auto load_tile = [&](int t) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (DK / 4);
            const int d = (idx % (DK / 4)) * 4;
            const int64_t kt = (int64_t)t * kTile + key;
            const bool in = kt < p.nkeys && d < p.dim;
            const int64_t ks = in ? kt : 0;
            kr[i] = in ? *(const f4 *)(key_row(p, ks) + (int64_t)kh * p.dim + d)
                       : f4{0.f, 0.f, 0.f, 0.f};
            vr[i] = in ? *(const f4 *)(value_row(p, ks) + (int64_t)kh * p.dim + d)
                       : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store_tile = [&](int buf) {
        float *ks = lds + buf * L::stage;
        float *vs = ks + L::kFloats;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (DK / 4);
            const int d = (idx % (DK / 4)) * 4;
            *(f4 *)(ks + key * KLD + d) = kr[i];
            *(f4 *)(vs + key * DK + d) = vr[i];
        }
    };
    auto merge_chunk = [&]() {
        const MergeFactors f = merge_factors(M, m);
        Lsum = merge_value(Lsum, l, f);
#pragma unroll
        for (int a = 0; a < NQ; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    Acc[a][j][i] = merge_value(Acc[a][j][i], O[a][j][i], f);
        M = f.m;
    };

    if (t_lo < t_hi) {
        load_tile(t_lo);
        store_tile(0);
    }
    __syncthreads();
    for (int t = t_lo; t < t_hi; ++t) {
        const int buf = (t - t_lo) & 1;
        if (t + 1 < t_hi)
            load_tile(t + 1);
        const float *ks = lds + buf * L::stage;
        const float *vs = ks + L::kFloats;

        bool ok[2][4];
        bool any = false;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ok[b][r] = allowed(p, row, (int64_t)t * kTile + 16 * b + 4 * g + r);
                any |= ok[b][r];
            }
        if (__any(any)) {
            f4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const int d = 32 * u + 8 * g;
                f4 ka[2][2];
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        ka[b][hh] = *(const f4 *)(ks + (16 * b + col) * KLD + d + 4 * hh);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        acc[b] = mfma(ka[b][jj >> 2][jj & 3], q[u][jj], acc[b]);
            }
            float s[2][4];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[b][r] = acc[b][r];
            bad |= bad_scores(s, ok);
            const float mn = fmaxf(m, tile_max(s, ok));
            const float ms = safe_max(mn);
            const float alpha = fexp(m - ms);
            float pr[2][4];
            const float rs = tile_probs(s, ok, ms, pr);
            l = __builtin_fmaf(l, alpha, rs);
            m = mn;
#pragma unroll
            for (int a = 0; a < NQ; ++a) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[a][j] = O[a][j] * alpha;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const f4 v = *(const f4 *)(vs + (16 * b + 4 * g + r) * DK + 64 * a +
                                                   4 * col);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            O[a][j] = mfma(v[j], pr[b][r], O[a][j]);
                    }
            }
            processed = true;
        }

        if (t + 1 < t_hi)
            store_tile(buf ^ 1);
        __syncthreads();

        if (!split && (((t + 1) % kTilesPerChunk) == 0 || t + 1 == t_hi)) {
            if (processed) {
                merge_chunk();
                m = kNegInf;
                l = 0.f;
#pragma unroll
                for (int a = 0; a < NQ; ++a)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
                processed = false;
            }
        }
    }
    if (bad)
        atomicOr(p.err, kErrScore);
    if (row >= p.nrows)
        return;

    // O[a][j][i] / Acc[a][j][i] hold dim 64a + 16g + 4i + j of `row`.
    if (split) {
        const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + blockIdx.z;
        float *wo = p.ws_o + slot * p.dk;
#pragma unroll
        for (int a = 0; a < NQ; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 64 * a + 16 * g + 4 * i;
                if (d >= p.dim)
                    continue;
                f4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[j] = O[a][j][i];
                *(f4 *)(wo + d) = v;
            }
        if (g == 0) {
            p.ws_ml[2 * slot] = m;
            p.ws_ml[2 * slot + 1] = l;
        }
        return;
    }
    const int query = row / p.group;
    const int h = kh * p.group + row % p.group;
    if (h < p.h_lo || h >= p.h_hi)
        return;
    float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
    bool nonfinite = false;
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 64 * a + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = Acc[a][j][i] / Lsum;
                nonfinite |= !is_finite(v[j]);
            }
            *(f4 *)(o + d) = v;
        }
    if (nonfinite)
        atomicOr(p.err, kErrOutput);
}

template <int DK> static hipError_t launch_tiled_dk(const Params &p, int split, hipStream_t stream)
{
    static bool configured = false; // dynamic LDS above 64 KiB must be allowed once
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void *)tiled_kernel<DK>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)TiledLds<DK>::bytes);
        if (e != hipSuccess)
            return e;
        configured = true;
    }
    constexpr int rows = TiledShape<DK>::rows;
    const dim3 grid((p.nrows + rows - 1) / rows, p.nkv, split ? p.nch : 1);
    tiled_kernel<DK><<<grid, TiledShape<DK>::threads, TiledLds<DK>::bytes, stream>>>(p, split);
    return hipGetLastError();
}

int tiled_rows(int dk)
{
    return dk > 128 ? TiledShape<256>::rows : TiledShape<128>::rows;
}

hipError_t launch_tiled(const Params &p, int split, hipStream_t stream)
{
    switch (p.dk) {
    case 64: return launch_tiled_dk<64>(p, split, stream);
    case 128: return launch_tiled_dk<128>(p, split, stream);
    case 256: return launch_tiled_dk<256>(p, split, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl
