// Two-pass split-KV decode for gfx950: a K pass, then a V pass.
//
// A decode step streams the attended K and V once each. On MI355X a grid that
// streams only K or only V reaches 6.5-7.0 TB/s, while workgroups that stream
// K and V together reach ~5.2 TB/s, and more loads in flight per wave do not
// help: HBM efficiency here is set by how many distinct rows are being read
// at once. So decode runs as two launches, each a single HBM stream that
// reads whole cache rows:
//
//   score pass  one wave per (256-key chunk, 16-row unit, KV head) streams the
//               chunk's K rows straight into MFMA A operands (a ring of
//               register pieces keeps the next loads in flight behind the
//               current MFMAs), runs the canonical score chain of
//               attention_device.hpp per 16-key block, and stores the raw
//               scores of the unit's real rows in a chunk record, laid out as
//               the MFMA left them;
//   value pass  one workgroup per (chunk, unit, KV head), one wave per 256
//               output dims, reads the scores back in the same layout, runs
//               the canonical per-tile online softmax itself, streams whole V
//               rows through the P.V chain and writes the chunk partial
//               (m, l, O), or the output when the launch has a single chunk.
//
// No step of the canonical arithmetic moves between passes except the raw
// MFMA scores, which are stored and reloaded bit for bit, so the results are
// bitwise those of the one-kernel split-KV decode. The extra traffic is the
// score record: 4 bytes per (key, real row), 0.4 % of the K/V bytes at GQA 2
// and 1.6 % at GQA 8.
#include "attention_device.hpp"

namespace pcl {

// Score record of one (KV head, unit, chunk): [tile][b][lane] f4, the scores
// of keys 32 tile + 16 b + 4 (lane / 16) + 0..3 for row lane % 16.
constexpr int kRecFloats = kTilesPerChunk * 2 * 64 * 4;

int rec_floats()
{
    return kRecFloats;
}

__device__ __forceinline__ float *record(const Params &p, int kvl, int unit, int chunk_local)
{
    return p.ws_rec + (((int64_t)kvl * p.units + unit) * p.nch + chunk_local) * kRecFloats;
}

// Streaming-load hint per head-dim class (measured: the nontemporal hint helps
// the 2 KiB rows of head dim 512 and costs ~20 % on 1 KiB rows).
template <int DK> __device__ __forceinline__ f4 ldg4_kv(const float *p)
{
    if constexpr (DK >= 512)
        return ldg4_stream(p);
    else
        return ldg4(p);
}

// K pieces: PU u-steps (32 dims each) of one 16-key block; RING pieces in
// flight.
template <int DK> struct ScoreCfg {
    static constexpr int NU = DK / 32;
    static constexpr int PU = NU < 4 ? NU : 4;
    static constexpr int PB = NU / PU; // pieces per 16-key block
    static constexpr int RING = 3;
};

template <int DK, bool FULL>
__global__ __launch_bounds__(64) void score_pass_kernel(Params p)
{
    using C = ScoreCfg<DK>;
    constexpr int NU = C::NU, PU = C::PU, PB = C::PB, RING = C::RING;
    constexpr int NP = 16 * PB; // pieces per chunk

    const int lane = threadIdx.x;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int c = p.c_lo + blockIdx.x;
    const int unit = blockIdx.y % p.units;
    const int kvl = blockIdx.y / p.units;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const int real = min(kRows, p.nrows - unit * kRows);
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;
    float *rec = record(p, kvl, unit, blockIdx.x);

    f4 kr[RING][PU][2];
    auto load_piece = [&](int pi, int slot) {
        const int64_t key = cbase + 16 * (pi / PB) + col;
        const float *kp = key_row(p, key < klast ? key : klast) + hoff;
        const int u0 = (pi % PB) * PU;
#pragma unroll
        for (int uu = 0; uu < PU; ++uu)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int d = 32 * (u0 + uu) + 8 * g + 4 * h;
                const bool din = FULL || d < p.dim;
                const f4 x = ldg4_kv<DK>(kp + (din ? d : 0));
                kr[slot][uu][h] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
            }
    };
#pragma unroll
    for (int s = 0; s < RING; ++s)
        load_piece(s, s);

    // Q^T B operands: q[u][jj] = Q[row][32u + 8g + jj] * q_scale (0 for padding).
    float q[NU][8];
    {
        const bool rin = row < p.nrows;
        const int query = rin ? row / p.group : 0;
        const int head = kh * p.group + (rin ? row % p.group : 0);
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)head * p.dim;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int d = 32 * u + 8 * g + 4 * hh;
                const bool din = FULL || d < p.dim;
                const f4 x = ldg4(qp + (din ? d : 0)) * p.q_scale;
                const f4 v = (rin && din) ? x : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[u][4 * hh + j] = v[j];
            }
    }

    // 16-key blocks with an allowed key for some row of the unit, one bit per
    // block (wave-uniform); the others' scores are never read, so their MFMAs
    // are skipped.
    uint32_t live = 0;
    const ChunkKeys ck = chunk_keys(p, row, cbase);
#pragma nounroll
    for (int blk = 0; blk < 16; ++blk) {
        bool ok[4];
        const bool any = block_keys(ck, 16 * blk, g, ok);
        live |= (uint32_t)__any(any) << blk;
    }
    live = __builtin_amdgcn_readfirstlane(live);

    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pi = 0; pi < NP; ++pi) {
        const int slot = pi % RING;
        const int pb = pi % PB;
        const int blk = pi / PB; // 16-key block of the chunk: tile blk / 2, b = blk % 2
        if (pb == 0)
            acc = f4{0.f, 0.f, 0.f, 0.f};
        __builtin_amdgcn_sched_barrier(0);
        if ((live >> blk) & 1) {
#pragma unroll
            for (int uu = 0; uu < PU; ++uu)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
                    acc = mfma(kr[slot][uu][jj >> 2][jj & 3], q[pb * PU + uu][jj], acc);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (pi + RING < NP)
            load_piece(pi + RING, slot); // the slot's registers are free again
        if (pb == PB - 1 && col < real)
            stg4(rec + (blk * 64 + lane) * 4, acc);
    }
}

// Output modes of the value pass.
enum ValueMode { kValueDirect = 0, kValuePartial = 1 };

// Waves per value-pass workgroup: one per 256 output dims.
template <int DK> constexpr int value_waves()
{
    return DK > 256 ? DK / 256 : 1;
}

template <int DK, int MODE>
__global__ __launch_bounds__(64 * value_waves<DK>()) void value_pass_kernel(Params p)
{
    constexpr int NQ = DK > 256 ? 4 : DK / 64; // 64-dim output groups per wave
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int d0 = 256 * (threadIdx.x >> 6); // the wave's first output dim
    const int c = p.c_lo + blockIdx.x;
    const int unit = blockIdx.y % p.units;
    const int kvl = blockIdx.y / p.units;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const int real = min(kRows, p.nrows - unit * kRows);
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;
    const float *rec = record(p, kvl, unit, blockIdx.x);

    // V of one 16-key half tile: vv[r][a] = V[key 16b + 4g + r][d0 + 64a + 4col ..].
    f4 vv[4][NQ];
    auto load_half = [&](int hi) {
        const int t = hi >> 1, b = hi & 1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t key = cbase + t * kTile + 16 * b + 4 * g + r;
            const float *vp = value_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
            for (int a = 0; a < NQ; ++a) {
                const int d = d0 + 64 * a + 4 * col;
                const bool din = d < p.dim;
                const f4 x = ldg4_stream(vp + (din ? d : 0));
                vv[r][a] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    load_half(0);
    // The chunk's scores (every block's record is written by the score pass).
    f4 sv[kTilesPerChunk][2];
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t)
#pragma unroll
        for (int b = 0; b < 2; ++b)
            sv[t][b] = ldg4(rec + ((t * 2 + b) * 64 + (col < real ? lane : 0)) * 4);

    float m = kNegInf, l = 0.f;
    bool bad = false;
    f4 O[NQ][4];
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
    const ChunkKeys ck = chunk_keys(p, row, cbase);
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        bool ok[2][4];
        const bool any = tile_keys(ck, t, g, ok);
        const bool tile_any = __any(any);
        float pr[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float alpha, rs = 0.f;
        if (tile_any) {
            float sc[2][4];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sc[b][r] = col < real ? sv[t][b][r] : 0.f;
            cap_scores(p, sc);
            bad |= bad_scores(sc, ok);
            const float mn = fmaxf(m, tile_max(sc, ok));
            const float ms = safe_max(mn);
            alpha = fexp(m - ms);
            rs = tile_probs(sc, ok, ms, pr);
            m = mn;
        } else {
            // nothing allowed for the unit: alpha = exp(m - safe(m)), rs = 0
            alpha = fexp(m - safe_max(m));
        }
        l = __builtin_fmaf(l, alpha, rs);
        if (tile_any) {
#pragma unroll
            for (int a = 0; a < NQ; ++a)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[a][j] = O[a][j] * alpha;
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int hi = 2 * t + b;
            __builtin_amdgcn_sched_barrier(0);
            if (tile_any) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int a = 0; a < NQ; ++a)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            O[a][j] = mfma(vv[r][a][j], pr[b][r], O[a][j]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (hi + 1 < 2 * kTilesPerChunk)
                load_half(hi + 1);
        }
    }
    if (bad && d0 == 0)
        atomicOr(p.err, kErrScore);

    // O[a][j][i] is dim d0 + 64a + 16g + 4i + j of row `row`.
    if (row >= p.nrows)
        return;
    if (MODE == kValueDirect) {
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
                const int d = d0 + 64 * a + 16 * g + 4 * i;
                if (d >= p.dim)
                    continue;
                f4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[j] = O[a][j][i] / l;
                    nonfinite |= !is_finite(v[j]);
                }
                stg4(o + d, v);
            }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }
    const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + blockIdx.x;
    float *wo = p.ws_o + slot * p.dk;
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = d0 + 64 * a + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[j] = O[a][j][i];
            stg4(wo + d, v);
        }
    if (d0 == 0 && g == 0) {
        stg(p.ws_ml + 2 * slot, m);
        stg(p.ws_ml + 2 * slot + 1, l);
    }
}

template <int DK> static hipError_t launch_dk(const Params &p, hipStream_t stream)
{
    const dim3 grid(p.nch, p.nkv * p.units);
    if (p.dim == DK)
        score_pass_kernel<DK, true><<<grid, 64, 0, stream>>>(p);
    else
        score_pass_kernel<DK, false><<<grid, 64, 0, stream>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    const int threads = 64 * value_waves<DK>();
    if (p.ws_o)
        value_pass_kernel<DK, kValuePartial><<<grid, threads, 0, stream>>>(p);
    else
        value_pass_kernel<DK, kValueDirect><<<grid, threads, 0, stream>>>(p);
    return hipGetLastError();
}

// Score pass, then value pass (chunk partials when ws_o is set, else the
// output of the single chunk).
hipError_t launch_two_pass(const Params &p, hipStream_t stream)
{
    switch (p.dk) {
    case 64: return launch_dk<64>(p, stream);
    case 128: return launch_dk<128>(p, stream);
    case 256: return launch_dk<256>(p, stream);
    case 512: return launch_dk<512>(p, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl
