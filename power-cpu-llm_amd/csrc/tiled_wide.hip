// LDS-tiled prefill / canvas attention at head dim 512 for gfx950.
//
// At head dim 512 one 16-row unit's Q^T (MFMA B operands) and its output
// state O are 128 floats per lane each, more than a wave can hold next to
// its operands. So each unit is worked by a pair of waves that split the
// head dim: wave half h (h = 0, 1) holds Q^T and O for dims
// [256h, 256h + 256). A tile's score chains run across the pair in the
// canonical order (attention_device.hpp): half 0 runs u = 0..7 of both 16-key
// blocks and leaves the two accumulators in LDS, half 1 continues them over
// u = 8..15 (an MFMA takes its accumulator as an operand, so the chain is
// the same chain) and leaves the raw scores in LDS. Both waves then run the
// tile's online softmax (the same values, bit for bit) and the P.V chain of
// their own dims.
//
// One workgroup of 8 waves owns 64 flat (query, head) rows of one KV head
// (4 units; on each SIMD one half-0 and one half-1 wave, so the halves'
// score phases alternate on the MFMA pipe). K and V tiles of 32 keys (64 KiB
// each) are copied HBM -> LDS by global_load_lds_dwordx4, single-buffered:
// a tile's K is needed only until the score chains finish, so the next K is
// requested while the P.V chains run, and the next V while the next scores
// run. K rows are stored with their 16-byte chunks XOR-swizzled by (key & 7)
// as in the other tiled kernel.
//
// The chunk, span and total merges, split launches and masks follow the
// other tiled kernel (tiled.hip); each wave merges its own dims.
#include "attention_device.hpp"

#include <atomic>

namespace pcl {

constexpr int kWideDk = 512;
constexpr int kWideUnits = 4;
constexpr int kWideWaves = 2 * kWideUnits;
constexpr int kWideRows = kWideUnits * kRows; // 64
constexpr int kWideTileFloats = kTile * kWideDk;
// K tile, V tile, half 0's partial score accumulators and half 1's scores
// ([unit][block][lane] f4 each)
constexpr int kWideLdsFloats = 2 * kWideTileFloats + 2 * kWideUnits * 2 * 64 * 4;
constexpr size_t kWideLdsBytes = kWideLdsFloats * sizeof(float);

typedef __attribute__((address_space(3))) void *wide_lds_t;
typedef const __attribute__((address_space(1))) void *wide_gbl_t;

__device__ __forceinline__ void wide_dma16(const float *g, float *l)
{
    __builtin_amdgcn_global_load_lds((wide_gbl_t)g, (wide_lds_t)l, 16, 0, 0);
}

// True when every row in [row_lo, row_hi] may attend every key of tile t.
__device__ __forceinline__ bool wide_tile_whole(const Params &p, int row_lo, int row_hi, int t)
{
    if (p.mask || row_lo > row_hi)
        return false;
    const int64_t k0 = (int64_t)t * kTile;
    if (k0 + kTile > p.nkeys)
        return false;
    if (!p.causal)
        return true;
    const int64_t kmin = p.first_key + k0;
    const int64_t kmax = kmin + kTile - 1;
    const int64_t qlo = p.first_query + row_lo / p.group;
    const int64_t qhi = p.first_query + row_hi / p.group;
    return kmax <= qlo && (p.window == 0 || qhi - kmin < p.window);
}

template <bool CAP>
__global__ __launch_bounds__(64 * kWideWaves, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_wide_kernel(Params p, int split, int z0)
{
    constexpr int NU = 8; // score chain steps per half
    constexpr int NQ = 4; // 64-dim output groups per half
    constexpr int NI = kWideTileFloats / 256 / kWideWaves; // 1 KiB DMA pieces per wave per array
    extern __shared__ float lds[];
    float *ks = lds;
    float *vs = lds + kWideTileFloats;
    f4 *part = reinterpret_cast<f4 *>(lds + 2 * kWideTileFloats); // [unit][b][lane]
    f4 *fin = part + kWideUnits * 2 * 64;                          // [unit][b][lane]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int unit = wv % kWideUnits;
    const int half = wv / kWideUnits;
    const int col = lane & 15;
    const int g = lane >> 4;
    // blocks cycle over the KV heads first; query blocks run last-to-first
    const int nqb = gridDim.x / p.nkv;
    const int kvl = blockIdx.x % p.nkv;
    const int qb = nqb - 1 - (int)(blockIdx.x / p.nkv);
    const int kh = p.kh_first + kvl;
    const int fa = qb * kWideRows;
    const int row = fa + unit * kRows + col;
    const int wrow_lo = fa + unit * kRows;
    const int wrow_hi = min(wrow_lo + kRows, p.nrows) - 1;
    const bool rin = row < p.nrows;
    const int query = rin ? row / p.group : 0;
    const int head = kh * p.group + (rin ? row % p.group : 0);
    const bool rout = rin && head >= p.h_lo && head < p.h_hi;
    const int dh = 256 * half; // this wave's first dim

    const RowKeys rk = row_keys(p, row);
    int64_t k_lo = 0, k_hi = p.nkeys;
    if (!p.mask && p.causal) {
        const int fb = min(fa + kWideRows, p.nrows) - 1;
        const int64_t qa = p.first_query + fa / p.group;
        const int64_t qz = p.first_query + fb / p.group;
        k_hi = min(max(qz - p.first_key + 1, (int64_t)0), p.nkeys);
        if (p.window)
            k_lo = min(max(qa - p.window + 1 - p.first_key, (int64_t)0), p.nkeys);
    }
    int t_lo = (int)(k_lo / kTile);
    int t_hi = (int)((k_hi + kTile - 1) / kTile);
    if (split) {
        const int c = p.c_lo + z0 + (int)blockIdx.z;
        t_lo = max(t_lo, c * kTilesPerChunk);
        t_hi = min(t_hi, (c + 1) * kTilesPerChunk);
    }

    // Q^T B operands of this half: q[u][jj] = Q[row][dh + 32u + 8g + jj] * q_scale.
    float q[NU][8];
    {
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)head * p.dim;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int d = dh + 32 * u + 8 * g + 4 * hh;
                const f4 x = ldg4(qp + (d < p.dim ? d : 0)) * p.q_scale;
                const f4 v = (rin && d < p.dim) ? x : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[u][4 * hh + j] = v[j];
            }
    }

    float m = kNegInf, l = 0.f, M1 = kNegInf, L1 = 0.f, M2 = kNegInf, L2 = 0.f;
    f4 O[NQ][4];
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
    bool processed = false;
    bool bad = false;
    float *acc1 = p.out + (int64_t)query * p.o_stride + (int64_t)(head - p.h_base) * p.dim;
    float *acc2 = p.ws_o ? p.ws_o + ((int64_t)kvl * p.nrows_pad + row) * p.dk : nullptr;

    // HBM -> LDS copies of tile t's K (swizzled) or V (plain). A slot past
    // the head's last dim copies the head's first four dims (Q is zero there
    // and those outputs are dropped), so no copy leaves the head's row.
    auto load_k = [&](int t) {
        const int64_t klast = p.nkeys - 1;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = wv * NI + i;
            const int f = 256 * j + 4 * lane;
            const int key = f / kWideDk;
            const int pos = (f % kWideDk) / 4;
            const int64_t kt = (int64_t)t * kTile + key;
            const int64_t kc = kt < klast ? kt : klast;
            const int kd = 4 * (pos ^ (key & 7));
            wide_dma16(key_row(p, kc) + (int64_t)kh * p.dim + (kd < p.dim ? kd : 0), ks + 256 * j);
        }
    };
    auto load_v = [&](int t) {
        const int64_t klast = p.nkeys - 1;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = wv * NI + i;
            const int f = 256 * j + 4 * lane;
            const int key = f / kWideDk;
            const int vd = f % kWideDk;
            const int64_t kt = (int64_t)t * kTile + key;
            const int64_t kc = kt < klast ? kt : klast;
            wide_dma16(value_row(p, kc) + (int64_t)kh * p.dim + (vd < p.dim ? vd : 0),
                       vs + 256 * j);
        }
    };

    // Where the span accumulator (the row's output slot until the last
    // merge) and the running total keep natural dims dh + 64a + 16g + 4i ..:
    // in a whole 64-dim block the 16-byte slots are stored with g and i
    // swapped, so the four lanes of a row in one load or store cover one
    // contiguous 64-byte sector; a partial last block keeps the natural order.
    auto acc_pos = [&](int a, int i) {
        return dh + 64 * a + 64 <= p.dim ? dh + 64 * a + 16 * i + 4 * g
                                         : dh + 64 * a + 16 * g + 4 * i;
    };

    // Chunk merge into the span, and at a span end the span merge into the
    // total (this wave's dims; not the last merge: flush_last below).
    auto flush = [&](bool chunk, bool span_end) {
        float *a1 = acc1, *a2 = acc2;
        asm volatile("" : "+v"(a1), "+v"(a2));
        const bool first1 = M1 == kNegInf;
        MergeFactors f1 = {M1, 1.f, 0.f};
        if (chunk) {
            f1 = merge_factors(M1, m);
            L1 = merge_value(L1, l, f1);
            M1 = f1.m;
        }
        const bool add2 = span_end && M1 != kNegInf;
        const bool first2 = M2 == kNegInf;
        MergeFactors f2 = {M2, 1.f, 0.f};
        if (add2) {
            f2 = merge_factors(M2, M1);
            L2 = merge_value(L2, L1, f2);
            M2 = f2.m;
        }
        if (rout) {
#pragma unroll
            for (int a = 0; a < NQ; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (dh + 64 * a + 16 * g + 4 * i >= p.dim)
                        continue;
                    const int dm = acc_pos(a, i);
                    f4 s1 = f4{0.f, 0.f, 0.f, 0.f};
                    if (!first1)
                        s1 = ldg4(a1 + dm);
                    if (chunk) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            s1[j] = merge_value(s1[j], O[a][j][i], f1);
                    }
                    if (!span_end) {
                        stg4(a1 + dm, s1);
                        continue;
                    }
                    f4 s2 = f4{0.f, 0.f, 0.f, 0.f};
                    if (!first2)
                        s2 = ldg4(a2 + dm);
                    if (add2) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            s2[j] = merge_value(s2[j], s1[j], f2);
                    }
                    stg4(a2 + dm, s2);
                }
        }
        if (chunk) {
            m = kNegInf;
            l = 0.f;
#pragma unroll
            for (int a = 0; a < NQ; ++a)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        if (span_end) {
            M1 = kNegInf;
            L1 = 0.f;
        }
    };

    // The last merge, normalised into the output (this wave's dims). The
    // output's natural order overwrites the span accumulator's slots in
    // another order, so every accumulator value is loaded first (after the
    // tiles: Q^T's registers are free).
    auto flush_last = [&](bool chunk) {
        float *a1 = acc1, *a2 = acc2;
        asm volatile("" : "+v"(a1), "+v"(a2));
        const bool first1 = M1 == kNegInf;
        MergeFactors f1 = {M1, 1.f, 0.f};
        if (chunk) {
            f1 = merge_factors(M1, m);
            L1 = merge_value(L1, l, f1);
            M1 = f1.m;
        }
        const bool add2 = M1 != kNegInf;
        const bool first2 = M2 == kNegInf;
        MergeFactors f2 = {M2, 1.f, 0.f};
        if (add2) {
            f2 = merge_factors(M2, M1);
            L2 = merge_value(L2, L1, f2);
            M2 = f2.m;
        }
        if (!rout)
            return;
        f4 s1v[NQ][4];
#pragma unroll
        for (int a = 0; a < NQ; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s1v[a][i] = f4{0.f, 0.f, 0.f, 0.f};
                if (!first1 && dh + 64 * a + 16 * g + 4 * i < p.dim)
                    s1v[a][i] = ldg4(a1 + acc_pos(a, i));
            }
        // Write-after-read across lanes: lane (g, i)'s slot 64a + 16i + 4g is
        // where the lane with g' = i stores dims 64a + 16g' + 4i' below, so
        // every load above must complete before the first store. The wait
        // (and its memory clobber, which keeps the compiler from sinking a
        // load past a store it cannot prove disjoint) orders them.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bool nonfinite = false;
#pragma unroll
        for (int a = 0; a < NQ; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = dh + 64 * a + 16 * g + 4 * i;
                if (d >= p.dim)
                    continue;
                f4 s1 = s1v[a][i];
                if (chunk) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        s1[j] = merge_value(s1[j], O[a][j][i], f1);
                }
                f4 s2 = f4{0.f, 0.f, 0.f, 0.f};
                if (!first2)
                    s2 = ldg4(a2 + acc_pos(a, i));
                if (add2) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        s2[j] = merge_value(s2[j], s1[j], f2);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s2[j] = s2[j] / L2;
                    nonfinite |= !is_finite(s2[j]);
                }
                stg4(a1 + d, s2);
            }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
    };

    // This half's part of tile t's two score chains: half 0 runs u = 0..7
    // from zero accumulators, half 1 continues over u = 8..15 from half 0's
    // accumulators in LDS; the results go to `to`.
    auto chains = [&](const f4 *from, f4 *to) {
        f4 acc[2];
        acc[0] = from ? from[lane] : f4{0.f, 0.f, 0.f, 0.f};
        acc[1] = from ? from[64 + lane] : f4{0.f, 0.f, 0.f, 0.f};
        f4 ka[2][2][2]; // [u parity][b][hh]
        const float *kh0 = ks + col * kWideDk;
        auto read_k = [&](int u, int sl) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int c4 = 64 * half + 8 * u + 2 * g + hh;
                    ka[sl][b][hh] = *(const f4 *)(kh0 + 16 * b * kWideDk + 4 * (c4 ^ (col & 7)));
                }
        };
        read_k(0, 0);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (u + 1 < NU)
                read_k(u + 1, (u + 1) & 1);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[b] = mfma(ka[u & 1][b][jj >> 2][jj & 3], q[u][jj], acc[b]);
        }
        to[lane] = acc[0];
        to[64 + lane] = acc[1];
    };

    if (t_lo < t_hi) {
        load_k(t_lo);
        load_v(t_lo);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    for (int t = t_lo; t < t_hi; ++t) {
        // masks (both halves of a unit derive the same ones)
        bool ok[2][4];
        bool any = false;
        if (wide_tile_whole(p, wrow_lo, wrow_hi, t)) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ok[b][r] = true;
            any = true;
        } else {
            any = tile_keys(chunk_of(rk, (int64_t)t * kTile), 0, g, ok);
        }
        const bool tile_any = __any(any);
        f4 *upart = part + unit * 2 * 64;
        f4 *ufin = fin + unit * 2 * 64;

        // scores: half 0, then half 1 from half 0's accumulators (#A: the
        // partial accumulators in LDS; #B: the scores in LDS, this tile's V
        // landed (each wave waits for its own copies, the barrier for
        // everyone's), K free)
#pragma unroll 1
        for (int phase = 0; phase < 2; ++phase) {
            if (phase == half && tile_any)
                chains(phase ? upart : nullptr, phase ? ufin : upart);
            if (phase == 1)
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        if (t + 1 < t_hi)
            load_k(t + 1);

        if (tile_any) {
            float s[2][4], pr[2][4];
            const f4 s0 = ufin[lane], s1 = ufin[64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[0][r] = s0[r];
                s[1][r] = s1[r];
            }
            cap_scores<CAP>(p, s);
            if (half == 0)
                bad |= bad_scores(s, ok);
            const float mn = fmaxf(m, tile_max(s, ok));
            const float ms = safe_max(mn);
            const float alpha = fexp(m - ms);
            const float rs = tile_probs(s, ok, ms, pr);
            l = __builtin_fmaf(l, alpha, rs);
            m = mn;
            f4 vb[2][4];
            auto read_v = [&](int hg, int sl) { // half-group hg = 2a + b
                const int a = hg >> 1, b = hg & 1;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    vb[sl][r] = *(const f4 *)(vs + (16 * b + 4 * g + r) * kWideDk + dh + 64 * a +
                                              4 * col);
            };
            read_v(0, 0);
#pragma unroll
            for (int hg = 0; hg < 2 * NQ; ++hg) {
                const int a = hg >> 1, b = hg & 1;
                if (hg + 1 < 2 * NQ)
                    read_v(hg + 1, (hg + 1) & 1);
                if (b == 0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        O[a][j] = O[a][j] * alpha;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        O[a][j] = mfma(vb[hg & 1][r][j], pr[b][r], O[a][j]);
            }
            processed = true;
        }

        if (!split && t + 1 < t_hi) { // (the last tile's merge follows the loop)
            const bool chunk_end = ((t + 1) % kTilesPerChunk) == 0;
            const bool span_end = ((t + 1) % kSpanTiles) == 0;
            if ((chunk_end && processed) || span_end)
                flush(chunk_end && processed, span_end);
            if (chunk_end)
                processed = false;
        }
        // the next K has landed; V free for the next tile
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads(); // #C
        if (t + 1 < t_hi)
            load_v(t + 1);
    }
    if (bad)
        atomicOr(p.err, kErrScore);
    if (!split) {
        // with no key at all: 0/0, flagged like any non-finite output
        flush_last(t_lo < t_hi && processed);
        return;
    }

    // O[a][j][i] holds dim dh + 64a + 16g + 4i + j of `row`.
    if (!rin)
        return;
    const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + z0 + blockIdx.z;
    float *wo = p.ws_o + slot * p.dk;
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = dh + 64 * a + 16 * g + 4 * i;
            if (d >= p.dim)
                continue;
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[j] = O[a][j][i];
            stg4(wo + d, v);
        }
    if (half == 0 && g == 0) {
        stg(p.ws_ml + 2 * slot, m);
        stg(p.ws_ml + 2 * slot + 1, l);
    }
}

constexpr int kWideMaxDevices = 64;


template <bool CAP>
static hipError_t launch_wide(const Params &p, int split, dim3 grid, hipStream_t stream)
{
    static std::atomic<bool> configured[kWideMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= kWideMaxDevices)
        return hipErrorInvalidDevice;
    if (!configured[dev].load(std::memory_order_acquire)) {
        e = hipFuncSetAttribute((const void *)tiled_wide_kernel<CAP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWideLdsBytes);
        if (e != hipSuccess)
            return e;
        configured[dev].store(true, std::memory_order_release);
    }
    tiled_wide_kernel<CAP><<<grid, 64 * kWideWaves, kWideLdsBytes, stream>>>(p, split, 0);
    return hipGetLastError();
}

int device_cus();
int tiled_tail_chunks(const Params &p, int nqb, int cus);
hipError_t launch_fan_chunk(const Params &p, int ci, bool merge_out, hipStream_t stream);

// A split launch whose chunk items leave a small last round runs that
// round's chunk as fanned (16-row unit, chunk) items (fan_kv.hip), as the
// other tiled kernel does; with all chunks in one span that tail also
// merges every chunk partial into the output (*merged: no combine needed).
hipError_t launch_tiled_wide(const Params &p, int split, hipStream_t stream, bool *merged)
{
    const int nqb = (p.nrows + kWideRows - 1) / kWideRows;
    const int tail = split ? tiled_tail_chunks(p, nqb, device_cus()) : 0;
    const dim3 grid(nqb * p.nkv, 1, split ? p.nch - tail : 1);
    hipError_t e = p.softcap > 0.0f ? launch_wide<true>(p, split, grid, stream)
                                    : launch_wide<false>(p, split, grid, stream);
    if (e != hipSuccess || !tail)
        return e;
    const bool merge_out = p.nspan == 1;
    e = launch_fan_chunk(p, p.nch - 1, merge_out, stream);
    if (e == hipSuccess && merge_out)
        *merged = true;
    return e;
}

int tiled_wide_rows()
{
    return kWideRows;
}

} // namespace pcl
