// Pipelined split-KV decode for gfx950: score waves and value waves per
// (256-key chunk, 16-row unit, KV head).
//
// The narrow layout (head dims 64 and 256 in long launches): one score wave
// and one value wave. The score wave streams K, runs the canonical score
// chain and online softmax of each tile (attention_device.hpp) and hands the
// tile's probabilities, alpha and row sum to the value wave through a
// double-buffered LDS slot. The value wave streams V and runs the P.V chain
// one tile behind. One barrier per tile keeps the workgroup in step; at head
// dim 256 the score and value waves' MFMA work is balanced (128 MFMAs each
// per tile). The wide layout (head dim 512; 128; 256 in short launches): two
// score waves sharing Q^T in LDS and two value waves splitting the output
// dims (pipe_dual below).
//
// In the narrow layout each wave keeps exactly one 16-key block of K or V in
// flight, loading the next block into the same registers as its MFMAs
// consume them: each 32-dim K slice (each 4-key V slice) is reloaded right
// after the MFMAs that read it, so a block's MFMA time overlaps the next
// block's memory latency (issuing the whole next block only after the last
// MFMA cost ~10 % at 32K). The wide layout reloads whole pieces after the
// MFMAs (early reloads there cost 9-40 %). At head dim 512 each wave holds
// 8 KiB (16 keys x 128 dims of K, 8 keys x 256 dims of V): at 127 VGPRs four
// workgroups share a CU, so a 128K decode's 1024 workgroups are all resident
// (3.5 % faster than 16 KiB pieces at three per CU, which left a third
// round).
template <int DK, bool WIDE> constexpr bool pipe_slice_loads();
// Measured on MI355X with inputs larger than the last-level cache, one block
// in flight per wave streams at the HBM limit (~6.9 TB/s for a pure K+V read)
// even with a microsecond of compute between loads, while two blocks in
// flight drop to ~6.0 TB/s and three to ~4.5 TB/s: more outstanding requests
// only thrash the DRAM row buffers.
//
// Output: for a launch of a single chunk, the output itself; otherwise the
// chunk partial (m, l, O) for the combine kernel (split_kv.hip).
#include "attention_device.hpp"
#include "step_prologue.hpp"

namespace pcl {

// The wide layout: two score waves (one per 16-key block of each tile; the
// second runs a tile ahead and hands its raw scores to the first, which owns
// the softmax, through LDS, where both read Q^T) and two value waves (half
// the output dims each). Always above head dim 256, where a tile's K is as
// many bytes as its V; at 128 always and at 256 for launches of few
// workgroups (WIDE), which are bound by each wave's chain of memory round
// trips: a chunk then takes 8 round trips per wave instead of 16.
template <int DK, bool WIDE> constexpr bool pipe_dual()
{
    return DK > 256 || WIDE;
}

template <int DK, bool WIDE> constexpr int pipe_score_waves()
{
    return pipe_dual<DK, WIDE>() ? 2 : 1;
}

template <int DK, bool WIDE> constexpr int pipe_value_waves()
{
    return pipe_dual<DK, WIDE>() ? 2 : 1;
}

// Output dims of a value wave (whole 64-dim groups).
template <int DK, bool WIDE> constexpr int pipe_value_dims()
{
    return DK / pipe_value_waves<DK, WIDE>();
}

// V slices (4 keys x the wave's dims each) a value wave keeps in flight: a
// 16-key block in the narrow layout; a whole tile in the wide layout up to
// head dim 256 (16 KiB at 256); half a block at 512, where a workgroup holds
// 8 KiB per wave so that four workgroups fit on a CU.
template <int DK, bool WIDE> constexpr int pipe_v_slices()
{
    return DK > 256 ? 2 : pipe_dual<DK, WIDE>() ? 8 : 4;
}

// Dims of the K piece a score wave keeps in flight: the whole 16-key block up
// to head dim 256; 128 dims (8 KiB; four pieces per block) at 512.
template <int DK> constexpr int pipe_k_piece_dims()
{
    return DK > 256 ? 128 : DK;
}

// The wide layout keeps Q^T in LDS (the score waves' registers hold the K
// block in flight); padded rows avoid bank conflicts.
template <int DK, bool WIDE> constexpr bool pipe_q_lds()
{
    return pipe_dual<DK, WIDE>();
}

// The narrow layout reloads each slice right after its MFMAs (see above).
template <int DK, bool WIDE> constexpr bool pipe_slice_loads()
{
    return !pipe_dual<DK, WIDE>();
}

// LDS hand-over between the score wave and the value waves.
// 16-byte aligned, with q and sb at 16-byte offsets: their 16-byte reads
// and writes stay single ds_read_b128 / ds_write_b128 instructions (at
// 4-byte alignment each one split into two ds_read2_b32).
// With a one-token step's head transform folded in (STEP), the narrow
// layout's score wave prepares its unit's query rows in q as well, and the
// new key's K and V rows are prepared through `row` there (the score wave
// may be in its first tile meanwhile) and through sb and p in the wide
// layout (free until its prologue barriers).
template <int DK, bool WIDE, bool STEP> struct __attribute__((aligned(16))) PipeLds {
    float p[2][8][64];    // probabilities, [slot][4b + r][lane]
    float alpha[2][kRows];
    float rs[2][kRows];
    float m[kRows];       // chunk maximum
    float q[pipe_q_lds<DK, WIDE>() || STEP ? kRows * (DK + 4) : 4];
    float row[STEP && !pipe_dual<DK, WIDE>() ? DK : 4];
    // raw scores of a tile's second 16-key block from the second score
    // wave, [tile & 1][r][lane]
    float sb[pipe_score_waves<DK, WIDE>() > 1 ? 2 : 1][4][64];
    int any[2];
};

// With a one-token step's transform folded in: whether chunk c holds the
// step's new key (the launch's last key) among its first `keys` keys, so
// that its first K or V requests would read that key's row (directly, or
// as the clamped row of a padding key) before it is written.
__device__ __forceinline__ bool step_row_wait(const Params &p, int c, int keys)
{
    const int64_t cbase = (int64_t)c * kChunk;
    return cbase + kChunk >= p.nkeys && p.nkeys - 1 < cbase + keys;
}

template <int DK, bool FULL, bool STEP>
__device__ __forceinline__ void score_wave(const Params &p, int unit, int kvl, int c, int ci,
                                           PipeLds<DK, false, STEP> &s)
{
    static_assert(!pipe_dual<DK, false>(), "head dims above 256 take the two score waves");
    constexpr int NU = DK / 32; // score chain steps
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;

    // The K piece in flight: a whole 16-key block (16 keys x DK dims).
    constexpr int PD = DK;
    constexpr int PU = PD / 32; // u-steps per piece
    constexpr int PB = DK / PD; // pieces per 16-key block
    f4 kb[PU][2];
    auto load_k_u = [&](int t, int b, int pc, int uu) {
        const int64_t key = cbase + t * kTile + 16 * b + col;
        const float *kp = key_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int d = 32 * (pc * PU + uu) + 8 * g + 4 * h;
            const bool din = FULL || d < p.dim;
            const f4 x = ldg4_stream(kp + (din ? d : 0));
            kb[uu][h] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // slice uu of the piece after (t, b, pc), if any
    auto load_next_u = [&](int t, int b, int pc, int uu) {
        if (pc + 1 < PB)
            load_k_u(t, b, pc + 1, uu);
        else if (b == 0)
            load_k_u(t, 1, 0, uu);
        else if (t + 1 < kTilesPerChunk)
            load_k_u(t + 1, 0, 0, uu);
    };
    auto load_k = [&](int t, int b, int pc) {
        const int64_t key = cbase + t * kTile + 16 * b + col;
        const float *kp = key_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
        for (int uu = 0; uu < PU; ++uu)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int d = 32 * (pc * PU + uu) + 8 * g + 4 * h;
                const bool din = FULL || d < p.dim;
                const f4 x = ldg4_stream(kp + (din ? d : 0));
                kb[uu][h] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
            }
    };
    // Q^T B operands: Q[row][32u + 8g + jj] * q_scale (0 for padding rows).
    float q[NU][8];
    if constexpr (STEP) {
        // The step's query rows, prepared here while the first K block is
        // in flight. The step's new key (the launch's last) is written into
        // the cache by the value wave of its chunk before that wave's first
        // barrier (tile 0 handed over); the K blocks requested before this
        // wave reaches it, (0,0), (0,1) and (1,0), hold the chunk's first 48
        // keys, so only a chunk whose new key is among those (a block past
        // the key reads the key's row: clamped) waits for the row first
        // (#S), and the others stream from the start.
        const bool wait = step_row_wait(p, c, 48);
        StepQueryRows<DK> sqr;
        sqr.issue(p, unit, kh);
        if (!wait)
            load_k(0, 0, 0);
        if (sqr.finish(p, unit, kh, s.q, DK + 4, ci == 0 && p.sqo))
            atomicOr(p.err, kErrTransform);
        if (wait) {
            __syncthreads(); // #S: the new key's rows written
            load_k(0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const f4 v = *(const f4 *)(s.q + col * (DK + 4) + 32 * u + 8 * g + 4 * hh);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[u][4 * hh + j] = v[j];
            }
    } else {
        const bool rin = row < p.nrows;
        const int query = rin ? row / p.group : 0;
        const int h = kh * p.group + (rin ? row % p.group : 0);
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim;
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
        load_k(0, 0, 0);
    }
    const ChunkKeys ck = chunk_keys(p, row, cbase);
    float m = kNegInf;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        bool ok[2][4];
        const bool any = tile_keys(ck, t, g, ok);
        const bool tile_any = __any(any);
        f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int pc = 0; pc < PB; ++pc) {
                __builtin_amdgcn_sched_barrier(0);
                if (tile_any) {
#pragma unroll
                    for (int uu = 0; uu < PU; ++uu) {
                        const int u = pc * PU + uu;
#pragma unroll
                        for (int jj = 0; jj < 8; ++jj)
                            acc[b] = mfma(kb[uu][jj >> 2][jj & 3], q[u][jj], acc[b]);
                        if constexpr (pipe_slice_loads<DK, false>()) {
                            // this slice's registers are consumed: the next piece's slice
                            __builtin_amdgcn_sched_barrier(0);
                            load_next_u(t, b, pc, uu);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (!tile_any || !pipe_slice_loads<DK, false>()) { // the whole next piece at once
                    if (pc + 1 < PB)
                        load_k(t, b, pc + 1);
                    else if (b == 0)
                        load_k(t, 1, 0);
                    else if (t + 1 < kTilesPerChunk)
                        load_k(t + 1, 0, 0);
                }
            }
        float pr[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float alpha = 1.f, rs = 0.f;
        if (tile_any) {
            float sc[2][4];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sc[b][r] = acc[b][r];
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
        const int slot = t & 1;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s.p[slot][4 * b + r][lane] = pr[b][r];
        if (g == 0) {
            s.alpha[slot][col] = alpha;
            s.rs[slot][col] = rs;
        }
        if (lane == 0)
            s.any[slot] = tile_any;
        __syncthreads(); // tile t handed over
    }
    if (g == 0)
        s.m[col] = m;
    if (bad)
        atomicOr(p.err, kErrScore);
    __syncthreads(); // chunk maximum handed over
}

// The two score waves of head dims above 256. ROLE 0 scores the first 16-key
// block of every tile and runs the tile's softmax; ROLE 1 scores the second
// block one tile ahead and leaves its raw scores in s.sb. Each block's score
// chain is the canonical one, so the results equal the one-wave kernel's.
// Barriers (the value waves keep the same count): #Q after Q^T is staged,
// #0 after the second wave's tile-0 scores, #t+1 after tile t is handed over,
// and one after the chunk maximum.
template <int DK, bool FULL, int ROLE, bool WIDE, bool STEP>
__device__ __forceinline__ void score_wave_dual(const Params &p, int unit, int kvl, int c, int ci,
                                                PipeLds<DK, WIDE, STEP> &s)
{
    static_assert(pipe_q_lds<DK, WIDE>(), "the two score waves share Q^T in LDS");
    constexpr int QLD = DK + 4;
    constexpr int PD = pipe_k_piece_dims<DK>(); // dims per K piece
    constexpr int PU = PD / 32; // u-steps per piece
    constexpr int PB = DK / PD; // pieces per 16-key block
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;

    f4 kb[PU][2]; // the K piece in flight: 16 keys (this wave's block) x PD dims
    auto load_k = [&](int t, int pc) {
        const int64_t key = cbase + t * kTile + 16 * ROLE + col;
        const float *kp = key_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
        for (int uu = 0; uu < PU; ++uu)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int d = 32 * (pc * PU + uu) + 8 * g + 4 * h;
                const bool din = FULL || d < p.dim;
                const f4 x = ldg4_stream(kp + (din ? d : 0));
                kb[uu][h] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
            }
    };
    // the first piece is requested before Q^T is staged, so the two loads'
    // latencies overlap (a barrier waits on LDS traffic only); with a step's
    // transform folded in (STEP), the new key's K and V rows are written
    // before #Q, so only a chunk whose first tile holds the new key (or a
    // clamped key past it) requests the tile after #Q
    const bool last = STEP && (int64_t)(c + 1) * kChunk >= p.nkeys;
    const bool wait = STEP && step_row_wait(p, c, kTile);
    StepQueryRows<DK> sqr;
    if constexpr (STEP && ROLE == 0)
        sqr.issue(p, unit, kh);
    if (!wait)
        load_k(0, 0);

    if constexpr (STEP) {
        // the first score wave prepares the unit's query rows; in the new
        // key's chunk the second prepares its K row (V: the first value wave)
        if constexpr (ROLE == 0) {
            if (sqr.finish(p, unit, kh, s.q, QLD, ci == 0 && p.sqo))
                atomicOr(p.err, kErrTransform);
        } else if (last) {
            if (step_kv_row<DK, true>(p, kh, &s.sb[0][0][0]))
                atomicOr(p.err, kErrTransform);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // the row is in L2 before #Q
        }
        __syncthreads(); // #Q: Q^T staged, the new key's rows written
        if (wait)
            load_k(0, 0);
    } else {
        // Q^T, staged by both score waves: every load is issued before the
        // first LDS store (a load-store loop would wait out one round trip
        // per row). Padding rows and dims read a valid row and store zeros.
        constexpr int QN = kRows * (DK / 4) / 128; // f4 per lane
        auto q_in = [&](int it, int *f, int *d) {
            const int i = lane + 64 * ROLE + 128 * it;
            *f = unit * kRows + i / (DK / 4);
            *d = (i % (DK / 4)) * 4;
            return *f < p.nrows && (FULL || *d < p.dim);
        };
        f4 qs[QN];
#pragma unroll
        for (int it = 0; it < QN; ++it) {
            int f, d;
            const bool in = q_in(it, &f, &d);
            const int ff = in ? f : 0;
            qs[it] = ldg4(p.q + (int64_t)(ff / p.group) * p.q_stride +
                          (int64_t)(kh * p.group + ff % p.group) * p.dim + (in ? d : 0));
        }
#pragma unroll
        for (int it = 0; it < QN; ++it) {
            int f, d;
            const bool in = q_in(it, &f, &d);
            f4 x = qs[it];
            // an unconditional use: keeps the (wave-uniform) row test from
            // sinking each load into a branch that waits for it alone
            asm volatile("" : "+v"(x));
            *(f4 *)(s.q + (f - unit * kRows) * QLD + d) =
                in ? x * p.q_scale : f4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads(); // #Q: Q^T staged
    }

    // this wave's block of tile t: its canonical score chain (run: any key of
    // the block allowed for the unit), the next piece loaded as registers free
    auto chain = [&](int t, bool run) {
        f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pc = 0; pc < PB; ++pc) {
            __builtin_amdgcn_sched_barrier(0);
            if (run) {
#pragma unroll
                for (int uu = 0; uu < PU; ++uu) {
                    const int u = pc * PU + uu;
                    const f4 qa0 = *(const f4 *)(s.q + col * QLD + 32 * u + 8 * g);
                    const f4 qa1 = *(const f4 *)(s.q + col * QLD + 32 * u + 8 * g + 4);
                    float qv[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        qv[j] = qa0[j];
                        qv[4 + j] = qa1[j];
                    }
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj)
                        acc = mfma(kb[uu][jj >> 2][jj & 3], qv[jj], acc);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (pc + 1 < PB)
                load_k(t, pc + 1);
            else if (t + 1 < kTilesPerChunk)
                load_k(t + 1, 0);
        }
        return acc;
    };
    // whether any key of this wave's block of tile t is allowed for the unit
    const ChunkKeys ck = chunk_keys(p, row, cbase);
    auto block_any = [&](int t, bool ok[4]) {
        const bool any = block_keys(ck, t * kTile + 16 * ROLE, g, ok);
        return (bool)__any(any);
    };

    if constexpr (ROLE == 1) {
        {
            bool ok[4];
            const f4 acc = chain(0, block_any(0, ok));
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s.sb[0][r][lane] = acc[r];
        }
        __syncthreads(); // #0: tile 0's second block scored
#pragma unroll 1
        for (int t = 0; t < kTilesPerChunk; ++t) {
            if (t + 1 < kTilesPerChunk) {
                bool ok[4];
                const f4 acc = chain(t + 1, block_any(t + 1, ok));
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s.sb[(t + 1) & 1][r][lane] = acc[r];
            }
            __syncthreads(); // #t+1
        }
        __syncthreads(); // chunk maximum
        return;
    }
    __syncthreads(); // #0
    float m = kNegInf;
    bool bad = false;
#pragma unroll 1
    for (int t = 0; t < kTilesPerChunk; ++t) {
        bool ok[2][4];
        const bool any0 = block_any(t, ok[0]);
        const bool any1 = block_keys(ck, t * kTile + 16, g, ok[1]);
        const bool tile_any = any0 || __any(any1);
        const f4 acc0 = chain(t, any0);
        float pr[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float alpha = 1.f, rs = 0.f;
        if (tile_any) {
            float sc[2][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sc[0][r] = acc0[r];
                sc[1][r] = s.sb[t & 1][r][lane];
            }
            cap_scores(p, sc);
            bad |= bad_scores(sc, ok);
            const float mn = fmaxf(m, tile_max(sc, ok));
            const float ms = safe_max(mn);
            alpha = fexp(m - ms);
            rs = tile_probs(sc, ok, ms, pr);
            m = mn;
        } else {
            alpha = fexp(m - safe_max(m));
        }
        const int slot = t & 1;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s.p[slot][4 * b + r][lane] = pr[b][r];
        if (g == 0) {
            s.alpha[slot][col] = alpha;
            s.rs[slot][col] = rs;
        }
        if (lane == 0)
            s.any[slot] = tile_any;
        __syncthreads(); // #t+1: tile t handed over
    }
    if (g == 0)
        s.m[col] = m;
    if (bad)
        atomicOr(p.err, kErrScore);
    __syncthreads(); // chunk maximum handed over
}

// Output modes of the pipelined kernel: the output of a launch's only
// chunk; a chunk partial for the combine kernel; or, for the last chunk of
// a one-span chunk-split launch run after the chunks before it
// (kMergeOut), the ordered merge of all the launch's chunk partials, this
// chunk's from registers, into the output: the combine kernel's arithmetic
// (split_kv.hip) without its launch.
enum PipeMode { kDirect = 0, kPartial = 1, kMergeOut = 2 };

template <int DK, int MODE, bool FULL, bool WIDE, bool STEP>
__device__ __forceinline__ void value_wave(const Params &p, int unit, int kvl, int c,
                                           PipeLds<DK, WIDE, STEP> &s, int vw, int ci)
{
    constexpr int VD = pipe_value_dims<DK, WIDE>();
    static_assert(VD % 64 == 0, "whole 64-dim output groups per value wave");
    constexpr int NQ = VD / 64; // 64-dim output groups of this wave
    const int d0 = VD * vw;     // the wave's first output dim
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;

    const int dv = d0 + 4 * col; // + 64a
    // V in flight: a group of VS 4-key slices; slice br = 4b + r of a tile
    // holds keys 16b + 4g + r (lane group g)
    constexpr int VS = pipe_v_slices<DK, WIDE>();
    constexpr int NG = 8 / VS; // groups per tile
    f4 vv[VS][NQ];             // [slice][64-dim group]
    auto load_v_sl = [&](int t, int grp, int sl) {
        const int br = VS * grp + sl;
        const int64_t key = cbase + t * kTile + 16 * (br >> 2) + 4 * g + (br & 3);
        const float *vp = value_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
        for (int a = 0; a < NQ; ++a) {
            const int d = 64 * a + dv;
            const bool din = FULL || d < p.dim;
            const f4 x = ldg4_stream(vp + (din ? d : 0));
            vv[sl][a] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // slice sl of the group after (t, grp), if any
    auto load_next_sl = [&](int t, int grp, int sl) {
        if (grp + 1 < NG)
            load_v_sl(t, grp + 1, sl);
        else if (t + 1 < kTilesPerChunk)
            load_v_sl(t + 1, 0, sl);
    };
    auto load_next = [&](int t, int grp) {
#pragma unroll
        for (int sl = 0; sl < VS; ++sl)
            load_next_sl(t, grp, sl);
    };
    // With a step's transform folded in (STEP), the chunk of the step's new
    // key prepares that key's V row (and in the narrow layout its K row) and
    // writes both into the cache before the wave's first barrier. The first
    // V group is requested before that unless its tile (the first) holds
    // the new key or a clamped key past it; the narrow layout's score wave
    // requests blocks of the first 48 keys before that barrier, so there
    // a chunk whose new key is among them waits for the rows first (#S).
    const bool last = STEP && (int64_t)(c + 1) * kChunk >= p.nkeys;
    const bool wait_s = STEP && pipe_score_waves<DK, WIDE>() == 1 && step_row_wait(p, c, 48);
    const bool early = !(STEP && step_row_wait(p, c, kTile)) && !wait_s;
    if (early) {
#pragma unroll
        for (int sl = 0; sl < VS; ++sl)
            load_v_sl(0, 0, sl);
    }
    if constexpr (STEP) {
        if (last) {
            bool bad = false;
            if constexpr (pipe_score_waves<DK, WIDE>() == 1) {
                bad = step_kv_row<DK, true>(p, kh, s.row);
                bad |= step_kv_row<DK, false>(p, kh, s.row);
            } else if (vw == 0) {
                bad = step_kv_row<DK, false>(p, kh, &s.p[0][0][0]);
            }
            if (bad)
                atomicOr(p.err, kErrTransform);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // the rows are in L2 before the barrier
        }
    }
    if constexpr (pipe_score_waves<DK, WIDE>() > 1) {
        // the score waves' prologue barriers (Q^T staged, the first block
        // scored) pass with the first group already requested
        __syncthreads(); // #Q
        if (!early) {
#pragma unroll
            for (int sl = 0; sl < VS; ++sl)
                load_v_sl(0, 0, sl);
        }
        __syncthreads(); // #0
    } else if (!early) {
        if (wait_s)
            __syncthreads(); // #S: the new key's rows written
#pragma unroll
        for (int sl = 0; sl < VS; ++sl)
            load_v_sl(0, 0, sl);
    }
    float l = 0.f;
    f4 O[NQ][4];
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
    __syncthreads(); // tile 0 handed over
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        const int slot = t & 1;
        const float a_t = s.alpha[slot][col];
        l = __builtin_fmaf(l, a_t, s.rs[slot][col]);
        const bool tile_any = s.any[slot];
        if (tile_any) {
#pragma unroll
            for (int a = 0; a < NQ; ++a)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    O[a][j] = O[a][j] * a_t;
        }
#pragma unroll
        for (int grp = 0; grp < NG; ++grp) {
            __builtin_amdgcn_sched_barrier(0);
            if (tile_any) {
#pragma unroll
                for (int sl = 0; sl < VS; ++sl) {
                    const float pb = s.p[slot][VS * grp + sl][lane];
#pragma unroll
                    for (int a = 0; a < NQ; ++a)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            O[a][j] = mfma(vv[sl][a][j], pb, O[a][j]);
                    if constexpr (pipe_slice_loads<DK, WIDE>()) {
                        // this slice's registers are consumed: the next group's slice
                        __builtin_amdgcn_sched_barrier(0);
                        load_next_sl(t, grp, sl);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!tile_any || !pipe_slice_loads<DK, WIDE>()) // the whole next group at once
                load_next(t, grp);
        }
        __syncthreads(); // tile t + 1 handed over (the last one: the chunk maximum)
    }
    const float m = s.m[col];

    // O[a][j][i] is dim 64a + 16g + 4i + j of row `row`.
    if (row >= p.nrows)
        return;
    if (MODE == kDirect) { // the launch's only chunk: final output
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
    { // chunk partial for the combine kernel
        const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + ci;
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
        if (g == 0 && d0 == 0) {
            stg(p.ws_ml + 2 * slot, m);
            stg(p.ws_ml + 2 * slot + 1, l);
        }
        return;
    }
}

template <int DK, bool WIDE> constexpr int pipe_threads()
{
    return 64 * (pipe_score_waves<DK, WIDE>() + pipe_value_waves<DK, WIDE>());
}

// Waves per SIMD the register budget is sized for: four workgroups per CU at
// head dim 512 (all 1024 workgroups of a 128K two-KV-head decode resident at
// once, 128 KiB in flight per CU); a padded head dim keeps the larger budget
// (its clamped loads would spill at 128 VGPRs).
template <int DK, bool FULL> constexpr int pipe_waves_per_simd()
{
    return DK > 256 && FULL ? 4 : 2;
}

// FULL: the head dim equals the padded head dim (no dim clamping). WIDE: the
// wide layout at head dims up to 256.
template <int DK, int MODE, bool FULL, bool WIDE, bool STEP>
__global__ __launch_bounds__((pipe_threads<DK, WIDE>()), (pipe_waves_per_simd<DK, FULL>()))
void pipe_kv_kernel(Params p, int c0)
{
    __shared__ PipeLds<DK, WIDE, STEP> s;
    const int ci = c0 + (int)blockIdx.x; // the launch's chunk index
    const int c = p.c_lo + ci;
    const int unit = blockIdx.y % p.units;
    const int kvl = blockIdx.y / p.units;
    const int wave = threadIdx.x >> 6;
    // the value waves write a chunk partial in both partial modes
    constexpr int VMODE = MODE == kMergeOut ? kPartial : MODE;
    if constexpr (pipe_score_waves<DK, WIDE>() == 1) {
        if (wave == 0)
            score_wave<DK, FULL, STEP>(p, unit, kvl, c, ci, s);
        else
            value_wave<DK, VMODE, FULL, WIDE, STEP>(p, unit, kvl, c, s, wave - 1, ci);
    } else {
        if (wave == 0) {
            score_wave_dual<DK, FULL, 0, WIDE, STEP>(p, unit, kvl, c, ci, s);
        } else if (wave == 1) {
            score_wave_dual<DK, FULL, 1, WIDE, STEP>(p, unit, kvl, c, ci, s);
        } else {
            value_wave<DK, VMODE, FULL, WIDE, STEP>(p, unit, kvl, c, s, wave - 2, ci);
        }
    }
    if constexpr (MODE == kMergeOut) {
        // The unit's rows, merged by every thread of the workgroup, four
        // consecutive dims of one row at a time: the launch's chunks (one
        // span; this chunk's partial just written, the others by the launch
        // before) in the combine kernel's order and arithmetic.
        __syncthreads(); // this chunk's partials visible to the workgroup
        const int q4 = p.dim / 4;
        const int kh = p.kh_first + kvl;
        for (int e = threadIdx.x; e < kRows * q4; e += blockDim.x) {
            const int row = unit * kRows + e / q4;
            const int d = 4 * (e % q4);
            if (row >= p.nrows)
                continue;
            const int query = row / p.group;
            const int h = kh * p.group + row % p.group;
            if (h < p.h_lo || h >= p.h_hi)
                continue;
            const int64_t slot0 = ((int64_t)kvl * p.nrows_pad + row) * p.nch;
            const Merged4 sv = merge_chunks4(p, slot0, d, 0, p.nch);
            const MergeFactors f = merge_factors(kNegInf, sv.M);
            const float L = merge_value(0.f, sv.L, f);
            f4 v;
            bool nonfinite = false;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = merge_value(0.f, sv.acc[j], f) / L;
                nonfinite |= !is_finite(v[j]);
            }
            stg4(p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim + d, v);
            if (nonfinite)
                atomicOr(p.err, kErrOutput);
        }
    }
}

// Which launches take the wide layout. Head dim 128: all (its narrow
// workgroup keeps only 16 KiB in flight; measured on MI355X the wide one was
// 1.1-1.7x faster from 2K to 32K keys with 8 KV heads). Head dim 256: fewer
// (chunk, unit, KV head) items than this, where each workgroup's chain of
// round trips is the time (1.04-1.14x faster at 32-256 items, even at 512;
// at 1024 items, the 32K decode, the narrow layout is 5 % faster).
constexpr int64_t kPipeWideMaxItems256 = 512;

template <int DK, int MODE, bool FULL, bool WIDE, bool STEP>
static void launch_dk(const Params &p, dim3 grid, int c0, hipStream_t stream)
{
    pipe_kv_kernel<DK, MODE, FULL, WIDE, STEP>
        <<<grid, pipe_threads<DK, WIDE>(), 0, stream>>>(p, c0);
}

// Chunks [c0, c0 + n) of the launch.
template <int MODE, bool FULL, bool STEP>
hipError_t launch_mode(const Params &p, int c0, int n, hipStream_t stream)
{
    const dim3 grid(n, p.nkv * p.units);
    const bool wide = (int64_t)n * p.nkv * p.units < kPipeWideMaxItems256;
    switch (p.dk) {
    case 64: launch_dk<64, MODE, FULL, false, STEP>(p, grid, c0, stream); break;
    case 128: launch_dk<128, MODE, FULL, true, STEP>(p, grid, c0, stream); break;
    case 256:
        wide ? launch_dk<256, MODE, FULL, true, STEP>(p, grid, c0, stream)
             : launch_dk<256, MODE, FULL, false, STEP>(p, grid, c0, stream);
        break;
    case 512: launch_dk<512, MODE, FULL, true, STEP>(p, grid, c0, stream); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// A one-token step's head transform folds in (Params::sq) only where the
// head dim is the padded one (the transform's own head dims from 64 up).
template <bool FULL>
hipError_t launch_full(const Params &p, int c0, int n, bool merge_out, hipStream_t stream)
{
    if (p.sq) {
        if constexpr (FULL) {
            if (merge_out || c0 != 0 || n != p.nch || p.nq != 1)
                return hipErrorInvalidValue;
            return p.ws_o == nullptr ? launch_mode<kDirect, true, true>(p, c0, n, stream)
                                     : launch_mode<kPartial, true, true>(p, c0, n, stream);
        }
        return hipErrorInvalidValue;
    }
    if (merge_out)
        return launch_mode<kMergeOut, FULL, false>(p, c0, n, stream);
    return p.ws_o == nullptr ? launch_mode<kDirect, FULL, false>(p, c0, n, stream)
                             : launch_mode<kPartial, FULL, false>(p, c0, n, stream);
}

// Chunks [c0, c0 + n) of the launch, their partials in the launch's chunk
// slots (the chunk-split prefill runs its last round's chunk this way at
// head dim 64; fan_kv.hip at the others); with merge_out (n = 1, the
// launch's last chunk, one span, the earlier chunks' partials already
// written) the merged output instead.
hipError_t launch_pipe_kv_chunks(const Params &p, int c0, int n, bool merge_out,
                                 hipStream_t stream)
{
    return p.dim == p.dk ? launch_full<true>(p, c0, n, merge_out, stream)
                         : launch_full<false>(p, c0, n, merge_out, stream);
}

// Direct output for a single chunk, chunk partials otherwise.
hipError_t launch_pipe_kv(const Params &p, hipStream_t stream)
{
    return launch_pipe_kv_chunks(p, 0, p.nch, false, stream);
}

} // namespace pcl
