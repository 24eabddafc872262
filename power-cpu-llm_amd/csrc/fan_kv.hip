// Fanned chunk kernel for gfx950: one (16-row unit, 256-key chunk, KV head)
// item over the eight waves of one workgroup.
//
// A chunk-split prefill or canvas whose chunk items leave a last round of
// one chunk per row block (the canvas: 288 items of 128 rows on 256 CUs; at
// head dim 512, 576 items of 64 rows) runs that chunk here, one workgroup
// per 16-row unit: 256 items for either canvas, one per CU. A unit-chunk is
// 4.2 MFLOP at head dim 256 (6.8 us of one CU's matrix peak), so the item
// is spread over all four SIMDs:
//
//   wave w forms the raw scores of tile w (its two 16-key blocks): the
//   canonical score chain of attention_device.hpp, K read straight into MFMA
//   A operands (at head dim 512 in four pieces, two in flight), Q (shared
//   by the waves) read from LDS;
//   wave w takes its tile's maximum; after a barrier every wave runs the
//   running-maximum chain over the tile maxima, and wave w forms its tile's
//   probabilities and row sum against the running maximum at its tile;
//   after a second barrier every wave runs the l chain and the P.V chain of
//   its own DK/8 output dims over all eight tiles, probabilities from LDS,
//   V of the first LT tiles from LDS (copied HBM -> LDS while the scores are
//   formed) and of the rest from registers (requested once the score chain
//   has consumed K, VB tiles in flight).
//
// Every value is the one the sequential per-tile online softmax forms (the
// same operations on the same operands in the same order), so the results
// are the other kernels' bits; each wave computes one tile's exponentials
// instead of all eight.
//
// Output: with merge_out (the launch's last chunk, one span, the earlier
// chunks' partials already written by the chunk items) the chunk state is
// transposed through LDS to a row-contiguous layout, and every thread
// merges the earlier partials of its row and dims in ascending order and
// then its own chunk state, which is the combine's ordered merge bit for bit
// (empty slots merge as no-ops), and writes the output; otherwise it writes
// the chunk partial for the combine kernels.
#include "attention_device.hpp"

#include <atomic>
#include <type_traits>

namespace pcl {

constexpr int kFanWaves = 8;
constexpr int kFanThreads = 64 * kFanWaves;

template <int DK, int SPLIT = 1> struct FanCfg {
    static constexpr int NU = DK / 32;        // score chain steps
    // output dims of a wave: a workgroup owns DK / SPLIT of them
    static constexpr int VD = DK / (kFanWaves * SPLIT);
    static constexpr int VW = VD / 16;        // output blocks of a wave (dims of a lane per key)
    // K of a wave's tile staged through LDS in pieces of KU score steps
    // (32 keys x 32 KU dims, 4 KU one-KiB copies), KB pieces in flight
    static constexpr int KU = DK <= 128 ? 4 : DK <= 256 ? 2 : 1;
    static constexpr int KPN = NU / KU;
    static constexpr int KB = KPN > 1 ? 2 : 1;
    static constexpr int KCOPIES = 4 * KU;
    static constexpr int kpFloats = kTile * 32 * KU;
    // V through registers: the first VB0 tiles requested up front; then the
    // rest once K is issued (VB = 8: every tile's V held at once), or VB
    // tiles in flight, each slot refilled once its tile's P.V has run
    static constexpr int VB = DK <= 256 ? kTilesPerChunk : 4;
    static constexpr int VB0 = 4;
    // merge: f4 columns of a thread's row; the earlier partials are copied
    // into the freed K staging area while the tiles run when they fit it
    static constexpr int NK = DK / 128;
    // LDS, in floats: region A holds Q (row-major, each row's f4 columns
    // XOR-swizzled by (row & 7)) during the score chains, the
    // probabilities ([tile][4b + r][lane]) after them and the chunk state
    // ([row][DK], swizzled like Q) after the tiles; region K holds each
    // wave's K pieces, then the earlier partials ([row][chunk][DK]);
    // region C holds each tile's row maxima and row sums, whether it has any
    // allowed key, and each row's (m, l)
    static constexpr int qFloats = kRows * DK;
    static constexpr int pFloats = kTilesPerChunk * 8 * 64;
    static constexpr int aFloats = qFloats > pFloats ? qFloats : pFloats;
    static constexpr int kFloats = kFanWaves * KB * kpFloats;
    static constexpr bool PREFETCH = kRows * 8 * DK <= kFloats;
    static constexpr int cFloats = 2 * kTilesPerChunk * kRows + kTilesPerChunk + 2 * kRows;
    static constexpr size_t bytes = (size_t)(aFloats + kFloats + cFloats) * sizeof(float);
    static_assert(VW >= 1 && VW * 16 * kFanWaves * SPLIT == DK, "whole 16-dim output blocks");
    static_assert(KU * KPN == NU, "whole K pieces");
};

typedef __attribute__((address_space(3))) void *fan_lptr_t;
typedef const __attribute__((address_space(1))) void *fan_gptr_t;

// A workgroup barrier that leaves vector-memory loads in flight (the caller
// has waited for whatever the other waves must see; __syncthreads would
// also wait for every LDS copy still in flight). The empty statements keep
// the compiler from moving memory accesses across it.
__device__ __forceinline__ void fan_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// f(std::integral_constant<int, i>) for i = I .. N-1, in order (compile-time
// indices where a builtin needs a constant).
template <int I, int N, typename F> __device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Vector-memory operations a wave has issued after its copies of K piece pc
// when that piece's score steps run. Issue order: Q, pieces 0 .. KB-1, V
// tiles 0 .. VB0-1; after piece j's steps, piece j + KB (while there is
// one), and after piece KPN - KB's steps V tiles VB0 .. 7 when every tile's
// V is held at once.
template <typename C> __device__ constexpr int ops_after_piece(int pc)
{
    int n = 0;
    // prologue entries after piece pc
    for (int q = pc + 1; q < C::KB && q < C::KPN; ++q)
        n += C::KCOPIES;
    if (pc < C::KB)
        n += 8 * C::VB0;
    // entries issued after piece j's steps, j < pc (all after piece pc's
    // copies when the entry is issued later than piece pc)
    for (int j = 0; j < pc; ++j) {
        if (j + C::KB < C::KPN && j + C::KB > pc)
            n += C::KCOPIES;
        if (C::VB == kTilesPerChunk && j == C::KPN - C::KB)
            n += 8 * (kTilesPerChunk - C::VB0);
    }
    return n;
}

// Earlier chunk partials a merging thread requests in one batch (the rest,
// in a span of more chunks, one at a time after them).
constexpr int kMergeHead = 8;

// FULL: the head dim equals the padded head dim (no dim clamping). MERGE:
// the launch's last chunk of one span, merged into the output.
// SPLIT (a launch of every chunk): SPLIT workgroups share an item, each
// forming all its scores and the P.V of DK / SPLIT output dims.
template <int DK, bool FULL, bool CAP, bool MERGE, int SPLIT>
__global__ __launch_bounds__(kFanThreads, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fan_kv_kernel(Params p, int ci)
{
    static_assert(SPLIT == 1 || !MERGE, "a merging launch keeps whole items");
    using C = FanCfg<DK, SPLIT>;
    int split = 0;
    // consecutive workgroups cycle over the KV heads (each XCD's L2 then
    // serves one head's K and V when there are eight)
    int kvl = (int)blockIdx.x % p.nkv;
    int unit = (int)blockIdx.x / p.nkv;
    if constexpr (!MERGE) {
        if (ci < 0) {
            // A launch of every chunk: item group gi = (chunk, KV head) has
            // its units in workgroups congruent mod 8, which the dispatcher
            // deals to one XCD, so they share the chunk's K and V in its L2:
            // workgroup b runs unit (b / 8) % units of group
            // ((b / 8) / units) * 8 + b % 8 (with SPLIT, (unit, split) pairs
            // in place of units).
            const int b = (int)blockIdx.x;
            const int k = b >> 3;
            const int gi = (k / (p.units * SPLIT)) * 8 + (b & 7);
            if (gi >= p.nkv * p.nch)
                return; // padding to whole groups of eight
            unit = k % (p.units * SPLIT) / SPLIT;
            split = k % SPLIT;
            kvl = gi % p.nkv;
            ci = gi / p.nkv;
        }
    }
    constexpr int VD = C::VD, VW = C::VW, KU = C::KU, KPN = C::KPN, KB = C::KB;
    constexpr int VB = C::VB, VB0 = C::VB0, NK = C::NK;
    constexpr int NQC = kRows * DK / 256 / kFanWaves; // Q copies per wave
    static_assert(NQC * 256 * kFanWaves == kRows * DK, "whole 1 KiB copies per wave");
    extern __shared__ float lds[];
    float *qs = lds;                  // region A: Q, the probabilities, the chunk state
    float *kst = lds + C::aFloats;    // region K: K pieces, then the earlier partials
    float *tmx = kst + C::kFloats;    // region C: [tile][row] maxima,
    float *trs = tmx + kTilesPerChunk * kRows;  // [tile][row] row sums,
    float *tany = trs + kTilesPerChunk * kRows; // [tile] any allowed key (0 / 1),
    float *mlst = tany + kTilesPerChunk;        // [row] (m, l)

    const int c = p.c_lo + ci;
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int lane = tid & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const bool rin = row < p.nrows;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;
    const int d0 = VD * w + DK / SPLIT * split; // the wave's output dims

    // Allowed flags of the lane's keys of tile w. A chunk that every real
    // row of the unit sees whole needs no per-key test (padding rows then
    // count as allowed: their columns never reach a real row's state); a
    // tile with no allowed key for any row of the unit is skipped, which
    // leaves the state bit-unchanged. (Mask bytes are read here, before the
    // large loads.)
    const ChunkKeys ck = chunk_keys(p, row, cbase);
    bool ok[2][4];
    bool any = true;
    if (!p.mask && __all(!rin || (ck.lo <= 0 && ck.hi >= kChunk - 1))) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                ok[b][r] = true;
    } else {
        any = tile_keys(ck, w, g, ok);
    }
    const bool tile_any = __any(any);

    // The merge's own layout (after the tiles): thread tid owns row
    // mrow = tid / 32 of the unit and the f4 columns tid % 32 + 32k (k < NK),
    // so a wave's accesses of a chunk partial are two rows' contiguous bytes.
    // With MERGE the earlier chunks' (m, l) are requested first.
    const int mrow = unit * kRows + tid / 32;
    const bool mrin = mrow < p.nrows;
    const int64_t mslot0 = ((int64_t)kvl * p.nrows_pad + (mrin ? mrow : 0)) * p.nch;
    constexpr int EH = MERGE ? kMergeHead : 1;
    f2 eml[EH];
    if constexpr (MERGE) {
#pragma unroll
        for (int c0 = 0; c0 < EH; ++c0) // slots past ci re-read the last earlier chunk
            eml[c0] = ldg2(p.ws_ml + 2 * (mslot0 + (c0 < ci ? c0 : ci - 1)));
    }

    // Q of the unit's 16 rows, HBM -> LDS (region A, unscaled): copy j moves
    // 1 KiB (256 floats) of the row-major [16][DK] block, each row's 16-byte
    // pieces XOR-swizzled by (row & 7) so that the eight rows an MFMA operand
    // read touches hit distinct banks. Padding rows copy the last real row
    // and dims past the head's last its first dims: both read as zero below.
#pragma unroll
    for (int i = 0; i < NQC; ++i) {
        const int j = w * NQC + i;
        const int f = 256 * j + 4 * lane;
        const int r = f / DK;
        const int qd = 4 * (((f % DK) / 4) ^ (r & 7));
        const int qrow = min(unit * kRows + r, p.nrows - 1);
        const int query = qrow / p.group;
        const int h = kh * p.group + qrow % p.group;
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim +
                          (FULL || qd < p.dim ? qd : 0);
        __builtin_amdgcn_global_load_lds((fan_gptr_t)qp, (fan_lptr_t)(qs + 256 * j), 16, 0, 0);
    }
    // K piece pc of tile w (keys 32w .. 32w+31, dims [32 KU pc, 32 KU (pc+1))),
    // HBM -> this wave's buffer in region K as contiguous copies (four keys'
    // 128 KU bytes each): [key][8 KU f4 slots], slot s of key k stored at
    // s ^ (k & 7) (an MFMA operand read's eight keys then hit distinct
    // banks). A dim past the head's last copies the head's first dims (Q is
    // zero there); keys past the last copy the last key (masked).
    auto load_k = [&](int pc, int buf) {
        float *dst = kst + (w * KB + buf) * C::kpFloats;
#pragma unroll
        for (int i = 0; i < C::KCOPIES; ++i) {
            const int f = 256 * i + 4 * lane;
            const int key = f / (32 * KU);
            const int pos = (f % (32 * KU)) / 4;
            const int kd = 32 * KU * pc + 4 * (pos ^ (key & 7));
            const int64_t kt = cbase + kTile * w + key;
            const float *kp = key_row(p, kt < klast ? kt : klast) + hoff +
                              (FULL || kd < p.dim ? kd : 0);
            __builtin_amdgcn_global_load_lds((fan_gptr_t)kp, (fan_lptr_t)(dst + 256 * i), 16, 0,
                                             0);
        }
    };
#pragma unroll
    for (int pc = 0; pc < KB; ++pc)
        load_k(pc, pc);

    // V for the wave's dims into registers: vr[slot][b][r][x] =
    // V[key 32t + 16b + 4g + r][d0 + VW col + x] for tile t in slot t % VB
    float vr[VB][2][4][VW];
    auto load_v = [&](int t) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t kt = cbase + kTile * t + 16 * b + 4 * g + r;
                const int vd = d0 + VW * col;
                const float *vp = value_row(p, kt < klast ? kt : klast) + hoff +
                                  (FULL || vd < p.dim ? vd : 0);
                float *dst = vr[t % VB][b][r];
                if constexpr (VW == 4) {
                    const f4 x = ldg4(vp);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        dst[e] = x[e];
                } else if constexpr (VW == 2) {
                    const f2 x = ldg2(vp);
                    dst[0] = x.x;
                    dst[1] = x.y;
                } else {
                    dst[0] = ldg(vp);
                }
            }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < VB0; ++t)
        load_v(t);
    __builtin_amdgcn_sched_barrier(0);

    // Q has landed (each wave waits for its own copies, the barrier for
    // all; K and V stay in flight).
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(KB * C::KCOPIES + 8 * VB0));
    fan_barrier();

    // the score chains of blocks 2w and 2w + 1: A operands from this wave's
    // K pieces (each piece waited for by count), B operands
    // Q[row][32u + 8g + jj] * q_scale (zero for padding rows and dims)
    f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
    static_for<0, KPN>([&](auto pcc) {
        constexpr int pc = decltype(pcc)::value;
        constexpr int buf = pc % KB;
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(ops_after_piece<C>(pc)));
        const float *kb = kst + (w * KB + buf) * C::kpFloats;
#pragma unroll
        for (int uu = 0; uu < KU; ++uu) {
            const int u = KU * pc + uu;
            float q[8];
            f4 ka[2][2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int c4 = 8 * u + 2 * g + hh;
                const bool qin = rin && (FULL || 4 * c4 < p.dim);
                const f4 x = *(const f4 *)(qs + col * DK + 4 * (c4 ^ (col & 7))) * p.q_scale;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[4 * hh + j] = qin ? x[j] : 0.f;
                const int s4 = 8 * uu + 2 * g + hh; // the f4 slot within the piece
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    ka[b][hh] = *(const f4 *)(kb + (16 * b + col) * 32 * KU + 4 * (s4 ^ (col & 7)));
            }
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[b] = mfma(ka[b][jj >> 2][jj & 3], q[jj], acc[b]);
        }
        // this buffer's operands are read: the next piece (or, after the
        // last piece is requested, the remaining V)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (pc + KB < KPN)
            load_k(pc + KB, buf);
        if constexpr (VB == kTilesPerChunk && pc == KPN - KB) {
#pragma unroll
            for (int t = VB0; t < kTilesPerChunk; ++t)
                load_v(t);
        }
        __builtin_amdgcn_sched_barrier(0);
    });

    // The tile's maximum (wave w), and whether it has a non-finite allowed
    // score. The lanes of each row agree on the maximum.
    float s[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            s[b][r] = acc[b][r];
    cap_scores<CAP>(p, s);
    bool bad = false;
    float tm = kNegInf;
    if (tile_any) {
        bad = bad_scores(s, ok);
        tm = tile_max(s, ok);
    }
    if (g == 0)
        tmx[w * kRows + col] = tm;
    if (lane == 0)
        tany[w] = tile_any ? 1.f : 0.f;

    // Every tile maximum in LDS, and every wave past its score chain
    // (regions A and K are free). The running maximum after each tile (the
    // same on every wave), then wave w's probabilities and row sum against
    // it.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    fan_barrier();
    if constexpr (MERGE && C::PREFETCH) {
        // the earlier chunks' partials of the unit's rows, HBM -> region K
        // ([row][kMergeHead][DK]; chunks past ci re-read the last earlier
        // one, rows past the launch's the last real row), landing while the
        // tiles run
        constexpr int NPC = kRows * kMergeHead * DK / 256 / kFanWaves;
        static_assert(NPC * 256 * kFanWaves == kRows * kMergeHead * DK, "whole copies");
#pragma unroll
        for (int i = 0; i < NPC; ++i) {
            const int f = 256 * (w * NPC + i) + 4 * lane;
            const int r = f / (kMergeHead * DK);
            const int c0 = (f / DK) % kMergeHead;
            const int d = f % DK;
            const int prow = min(unit * kRows + r, p.nrows - 1);
            const int64_t slot = ((int64_t)kvl * p.nrows_pad + prow) * p.nch +
                                 (c0 < ci ? c0 : ci - 1);
            __builtin_amdgcn_global_load_lds((fan_gptr_t)(p.ws_o + slot * p.dk + d),
                                             (fan_lptr_t)(kst + 256 * (w * NPC + i)), 16, 0, 0);
        }
    }
    float tmr[kTilesPerChunk];
    bool tan[kTilesPerChunk];
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        tmr[t] = tmx[t * kRows + col];
        tan[t] = tany[t] != 0.f;
    }
    {
        float mrun = kNegInf, msw = 0.f;
#pragma unroll
        for (int t = 0; t < kTilesPerChunk; ++t) {
            if (tan[t])
                mrun = fmaxf(mrun, tmr[t]);
            if (t == w)
                msw = safe_max(mrun);
        }
        if (tile_any) {
            float pr[2][4];
            const float rs = tile_probs(s, ok, msw, pr);
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    qs[(w * 8 + 4 * b + r) * 64 + lane] = pr[b][r];
            if (g == 0)
                trs[w * kRows + col] = rs;
        }
    }
    if (bad)
        atomicOr(p.err, kErrScore);
    // the probabilities and row sums in LDS
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    fan_barrier();

    // The l chain and the P.V chains of the wave's VW output blocks, tile
    // by tile. Output block x: A operand V[key][d0 + VW col + x], so O[x][i]
    // is dim d0 + VW (4g + i) + x.
    float m = kNegInf, l = 0.f;
    f4 O[VW];
#pragma unroll
    for (int x = 0; x < VW; ++x)
        O[x] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kTilesPerChunk; ++t) {
        if (tan[t]) {
            const float mn = fmaxf(m, tmr[t]);
            const float ms = safe_max(mn);
            const float alpha = fexp(m - ms);
            l = __builtin_fmaf(l, alpha, trs[t * kRows + col]);
            m = mn;
            float pr[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                pr[e] = qs[(t * 8 + e) * 64 + lane];
#pragma unroll
            for (int x = 0; x < VW; ++x)
                O[x] = O[x] * alpha;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int x = 0; x < VW; ++x)
                        O[x] = mfma(vr[t % VB][b][r][x], pr[4 * b + r], O[x]);
        }
        if (VB < kTilesPerChunk && t + VB < kTilesPerChunk) { // this slot is free: a later tile
            __builtin_amdgcn_sched_barrier(0);
            load_v(t + VB);
        }
    }
    // without the copies of region K: the earlier partials into registers
    f4 eo[MERGE && !C::PREFETCH ? kMergeHead : 1][NK];
    if constexpr (MERGE && !C::PREFETCH) {
#pragma unroll
        for (int c0 = 0; c0 < kMergeHead; ++c0) {
            const int64_t cc = mslot0 + (c0 < ci ? c0 : ci - 1);
#pragma unroll
            for (int k = 0; k < NK; ++k)
                eo[c0][k] = ldg4(p.ws_o + cc * p.dk + 4 * (tid % 32 + 32 * k));
        }
    }

    // The chunk state into region A (free once every wave is past its
    // tiles), row-major [16][DK] with each row's f4 columns XOR-swizzled by
    // (row & 7), and (m, l) per row: lane (col, g) holds the 4 VW
    // consecutive dims d0 + 4 VW g .. of row col (dim d0 + VW (4g + i) + x
    // is O[x][i]).
    float *ost = qs;
    fan_barrier();
#pragma unroll
    for (int k = 0; k < VW; ++k) {
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int n = 4 * k + e;
            v[e] = O[n % VW][n / VW];
        }
        const int c4 = (d0 + 4 * VW * g + 4 * k) / 4;
        *(f4 *)(ost + col * DK + 4 * (c4 ^ (col & 7))) = v;
    }
    if (w == 0 && g == 0) {
        mlst[2 * col] = m;
        mlst[2 * col + 1] = l;
    }
    // the columns this workgroup formed (all but with SPLIT)
    auto own = [&](int k) {
        return SPLIT == 1 || (tid % 32 + 32 * k) / (32 * C::NK / SPLIT) == split;
    };
    // (the earlier partials' copies have landed too)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    fan_barrier();
    if (!mrin)
        return;
    const int mr = tid / 32; // the merge row within the unit
    const float mm = mlst[2 * mr], ml = mlst[2 * mr + 1];
    f4 ov[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int c4 = tid % 32 + 32 * k;
        ov[k] = own(k) ? *(const f4 *)(ost + mr * DK + 4 * (c4 ^ (mr & 7))) : f4{};
    }
    if constexpr (!MERGE) { // chunk partial for the combine kernels
        const int64_t slot = mslot0 + ci;
        float *wo = p.ws_o + slot * p.dk;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int d = 4 * (tid % 32 + 32 * k);
            if ((FULL || d < p.dim) && own(k))
                stg4(wo + d, ov[k]);
        }
        if (tid % 32 == 0 && split == 0) {
            stg(p.ws_ml + 2 * slot, mm);
            stg(p.ws_ml + 2 * slot + 1, ml);
        }
        return;
    } else {
        const int query = mrow / p.group;
        const int h = kh * p.group + mrow % p.group;
        if (h < p.h_lo || h >= p.h_hi)
            return;
        float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
        bool nonfinite = false;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int d = 4 * (tid % 32 + 32 * k);
            if (!FULL && d >= p.dim)
                continue;
            // the span's earlier chunks in ascending order (the combine's
            // order, without its empty slots, which merge as no-ops), then
            // this chunk, the span's last; then the span into the empty total
            Merged4 sv = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int c0 = 0; c0 < kMergeHead; ++c0)
                if (c0 < ci) {
                    f4 x;
                    if constexpr (C::PREFETCH)
                        x = *(const f4 *)(kst + (mr * kMergeHead + c0) * DK + d);
                    else
                        x = eo[c0][k];
                    merge_into4(sv, eml[c0].x, eml[c0].y, x);
                }
            for (int c0 = kMergeHead; c0 < ci; ++c0) {
                const int64_t cc = mslot0 + c0;
                const f2 x = ldg2(p.ws_ml + 2 * cc);
                merge_into4(sv, x.x, x.y, ldg4(p.ws_o + cc * p.dk + d));
            }
            merge_into4(sv, mm, ml, ov[k]);
            const MergeFactors f = merge_factors(kNegInf, sv.M);
            const float L = merge_value(0.f, sv.L, f);
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = merge_value(0.f, sv.acc[j], f) / L;
                nonfinite |= !is_finite(v[j]);
            }
            stg4(o + d, v);
        }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
    }
}

constexpr int kFanMaxDevices = 64;

// Dynamic LDS above 64 KiB must be allowed once per kernel and device; a
// repeated call from a racing thread is harmless.
template <int DK, bool FULL, bool CAP, bool MERGE, int SPLIT> static hipError_t configure_fan()
{
    static std::atomic<bool> configured[kFanMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= kFanMaxDevices)
        return hipErrorInvalidDevice;
    if (!configured[dev].load(std::memory_order_acquire)) {
        e = hipFuncSetAttribute((const void *)fan_kv_kernel<DK, FULL, CAP, MERGE, SPLIT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)FanCfg<DK, SPLIT>::bytes);
        if (e != hipSuccess)
            return e;
        configured[dev].store(true, std::memory_order_release);
    }
    return hipSuccess;
}

// ci < 0: every chunk of the launch (grid y), partials for the combine.
template <int DK, bool FULL, bool CAP, bool MERGE, int SPLIT>
static hipError_t launch_fan_split(const Params &p, int ci, hipStream_t stream)
{
    const hipError_t e = configure_fan<DK, FULL, CAP, MERGE, SPLIT>();
    if (e != hipSuccess)
        return e;
    // every chunk: (chunk, KV head) groups padded to a multiple of eight,
    // each group's units (and their splits) on one XCD (see the kernel)
    const int groups8 = (p.nkv * p.nch + 7) / 8 * 8;
    const dim3 grid(ci < 0 ? groups8 * p.units * SPLIT : p.units * p.nkv);
    fan_kv_kernel<DK, FULL, CAP, MERGE, SPLIT>
        <<<grid, kFanThreads, FanCfg<DK, SPLIT>::bytes, stream>>>(p, ci);
    return hipGetLastError();
}

// Items (chunk, unit, KV head) up to which a launch of every chunk at head
// dim 256 or 512 splits each item's output dims over two workgroups (at 512
// four up to half as many): one workgroup a CU (its LDS), so at most half
// (a quarter of) the CUs would hold an item otherwise. The split workgroups
// of an item share its K and V through their XCD's L2.
constexpr int64_t kFanSplitItems = 128;

template <int DK, bool FULL, bool CAP, bool MERGE>
static hipError_t launch_fan_dk(const Params &p, int ci, hipStream_t stream)
{
    if constexpr (DK == 512 && !MERGE) {
        if (ci < 0 && (int64_t)p.nkv * p.nch * p.units <= kFanSplitItems / 2)
            return launch_fan_split<DK, FULL, CAP, MERGE, 4>(p, ci, stream);
        if (ci < 0 && (int64_t)p.nkv * p.nch * p.units <= kFanSplitItems)
            return launch_fan_split<DK, FULL, CAP, MERGE, 2>(p, ci, stream);
    }
    if constexpr (DK == 256 && !MERGE) {
        if (ci < 0 && (int64_t)p.nkv * p.nch * p.units <= kFanSplitItems)
            return launch_fan_split<DK, FULL, CAP, MERGE, 2>(p, ci, stream);
    }
    return launch_fan_split<DK, FULL, CAP, MERGE, 1>(p, ci, stream);
}

template <int DK, bool MERGE>
static hipError_t launch_fan_mode(const Params &p, int ci, hipStream_t stream)
{
    const bool full = p.dim == DK;
    if (p.softcap > 0.0f)
        return full ? launch_fan_dk<DK, true, true, MERGE>(p, ci, stream)
                    : launch_fan_dk<DK, false, true, MERGE>(p, ci, stream);
    return full ? launch_fan_dk<DK, true, false, MERGE>(p, ci, stream)
                : launch_fan_dk<DK, false, false, MERGE>(p, ci, stream);
}

template <int DK>
static hipError_t launch_fan_cap(const Params &p, int ci, bool merge_out, hipStream_t stream)
{
    return merge_out ? launch_fan_mode<DK, true>(p, ci, stream)
                     : launch_fan_mode<DK, false>(p, ci, stream);
}

// Whether launch chunk items at padded head dim dk can run fanned.
bool fan_supported(int dk)
{
    return dk == 128 || dk == 256 || dk == 512;
}

// The launch's chunk ci (its last) as one fanned item per (16-row unit, KV
// head). merge_out: the launch is one span and every other chunk's partial
// is written; the output is then the merged result. Otherwise the chunk's
// partial is written for the combine kernels.
hipError_t launch_fan_chunk(const Params &p, int ci, bool merge_out, hipStream_t stream)
{
    if (ci < 0 || ci >= p.nch ||
        (merge_out && (p.nspan != 1 || ci < 1 || ci != p.nch - 1 || p.nch > kSpanChunks)))
        return hipErrorInvalidValue;
    switch (p.dk) {
    case 128: return launch_fan_cap<128>(p, ci, merge_out, stream);
    case 256: return launch_fan_cap<256>(p, ci, merge_out, stream);
    case 512: return launch_fan_cap<512>(p, ci, merge_out, stream);
    default: return hipErrorInvalidValue;
    }
}

// A decode (or any split-KV launch of at least two chunks): every (chunk,
// 16-row unit, KV head) item as one fanned workgroup, each writing its chunk
// partial for the combine kernels.
hipError_t launch_fan_kv(const Params &p, hipStream_t stream)
{
    if (p.nch < 2 || !p.ws_o)
        return hipErrorInvalidValue;
    switch (p.dk) {
    case 128: return launch_fan_cap<128>(p, -1, false, stream);
    case 256: return launch_fan_cap<256>(p, -1, false, stream);
    case 512: return launch_fan_cap<512>(p, -1, false, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl
