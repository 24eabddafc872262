// Spread split-KV decode for gfx950: one 256-key chunk over S = DK/32
// slices of two waves, for short decodes whose (chunk, 16-row unit, KV head)
// items are too few to fill the chip (a 2K decode has 64 of them on 256
// CUs).
//
// Slice j of an item takes
//   the scores of 16 / S of the chunk's 16 key blocks (one 16-key block per
//   wave at head dim 256): the canonical score chain of attention_device.hpp
//   on K read straight into MFMA operands, published to the workspace;
//   output dims [32j, 32j + 32) (16 per wave): V for those dims and all 256
//   keys, requested behind the wave's K and kept in LDS.
// A workgroup runs one slice (two waves) or two (four waves, so that a
// launch of up to two slices per CU still has one workgroup per CU). Its
// waves then read the chunk's raw scores back (a share each, shared through
// LDS) and each runs the tile-by-tile online softmax and the P.V chain for
// its own dims exactly as the other kernels do (every workgroup of the item
// derives the same m, l and probabilities, bit for bit). So each slice
// reads 1/S of the chunk's K and 1/S of its V, and a 2K decode runs 512
// slices.
//
// Publication needs no flag and no fence: every score is stored as one
// 64-bit word (the launch's epoch, the score's bits), which lands whole, and
// a reader takes a word only with a device-coherent load and only when it
// carries the current epoch. The words live in a region at the start of the
// workspace that holds nothing else (zero when allocated and after every
// wrap of the epoch counter; epochs are never zero), so a stale word
// carries an earlier epoch.
//
// Local form (the (KV head, 16-row unit) groups come in whole eights, as
// with 8 KV heads): a one-dimensional grid deals each group's workgroups,
// its items' and then its merge workgroups, to one XCD (the dispatcher
// deals workgroup b to XCD b % 8), and the words are stored plainly, so
// they stay in that XCD's L2, where the readers find them (a score is seen
// about 240 ns after its store instead of 400-530 ns, and the exchange adds
// no HBM traffic). Otherwise the three-dimensional grid (slice groups,
// chunks, groups plus merge planes) and device-coherent stores.
//
// The wait is bounded: after max_polls reads a wave stops waiting and forms
// every score block whose words have not arrived itself, by the same chain
// from K and Q (the same bits), so every wave exits with a valid result even
// when some workgroups of its item never ran alongside it. The host picks
// this kernel only for launches whose workgroups all fit on the chip at
// once, and a wave waits only for the workgroups of its own item, adjacent
// in dispatch order, so the fallback is for a GPU shared with other work.
//
// Output: for a launch of a single chunk, the output itself. Otherwise each
// workgroup publishes its chunk partial (m, l, O) as (epoch, bits) words,
// and merge workgroups appended to the grid (dispatched after every item's
// workgroups, so they wait only for workgroups already running) take them
// and run the ordered chunk and span merges of the combine kernels
// (split_kv.hip) for four dims of one row per thread, writing the output:
// no combine launch. (Merging by the last workgroup of each slice to finish
// instead was measured slower: its chain of dependent round trips outlasted
// the separate combine launch.)
#include "attention_device.hpp"

namespace pcl {

constexpr int kSliceWaves = 2; // waves per 32-dim slice
constexpr int kSpreadSliceDims = 32;
constexpr int kBlocksPerChunk = 2 * kTilesPerChunk; // 16-key blocks

typedef __attribute__((address_space(3))) void *spread_lptr_t;
typedef const __attribute__((address_space(1))) void *spread_gptr_t;


// Merge role: thread e of the merge workgroups owns four dims of one row of
// one KV head; it takes every chunk partial of that row as published words
// and merges them exactly as the combine kernels do (per span the span's
// kSpanChunks slots in ascending order from (-inf, 0, 0), absent chunks as
// empty parts; then the spans in ascending order), then writes the output.
template <bool LOCAL>
__device__ __forceinline__ void spread_merge_row(const Params &p, int kvl, int row, int d)
{
    const int q4 = p.dim / 4;
    const int64_t slot0 = ((int64_t)kvl * p.nrows + row) * p.nch;
    // the threads of each wave of the row poll one word of each chunk
    // partial between them (a row of more than 64 threads spans two waves,
    // each of which waits for all chunks)
    const int wq = q4 < 64 ? q4 : 64;
    if (!wait_partials<LOCAL ? 1 : 8>(p, slot0, (d / 4) % wq, wq, p.nch)) {
        atomicOr(p.err, kErrWait);
        return;
    }
    Merged4 tot = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
    bool ok = true;
    for (int sl = 0; sl < p.nspan; ++sl) {
        const int span = p.s_lo + sl;
        const int c0 = max(span * kSpanChunks, p.c_lo) - p.c_lo;
        const int c1 = min((span + 1) * kSpanChunks, p.c_lo + p.nch) - p.c_lo;
        Merged4 sm = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
        // (batches of absent chunks only are not run; four or fewer
        // chunks left take a batch of four)
        for (int b0 = 0; b0 < kSpanChunks && c0 + b0 < c1; b0 += kMergeBatch)
            ok &= c1 - (c0 + b0) <= kMergeBatch / 2
                      ? merge_words_batch<kMergeBatch / 2, LOCAL ? 1 : 2>(p, slot0, c0, b0, c1,
                                                                          d, sm)
                      : merge_words_batch<kMergeBatch, LOCAL ? 1 : 2>(p, slot0, c0, b0, c1, d, sm);
        merge_into4(tot, sm.M, sm.L, sm.acc);
    }
    if (!ok) {
        atomicOr(p.err, kErrWait);
        return;
    }
    const int kh = p.kh_first + kvl;
    const int query = row / p.group;
    const int h = kh * p.group + row % p.group;
    if (h < p.h_lo || h >= p.h_hi)
        return;
    float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
    f4 v;
    bool nonfinite = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = tot.acc[j] / tot.L;
        nonfinite |= !is_finite(v[j]);
    }
    stg4(o + d, v);
    if (nonfinite)
        atomicOr(p.err, kErrOutput);
}

// Thread e of the merge planes (the three-dimensional form): rows of every
// KV head in turn.
__device__ __forceinline__ void spread_merge(const Params &p, int64_t e)
{
    const int q4 = p.dim / 4;
    const int64_t per_kv = (int64_t)p.nrows * q4;
    if (e >= p.nkv * per_kv)
        return;
    spread_merge_row<false>(p, (int)(e / per_kv), (int)(e % per_kv) / q4,
                            4 * (int)(e % per_kv % q4));
}

// Thread e of group z's merge workgroups (the local form): the rows of the
// group's 16-row unit.
__device__ __forceinline__ void spread_merge_group(const Params &p, int z, int e)
{
    const int q4 = p.dim / 4;
    const int unit = z % p.units;
    const int row = unit * kRows + e / q4;
    if (e >= kRows * q4 || row >= p.nrows)
        return;
    spread_merge_row<true>(p, z / p.units, row, 4 * (e % q4));
}

// The local form's merge workgroups per (KV head, unit) group: one thread
// per four dims of each real row of a unit.
__host__ __device__ inline int spread_group_merge_wgs(const Params &p, int threads)
{
    if (p.ws_ptag == nullptr)
        return 0;
    const int rows = p.nrows < kRows ? p.nrows : kRows;
    return (rows * (p.dim / 4) + threads - 1) / threads;
}

// The canonical score chain of the 16-key block at key0 for the rows of the
// lane's unit (lane (col, g): row `row`, keys key0 + 4g + r in the result),
// loaded and formed on its own: the operands and the order of the kernel's
// own chains, for a block whose published words did not arrive.
template <int DK, bool FULL>
__device__ __forceinline__ f4 spread_block_scores(const Params &p, int64_t key0, int kh, int row,
                                               bool rin, int col, int g)
{
    constexpr int NU = DK / 32;
    const int64_t klast = p.nkeys - 1;
    const int64_t key = key0 + col;
    const float *kp = key_row(p, key < klast ? key : klast) + (int64_t)kh * p.dim;
    const int query = rin ? row / p.group : 0;
    const int h = kh * p.group + (rin ? row % p.group : 0);
    const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim;
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int u = 0; u < NU; ++u) {
        float q[8], k[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int d = 32 * u + 8 * g + 4 * hh;
            const bool din = FULL || d < p.dim;
            const f4 x = ldg4(qp + (din ? d : 0)) * p.q_scale;
            const f4 y = ldg4(kp + (din ? d : 0));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                q[4 * hh + j] = (rin && din) ? x[j] : 0.f;
                k[4 * hh + j] = din ? y[j] : 0.f;
            }
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            acc = mfma(k[jj], q[jj], acc);
    }
    return acc;
}

// LOCAL: the one-dimensional grid that places each (KV head, 16-row unit)
// group's workgroups, its items' and then its merge workgroups, on one XCD
// (the dispatcher deals workgroup b to XCD b % 8), so that the exchanged
// words are read through that XCD's L2; otherwise the three-dimensional
// grid (slice groups, chunks, groups + merge planes). WHOLE: the host found
// that every real row sees every chunk of the launch whole (no per-key
// test anywhere; the kernel then carries no per-key tile path, which made
// the compiler fold the two tile loops into one loop with per-tile branches:
// the 1024-key window 12.1 -> 11.5 us without it).
template <int DK, bool FULL, bool CAP, bool EARLY, int WV, bool LOCAL, bool WHOLE>
__global__ __launch_bounds__(64 * WV, 2) void spread_kv_kernel(Params p)
{
    constexpr int S = DK / kSpreadSliceDims;                 // slices per item
    constexpr int SPW = WV / kSliceWaves;                    // slices per workgroup
    int xs, ci, z; // slice group, launch chunk, (KV head, unit) group
    if constexpr (LOCAL) {
        // group z = 8 j + (b % 8) takes workgroups b = 8 (j W + w) + z % 8,
        // w < W: items (chunk w / (S / SPW), slice group w % (S / SPW)),
        // then its merge workgroups
        constexpr int X = S / SPW;
        const int b = (int)blockIdx.x;
        const int k = b >> 3;
        const int W = p.nch * X + spread_group_merge_wgs(p, 64 * WV);
        z = (k / W) * 8 + (b & 7);
        const int w = k % W;
        if (z >= p.nkv * p.units)
            return;
        if (w >= p.nch * X) {
            spread_merge_group(p, z, (w - p.nch * X) * (64 * WV) + (int)threadIdx.x);
            return;
        }
        ci = w / X;
        xs = w % X;
    } else {
        if ((int)blockIdx.z >= p.nkv * p.units) { // an appended merge workgroup
            const int64_t mw = blockIdx.x + (int64_t)gridDim.x *
                                                (blockIdx.y + (int64_t)gridDim.y *
                                                                  (blockIdx.z - p.nkv * p.units));
            spread_merge(p, mw * (64 * WV) + threadIdx.x);
            return;
        }
        xs = blockIdx.x;
        ci = blockIdx.y;
        z = blockIdx.z;
    }
    constexpr int BPW = kBlocksPerChunk / (S * kSliceWaves); // score blocks per wave
    constexpr int NU = DK / 32;                              // score chain steps
    static_assert(BPW >= 1 && BPW * S * kSliceWaves == kBlocksPerChunk, "whole blocks");
    static_assert(SPW >= 1 && S % SPW == 0 && kBlocksPerChunk % WV == 0, "whole slices");

    // V of each wave's 16 dims for the chunk's 256 keys, 1 KiB per 16-key
    // block: slot j of a block (64 bytes, 16 dims) holds key 4(j % 4) + j / 4
    // of the block, so the four keys 4g + r an MFMA step reads sit in four
    // different 64-byte bank groups
    __shared__ float vlds[WV][kBlocksPerChunk][16][16];
    // the chunk's raw scores, [block][r][lane], gathered by all waves
    __shared__ float slds[kBlocksPerChunk][4][64];
    const int c = p.c_lo + ci;
    const int unit = z % p.units;
    const int kvl = z / p.units;
    const int64_t item = ((int64_t)z * p.nch + ci);
    const int w = threadIdx.x >> 6;
    const int slice = xs * SPW + w / kSliceWaves;
    const int ws = w % kSliceWaves; // the wave within its slice
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const bool rin = row < p.nrows;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;
    // the item's words: [block][r][lane]
    uint64_t *words = p.ws_tag + item * (kBlocksPerChunk * 64 * 4);
    const int d0 = kSpreadSliceDims * slice + 16 * ws; // the wave's output dims

    {
        // K of this wave's score blocks (MFMA A operands), Q^T (B operands:
        // Q[row][32u + 8g + jj] * q_scale, 0 for padding rows) and V of the
        // wave's 16 dims for the chunk's 256 keys: lane L of block i moves
        // 16 bytes (dims d0 + 4(L % 4) ..) of key 16i + 4(s % 4) + s / 4
        // into LDS slot s = L / 4. A dim past the head's last reads the
        // head's first dims instead (that output is dropped).
        const int blk0 = (slice * kSliceWaves + ws) * BPW;
        f4 kb[BPW][NU][2];
        float q[NU][8];
        f4 vr[EARLY ? kBlocksPerChunk : 1];
        const int query = rin ? row / p.group : 0;
        const int h = kh * p.group + (rin ? row % p.group : 0);
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim;
        const int sl = lane >> 2;
        const int kin = 4 * (sl & 3) + (sl >> 2);
        const int vd = 4 * (lane & 3);
        const int dv = FULL || d0 + vd < p.dim ? d0 + vd : 0;
        if constexpr (EARLY) {
            // At most one workgroup per CU: every request goes out before
            // the first wait, K (from HBM) first, then Q (from L2), then V
            // into registers (written to LDS once the scores are out;
            // register loads, because with LDS copies also in flight the
            // compiler would wait for all of them before the first score
            // step).
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int64_t key = cbase + 16 * (blk0 + i) + col;
                const float *kp = key_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
                for (int u = 0; u < NU; ++u)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int d = 32 * u + 8 * g + 4 * hh;
                        kb[i][u][hh] = ldg4_stream(kp + (FULL || d < p.dim ? d : 0));
                    }
            }
            f4 qr[NU][2];
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int d = 32 * u + 8 * g + 4 * hh;
                    qr[u][hh] = ldg4(qp + (FULL || d < p.dim ? d : 0));
                }
#pragma unroll
            for (int i = 0; i < kBlocksPerChunk; ++i) {
                const int64_t key = cbase + 16 * i + kin;
                vr[i] = ldg4_stream(value_row(p, key < klast ? key : klast) + hoff + dv);
            }
            // K and Q have landed; V may still be in flight
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(kBlocksPerChunk));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int d = 32 * u + 8 * g + 4 * hh;
                    const bool din = FULL || d < p.dim;
                    const f4 x = qr[u][hh] * p.q_scale;
                    const f4 v = (rin && din) ? x : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        q[u][4 * hh + j] = v[j];
                    if (!din) {
#pragma unroll
                        for (int i = 0; i < BPW; ++i)
                            kb[i][u][hh] = f4{0.f, 0.f, 0.f, 0.f};
                    }
                }
        } else {
            // Two or three workgroups per CU: Q, then K, then V copied
            // HBM -> LDS with no register staging behind each wave's K (all
            // requested up front measured slower with two two-wave
            // workgroups per CU: the second one's K then queued behind the
            // first one's V).
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
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int64_t key = cbase + 16 * (blk0 + i) + col;
                const float *kp = key_row(p, key < klast ? key : klast) + hoff;
#pragma unroll
                for (int u = 0; u < NU; ++u)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int d = 32 * u + 8 * g + 4 * hh;
                        const bool din = FULL || d < p.dim;
                        const f4 x = ldg4_stream(kp + (din ? d : 0));
                        kb[i][u][hh] = din ? x : f4{0.f, 0.f, 0.f, 0.f};
                    }
            }
            float *vl = &vlds[w][0][0][0];
#pragma unroll
            for (int i = 0; i < kBlocksPerChunk; ++i) {
                const int64_t key = cbase + 16 * i + kin;
                const float *vp = value_row(p, key < klast ? key : klast) + hoff + dv;
                __builtin_amdgcn_global_load_lds((spread_gptr_t)vp,
                                                 (spread_lptr_t)(vl + i * 256), 16, 0, 0);
            }
        }
        // the score chains, each block published
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
                    acc = mfma(kb[i][u][jj >> 2][jj & 3], q[u][jj], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                publish_to<LOCAL>(words + ((blk0 + i) * 4 + r) * 64 + lane, p.epoch, acc[r]);
        }
        if constexpr (EARLY) {
            float *vl = &vlds[w][0][0][0];
#pragma unroll
            for (int i = 0; i < kBlocksPerChunk; ++i)
                *(f4 *)(vl + i * 256 + 4 * lane) = vr[i];
        }
    }

    // The chunk's raw scores once every word carries this launch's epoch
    // (bounded): each wave takes its share of the blocks and leaves them in
    // LDS. A block whose words have not all arrived when the wait runs out
    // (a workgroup of the item that is not running: a GPU shared with other
    // work, or too few CUs) is formed here by the same score chain from K and
    // Q, so the launch completes with the same bits either way.
    {
        constexpr int HB = kBlocksPerChunk / WV;
        uint64_t x[HB][4];
        bool gave_up = false;
        for (int polls = 0;;) {
            // an opaque base each pass: the loads' addresses are formed here
            // from it (otherwise the compiler keeps them all live across the
            // loop)
            const uint64_t *base = words + (w * HB * 4) * 64 + lane;
            asm volatile("" : "+v"(base));
            bool fresh = true;
#pragma unroll
            for (int b = 0; b < HB; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    x[b][r] = take(base + (b * 4 + r) * 64);
                    fresh &= (uint32_t)(x[b][r] >> 32) == p.epoch;
                }
            if (__all(fresh))
                break;
            if (++polls >= p.max_polls) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(LOCAL ? 1 : 2);
        }
        if (gave_up) {
#pragma unroll
            for (int b = 0; b < HB; ++b) {
                bool got = true;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    got &= (uint32_t)(x[b][r] >> 32) == p.epoch;
                if (__all(got))
                    continue;
                const f4 acc = spread_block_scores<DK, FULL>(p, cbase + 16 * (w * HB + b),
                                                             kh, row, rin, col, g);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    x[b][r] = (uint64_t)__float_as_uint(acc[r]);
            }
        }
#pragma unroll
        for (int b = 0; b < HB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                slds[w * HB + b][r][lane] = __uint_as_float((uint32_t)x[b][r]);
    }
    // the V copies have landed (s_waitcnt covers LDS copies too) and both
    // halves of the scores are in LDS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // Online softmax and the P.V chain of this wave's 16 dims, tile by tile.
    float m = kNegInf, l = 0.f;
    f4 O = f4{0.f, 0.f, 0.f, 0.f};
    bool bad = false;
    const ChunkKeys ck = chunk_keys(p, row, cbase);
    // one tile: ok the lane's allowed keys, tile_any whether the unit has any
    auto tile_step = [&](int t, const bool ok[2][4], bool tile_any) {
        float pr[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float alpha, rs = 0.f;
        if (tile_any) {
            float sv[2][4];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sv[b][r] = slds[2 * t + b][r][lane];
            cap_scores<CAP>(p, sv);
            bad |= bad_scores(sv, ok);
            const float mn = fmaxf(m, tile_max(sv, ok));
            const float ms = safe_max(mn);
            alpha = fexp(m - ms);
            rs = tile_probs(sv, ok, ms, pr);
            m = mn;
        } else {
            // nothing allowed for the unit: alpha = exp(m - safe(m)), rs = 0
            alpha = fexp(m - safe_max(m));
        }
        l = __builtin_fmaf(l, alpha, rs);
        if (tile_any) {
            O = O * alpha;
#pragma unroll
            for (int br = 0; br < 8; ++br) {
                // key 16b + 4g + r of block 2t + b sits in slot 4r + g
                const int b = br >> 2, r = br & 3;
                O = mfma(vlds[w][2 * t + b][4 * r + g][col], pr[b][r], O);
            }
        }
    };
    // A chunk that every real row of the unit sees whole (the usual decode
    // chunk) needs no per-key test and runs its tiles as one branch-free
    // sequence (padding rows then count as allowed: their columns never
    // reach a real row's state, and any non-finite score they see a real row
    // sees too). In other chunks each tile that every real row sees whole
    // takes the same step (a sliding window's first chunk or the cache's
    // last: 1.1-2 us less per decode than testing every key of the chunk).
    if (WHOLE || (!p.mask && __all(!rin || (ck.lo <= 0 && ck.hi >= kChunk - 1)))) {
        const bool ok[2][4] = {{true, true, true, true}, {true, true, true, true}};
#pragma unroll
        for (int t = 0; t < kTilesPerChunk; ++t)
            tile_step(t, ok, true);
    } else if constexpr (!WHOLE) {
#pragma unroll
        for (int t = 0; t < kTilesPerChunk; ++t) {
            if (!p.mask && __all(!rin || (ck.lo <= kTile * t && ck.hi >= kTile * t + kTile - 1))) {
                const bool ok[2][4] = {{true, true, true, true}, {true, true, true, true}};
                tile_step(t, ok, true);
            } else {
                bool ok[2][4];
                const bool any = tile_keys(ck, t, g, ok);
                tile_step(t, ok, __any(any));
            }
        }
    }
    if (bad && slice == 0 && ws == 0)
        atomicOr(p.err, kErrScore);

    // O[i] is dim d0 + 4g + i of row `row`.
    const int d = d0 + 4 * g;
    const bool dout = rin && (FULL || d < p.dim);
    if (p.ws_ptag == nullptr) { // the launch's only chunk: final output
        if (!rin)
            return;
        const int query = row / p.group;
        const int h = kh * p.group + row % p.group;
        if (h < p.h_lo || h >= p.h_hi || !dout)
            return;
        float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
        f4 v;
        bool nonfinite = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = O[i] / l;
            nonfinite |= !is_finite(v[i]);
        }
        stg4(o + d, v);
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }

    // the chunk partial for the merge workgroups
    if (!rin)
        return;
    uint64_t *pw = partial_words(p, kvl, row, ci);
    if (dout) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            publish_to<LOCAL>(pw + d + i, p.epoch, O[i]);
    }
    if (slice == 0 && ws == 0 && g == 0) {
        publish_to<LOCAL>(pw + p.dk, p.epoch, m);
        publish_to<LOCAL>(pw + p.dk + 1, p.epoch, l);
    }
}

// ---- Head dim 512 ---------------------------------------------------------
// The spread decode of short head-dim-512 launches (global layers: 16 query
// and 2 KV heads, a few thousand keys, which give too few (chunk, unit, KV
// head) items to fill the chip otherwise). An item's 16 slices are one wave
// each (a one-wave workgroup): slice j forms the raw scores of the chunk's
// key block j (its canonical chain over all 512 dims, 128 dependent MFMAs)
// and owns output dims [32j, 32j + 32) (two 16-dim output blocks, two
// independent P.V chains). K streams in four pieces of 128 dims, two in
// flight, each with its Q^T piece (B operands from L2); V of the wave's
// dims for the chunk's 256 keys goes straight to LDS (32 KiB), requested
// once the last K piece is (requested behind the first two pieces instead,
// the later pieces' waits also waited for V: 0.5 us slower at 2K and 4K
// keys). The scores are published as (epoch, bits)
// words and every slice gathers all 16 blocks, exactly as the head-dim-256
// form does, so every kernel's bits follow.
//
// A one-dimensional grid deals item i (i = group * nch + chunk) to XCD
// i % 8 (workgroup b = 8 (16 (i / 8) + j) + i % 8 for slice j): an item's
// score words are stored plainly into its XCD's L2 and read there. Its
// chunk partial goes out as device-coherent words to the merge workgroups
// appended to the grid (one thread per four dims of a row), which may run
// on any XCD.
int device_cus();

constexpr int kWideSlices = 16;  // slices per item: one key block each
constexpr int kWidePieceU = 4;   // score chain steps (32 dims each) per K piece
constexpr int kWidePieces = 512 / 32 / kWidePieceU;

// Item workgroups of a launch of SL slices per item (a whole number of
// eights of items, so that item i's slices all sit on XCD i % 8).
template <int SL> __host__ __device__ inline int spread_wide_item_wgs(const Params &p)
{
    const int items = p.nch * p.nkv * p.units;
    return SL * 8 * ((items + 7) / 8);
}

// SL slices per item (kWideSlices: one key block and 32 output dims per
// slice). Eight slices of two blocks each (their chains interleaved, 64
// dims, 80 KiB of LDS, two per CU), for launches of up to 64 items, were
// slower than the fanned kernel at 8K keys (43.3 against 36.2 us) and than
// sixteen slices at 2K-6K (31.3 against 21.0 us at 2K), so only sixteen run.
template <bool FULL, bool CAP, int SL>
__global__ __launch_bounds__(64) void spread_wide_kernel(Params p)
{
    constexpr int DK = 512;
    constexpr int BPW = kBlocksPerChunk / SL; // score blocks of a slice
    constexpr int VD = DK / SL;               // output dims of a slice
    constexpr int NH = VD / 16;               // its 16-dim output blocks
    const int b = (int)blockIdx.x;
    const int item_wgs = spread_wide_item_wgs<SL>(p);
    if (b >= item_wgs) { // an appended merge workgroup
        spread_merge(p, (int64_t)(b - item_wgs) * 64 + threadIdx.x);
        return;
    }
    const int item = 8 * ((b >> 3) / SL) + (b & 7);
    const int slice = (b >> 3) % SL;
    if (item >= p.nch * p.nkv * p.units)
        return;
    const int z = item / p.nch, ci = item % p.nch;

    // V of the wave's dims for the chunk's 256 keys, as the head-dim-256
    // form lays out 16 dims: [16-dim block][key block][slot][dim], slot j of
    // a key block holding key 4(j % 4) + j / 4
    __shared__ float vlds[NH][kBlocksPerChunk][16][16];
    // the chunk's raw scores, [block][r][lane]
    __shared__ float slds[kBlocksPerChunk][4][64];
    const int c = p.c_lo + ci;
    const int unit = z % p.units;
    const int kvl = z / p.units;
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int kh = p.kh_first + kvl;
    const int row = unit * kRows + col;
    const bool rin = row < p.nrows;
    const int64_t cbase = (int64_t)c * kChunk;
    const int64_t klast = p.nkeys - 1;
    const int64_t hoff = (int64_t)kh * p.dim;
    uint64_t *words = p.ws_tag + (int64_t)item * (kBlocksPerChunk * 64 * 4);
    const int d0 = VD * slice; // the wave's first output dim

    {
        const int query = rin ? row / p.group : 0;
        const int h = kh * p.group + (rin ? row % p.group : 0);
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)h * p.dim;
        const float *kp[BPW];
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            const int64_t key = cbase + 16 * (BPW * slice + i) + col;
            kp[i] = key_row(p, key < klast ? key : klast) + hoff;
        }
        // piece pc in register slot s: K[key][32u + 8g + 4hh ..] of each of
        // the slice's blocks and Q[row][32u + 8g + jj] * q_scale for u =
        // 4pc + uu (a dim past the head's last reads dim 0 and becomes 0)
        f4 kb[2][BPW][kWidePieceU][2];
        f4 qr[2][kWidePieceU][2];
        auto load_piece = [&](int pc, int sl) {
#pragma unroll
            for (int uu = 0; uu < kWidePieceU; ++uu)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int d = 32 * (kWidePieceU * pc + uu) + 8 * g + 4 * hh;
                    const int dd = FULL || d < p.dim ? d : 0;
#pragma unroll
                    for (int i = 0; i < BPW; ++i)
                        kb[sl][i][uu][hh] = ldg4_stream(kp[i] + dd);
                    qr[sl][uu][hh] = ldg4(qp + dd);
                }
        };
        load_piece(0, 0);
        load_piece(1, 1);
        // V: lane L of key block i moves 16 bytes (dims d0 + 16 n + 4(L % 4)
        // ..) of key 16i + 4(s % 4) + s / 4 into slot s = L / 4
        auto load_v = [&]() {
            const int sl = lane >> 2;
            const int kin = 4 * (sl & 3) + (sl >> 2);
#pragma unroll
            for (int n = 0; n < NH; ++n) {
                const int dv = d0 + 16 * n + 4 * (lane & 3);
                const int dd = FULL || dv < p.dim ? dv : 0;
#pragma unroll
                for (int i = 0; i < kBlocksPerChunk; ++i) {
                    const int64_t vk = cbase + 16 * i + kin;
                    const float *vp = value_row(p, vk < klast ? vk : klast) + hoff + dd;
                    __builtin_amdgcn_global_load_lds((spread_gptr_t)vp,
                                                     (spread_lptr_t)(&vlds[n][i][0][0]), 16,
                                                     0, 0);
                }
            }
        };
        f4 acc[BPW];
#pragma unroll
        for (int i = 0; i < BPW; ++i)
            acc[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pc = 0; pc < kWidePieces; ++pc) {
            const int sl = pc & 1;
#pragma unroll
            for (int uu = 0; uu < kWidePieceU; ++uu) {
                const int u = kWidePieceU * pc + uu;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int d = 32 * u + 8 * g + 4 * hh;
                    const bool din = FULL || d < p.dim;
                    const f4 x = qr[sl][uu][hh] * p.q_scale;
                    const f4 qv = (rin && din) ? x : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int i = 0; i < BPW; ++i) {
                            const float kv = din ? kb[sl][i][uu][hh][j] : 0.f;
                            acc[i] = mfma(kv, qv[j], acc[i]);
                        }
                }
            }
            if (pc + 2 < kWidePieces)
                load_piece(pc + 2, sl);
            if (pc == kWidePieces - 3)
                load_v(); // behind the last K piece
        }
#pragma unroll
        for (int i = 0; i < BPW; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                publish_to<true>(words + ((BPW * slice + i) * 4 + r) * 64 + lane, p.epoch,
                                 acc[i][r]);
    }

    // Every block's raw scores once its words carry this launch's epoch, in
    // two halves of eight blocks (bounded; a block whose words have not all
    // arrived when the wait runs out is formed here by the same chain).
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        constexpr int HB = kBlocksPerChunk / 2;
        uint64_t x[HB][4];
        bool gave_up = false;
        for (int polls = 0;;) {
            const uint64_t *base = words + (half * HB * 4) * 64 + lane;
            asm volatile("" : "+v"(base));
            bool fresh = true;
#pragma unroll
            for (int bb = 0; bb < HB; ++bb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    x[bb][r] = take(base + (bb * 4 + r) * 64);
                    fresh &= (uint32_t)(x[bb][r] >> 32) == p.epoch;
                }
            if (__all(fresh))
                break;
            if (++polls >= p.max_polls) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (gave_up) {
#pragma unroll
            for (int bb = 0; bb < HB; ++bb) {
                bool got = true;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    got &= (uint32_t)(x[bb][r] >> 32) == p.epoch;
                if (__all(got))
                    continue;
                const f4 acc = spread_block_scores<DK, FULL>(p, cbase + 16 * (half * HB + bb), kh,
                                                             row, rin, col, g);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    x[bb][r] = (uint64_t)__float_as_uint(acc[r]);
            }
        }
#pragma unroll
        for (int bb = 0; bb < HB; ++bb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                slds[half * HB + bb][r][lane] = __uint_as_float((uint32_t)x[bb][r]);
    }
    // the V copies have landed (s_waitcnt covers LDS copies too); the
    // scores are this wave's own LDS writes
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

    // Online softmax and the P.V chains of the wave's two 16-dim blocks.
    float m = kNegInf, l = 0.f;
    f4 O[NH];
#pragma unroll
    for (int n = 0; n < NH; ++n)
        O[n] = f4{0.f, 0.f, 0.f, 0.f};
    bool bad = false;
    const ChunkKeys ck = chunk_keys(p, row, cbase);
    auto tile_step = [&](int t, const bool ok[2][4], bool tile_any) {
        float pr[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float alpha, rs = 0.f;
        if (tile_any) {
            float sv[2][4];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sv[bb][r] = slds[2 * t + bb][r][lane];
            cap_scores<CAP>(p, sv);
            bad |= bad_scores(sv, ok);
            const float mn = fmaxf(m, tile_max(sv, ok));
            const float ms = safe_max(mn);
            alpha = fexp(m - ms);
            rs = tile_probs(sv, ok, ms, pr);
            m = mn;
        } else {
            alpha = fexp(m - safe_max(m));
        }
        l = __builtin_fmaf(l, alpha, rs);
        if (tile_any) {
#pragma unroll
            for (int n = 0; n < NH; ++n)
                O[n] = O[n] * alpha;
#pragma unroll
            for (int br = 0; br < 8; ++br) {
                // key 16b + 4g + r of block 2t + b sits in slot 4r + g
                const int bb = br >> 2, r = br & 3;
#pragma unroll
                for (int n = 0; n < NH; ++n)
                    O[n] = mfma(vlds[n][2 * t + bb][4 * r + g][col], pr[bb][r], O[n]);
            }
        }
    };
    if (!p.mask && __all(!rin || (ck.lo <= 0 && ck.hi >= kChunk - 1))) {
        const bool ok[2][4] = {{true, true, true, true}, {true, true, true, true}};
#pragma unroll
        for (int t = 0; t < kTilesPerChunk; ++t)
            tile_step(t, ok, true);
    } else {
#pragma unroll
        for (int t = 0; t < kTilesPerChunk; ++t) {
            if (!p.mask && __all(!rin || (ck.lo <= kTile * t && ck.hi >= kTile * t + kTile - 1))) {
                const bool ok[2][4] = {{true, true, true, true}, {true, true, true, true}};
                tile_step(t, ok, true);
            } else {
                bool ok[2][4];
                const bool any = tile_keys(ck, t, g, ok);
                tile_step(t, ok, __any(any));
            }
        }
    }
    if (bad && slice == 0)
        atomicOr(p.err, kErrScore);

    // O[n][i] is dim d0 + 16n + 4g + i of row `row`.
    if (!rin)
        return;
    if (p.ws_ptag == nullptr) { // the launch's only chunk: final output
        const int query = row / p.group;
        const int h = kh * p.group + row % p.group;
        if (h < p.h_lo || h >= p.h_hi)
            return;
        float *o = p.out + (int64_t)query * p.o_stride + (int64_t)(h - p.h_base) * p.dim;
        bool nonfinite = false;
#pragma unroll
        for (int n = 0; n < NH; ++n) {
            const int d = d0 + 16 * n + 4 * g;
            if (!(FULL || d < p.dim))
                continue;
            f4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = O[n][i] / l;
                nonfinite |= !is_finite(v[i]);
            }
            stg4(o + d, v);
        }
        if (nonfinite)
            atomicOr(p.err, kErrOutput);
        return;
    }
    // the chunk partial for the merge workgroups (on any XCD)
    uint64_t *pw = partial_words(p, kvl, row, ci);
#pragma unroll
    for (int n = 0; n < NH; ++n) {
        const int d = d0 + 16 * n + 4 * g;
        if (!(FULL || d < p.dim))
            continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            publish_to<false>(pw + d + i, p.epoch, O[n][i]);
    }
    if (slice == 0 && g == 0) {
        publish_to<false>(pw + p.dk, p.epoch, m);
        publish_to<false>(pw + p.dk + 1, p.epoch, l);
    }
}

template <bool CAP, int SL>
static void launch_wide_sl(const Params &p, hipStream_t stream)
{
    int wgs = spread_wide_item_wgs<SL>(p);
    if (p.ws_ptag)
        wgs += (int)(((int64_t)p.nkv * p.nrows * (p.dim / 4) + 63) / 64);
    if (p.dim == 512)
        spread_wide_kernel<true, CAP, SL><<<wgs, 64, 0, stream>>>(p);
    else
        spread_wide_kernel<false, CAP, SL><<<wgs, 64, 0, stream>>>(p);
}

template <bool CAP>
static hipError_t launch_wide(const Params &p, hipStream_t stream)
{
    launch_wide_sl<CAP, kWideSlices>(p, stream);
    return hipGetLastError();
}

int spread_slices(int dk)
{
    return dk / kSpreadSliceDims;
}

// Whether every real row of a launch sees each of its chunks whole: no mask,
// and each row's key range covers chunks c_lo .. c_lo + nch - 1 entirely.
// A row's range grows with its query, so the first and the last real row
// decide (the device's per-chunk test would pass everywhere).
bool spread_whole_chunks(const Params &p)
{
    if (p.mask)
        return false;
    const int64_t first = (int64_t)p.c_lo * kChunk;
    const int64_t last = (int64_t)(p.c_lo + p.nch) * kChunk - 1;
    const int rows[2] = {0, p.nrows - 1};
    for (int row : rows) {
        int64_t lo = 0, hi = p.nkeys - 1;
        if (p.causal) {
            const int64_t rel = p.first_query + row / p.group - p.first_key;
            hi = hi < rel ? hi : rel;
            if (p.window)
                lo = rel - p.window + 1;
        }
        if (lo > first || hi < last)
            return false;
    }
    return true;
}

template <int DK, bool CAP, bool EARLY, int WV, bool LOCAL, bool WHOLE>
static void launch_whole(const Params &p, dim3 grid, hipStream_t stream)
{
    if (p.dim == DK)
        spread_kv_kernel<DK, true, CAP, EARLY, WV, LOCAL, WHOLE><<<grid, 64 * WV, 0, stream>>>(p);
    else
        spread_kv_kernel<DK, false, CAP, EARLY, WV, LOCAL, WHOLE><<<grid, 64 * WV, 0, stream>>>(p);
}

// The early forms (the shortest decodes, where it pays) have a whole-chunk
// instantiation.
template <int DK, bool CAP, bool EARLY, int WV, bool LOCAL>
static void launch_grid(const Params &p, dim3 grid, hipStream_t stream)
{
    if constexpr (EARLY) {
        if (spread_whole_chunks(p)) {
            launch_whole<DK, CAP, EARLY, WV, LOCAL, true>(p, grid, stream);
            return;
        }
    }
    launch_whole<DK, CAP, EARLY, WV, LOCAL, false>(p, grid, stream);
}

template <int DK, bool CAP, bool EARLY, int WV>
static void launch_form(const Params &p, hipStream_t stream)
{
    constexpr int S = DK / kSpreadSliceDims;
    constexpr int X = S / (WV / kSliceWaves); // item workgroups per chunk
    const int groups = p.nkv * p.units;
    if (groups % 8 == 0) {
        // the local form: each group's workgroups on one XCD
        const int W = p.nch * X + spread_group_merge_wgs(p, 64 * WV);
        launch_grid<DK, CAP, EARLY, WV, true>(p, dim3(groups * W), stream);
        return;
    }
    // merge workgroups (one thread per four dims of a row) as whole planes
    // after the items' planes
    int merge_planes = 0;
    if (p.ws_ptag) {
        const int64_t threads = (int64_t)p.nkv * p.nrows * (p.dim / 4);
        const int64_t per_plane = (int64_t)X * p.nch * 64 * WV;
        merge_planes = (int)((threads + per_plane - 1) / per_plane);
    }
    launch_grid<DK, CAP, EARLY, WV, false>(p, dim3(X, p.nch, groups + merge_planes), stream);
}

template <int DK, bool CAP>
static hipError_t launch_cap(const Params &p, hipStream_t stream)
{
    constexpr int S = DK / kSpreadSliceDims;
    // Every request goes out up front when the item workgroups take at most
    // one CU each: two-wave workgroups (one slice) when they fit so, four-wave
    // ones (two slices) when those do; otherwise two-wave workgroups, two or
    // three per CU, in the compiler's order.
    const int64_t slices = (int64_t)S * p.nch * p.nkv * p.units;
    const int cus = device_cus();
    if (cus > 0 && slices <= cus)
        launch_form<DK, CAP, true, 2>(p, stream);
    else if (cus > 0 && S % 2 == 0 && slices <= 2 * (int64_t)cus)
        launch_form<DK, CAP, true, 4>(p, stream);
    else
        launch_form<DK, CAP, false, 2>(p, stream);
    return hipGetLastError();
}

template <int DK>
static hipError_t launch_dk(const Params &p, hipStream_t stream)
{
    return p.softcap > 0.0f ? launch_cap<DK, true>(p, stream) : launch_cap<DK, false>(p, stream);
}

hipError_t launch_spread_kv(const Params &p, hipStream_t stream)
{
    switch (p.dk) {
    case 64: return launch_dk<64>(p, stream);
    case 128: return launch_dk<128>(p, stream);
    case 256: return launch_dk<256>(p, stream);
    case 512:
        return p.softcap > 0.0f ? launch_wide<true>(p, stream) : launch_wide<false>(p, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl
