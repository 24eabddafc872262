// LDS-tiled prefill / canvas attention for gfx950.
//
// One workgroup of 8 waves (two per SIMD) owns 128 flat (query, head) rows of
// one KV head, one 16-row MFMA unit per wave. Q^T (MFMA B operands) and the
// chunk state O stay in registers. K and V tiles of 32 keys are copied
// HBM -> LDS by global_load_lds_dwordx4 (no register staging), double
// buffered. K rows are stored with their 16-byte chunks XOR-swizzled by
// (key & 7), so the 16 key rows of an MFMA A operand hit distinct banks
// without padding the rows.
//
// Per tile each wave runs the score chain, online softmax and P.V chain of
// the canonical arithmetic (attention_device.hpp). The merges are rare (every
// 8 and every 128 tiles), so their accumulators live outside the registers:
// the span accumulator's leading 64-dim blocks in the LDS beside the stages,
// the rest in the row's own output slot, the running total across spans in
// the workspace; the last merge writes the normalised output. Tiles wholly
// masked for the workgroup are never loaded; tiles wholly masked for a wave
// are skipped by that wave.
//
// split != 0: the workgroup computes the single chunk c_lo + z0 + blockIdx.z
// and writes its chunk partial for the combine kernels. A split launch whose
// chunk items leave a small last round runs that round's chunk as fanned
// items instead (fan_kv.hip: one (16-row unit, chunk) item per workgroup of
// eight waves: more, shorter items fill the CUs; the pipelined decode kernel
// at head dim 64); each row's arithmetic is the same either way.
#include "attention_device.hpp"

#include <algorithm>
#include <atomic>

namespace pcl {

hipError_t launch_pipe_kv_chunks(const Params &p, int c0, int n, bool merge_out,
                                 hipStream_t stream);
hipError_t launch_fan_chunk(const Params &p, int ci, bool merge_out, hipStream_t stream);
bool fan_supported(int dk);

constexpr int kTiledWaves = 8;
constexpr int kTiledRows = kTiledWaves * kRows; // 128

// LDS of one workgroup: two K/V stages, then the leading 64-dim blocks of
// the span accumulator (as many as the 160 KiB of a CU hold beside the
// stages: one at head dim 256, all of them at 128 and 64).
template <int DK> struct TiledLds {
    static constexpr int tileFloats = kTile * DK;
    static constexpr int stage = 2 * tileFloats; // K then V
    static constexpr int stageFloats = 2 * stage;
    static constexpr int blockFloats = kTiledRows * 64; // one 64-dim block of every row
    static constexpr int spanBlocks = std::min(DK / 64, (40960 - stageFloats) / blockFloats);
    static constexpr size_t bytes = (size_t)(stageFloats + spanBlocks * blockFloats) * sizeof(float);
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef const __attribute__((address_space(1))) void *gbl_ptr_t;

__device__ __forceinline__ void dma16(const float *g, float *l)
{
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)g, (lds_ptr_t)l, 16, 0, 0);
}

// True when every row in [row_lo, row_hi] may attend every key of tile t
// (no explicit mask; the tile inside the keys and inside every row's causal
// window).
__device__ __forceinline__ bool tile_whole(const Params &p, int row_lo, int row_hi, int t)
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

// One workgroup per CU (its K/V stages fill the LDS), so at most two waves
// per SIMD: each wave may hold 256 VGPRs, which the operand double-buffering
// below uses. W waves per workgroup, one 16-row unit each.
template <int DK, int W, bool CAP>
__global__ __launch_bounds__(64 * W, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_kernel(Params p, int split, int z0)
{
    using LD = TiledLds<DK>;
    constexpr int NU = DK / 32;                // score chain steps
    constexpr int NQ = DK / 64;                // 64-dim output groups
    constexpr int NI = kTile * DK / 256 / W;   // DMA pieces per wave per array
    constexpr int ROWS = W * kRows;            // rows of the workgroup
    constexpr int NL = LD::spanBlocks;         // span accumulator blocks kept in LDS
    static_assert(NI * W * 256 == kTile * DK, "whole 1 KiB pieces per wave");
    static_assert(ROWS == kTiledRows, "LDS span blocks sized for the workgroup");
    extern __shared__ float lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    // Blocks cycle over the KV heads first (the dispatcher deals consecutive
    // blocks to the 8 XCDs, so each XCD's L2 serves one head's K/V), and the
    // query blocks run last-to-first (longest causal blocks first).
    const int nqb = gridDim.x / p.nkv;
    const int kvl = blockIdx.x % p.nkv;
    const int qb = nqb - 1 - (int)(blockIdx.x / p.nkv);
    const int kh = p.kh_first + kvl;
    const int fa = qb * ROWS;
    const int row = fa + w * kRows + col;
    // the wave's real rows
    const int wrow_lo = fa + w * kRows;
    const int wrow_hi = min(wrow_lo + kRows, p.nrows) - 1;
    const bool rin = row < p.nrows;
    const int query = rin ? row / p.group : 0;
    const int head = kh * p.group + (rin ? row % p.group : 0);
    // rows that are written (others are computed and dropped)
    const bool rout = rin && head >= p.h_lo && head < p.h_hi;

    const RowKeys rk = row_keys(p, row); // the row's allowed keys (boundary tiles)
    // Key range the workgroup can see.
    int64_t k_lo = 0, k_hi = p.nkeys;
    if (!p.mask && p.causal) {
        const int fb = min(fa + ROWS, p.nrows) - 1;
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

    // Q^T B operands: q[u][jj] = Q[row][32u + 8g + jj] * q_scale.
    float q[NU][8];
    {
        const float *qp = p.q + (int64_t)query * p.q_stride + (int64_t)head * p.dim;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int d = 32 * u + 8 * g + 4 * hh;
                const f4 x = ldg4(qp + (d < p.dim ? d : 0)) * p.q_scale;
                const f4 v = (rin && d < p.dim) ? x : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[u][4 * hh + j] = v[j];
            }
    }

    // chunk state (m, l, O) in registers; span (M1, L1) and total (M2, L2)
    // scalars in registers, their vectors in memory
    float m = kNegInf, l = 0.f, M1 = kNegInf, L1 = 0.f, M2 = kNegInf, L2 = 0.f;
    f4 O[NQ][4];
#pragma unroll
    for (int a = 0; a < NQ; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            O[a][j] = f4{0.f, 0.f, 0.f, 0.f};
    bool processed = false; // this wave computed a tile of the current chunk
    bool bad = false;
    float *acc1 = p.out + (int64_t)query * p.o_stride + (int64_t)(head - p.h_base) * p.dim;
    float *acc2 = p.ws_o ? p.ws_o + ((int64_t)kvl * p.nrows_pad + row) * p.dk : nullptr;

    // HBM -> LDS copy of tile t into stage `buf` (K swizzled, V plain).
    // Below the padded head dim, a slot past the head's last dim copies the
    // head's first four dims instead, as the decode kernels load them: the
    // copy never leaves the head's row (the last head of the last key ends
    // the caller's buffer), Q is zero on those dims and their outputs are
    // dropped.
    auto load_tile = [&](int t, int buf) {
        float *ks = lds + buf * LD::stage;
        float *vs = ks + LD::tileFloats;
        const int64_t klast = p.nkeys - 1;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = w * NI + i;          // 1 KiB piece of the tile
            const int f = 256 * j + 4 * lane;  // float offset of this lane's 16 bytes
            const int key = f / DK;
            const int pos = (f % DK) / 4;      // 16-byte chunk slot in the row
            const int64_t kt = (int64_t)t * kTile + key;
            const int64_t kc = kt < klast ? kt : klast;
            const int64_t off = (int64_t)kh * p.dim;
            const int kd = 4 * (pos ^ (key & 7));
            const int vd = 4 * pos;
            dma16(key_row(p, kc) + off + (kd < p.dim ? kd : 0), ks + 256 * j);
            dma16(value_row(p, kc) + off + (vd < p.dim ? vd : 0), vs + 256 * j);
        }
    };

    // Where the span accumulator (the row's output slot until the last
    // merge) and the running total keep natural dims 64a + 16g + 4i ..: in a
    // whole 64-dim block the 16-byte slots are stored with g and i swapped,
    // so the four lanes of a row in one load or store (g = 0 .. 3) cover one
    // contiguous 64-byte sector instead of 16 bytes of four sectors; a
    // partial last block keeps the natural order.
    auto acc_pos = [&](int a, int i) {
        return 64 * a + 64 <= p.dim ? 64 * a + 16 * i + 4 * g : 64 * a + 16 * g + 4 * i;
    };
    // Blocks a < NL of the span accumulator stay in LDS instead, private to
    // the wave: 256 bytes per row, the lane's 16-byte slot 4g + i XOR-ed
    // with the row so that the 16 rows of one access hit distinct banks.
    float *const lspan = lds + LD::stageFloats + w * NL * kRows * 64;
    auto lacc = [&](int a, int i) -> f4 & {
        return *(f4 *)(lspan + a * kRows * 64 + col * 64 + 4 * ((4 * g + i) ^ col));
    };

    // Chunk merge into the span, and at a span end the span merge into the
    // total (not the last merge: flush_last below).
    auto flush = [&](bool chunk, bool span_end) {
        // Opaque copies of the accumulator bases: the per-dim addresses are
        // then formed here (base + immediate offset). Otherwise the compiler
        // hoists them out of the tile loop as 32 pointers, which spill to
        // scratch, and every flush first reloads an address (the kernel ran
        // 4-5 % slower that way).
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
                    if (64 * a + 16 * g + 4 * i >= p.dim)
                        continue;
                    const int dm = acc_pos(a, i);
                    f4 s1 = f4{0.f, 0.f, 0.f, 0.f};
                    if (!first1)
                        s1 = a < NL ? lacc(a, i) : ldg4(a1 + dm);
                    if (chunk) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            s1[j] = merge_value(s1[j], O[a][j][i], f1);
                    }
                    if (!span_end) {
                        if (a < NL)
                            lacc(a, i) = s1;
                        else
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

    // The last merge: the chunk into the span, the span into the total,
    // normalised into the output. The output's natural order overwrites the
    // span accumulator's slots in another order, so every accumulator value
    // is loaded first (after the tiles: Q^T's registers are free).
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
                if (!first1 && 64 * a + 16 * g + 4 * i < p.dim)
                    s1v[a][i] = a < NL ? lacc(a, i) : ldg4(a1 + acc_pos(a, i));
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
                const int d = 64 * a + 16 * g + 4 * i;
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

    if (t_lo < t_hi) {
        load_tile(t_lo, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    for (int t = t_lo; t < t_hi; ++t) {
        const int buf = (t - t_lo) & 1;
        if (t + 1 < t_hi)
            load_tile(t + 1, buf ^ 1);
        const float *ks = lds + buf * LD::stage;
        const float *vs = ks + LD::tileFloats;

        // Masks. Without an explicit mask, a tile that every row of the wave
        // sees whole needs no per-key test (padding rows may then count as
        // allowed: their columns never reach a real row's state).
        bool ok[2][4];
        bool any = false;
        if (tile_whole(p, wrow_lo, wrow_hi, t)) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ok[b][r] = true;
            any = true;
        } else {
            any = tile_keys(chunk_of(rk, (int64_t)t * kTile), 0, g, ok);
        }
        if (__any(any)) {
            // score chain, the next u-step's K operands read ahead of the MFMAs
            f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
            f4 ka[2][2][2]; // [u parity][b][hh]
            auto read_k = [&](int u, int sl) {
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int c4 = 8 * u + 2 * g + hh;
                        ka[sl][b][hh] =
                            *(const f4 *)(ks + (16 * b + col) * DK + 4 * (c4 ^ (col & 7)));
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
            // the first V operands are read while the softmax runs
            f4 vb[2][4]; // [half-group parity][r]
            auto read_v = [&](int hg, int sl) { // half-group hg = 2a + b
                const int a = hg >> 1, b = hg & 1;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    vb[sl][r] = *(const f4 *)(vs + (16 * b + 4 * g + r) * DK + 64 * a + 4 * col);
            };
            read_v(0, 0);
            float s[2][4], pr[2][4];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[b][r] = acc[b][r];
            cap_scores<CAP>(p, s);
            bad |= bad_scores(s, ok);
            const float mn = fmaxf(m, tile_max(s, ok));
            const float ms = safe_max(mn);
            const float alpha = fexp(m - ms);
            const float rs = tile_probs(s, ok, ms, pr);
            l = __builtin_fmaf(l, alpha, rs);
            m = mn;
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

        if (t + 1 < t_hi)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();

        if (!split && t + 1 < t_hi) { // (the last tile's merge follows the loop)
            const bool chunk_end = ((t + 1) % kTilesPerChunk) == 0;
            const bool span_end = ((t + 1) % kSpanTiles) == 0;
            if ((chunk_end && processed) || span_end)
                flush(chunk_end && processed, span_end);
            if (chunk_end)
                processed = false;
        }
    }
    if (bad)
        atomicOr(p.err, kErrScore);
    if (!split) {
        // with no key at all: 0/0, flagged like any non-finite output
        flush_last(t_lo < t_hi && processed);
        return;
    }

    // O[a][j][i] holds dim 64a + 16g + 4i + j of `row`.
    if (!rin)
        return;
    const int64_t slot = ((int64_t)kvl * p.nrows_pad + row) * p.nch + z0 + blockIdx.z;
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
            stg4(wo + d, v);
        }
    if (g == 0) {
        stg(p.ws_ml + 2 * slot, m);
        stg(p.ws_ml + 2 * slot + 1, l);
    }
}

constexpr int kMaxDevices = 64;

// Compute units of the current device (cached per device; callers on other
// threads with their own contexts may race here, so the cache is atomic).
int device_cus()
{
    static std::atomic<int> cached[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Dynamic LDS above 64 KiB must be allowed once per kernel and device; a
// repeated call from a racing thread is harmless.
template <int DK, int W, bool CAP> static hipError_t configure_tiled()
{
    static std::atomic<bool> configured[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= kMaxDevices)
        return hipErrorInvalidDevice;
    if (!configured[dev].load(std::memory_order_acquire)) {
        e = hipFuncSetAttribute((const void *)tiled_kernel<DK, W, CAP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)TiledLds<DK>::bytes);
        if (e != hipSuccess)
            return e;
        configured[dev].store(true, std::memory_order_release);
    }
    return hipSuccess;
}

// Chunks of a split launch to run as (16-row unit, chunk) items of the
// pipelined kernel: the last chunk when the tiled items (nqb row blocks per
// KV head, one workgroup per CU) leave a last round of at most one chunk's
// items and the tail's items fit one round. 0: none.
int tiled_tail_chunks(const Params &p, int nqb, int cus)
{
    const int64_t per_chunk = (int64_t)nqb * p.nkv;
    const int64_t items = per_chunk * p.nch;
    if (cus <= 0 || items <= cus || items % cus == 0 || items % cus > per_chunk)
        return 0;
    const int64_t units = (p.nrows + kRows - 1) / kRows;
    if (p.nch < 2 || units * p.nkv > cus)
        return 0;
    return 1;
}

template <int DK, bool CAP>
static hipError_t launch_tiled_grid(const Params &p, int split, dim3 grid, hipStream_t stream)
{
    const hipError_t e = configure_tiled<DK, kTiledWaves, CAP>();
    if (e != hipSuccess)
        return e;
    tiled_kernel<DK, kTiledWaves, CAP>
        <<<grid, 64 * kTiledWaves, TiledLds<DK>::bytes, stream>>>(p, split, 0);
    return hipGetLastError();
}

template <int DK>
static hipError_t launch_tiled_dk(const Params &p, int split, hipStream_t stream, bool *merged)
{
    const int nqb = (p.nrows + kTiledRows - 1) / kTiledRows;
    const int tail = split ? tiled_tail_chunks(p, nqb, device_cus()) : 0;
    const dim3 grid(nqb * p.nkv, 1, split ? p.nch - tail : 1);
    hipError_t e = p.softcap > 0.0f ? launch_tiled_grid<DK, true>(p, split, grid, stream)
                                    : launch_tiled_grid<DK, false>(p, split, grid, stream);
    if (e != hipSuccess || !tail)
        return e;
    // the tail runs after every other chunk's partial is written: with all
    // chunks in one span it merges them into the output itself
    const bool merge_out = p.nspan == 1;
    e = fan_supported(DK) ? launch_fan_chunk(p, p.nch - 1, merge_out, stream)
                          : launch_pipe_kv_chunks(p, p.nch - tail, tail, merge_out, stream);
    if (e == hipSuccess && merge_out)
        *merged = true;
    return e;
}

hipError_t launch_tiled_wide(const Params &p, int split, hipStream_t stream, bool *merged);
int tiled_wide_rows();

// Rows of one workgroup: 128 up to head dim 256; 64 at 512 (tiled_wide.hip).
int tiled_rows(int dk)
{
    return dk > 256 ? tiled_wide_rows() : kTiledRows;
}

// *merged: set when the launch itself wrote the merged output of a split
// launch (no combine needed).
hipError_t launch_tiled(const Params &p, int split, hipStream_t stream, bool *merged)
{
    *merged = false;
    switch (p.dk) {
    case 64: return launch_tiled_dk<64>(p, split, stream, merged);
    case 128: return launch_tiled_dk<128>(p, split, stream, merged);
    case 256: return launch_tiled_dk<256>(p, split, stream, merged);
    case 512: return launch_tiled_wide(p, split, stream, merged);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pcl
