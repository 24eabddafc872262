// Canonical arithmetic of the attention backend (gfx950 device code).
//
// Every kernel in this library computes one (query, head) row with exactly
// the operation sequence defined here, so results are bitwise independent of
// which kernel ran, how rows were batched and how keys were split between
// workgroups:
//
//   keys are cut into chunks of kChunk = 256 keys (by key index), a chunk
//   into tiles of kTile = 32 keys, a tile into two MFMA blocks of 16 keys;
//
//   score s[key][row]: one v_mfma_f32_16x16x4f32 chain (A = 16 keys x 4
//   dims, B = 4 dims x 16 rows) over u = 0..DK/32-1, jj = 0..7, the lane
//   group g = lane/16 supplying dim 32u + 8g + jj;
//
//   per tile, online softmax inside the chunk (state m, l, O):
//     t_max = max over allowed scores; m' = max(m, t_max);
//     ms = m' or 0 when m' = -inf; alpha = exp(m - ms);
//     p = allowed ? exp(s - ms) : 0; l = fma(l, alpha, rowsum(p));
//     O = O * alpha, then O += P.V by one MFMA chain per 16x16 output block
//     over (b, r) = (0..1, 0..3), the lane group g supplying key
//     16b + 4g + r;
//
//   merge of a partial (m, l, O) into (M, L, Acc): M' = max(M, m);
//   a = exp(M - Ms); b = exp(m - Ms) with Ms = M' or 0 when M' = -inf;
//   L = fma(L, a, l*b); Acc = fma(Acc, a, O*b);
//
//   chunks are grouped into spans of kSpanChunks = 16 chunks (4096 keys, by
//   chunk index): the chunks of a span are merged in ascending order from
//   (-inf, 0, 0), then the spans are merged in ascending order from
//   (-inf, 0, 0); the output is Acc / L. Two levels keep the longest serial
//   merge chain of the split-KV combine short (16 + keys/4096 steps).
//
// A tile, chunk or span with no allowed key for a row leaves that row's
// state bit-unchanged through these formulas, so kernels may skip such work.
// The P.V chain's assignment of output dims to lanes does not change any
// value, so kernels choose it freely; the score chain's assignment of dims to
// MFMA k slots is fixed as above.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pcl {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 32;
constexpr int kChunk = 256;
constexpr int kTilesPerChunk = kChunk / kTile;
constexpr int kSpanChunks = 16;
constexpr int kSpanTiles = kSpanChunks * kTilesPerChunk;
constexpr int kRows = 16;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kNegInf = -__builtin_huge_valf();

// Device error flag bits: a non-finite allowed score, a non-finite output, a
// non-finite head-transform value, (8: the output block's non-finite value,)
// a workgroup that gave up waiting for the scores of the other workgroups of
// its chunk (its results are not valid).
enum ErrorBits { kErrScore = 1, kErrOutput = 2, kErrTransform = 4, kErrWait = 16 };

// Launch parameters shared by every kernel (host fills, passed by value).
struct Params {
    // queries: query i, head h at q + i*q_stride + h*dim
    const float *q;
    int64_t q_stride;
    int nq;
    float q_scale;
    // logit soft-cap (0 = off) and its f32 reciprocal
    float softcap, inv_softcap;
    // keys/values: key t < n0 in segment 0, the rest in segment 1
    const float *k0, *v0;
    int64_t n0;
    const float *k1, *v1;
    int64_t nkeys;
    int64_t kv_stride; // floats between consecutive keys (kvheads*dim)
    int dim, group;
    int kh_first; // first KV head of the launch
    int nkv;      // KV heads in the launch
    int h_lo, h_hi; // query heads written
    // masks
    const uint8_t *mask;
    int64_t mask_stride;
    int causal;
    int64_t window;
    int64_t first_key, first_query;
    // output: query i, head h at out + i*o_stride + (h - h_base)*dim
    float *out;
    int64_t o_stride;
    int h_base;
    // rows: flat (query, head-in-group) index f = query*group + j
    int nrows;     // nq*group
    int nrows_pad; // rounded up to whole 16-row units
    int units;     // nrows_pad / 16
    // chunk partials for the ordered combine
    float *ws_o;  // [nkv][nrows_pad][nch][DK]
    float *ws_ml; // [nkv][nrows_pad][nch][2]
    int c_lo;     // first chunk of the launch (absolute chunk index)
    int nch;      // chunks of the launch
    // span partials of the two-level combine
    float *ws2_o;  // [nkv][nrows_pad][nspan][DK]
    float *ws2_ml; // [nkv][nrows_pad][nspan][2]
    int s_lo;      // first span of the launch (absolute span index)
    int nspan;     // spans of the launch
    int dk;        // padded head dim of the launch
    // the spread decode's published scores, [items][16 blocks][4][64 lanes]
    // words of (epoch, score bits), and the launch's epoch
    uint64_t *ws_tag;
    uint32_t epoch;
    int max_polls; // bound of every wait for another workgroup's words
    // the spread decode's chunk partials as published words (partial_words
    // below), which the launch's own merge workgroups combine
    uint64_t *ws_ptag;
    int *err;
    // A one-token decode step's head transform, fused (sq null: none; q
    // unused): the token's raw rows (Q [qheads][dim], K and V
    // [kvheads][dim]; sv null: V is the raw K), the learned Q and K scales,
    // the (sin, cos) pairs of its position and the norm epsilon. Its
    // prepared K and V rows (snk, snv: [kvheads][dim]) are the launch's
    // last key, which the workgroups of that key's chunk write before they
    // read the chunk; the workgroups of the launch's first chunk write the
    // prepared queries to sqo ([qheads][dim]).
    const float *sq, *sk, *sv, *sqs, *sks, *srot;
    float *snk, *snv, *sqo;
    float seps;
};

// Global-memory accessors. Pointers taken from Params are generic, and a
// generic (flat) load counts against both the vector-memory and the LDS
// counters, so every LDS wait would also drain all outstanding HBM loads;
// casting to the global address space keeps the two counters apart.
typedef const __attribute__((address_space(1))) f4 *gf4_cptr;
typedef __attribute__((address_space(1))) f4 *gf4_ptr;
typedef const __attribute__((address_space(1))) float *gf_cptr;
typedef __attribute__((address_space(1))) float *gf_ptr;
typedef const __attribute__((address_space(1))) uint8_t *gu8_cptr;

__device__ __forceinline__ f4 ldg4(const float *p)
{
    return *(gf4_cptr)p;
}

// Streaming load for data read exactly once (decode K/V): the nontemporal
// hint keeps it from displacing reused lines; the HBM stream runs faster.
// s_waitcnt immediate for vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0
// and 15:14; expcnt 7 and lgkmcnt 15 wait for nothing), for
// __builtin_amdgcn_s_waitcnt. The compiler's own waits know this form (an
// inline-asm wait they would not).
constexpr int waitcnt_vm(int n)
{
    return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

// The same with lgkmcnt(0): every LDS access of the wave complete too.
constexpr int waitcnt_vm_lgkm0(int n)
{
    return (n & 15) | ((n >> 4) << 14) | (7 << 4);
}

__device__ __forceinline__ f4 ldg4_stream(const float *p)
{
    return __builtin_nontemporal_load((gf4_cptr)p);
}

__device__ __forceinline__ void stg4(float *p, f4 v)
{
    *(gf4_ptr)p = v;
}

__device__ __forceinline__ float ldg(const float *p)
{
    return *(gf_cptr)p;
}

__device__ __forceinline__ void stg(float *p, float v)
{
    *(gf_ptr)p = v;
}

__device__ __forceinline__ f4 mfma(float a, float b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// exp(x) as 2^(x*log2 e) on the hardware exp2; exp(0) = 1 and exp(-inf) = 0
// exactly, which the skip rules above rely on.
__device__ __forceinline__ float fexp(float x)
{
    return __builtin_amdgcn_exp2f(x * kLog2e);
}

__device__ __forceinline__ bool is_finite(float x)
{
    return __builtin_isfinite(x);
}

__device__ __forceinline__ const float *key_row(const Params &p, int64_t t)
{
    return t < p.n0 ? p.k0 + t * p.kv_stride : p.k1 + (t - p.n0) * p.kv_stride;
}

__device__ __forceinline__ const float *value_row(const Params &p, int64_t t)
{
    return t < p.n0 ? p.v0 + t * p.kv_stride : p.v1 + (t - p.n0) * p.kv_stride;
}

// Whether flat row `row` may attend key index `t`.
__device__ __forceinline__ bool allowed(const Params &p, int row, int64_t t)
{
    if (row >= p.nrows || t >= p.nkeys)
        return false;
    const int query = row / p.group;
    if (p.mask)
        return ((gu8_cptr)p.mask)[(int64_t)query * p.mask_stride + t] != 0;
    if (!p.causal)
        return true;
    const int64_t kp = p.first_key + t;
    const int64_t qp = p.first_query + query;
    return kp <= qp && (p.window == 0 || qp - kp < p.window);
}

// allowed() for one row over the keys [base, base + kChunk), with the row's
// constants hoisted out of the key loop: a key's test is then a range check
// against two per-lane bounds (chunk-relative), and, with an explicit mask,
// a byte of the row's mask read only for keys inside the range (so never
// past the mask row). Equal to allowed() for every key of the range.
struct RowKeys {
    int64_t lo, hi; // keys t with lo <= t <= hi pass the range
    gu8_cptr mask;  // the row's mask bytes, or null
    bool masked;    // whether the launch has a mask (the same for every lane)
};

struct ChunkKeys {
    int lo, hi;    // chunk-relative keys k with lo <= k <= hi pass the range
    gu8_cptr mask; // the row's mask byte of the chunk's first key, or null
    bool masked;   // whether the launch has a mask (the same for every lane)
};

__device__ __forceinline__ RowKeys row_keys(const Params &p, int row)
{
    const bool in = row < p.nrows;
    const int query = in ? row / p.group : 0;
    RowKeys r;
    r.lo = 0;
    r.hi = in ? p.nkeys - 1 : -1;
    if (!p.mask && p.causal) {
        // kp <= qp and qp - kp < window with kp = first_key + t, qp = first_query + query
        const int64_t rel = p.first_query + query - p.first_key;
        r.hi = r.hi < rel ? r.hi : rel;
        if (p.window)
            r.lo = rel - p.window + 1;
    }
    r.mask = p.mask ? (gu8_cptr)p.mask + (int64_t)query * p.mask_stride : nullptr;
    r.masked = p.mask != nullptr;
    return r;
}

// The keys [base, base + kChunk) of a row.
__device__ __forceinline__ ChunkKeys chunk_of(const RowKeys &r, int64_t base)
{
    const int64_t lo = r.lo - base, hi = r.hi - base;
    ChunkKeys c;
    c.lo = (int)(lo < 0 ? 0 : lo > kChunk ? kChunk : lo);
    c.hi = (int)(hi < -1 ? -1 : hi > kChunk - 1 ? kChunk - 1 : hi);
    c.mask = r.mask ? r.mask + base : nullptr;
    c.masked = r.masked;
    return c;
}

__device__ __forceinline__ ChunkKeys chunk_keys(const Params &p, int row, int64_t base)
{
    return chunk_of(row_keys(p, row), base);
}

// Allowed flags of keys k0 + 4g + r (r = 0..3) of a chunk; true when any is.
__device__ __forceinline__ bool block_keys(const ChunkKeys &c, int k0, int g, bool ok[4])
{
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int k = k0 + 4 * g + r;
        ok[r] = k >= c.lo && k <= c.hi;
    }
    if (c.masked) {
        uint8_t m[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            m[r] = ok[r] ? c.mask[k0 + 4 * g + r] : (uint8_t)1;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            ok[r] = ok[r] && m[r] != 0;
    }
    bool any = false;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        any |= ok[r];
    return any;
}

// Allowed flags of the lane's eight keys of tile t (chunk-relative keys
// 32t + 16b + 4g + r); true when any is.
__device__ __forceinline__ bool tile_keys(const ChunkKeys &c, int t, int g, bool ok[2][4])
{
    const bool a0 = block_keys(c, t * kTile, g, ok[0]);
    const bool a1 = block_keys(c, t * kTile + 16, g, ok[1]);
    return a0 || a1;
}

// Butterflies across the four 16-lane groups: each lane combined with lane ^
// 16 or lane ^ 32. The gfx950 permlane swaps exchange 16-lane rows (32-lane
// halves) between two registers in a few cycles, where a shuffle goes
// through the LDS unit; given the same value twice, their two results hold
// every lane's own value and its partner's, and max and + are commutative,
// so the results equal x op shfl_xor(x, k) bit for bit.
__device__ __forceinline__ float max_xor16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float max_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float add_xor16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float add_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Max of a tile's allowed scores for the lane's row (column lane%16): the
// lane's eight values, then across the four lane groups.
__device__ __forceinline__ float tile_max(const float s[2][4], const bool ok[2][4])
{
    float m = kNegInf;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            m = ok[b][r] ? fmaxf(m, s[b][r]) : m;
    m = max_xor16(m);
    m = max_xor32(m);
    return m;
}

// p = exp(s - ms) for allowed keys (0 otherwise) and their row sum, by a
// fixed tree: in-lane pairs, then lane groups xor 16, xor 32.
__device__ __forceinline__ float tile_probs(const float s[2][4], const bool ok[2][4], float ms,
                                            float p[2][4])
{
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            p[b][r] = ok[b][r] ? fexp(s[b][r] - ms) : 0.0f;
    const float x0 = (p[0][0] + p[0][1]) + (p[0][2] + p[0][3]);
    const float x1 = (p[1][0] + p[1][1]) + (p[1][2] + p[1][3]);
    float x = x0 + x1;
    x = add_xor16(x);
    x = add_xor32(x);
    return x;
}

// Safe subtrahend for a running max (0 when nothing was allowed yet).
__device__ __forceinline__ float safe_max(float m)
{
    return m == kNegInf ? 0.0f : m;
}

// Factors of the ordered chunk merge.
struct MergeFactors {
    float m, a, b;
};

__device__ __forceinline__ MergeFactors merge_factors(float M, float m)
{
    MergeFactors f;
    f.m = fmaxf(M, m);
    const float ms = safe_max(f.m);
    f.a = fexp(M - ms);
    f.b = fexp(m - ms);
    return f;
}

__device__ __forceinline__ float merge_value(float acc, float o, const MergeFactors &f)
{
    return __builtin_fmaf(acc, f.a, o * f.b);
}

// Merge state of four consecutive dims of one row (the per-element merge
// above, with the shared M and L kept once).
struct Merged4 {
    float M, L;
    f4 acc;
};

// Branch-free: an empty part (m = -inf, l = 0, O = +0) leaves the state
// bit-unchanged through the formulas (a = 1 and b = 0, or a = b = 0 on an
// empty state), so the factors of consecutive merges, which depend only on
// the running maxima, can be computed ahead of the fma chain.
__device__ __forceinline__ void merge_into4(Merged4 &s, float m, float l, f4 o)
{
    const MergeFactors f = merge_factors(s.M, m);
    s.L = merge_value(s.L, l, f);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        s.acc[j] = merge_value(s.acc[j], o[j], f);
    s.M = f.m;
}

typedef float f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f2 ldg2(const float *p)
{
    return *(const __attribute__((address_space(1))) f2 *)p;
}

// The ordered merge of chunks [c0, c1) of one span (launch-relative chunk
// indices) for four consecutive dims of one row (slot0: the row's first
// chunk slot), as the combine kernels run it: one batch of loads over the
// span's kSpanChunks slots (slots past c1 re-read chunk c0 and merge as
// empty parts, which leave the state bit-unchanged), merged into
// (-inf, 0, 0) in ascending order.
__device__ __forceinline__ Merged4 merge_chunks4(const Params &p, int64_t slot0, int d, int c0,
                                                 int c1)
{
    f2 ml[kSpanChunks];
    f4 ov[kSpanChunks];
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i) {
        const int64_t cc = slot0 + (c0 + i < c1 ? c0 + i : c0);
        ml[i] = ldg2(p.ws_ml + 2 * cc);
        ov[i] = ldg4(p.ws_o + cc * p.dk + d);
    }
    Merged4 s = {kNegInf, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < kSpanChunks; ++i) {
        // chunks past the span merge as empty parts (no-ops)
        const bool in = c0 + i < c1;
        merge_into4(s, in ? ml[i].x : kNegInf, in ? ml[i].y : 0.f,
                    in ? ov[i] : f4{0.f, 0.f, 0.f, 0.f});
    }
    return s;
}

// ---- Published words -------------------------------------------------
// Data exchanged between workgroups of one launch without flags or fences:
// each value is one 64-bit word (the launch's epoch, the value's bits),
// written with a device-coherent 64-bit store, which lands whole; a reader
// accepts a word only when it carries the current epoch. The words live in
// a workspace region that holds nothing else (zero when allocated; epochs
// are never zero), so a stale word carries an earlier epoch. Every wait is
// bounded: a wait for another workgroup's scores by the launch's max_polls
// polls (kMaxPolls unless the context set another limit), after which the
// waiting wave forms what is missing itself; a wait of the merge workgroups
// (which only ever wait for workgroups dispatched before them, and those
// always finish) by kMergeMaxPolls, a guard against a fault elsewhere.

constexpr int kMaxPolls = 1 << 16;
constexpr int kMergeMaxPolls = 1 << 20;
// Chunks whose partial words a merging thread requests per batch of loads.
constexpr int kMergeBatch = 8;

typedef __attribute__((address_space(1))) uint64_t *gu64_ptr;

__device__ __forceinline__ uint64_t take(const uint64_t *p)
{
    return __hip_atomic_load((gu64_ptr)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Words of a launch whose writing and reading workgroups share one XCD (the
// spread decode's local form) are stored plainly: the store lands in that
// XCD's L2, where the readers' device-coherent loads (take) find it, and
// goes no further. Measured on MI355X (a workgroup writing one word, others
// polling it): a device-coherent store is seen 400 ns later on the same XCD
// and 530 ns later on another; a plain store 240 ns later on the same XCD
// (850 ns on another: it is still seen); plain and workgroup-scope loads
// never see another CU's store (they hit the reader's L1).
template <bool LOCAL>
__device__ __forceinline__ void publish_to(uint64_t *p, uint32_t epoch, float v)
{
    const uint64_t word = ((uint64_t)epoch << 32) | (uint64_t)__float_as_uint(v);
    if (LOCAL)
        __hip_atomic_store((gu64_ptr)p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
        __hip_atomic_store((gu64_ptr)p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Published chunk partials of the spread decode: row `row` (a real row) of
// launch KV head kvl, launch chunk ci, at
// ws_ptag + (((kvl * nrows + row) * nch + ci) * (dk + 2)): O[dk], then m, l.
__device__ __forceinline__ uint64_t *partial_words(const Params &p, int kvl, int row, int ci)
{
    return p.ws_ptag + (((int64_t)kvl * p.nrows + row) * p.nch + ci) * (p.dk + 2);
}

// Waits, cheaply, until the m words of chunks ci = first, first + step, ...
// below last of row slot0 (the row's first chunk slot) carry the epoch (the
// wave's lanes together cover their rows' chunks). Polling every word of
// every partial instead slowed the producing workgroups' own loads. False
// when the wait gave up.
template <int SLEEP = 8>
__device__ __forceinline__ bool wait_partials(const Params &p, int64_t slot0, int first,
                                              int step, int last)
{
    const int stride = p.dk + 2;
    for (int polls = 0;; ++polls) {
        bool fresh = true;
        for (int ci = first; ci < last; ci += step)
            fresh &= (uint32_t)(take(p.ws_ptag + (slot0 + ci) * stride + p.dk) >> 32) == p.epoch;
        if (__all(fresh))
            return true;
        if (polls >= kMergeMaxPolls)
            return false;
        __builtin_amdgcn_s_sleep(SLEEP);
    }
}

// One batch of a span's ordered chunk merge from published words: chunks
// c0 + b0 + i (i < B; those at or past c1 are neither loaded nor merged) of
// row slot0, four dims from d, merged into s in ascending order (c0, b0 and
// c1 must be the same for every lane of the wave). Every word is re-checked
// (and the batch reloaded until all carry the epoch). False when the wait
// gave up.
template <int B = kMergeBatch, int SLEEP = 2>
__device__ __forceinline__ bool merge_words_batch(const Params &p, int64_t slot0, int c0,
                                                  int b0, int c1, int d, Merged4 &s)
{
    const int stride = p.dk + 2;
    const int n = c1 - (c0 + b0); // chunks of the batch that exist (uniform)
    uint64_t wm[B], wl[B], wo[B][4];
    bool ok = true;
    for (int polls = 0; n > 0; ++polls) {
        // every present chunk's words requested back to back (the checks
        // below, outside these uniform branches, wait for them together)
#pragma unroll
        for (int i = 0; i < B; ++i) {
            if (i >= n)
                continue;
            const uint64_t *w = p.ws_ptag + (slot0 + c0 + b0 + i) * stride;
            wm[i] = take(w + p.dk);
            wl[i] = take(w + p.dk + 1);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wo[i][j] = take(w + d + j);
        }
        bool fresh = true;
#pragma unroll
        for (int i = 0; i < B; ++i) {
            if (i >= n)
                continue;
            fresh &= (uint32_t)(wm[i] >> 32) == p.epoch && (uint32_t)(wl[i] >> 32) == p.epoch;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                fresh &= (uint32_t)(wo[i][j] >> 32) == p.epoch;
        }
        if (__all(fresh))
            break;
        if (polls >= kMergeMaxPolls) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(SLEEP);
    }
    // absent chunks would merge as empty parts, which leave the state
    // bit-unchanged; skipping them takes their dependent merges off the chain
#pragma unroll
    for (int i = 0; i < B; ++i) {
        if (i >= n)
            continue;
        f4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            o[j] = __uint_as_float((uint32_t)wo[i][j]);
        merge_into4(s, __uint_as_float((uint32_t)wm[i]), __uint_as_float((uint32_t)wl[i]), o);
    }
    return ok;
}

// Logit soft-cap: cap * tanh(s / cap) in f32, one definition for every
// kernel. tanh(t) is an odd Taylor polynomial through t^9 for |t| < 1/4
// (truncation below 1e-8 relative) and (1 - e) / (1 + e) with e = exp(-2|t|)
// above (relative error a few 1e-7), so a capped score is within about 1e-6
// relative of the exact cap; +-inf becomes +-cap and NaN stays NaN.
__device__ __forceinline__ float soft_cap(float s, float cap, float inv_cap)
{
    const float t = s * inv_cap;
    const float a = fabsf(t);
    const float t2 = t * t;
    const float small =
        t + t * t2 * (-0.333333333f + t2 * (0.133333333f + t2 * (-0.0539682540f +
                                                                   t2 * 0.0218694885f)));
    const float e = fexp(-2.0f * a);
    const float large = copysignf((1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e), t);
    return cap * (a < 0.25f ? small : large);
}

// Applies the descriptor's soft-cap (when on) to a tile's raw scores.
// Kernels instantiated per cap setting pass CAP = false for launches without
// a cap, which removes the code; the others test the launch at run time.
template <bool CAP = true>
__device__ __forceinline__ void cap_scores(const Params &p, float s[2][4])
{
    if (CAP && p.softcap > 0.0f) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s[b][r] = soft_cap(s[b][r], p.softcap, p.inv_softcap);
    }
}

// True when any allowed score of the lane is not finite.
__device__ __forceinline__ bool bad_scores(const float s[2][4], const bool ok[2][4])
{
    bool bad = false;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            bad |= ok[b][r] && !is_finite(s[b][r]);
    return bad;
}

} // namespace pcl
