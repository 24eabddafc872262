// Host side of the attention backend: contexts, descriptor validation,
// kernel choice and the C ABI of include/pcl_attention.h.
#include "attention_device.hpp"
#include "pcl_attention.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

namespace pcl {
hipError_t launch_split_kv(const Params &p, hipStream_t stream);
hipError_t launch_combine(const Params &p, hipStream_t stream);
hipError_t launch_pipe_kv(const Params &p, hipStream_t stream);
hipError_t launch_tiled(const Params &p, int split, hipStream_t stream, bool *merged);
hipError_t launch_fan_kv(const Params &p, hipStream_t stream);
hipError_t launch_spread_kv(const Params &p, hipStream_t stream);
int tiled_rows(int dk);
int spread_slices(int dk);
int device_cus();
// published score words (64-bit) of one spread item: 16 key blocks x 4 x 64
// lanes
constexpr size_t kSpreadWordsPerItem = 2 * kTilesPerChunk * 4 * 64;
} // namespace pcl

using pcl::Params;

#include "context.hpp"

namespace {

constexpr int kMaxDim = 512;
constexpr int64_t kMaxKeys = (int64_t)1 << 30;
constexpr int64_t kMaxRowsTimesKvHeads = (int64_t)1 << 22;
constexpr int kTiledMaxDk = 512;
constexpr int kPipeMaxDk = 512;
// Launches of few (chunk, 16-row unit, KV head) items, each latency-bound
// in one workgroup, take the fanned kernel (each item over eight waves),
// where it was measured faster on MI355X (A/B of every kernel per shape,
// inputs larger than the last-level cache): at head dim 512 below 512
// items (2K-32K-key decodes of 2 KV heads: 34-58 us against 48-61 us for
// the four-phase and 59-67 us for the pipelined kernel; 8 queries over
// 1279 keys 34 against 97 us chunk-split tiled; at 512 items, a 64K decode,
// the pipelined kernel is 9 % faster); at head dim 256 up to 128 items
// (4K-key decode 28 against 33 us pipelined; at 256 items pipelined is
// 11 % faster), or up to 512 items of at least two units (8-32 queries over
// 3194 keys: 27-46 against 36-55 us). Head dim 128 never (pipelined 8 %
// faster at 256 items).
constexpr int64_t kFanMaxItems512 = 512;
constexpr int64_t kFanMaxItems256 = 128;
constexpr int64_t kFanMaxItems256Units = 512;

bool fan_preferred(int dk, int64_t units, int64_t items, int64_t nch)
{
    if (nch < 2)
        return false;
    if (dk == 512)
        return items < kFanMaxItems512;
    if (dk == 256)
        return items <= kFanMaxItems256 || (units >= 2 && items <= kFanMaxItems256Units);
    return false;
}
// The spread decode's slices (dk/32 per item; up to head dim 256 a two-wave
// workgroup with 48 KiB of LDS each, three per CU, or two per four-wave
// workgroup when they take at most two per CU; at 512 a one-wave workgroup
// with 48 KiB of LDS, three per CU) all fit on the chip at once up to this
// many per CU of the device the launch runs on (768 on a whole MI355X;
// fewer on a partitioned one). Its workgroups wait for each other, so it is chosen only
// within that bound and within the items its score-word region holds
// (requested beyond them, the pipelined kernel runs).
constexpr int64_t kSpreadSlicesPerCu = 3;
constexpr int kMi355xCus = 256;
// Every non-empty workspace begins with the spread decode's region of
// published words: the score words of up to kSpreadMaxItems (chunk, unit,
// KV head) items, then their chunk partials (16 rows x (256 + 2) words an
// item). No other data ever lands there, so a stale word carries an earlier
// launch's epoch and never the current one.
constexpr int64_t kSpreadMaxItems = 128;
constexpr size_t kSpreadScoreWords = (size_t)kSpreadMaxItems * pcl::kSpreadWordsPerItem;
constexpr size_t kSpreadPartWords = (size_t)kSpreadMaxItems * pcl::kRows * (256 + 2);
constexpr size_t kTagFloats = 2 * (kSpreadScoreWords + kSpreadPartWords);

// Epochs of spread launches, per device: every launch on a device takes a
// new one (shared by all contexts and the allocation-free scratch). The
// counter is 64-bit: its low word is the epoch a kernel compares, its high
// word the generation, which grows each time the epoch wraps. A region of
// published words holds only zeros and words of one generation's launches
// (whose epochs are unique); a launch of a later generation zeroes the
// region first, so a word left from before a wrap can never carry the
// current epoch.
constexpr int kMaxEpochDevices = 64;
std::atomic<uint64_t> g_epoch[kMaxEpochDevices];

struct Epoch {
    uint32_t epoch;
    uint32_t generation;
};

std::atomic<uint64_t> &epoch_counter(int device)
{
    return g_epoch[device >= 0 && device < kMaxEpochDevices ? device : 0];
}

Epoch next_epoch(int device)
{
    std::atomic<uint64_t> &e = epoch_counter(device);
    uint64_t v = e.fetch_add(1, std::memory_order_relaxed) + 1;
    while ((uint32_t)v == 0) // 0 is the value of a word never written
        v = e.fetch_add(1, std::memory_order_relaxed) + 1;
    return Epoch{(uint32_t)v, (uint32_t)(v >> 32)};
}

// The generation of the device's next launch (what a region zeroed now is
// valid for).
uint32_t current_generation(int device)
{
    return (uint32_t)((epoch_counter(device).load(std::memory_order_relaxed) + 1) >> 32);
}

void report(const char *what, hipError_t e)
{
    std::fprintf(stderr, "pcl_attention: %s: %s\n", what, hipGetErrorString(e));
}

bool aligned16(const void *p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int64_t round_up(int64_t x, int64_t m)
{
    return (x + m - 1) / m * m;
}

// A validated launch: parameters, kernel and workspace.
struct Plan {
    Params p;
    int kernel = PCL_KERNEL_SPLIT_KV;
    // workspace floats: the spread decode's score words, then chunk and
    // span partials (or the tiled kernel's running totals)
    size_t ws_floats = 0;
    size_t part_floats = 0;
    bool empty = false;    // nothing to compute
};

// Visible key chunks of the whole launch (descriptor masks only narrow it).
void chunk_range(const pcl_attention_desc &d, int64_t nkeys, int64_t *c_lo, int64_t *c_hi,
                 bool *none)
{
    int64_t k_lo = 0, k_hi = nkeys;
    if (!d.mask && d.causal) {
        k_hi = std::min(std::max(d.first_query + d.nq - 1 - d.first_key + 1, (int64_t)0), nkeys);
        if (d.window)
            k_lo = std::min(std::max(d.first_query - d.window + 1 - d.first_key, (int64_t)0),
                            nkeys);
    }
    *none = k_hi <= k_lo;
    *c_lo = k_lo / pcl::kChunk;
    *c_hi = (k_hi + pcl::kChunk - 1) / pcl::kChunk;
}

// Workgroups of a spread launch (its slices: two-wave ones up to head dim
// 256, one-wave ones at 512), or 0 when its items or their chunk partials
// exceed the published-word region.
int64_t spread_workgroups(int dk, int64_t nrows, int64_t nkv, int64_t nch)
{
    const int64_t units = (nrows + pcl::kRows - 1) / pcl::kRows;
    if (nch * nkv * units > kSpreadMaxItems)
        return 0;
    if (nch > 1 && nkv * nrows * nch * (dk + 2) > (int64_t)kSpreadPartWords)
        return 0;
    return nch * nkv * units * pcl::spread_slices(dk);
}

// cus: compute units of the device the launch runs on (the spread decode's
// workgroups must all be resident at once).
int choose_kernel(int requested, int dk, int64_t nrows, int64_t nkv, int64_t nch, int cus)
{
    const int64_t spread = spread_workgroups(dk, nrows, nkv, nch);
    const bool spread_fits = spread > 0 && spread <= kSpreadSlicesPerCu * (int64_t)cus;
    if (requested == PCL_KERNEL_SPREAD_KV)
        return spread_fits ? requested : dk <= kPipeMaxDk ? PCL_KERNEL_PIPE_KV
                                                           : PCL_KERNEL_SPLIT_KV;
    if (requested == PCL_KERNEL_TILED || requested == PCL_KERNEL_TILED_SPLIT)
        return dk <= kTiledMaxDk ? requested : PCL_KERNEL_SPLIT_KV;
    if (requested == PCL_KERNEL_SPLIT_KV)
        return requested;
    if (requested == PCL_KERNEL_PIPE_KV)
        return dk <= kPipeMaxDk ? requested : PCL_KERNEL_SPLIT_KV;
    if (requested == PCL_KERNEL_FAN_KV) {
        // its one-dimensional grid of 512-thread workgroups stays below 2^32
        // work-items up to 2^22 items
        const int64_t items = nch * nkv * ((nrows + pcl::kRows - 1) / pcl::kRows);
        return dk >= 128 && nch >= 2 && items <= ((int64_t)1 << 22) ? requested
                                                                    : PCL_KERNEL_PIPE_KV;
    }
    const int64_t units = (nrows + pcl::kRows - 1) / pcl::kRows;
    const bool fan = fan_preferred(dk, units, nch * nkv * units, nch);
    if (dk > kTiledMaxDk || nrows < 64) {
        // decode: short launches spread each chunk over several workgroups,
        // or fan each item over a workgroup's eight waves; otherwise the
        // pipelined kernel; a single chunk at head dim 512 the four-phase
        // kernel
        if (spread_fits)
            return PCL_KERNEL_SPREAD_KV;
        if (fan)
            return PCL_KERNEL_FAN_KV;
        if (dk > 256 && nch == 1)
            return PCL_KERNEL_SPLIT_KV;
        return PCL_KERNEL_PIPE_KV;
    }
    const int64_t rows = pcl::tiled_rows(dk);
    const int64_t blocks = (nrows + rows - 1) / rows * nkv;
    if (blocks >= 128 || nch <= 1)
        return PCL_KERNEL_TILED;
    // a chunk-split launch of few row blocks: fanned items where they are
    // few enough
    return fan ? PCL_KERNEL_FAN_KV : PCL_KERNEL_TILED_SPLIT;
}

// Validate a descriptor and build the plan. h_lo/h_hi/h_base select and place
// the written query heads (the whole KV-head range for the public entry).
int make_plan(const pcl_attention_desc &d, int64_t h_lo, int64_t h_hi, int64_t h_base,
              Plan *plan)
{
    if (d.qheads <= 0 || d.kvheads <= 0 || d.qheads % d.kvheads != 0 || d.dim <= 0 ||
        d.dim % 16 != 0 || d.dim > kMaxDim || d.nq < 0 || d.n0 < 0 || d.n1 < 0 ||
        d.kh_first < 0 || d.kh_first > d.kh_end || d.kh_end > d.kvheads || d.window < 0)
        return PCL_INVALID_SHAPE;
    if (d.kernel < PCL_KERNEL_AUTO || d.kernel > PCL_KERNEL_FAN_KV || d.kernel == 5)
        return PCL_INVALID_PARAMETER;
    // negative, NaN, infinite or subnormal caps, and caps whose f32
    // reciprocal (what the kernels multiply by) would be subnormal
    if (!(d.softcap >= 0.0f) || !std::isfinite(d.softcap) ||
        (d.softcap > 0.0f && (!std::isnormal(d.softcap) || !std::isnormal(1.0f / d.softcap))))
        return PCL_INVALID_PARAMETER;
    const int64_t group = d.qheads / d.kvheads;
    const int64_t nkeys = d.n0 + d.n1;
    const int64_t nkv = d.kh_end - d.kh_first;
    plan->empty = d.nq == 0 || nkv == 0 || h_lo >= h_hi;
    if (plan->empty)
        return PCL_OK;
    if (nkeys <= 0 || !d.q || !d.out || (d.n0 > 0 && (!d.k0 || !d.v0)) ||
        (d.n1 > 0 && (!d.k1 || !d.v1)))
        return PCL_INVALID_SHAPE;
    if (d.q_stride < d.qheads * d.dim || d.q_stride % 4 != 0 || d.o_stride % 4 != 0 ||
        (d.mask && d.mask_stride < nkeys) || !aligned16(d.q) || !aligned16(d.out) ||
        (d.n0 > 0 && (!aligned16(d.k0) || !aligned16(d.v0))) ||
        (d.n1 > 0 && (!aligned16(d.k1) || !aligned16(d.v1))))
        return PCL_INVALID_SHAPE;
    const int64_t nrows = d.nq * group;
    // size limits: every launch's grid stays below 2^31 work-items per
    // dimension (at most 2^22 chunks x 512 threads; 2^22 rows x 256 threads)
    // and chunk indices fit an int
    if (nkeys > kMaxKeys || nrows * nkv > kMaxRowsTimesKvHeads)
        return PCL_INVALID_SHAPE;
    int64_t c_lo, c_hi;
    bool none;
    chunk_range(d, nkeys, &c_lo, &c_hi, &none);
    if (none)
        return PCL_INVALID_PARAMETER; // no query sees any key
    // padded head dim: the kernels are instantiated for 64, 128, 256 and 512
    const int dk = d.dim <= 64 ? 64 : d.dim <= 128 ? 128 : d.dim <= 256 ? 256 : 512;
    const int64_t nch = c_hi - c_lo;

    Params &p = plan->p;
    std::memset(&p, 0, sizeof p);
    p.q = d.q;
    p.q_stride = d.q_stride;
    p.nq = (int)d.nq;
    p.q_scale = d.q_scale;
    if (d.softcap > 0.0f) {
        p.softcap = d.softcap;
        p.inv_softcap = 1.0f / d.softcap;
    }
    if (d.n0 > 0) {
        p.k0 = d.k0;
        p.v0 = d.v0;
        p.n0 = d.n0;
        p.k1 = d.n1 > 0 ? d.k1 : d.k0;
        p.v1 = d.n1 > 0 ? d.v1 : d.v0;
    } else {
        p.k0 = p.k1 = d.k1;
        p.v0 = p.v1 = d.v1;
        p.n0 = 0;
    }
    p.nkeys = nkeys;
    p.kv_stride = d.kvheads * d.dim;
    p.dim = (int)d.dim;
    p.group = (int)group;
    p.kh_first = (int)d.kh_first;
    p.nkv = (int)nkv;
    p.h_lo = (int)h_lo;
    p.h_hi = (int)h_hi;
    p.h_base = (int)h_base;
    p.mask = d.mask;
    p.mask_stride = d.mask_stride;
    p.causal = d.causal;
    p.window = d.window;
    p.first_key = d.first_key;
    p.first_query = d.first_query;
    p.out = d.out;
    p.o_stride = d.o_stride;
    p.nrows = (int)nrows;
    p.units = (int)((nrows + pcl::kRows - 1) / pcl::kRows);
    p.nrows_pad = p.units * pcl::kRows;
    p.c_lo = (int)c_lo;
    p.nch = (int)nch;
    p.dk = dk;

    // the current device's CU count; with no device to ask (host-only
    // queries: nothing launches there) a whole MI355X's
    const int cus = pcl::device_cus();
    plan->kernel = choose_kernel(d.kernel, dk, nrows, nkv, nch, cus > 0 ? cus : kMi355xCus);
    if (plan->kernel == PCL_KERNEL_TILED_SPLIT) {
        // the tiled kernel's rows come in whole workgroup blocks
        p.nrows_pad = (int)round_up(nrows, pcl::tiled_rows(dk));
    }
    const int64_t s_lo = c_lo / pcl::kSpanChunks;
    const int64_t s_hi = (c_hi - 1) / pcl::kSpanChunks + 1;
    p.s_lo = (int)s_lo;
    p.nspan = (int)(s_hi - s_lo);
    const bool partials = plan->kernel == PCL_KERNEL_TILED_SPLIT ||
                          ((plan->kernel == PCL_KERNEL_SPLIT_KV ||
                            plan->kernel == PCL_KERNEL_PIPE_KV ||
                            plan->kernel == PCL_KERNEL_FAN_KV) && nch > 1);
    plan->part_floats = 0;
    if (partials) {
        plan->part_floats = (size_t)nkv * p.nrows_pad * nch * (dk + 2);
        if (p.nspan > 1)
            plan->part_floats += (size_t)nkv * p.nrows_pad * p.nspan * (dk + 2);
    } else if (plan->kernel == PCL_KERNEL_TILED && p.nspan > 1) {
        // the tiled kernel's running totals across spans
        plan->part_floats = (size_t)nkv * p.nrows_pad * dk;
    }
    plan->part_floats = round_up((int64_t)plan->part_floats, 4);
    const size_t body = plan->part_floats;
    plan->ws_floats = body || plan->kernel == PCL_KERNEL_SPREAD_KV ? kTagFloats + body : 0;
    return PCL_OK;
}

__global__ void zero_words_kernel(uint32_t *words, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        words[i] = 0;
}

// Zeroes the published-word region at the start of a workspace of `bytes`
// on ctx's stream (a fill kernel rather than a memset node, should a caller
// capture this) and records the generation it is valid for in *gen.
int zero_tag_region(pcl_context *ctx, void *ws, size_t bytes, uint32_t *gen)
{
    const int nwords = (int)std::min<size_t>(kTagFloats, bytes / sizeof(uint32_t));
    *gen = current_generation(ctx->device);
    zero_words_kernel<<<(nwords + 255) / 256, 256, 0, ctx->stream>>>(
        static_cast<uint32_t *>(ws), nwords);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        report("workspace score words", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

int ensure_workspace(pcl_context *ctx, size_t bytes)
{
    if (bytes <= ctx->ws_bytes)
        return PCL_OK;
    if (ctx->ws) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    hipError_t e = hipMalloc(&ctx->ws, bytes);
    if (e != hipSuccess) {
        ctx->ws = nullptr;
        report("workspace allocation", e);
        return PCL_RESOURCE_LIMIT;
    }
    ctx->ws_bytes = bytes;
    // a new buffer's score-word region starts at zero, an epoch no launch
    // takes
    return zero_tag_region(ctx, ctx->ws, bytes, &ctx->ws_tag_gen);
}

hipEvent_t take_event(pcl_context *ctx)
{
    if (!ctx->free_events.empty()) {
        hipEvent_t e = ctx->free_events.back();
        ctx->free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

// Opens a timed span of `role` on the context's stream (no-op when timing is
// off); close_span records its end.
int open_span(pcl_context *ctx, int role)
{
    if (!ctx->timing)
        return -1;
    TimedSpan t;
    t.start = take_event(ctx);
    t.stop = take_event(ctx);
    t.role = role;
    if (!t.start || !t.stop || hipEventRecord(t.start, ctx->stream) != hipSuccess) {
        if (t.start)
            ctx->free_events.push_back(t.start);
        if (t.stop)
            ctx->free_events.push_back(t.stop);
        return -1;
    }
    ctx->spans.push_back(t);
    return (int)ctx->spans.size() - 1;
}

void close_span(pcl_context *ctx, int idx)
{
    if (idx >= 0)
        (void)hipEventRecord(ctx->spans[idx].stop, ctx->stream);
}

// Launches a plan with its workspace at `ws` (plan.ws_floats floats; its
// published-word region last zeroed for generation *tag_gen).
int run_plan_ws(pcl_context *ctx, Plan &plan, float *ws, uint32_t *tag_gen)
{
    Params &p = plan.p;
    p.err = ctx->err;
    if (plan.ws_floats) {
        float *body = ws + kTagFloats;
        if (plan.part_floats) {
            const size_t o_floats = (size_t)p.nkv * p.nrows_pad * p.nch * p.dk;
            const size_t ml_floats = (size_t)p.nkv * p.nrows_pad * p.nch * 2;
            p.ws_o = body;
            p.ws_ml = p.ws_o + o_floats;
            if (p.nspan > 1) {
                p.ws2_o = p.ws_ml + ml_floats;
                p.ws2_ml = p.ws2_o + (size_t)p.nkv * p.nrows_pad * p.nspan * p.dk;
            }
        }
        if (plan.kernel == PCL_KERNEL_SPREAD_KV) {
            p.ws_tag = reinterpret_cast<uint64_t *>(ws);
            if (p.nch > 1) // the launch merges its own chunk partials
                p.ws_ptag = p.ws_tag + kSpreadScoreWords;
            const Epoch ep = next_epoch(ctx->device);
            if (ep.generation != *tag_gen) {
                // the epoch wrapped since the region was zeroed: words of
                // the previous generation could carry this epoch
                const int rc = zero_tag_region(ctx, ws, kTagFloats * sizeof(float), tag_gen);
                if (rc != PCL_OK)
                    return rc;
                *tag_gen = ep.generation;
            }
            p.epoch = ep.epoch;
            p.max_polls = ctx->wait_polls;
        }
    }
    hipError_t e = hipSuccess;
    bool combine = plan.kernel == PCL_KERNEL_TILED_SPLIT ||
                         ((plan.kernel == PCL_KERNEL_SPLIT_KV || plan.kernel == PCL_KERNEL_PIPE_KV ||
                           plan.kernel == PCL_KERNEL_FAN_KV) &&
                          p.ws_o);
    int span = open_span(ctx, 0);
    switch (plan.kernel) {
    case PCL_KERNEL_SPLIT_KV:
        e = pcl::launch_split_kv(p, ctx->stream);
        break;
    case PCL_KERNEL_PIPE_KV:
        e = pcl::launch_pipe_kv(p, ctx->stream);
        break;
    case PCL_KERNEL_FAN_KV:
        e = pcl::launch_fan_kv(p, ctx->stream);
        break;
    case PCL_KERNEL_TILED: {
        bool merged = false;
        e = pcl::launch_tiled(p, 0, ctx->stream, &merged);
        break;
    }
    case PCL_KERNEL_TILED_SPLIT: {
        bool merged = false;
        e = pcl::launch_tiled(p, 1, ctx->stream, &merged);
        combine = !merged;
        break;
    }
    case PCL_KERNEL_SPREAD_KV:
        e = pcl::launch_spread_kv(p, ctx->stream);
        break;
    default:
        return PCL_INVALID_SHAPE;
    }
    close_span(ctx, span);
    if (e == hipSuccess && combine) {
        span = open_span(ctx, 1);
        e = pcl::launch_combine(p, ctx->stream);
        close_span(ctx, span);
    }
    if (e != hipSuccess) {
        report("kernel launch", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

int run_plan(pcl_context *ctx, Plan &plan)
{
    if (plan.empty)
        return PCL_OK;
    if (plan.ws_floats) {
        const int rc = ensure_workspace(ctx, plan.ws_floats * sizeof(float));
        if (rc != PCL_OK)
            return rc;
    }
    return run_plan_ws(ctx, plan, static_cast<float *>(ctx->ws), &ctx->ws_tag_gen);
}

// ---- the allocation-free entry's scratch ------------------------------------
//
// A file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, taken once per device when the first context on that
// device is created, and the kernels receive it as their workspace.
constexpr size_t kNoAllocScratchBytes = PCL_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxScratchDevices];
bool g_scratch_done[kMaxScratchDevices];
// epoch generation for which each device's scratch was last zeroed (its
// published-word region starts at zero, as the array does when the
// library loads, in generation 0)
uint32_t g_scratch_gen[kMaxScratchDevices];

// This device's scratch address (the device must be current), or null when
// its lookup failed.
void *noalloc_scratch(int device)
{
    if (device < 0 || device >= kMaxScratchDevices)
        return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_done[device]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            report("scratch address", e);
            ptr = nullptr;
        }
        g_scratch_ptr[device] = ptr;
        g_scratch_done[device] = true;
    }
    return g_scratch_ptr[device];
}

// ---- host-pointer entries: one shared context, one call at a time ----------

std::mutex g_abi_mutex;
pcl_context *g_abi_ctx = nullptr;

// Wait limit of the host-pointer entries' context (0: the default), set
// with pcl_context_set_wait_limit(NULL, polls).
std::atomic<int> g_abi_wait_polls{0};

pcl_context *abi_context()
{
    if (!g_abi_ctx) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess)
            dev = 0;
        if (pcl_context_create(dev, &g_abi_ctx) != PCL_OK)
            g_abi_ctx = nullptr;
    }
    return g_abi_ctx;
}

void *stage_buffer(pcl_context *ctx, int slot, size_t bytes)
{
    bytes = std::max<size_t>(bytes, 16);
    if (bytes > ctx->stage_bytes[slot]) {
        if (ctx->stage[slot])
            (void)hipFree(ctx->stage[slot]);
        ctx->stage[slot] = nullptr;
        ctx->stage_bytes[slot] = 0;
        const hipError_t e = hipMalloc(&ctx->stage[slot], bytes);
        if (e != hipSuccess) {
            report("staging allocation", e);
            return nullptr;
        }
        ctx->stage_bytes[slot] = bytes;
    }
    return ctx->stage[slot];
}

// The full K/V upload the host-pointer entries share: the engine runs one
// position's heads as concurrent calls from its workers, one head range
// each, over the same read-only K and V (src/engine/attention.rs:755-777).
// A call registers for its (keys, values, length) before it queues for the
// device; while any registered call of that key is pending, the upload
// stays valid, so the fan-out copies K and V once. Once the last of them
// returns, the entry is dropped (the caller may then rewrite the buffers).
// A call whose keys differ from an entry still in use copies privately.
struct HostUpload {
    const float *keys = nullptr, *values = nullptr;
    size_t kv_floats = 0;
    int users = 0;      // registered calls not yet returned
    bool valid = false; // the shared staging buffers hold this key's K and V
};
std::mutex g_upload_mutex;
HostUpload g_upload;

enum StageSlot { kStageQ, kStageK, kStageV, kStageMask, kStageOut, kStageKOwn, kStageVOwn };

// Copy the inputs to the device (K and V through the shared upload when
// possible), run, copy the output rows back. query: nq rows of q_floats
// (device stride q_stride); h_lo / h_hi / h_base: the written query heads and
// the output's first head.
bool run_host(const float *query, size_t q_floats, const float *keys, const float *values,
              size_t kv_floats, const uint8_t *allowed, size_t mask_bytes,
              pcl_attention_desc d, int64_t h_lo, int64_t h_hi, int64_t h_base, float *out,
              size_t out_rows, size_t out_row_floats, size_t out_pitch_floats)
{
    bool shared = false;
    {
        std::lock_guard<std::mutex> lock(g_upload_mutex);
        HostUpload &u = g_upload;
        if (u.users > 0 && u.keys == keys && u.values == values && u.kv_floats == kv_floats) {
            ++u.users;
            shared = true;
        } else if (u.users == 0) {
            u.keys = keys;
            u.values = values;
            u.kv_floats = kv_floats;
            u.valid = false;
            u.users = 1;
            shared = true;
        }
    }
    bool ok = false;
    {
        std::lock_guard<std::mutex> lock(g_abi_mutex);
        ok = [&]() {
            pcl_context *ctx = abi_context();
            if (!ctx)
                return false;
            (void)hipSetDevice(ctx->device);
            const int polls = g_abi_wait_polls.load(std::memory_order_relaxed);
            ctx->wait_polls = polls ? polls : 1 << 16;
            const size_t kv_bytes = kv_floats * sizeof(float);
            float *dq = static_cast<float *>(stage_buffer(ctx, kStageQ, q_floats * sizeof(float)));
            uint8_t *dm =
                allowed ? static_cast<uint8_t *>(stage_buffer(ctx, kStageMask, mask_bytes)) : nullptr;
            float *dout = static_cast<float *>(
                stage_buffer(ctx, kStageOut, out_rows * out_pitch_floats * sizeof(float)));
            bool upload = true;
            if (shared) {
                std::lock_guard<std::mutex> ul(g_upload_mutex);
                upload = !g_upload.valid;
            }
            // the shared buffers are only grown (reallocated) by the call
            // that uploads into them, which no other pending call relies on
            float *dk = static_cast<float *>(
                shared && !upload ? ctx->stage[kStageK]
                                  : stage_buffer(ctx, shared ? kStageK : kStageKOwn, kv_bytes));
            float *dv = static_cast<float *>(
                shared && !upload ? ctx->stage[kStageV]
                                  : stage_buffer(ctx, shared ? kStageV : kStageVOwn, kv_bytes));
            if (!dq || !dk || !dv || (allowed && !dm) || !dout)
                return false;
            hipError_t e = hipMemcpyAsync(dq, query, q_floats * sizeof(float),
                                          hipMemcpyHostToDevice, ctx->stream);
            if (e == hipSuccess && upload)
                e = hipMemcpyAsync(dk, keys, kv_bytes, hipMemcpyHostToDevice, ctx->stream);
            if (e == hipSuccess && upload)
                e = hipMemcpyAsync(dv, values, kv_bytes, hipMemcpyHostToDevice, ctx->stream);
            if (e == hipSuccess && allowed)
                e = hipMemcpyAsync(dm, allowed, mask_bytes, hipMemcpyHostToDevice, ctx->stream);
            if (e != hipSuccess) {
                report("host to device copy", e);
                return false;
            }
            if (shared && upload) {
                // later calls of this key run after the copies on this stream
                std::lock_guard<std::mutex> ul(g_upload_mutex);
                g_upload.valid = true;
            }
            d.q = dq;
            d.k0 = dk;
            d.v0 = dv;
            d.mask = dm;
            d.out = dout;
            d.o_stride = (int64_t)out_pitch_floats;
            Plan plan;
            if (make_plan(d, h_lo, h_hi, h_base, &plan) != PCL_OK)
                return false;
            if (run_plan(ctx, plan) != PCL_OK)
                return false;
            int derr = 0;
            if (pcl_context_sync(ctx, &derr) != PCL_OK)
                return false;
            if (derr & pcl::kErrWait) {
                // the spread decode's workgroups gave up waiting for each
                // other (a GPU shared with other work can keep some of them
                // from running): once more with the pipelined kernel, which
                // never waits, for the same bits
                d.kernel = PCL_KERNEL_PIPE_KV;
                if (make_plan(d, h_lo, h_hi, h_base, &plan) != PCL_OK ||
                    run_plan(ctx, plan) != PCL_OK ||
                    pcl_context_sync(ctx, &derr) != PCL_OK)
                    return false;
            }
            if (derr != 0)
                return false;
            e = hipMemcpy2DAsync(out, out_pitch_floats * sizeof(float), dout,
                                 out_pitch_floats * sizeof(float), out_row_floats * sizeof(float),
                                 out_rows, hipMemcpyDeviceToHost, ctx->stream);
            if (e == hipSuccess)
                e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) {
                report("device to host copy", e);
                return false;
            }
            return true;
        }();
    }
    if (shared) {
        std::lock_guard<std::mutex> lock(g_upload_mutex);
        if (--g_upload.users == 0)
            g_upload.valid = false;
    }
    return ok;
}

bool all_finite(const float *x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(x[i]))
            return false;
    return true;
}

} // namespace

extern "C" {

const char *pcl_version(void)
{
    return "pcl_attention 0.1 gfx950 (mfma_f32_16x16x4f32, chunk 256, tile 32)";
}

static int context_create(int device, bool own, void *stream, pcl_context **out)
{
    if (!out)
        return PCL_INVALID_SHAPE;
    *out = nullptr;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) {
        report("hipSetDevice", e);
        return PCL_NON_FINITE_VALUE;
    }
    auto *ctx = new pcl_context;
    ctx->device = device;
    if (!own) {
        ctx->stream = static_cast<hipStream_t>(stream);
    } else {
        e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            report("stream creation", e);
            delete ctx;
            return PCL_NON_FINITE_VALUE;
        }
        ctx->own_stream = true;
    }
    e = hipMalloc(&ctx->err, sizeof(int));
    if (e == hipSuccess)
        e = hipMemsetAsync(ctx->err, 0, sizeof(int), ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        report("error flag", e);
        pcl_context_destroy(ctx);
        return PCL_NON_FINITE_VALUE;
    }
    // the allocation-free entry's scratch on this device (null: that entry
    // reports the failure; every other entry works without it)
    ctx->noalloc_scratch = noalloc_scratch(device);
    *out = ctx;
    return PCL_OK;
}

int pcl_context_create(int device, pcl_context **out)
{
    return context_create(device, true, nullptr, out);
}

int pcl_context_create_on_stream(int device, void *stream, pcl_context **out)
{
    return context_create(device, false, stream, out);
}

void pcl_context_destroy(pcl_context *ctx)
{
    if (!ctx)
        return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream)
        (void)hipStreamSynchronize(ctx->stream);
    for (const TimedSpan &t : ctx->spans) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    for (hipEvent_t e : ctx->free_events)
        (void)hipEventDestroy(e);
    for (int i = 0; i < kStageSlots; ++i)
        if (ctx->stage[i])
            (void)hipFree(ctx->stage[i]);
    if (ctx->ws)
        (void)hipFree(ctx->ws);
    if (ctx->err)
        (void)hipFree(ctx->err);
    if (ctx->own_stream && ctx->stream)
        (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void *pcl_context_stream(pcl_context *ctx)
{
    return ctx ? ctx->stream : nullptr;
}

int pcl_context_reserve(pcl_context *ctx, size_t bytes)
{
    if (!ctx)
        return PCL_INVALID_SHAPE;
    (void)hipSetDevice(ctx->device);
    return ensure_workspace(ctx, bytes);
}

size_t pcl_attention_workspace_bytes(const pcl_attention_desc *desc)
{
    if (!desc)
        return 0;
    const int64_t group = desc->kvheads ? desc->qheads / desc->kvheads : 0;
    const int64_t h_lo = desc->kh_first * group, h_hi = desc->kh_end * group;
    Plan plan;
    if (make_plan(*desc, h_lo, h_hi, h_lo, &plan) != PCL_OK)
        return 0;
    size_t floats = plan.ws_floats;
    if (plan.kernel == PCL_KERNEL_SPREAD_KV && desc->kernel == PCL_KERNEL_AUTO) {
        // the same launch captured into a graph takes the pipelined kernel
        pcl_attention_desc d = *desc;
        d.kernel = PCL_KERNEL_PIPE_KV;
        if (make_plan(d, h_lo, h_hi, h_lo, &plan) == PCL_OK)
            floats = std::max(floats, plan.ws_floats);
    }
    return floats * sizeof(float);
}

int pcl_attention_resolve_kernel(const pcl_attention_desc *desc)
{
    if (!desc || desc->kvheads <= 0)
        return -1;
    const int64_t group = desc->qheads / desc->kvheads;
    Plan plan;
    if (make_plan(*desc, desc->kh_first * group, desc->kh_end * group, desc->kh_first * group,
                  &plan) != PCL_OK)
        return -1;
    return plan.kernel;
}

} // extern "C"

namespace {

// True while `stream` is being captured into a graph (an error of the query
// itself counts as not capturing and is cleared).
bool capturing(hipStream_t stream)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return st != hipStreamCaptureStatusNone;
}

// The plan of a device-resident launch on ctx's stream. A launch being
// captured into a graph never takes the spread decode: its workgroups accept
// a published word by the launch's epoch, a kernel argument that every
// replay of the graph repeats, so one replay could take the previous
// replay's words. AUTO then takes the pipelined kernel (the same bits); an
// explicit request for the spread decode is refused.
int launch_plan(pcl_context *ctx, const pcl_attention_desc &desc, Plan *plan)
{
    if (desc.kvheads <= 0 || desc.qheads % desc.kvheads != 0)
        return PCL_INVALID_SHAPE;
    const int64_t group = desc.qheads / desc.kvheads;
    const int64_t h_lo = desc.kh_first * group, h_hi = desc.kh_end * group;
    // the kernel choice reads the current device's CU count
    (void)hipSetDevice(ctx->device);
    int rc = make_plan(desc, h_lo, h_hi, h_lo, plan);
    if (rc != PCL_OK || plan->empty || plan->kernel != PCL_KERNEL_SPREAD_KV)
        return rc;
    if (!capturing(ctx->stream))
        return PCL_OK;
    if (desc.kernel != PCL_KERNEL_AUTO)
        return PCL_INVALID_PARAMETER;
    pcl_attention_desc d = desc;
    d.kernel = PCL_KERNEL_PIPE_KV;
    return make_plan(d, h_lo, h_hi, h_lo, plan);
}

} // namespace

int pcl::launch_step(pcl_context *ctx, const pcl_attention_desc &desc, const StepFold &f,
                     const std::function<int()> &separate)
{
    if (desc.nq != 1)
        return PCL_INVALID_SHAPE;
    Plan plan;
    int rc = launch_plan(ctx, desc, &plan);
    if (rc != PCL_OK)
        return rc;
    (void)hipSetDevice(ctx->device);
    Params &p = plan.p;
    if (!plan.empty && plan.kernel == PCL_KERNEL_PIPE_KV && p.dim == p.dk) {
        p.sq = f.rq;
        p.sk = f.rk;
        p.sv = f.rv;
        p.sqs = f.qs;
        p.sks = f.ks;
        p.srot = f.rot;
        p.snk = f.nk;
        p.snv = f.nv;
        p.sqo = f.qo;
        p.seps = f.eps;
    } else {
        rc = separate();
        if (rc != PCL_OK)
            return rc;
    }
    return run_plan(ctx, plan);
}

extern "C" {

int pcl_attention_launch(pcl_context *ctx, const pcl_attention_desc *desc)
{
    if (!ctx || !desc)
        return PCL_INVALID_SHAPE;
    Plan plan;
    const int rc = launch_plan(ctx, *desc, &plan);
    if (rc != PCL_OK)
        return rc;
    (void)hipSetDevice(ctx->device);
    return run_plan(ctx, plan);
}

int pcl_attention_launch_noalloc(pcl_context *ctx, const pcl_attention_desc *desc)
{
    if (!ctx || !desc)
        return PCL_INVALID_SHAPE;
    Plan plan;
    const int rc = launch_plan(ctx, *desc, &plan);
    if (rc != PCL_OK)
        return rc;
    if (plan.empty)
        return PCL_OK;
    if (plan.ws_floats * sizeof(float) > kNoAllocScratchBytes)
        return PCL_RESOURCE_LIMIT;
    if (!ctx->noalloc_scratch)
        return PCL_NON_FINITE_VALUE;
    (void)hipSetDevice(ctx->device);
    // no timing spans here: recording them creates events and grows a list
    const bool timing = ctx->timing;
    ctx->timing = false;
    const int dev = ctx->device >= 0 && ctx->device < kMaxScratchDevices ? ctx->device : 0;
    const int out = run_plan_ws(ctx, plan, static_cast<float *>(ctx->noalloc_scratch),
                                &g_scratch_gen[dev]);
    ctx->timing = timing;
    return out;
}

int pcl_context_set_wait_limit(pcl_context *ctx, int polls)
{
    if (polls < 0)
        return PCL_INVALID_PARAMETER;
    if (!ctx) { // the host-pointer entries' own context
        g_abi_wait_polls.store(polls, std::memory_order_relaxed);
        return PCL_OK;
    }
    ctx->wait_polls = polls == 0 ? 1 << 16 : polls;
    return PCL_OK;
}

int pcl_debug_set_epoch_counter(int device, uint64_t value)
{
    if (device < 0 || device >= kMaxEpochDevices)
        return PCL_INVALID_SHAPE;
    epoch_counter(device).store(value, std::memory_order_relaxed);
    return PCL_OK;
}

int pcl_context_set_timing(pcl_context *ctx, int enable)
{
    if (!ctx)
        return PCL_INVALID_SHAPE;
    ctx->timing = enable != 0;
    return PCL_OK;
}

int pcl_context_timing(pcl_context *ctx, double *ms, int64_t *launches)
{
    if (!ctx || !ms || !launches)
        return PCL_INVALID_SHAPE;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    for (const TimedSpan &t : ctx->spans) {
        float x = 0.f;
        if (e == hipSuccess)
            e = hipEventElapsedTime(&x, t.start, t.stop);
        if (e == hipSuccess) {
            ms[t.role] += x;
            launches[t.role] += 1;
        }
        ctx->free_events.push_back(t.start);
        ctx->free_events.push_back(t.stop);
    }
    ctx->spans.clear();
    if (e != hipSuccess) {
        report("timing", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

int pcl_context_sync(pcl_context *ctx, int *device_error)
{
    if (!ctx)
        return PCL_INVALID_SHAPE;
    (void)hipSetDevice(ctx->device);
    int h = 0;
    hipError_t e = hipMemcpyAsync(&h, ctx->err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess && h != 0)
        e = hipMemsetAsync(ctx->err, 0, sizeof(int), ctx->stream);
    if (e == hipSuccess && h != 0)
        e = hipStreamSynchronize(ctx->stream);
    if (device_error)
        *device_error = h;
    if (e != hipSuccess) {
        report("synchronize", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

bool pcl_hip_attention_f32_heads(const float *query, const float *keys, const float *values,
                                 size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                 const uint8_t *allowed, float *scratch, float *out,
                                 size_t h_first, size_t h_end)
{
    (void)scratch; // the device keeps its own score storage
    if (h_first > h_end || h_end > qheads)
        return false;
    if (dim % 16 != 0 || dim == 0 || kvheads == 0 || qheads % kvheads != 0 || dim > kMaxDim)
        return false;
    if (h_first == h_end)
        return true;
    if (nkeys == 0)
        return false;
    const size_t group = qheads / kvheads;
    pcl_attention_desc d;
    std::memset(&d, 0, sizeof d);
    d.q_stride = (int64_t)(qheads * dim);
    d.nq = 1;
    d.n0 = (int64_t)nkeys;
    d.qheads = (int64_t)qheads;
    d.kvheads = (int64_t)kvheads;
    d.dim = (int64_t)dim;
    d.kh_first = (int64_t)(h_first / group);
    d.kh_end = (int64_t)((h_end - 1) / group + 1);
    d.mask_stride = (int64_t)nkeys;
    d.q_scale = 1.0f;
    d.kernel = PCL_KERNEL_AUTO;
    const size_t olen = (h_end - h_first) * dim;
    return run_host(query, qheads * dim, keys, values, nkeys * kvheads * dim, allowed, nkeys, d,
                    (int64_t)h_first, (int64_t)h_end, (int64_t)h_first, out, 1, olen, olen);
}

bool pcl_hip_attention_f32_multi_kv(const float *query, size_t nq, size_t q_stride,
                                    const float *keys, const float *values, size_t qheads,
                                    size_t kvheads, size_t dim, size_t nkeys,
                                    const uint8_t *allowed, size_t mask_stride, float *scratch,
                                    float *out, size_t o_stride, size_t kh_first, size_t kh_end)
{
    (void)scratch;
    if (dim % 16 != 0 || dim == 0 || kvheads == 0 || qheads % kvheads != 0 || dim > kMaxDim)
        return false;
    if (kh_first >= kh_end || kh_end > kvheads)
        return false;
    const size_t group = qheads / kvheads;
    const size_t olen = (kh_end - kh_first) * group * dim;
    if (q_stride < qheads * dim || o_stride < olen || (allowed && mask_stride < nkeys))
        return false;
    if (nq == 0)
        return true;
    if (nkeys == 0)
        return false;
    // The device reads queries and outputs with 16-byte vectors: keep the
    // strides a multiple of four floats on the device side.
    const size_t dq_stride = (size_t)round_up((int64_t)q_stride, 4);
    const size_t do_stride = (size_t)round_up((int64_t)olen, 4);
    std::vector<float> qbuf;
    const float *qsrc = query;
    size_t q_floats = (nq - 1) * q_stride + qheads * dim;
    if (dq_stride != q_stride) {
        qbuf.assign(nq * dq_stride, 0.0f);
        for (size_t i = 0; i < nq; ++i)
            std::memcpy(&qbuf[i * dq_stride], query + i * q_stride, qheads * dim * sizeof(float));
        qsrc = qbuf.data();
        q_floats = qbuf.size();
    }
    pcl_attention_desc d;
    std::memset(&d, 0, sizeof d);
    d.q_stride = (int64_t)dq_stride;
    d.nq = (int64_t)nq;
    d.n0 = (int64_t)nkeys;
    d.qheads = (int64_t)qheads;
    d.kvheads = (int64_t)kvheads;
    d.dim = (int64_t)dim;
    d.kh_first = (int64_t)kh_first;
    d.kh_end = (int64_t)kh_end;
    d.mask_stride = (int64_t)mask_stride;
    d.q_scale = 1.0f;
    d.kernel = PCL_KERNEL_AUTO;
    const size_t mask_bytes = allowed ? (nq - 1) * mask_stride + nkeys : 0;
    std::vector<float> obuf;
    float *odst = out;
    if (do_stride != o_stride) {
        obuf.assign(nq * do_stride, 0.0f);
        odst = obuf.data();
    }
    const int64_t h0 = (int64_t)(kh_first * group);
    const bool ok = run_host(qsrc, q_floats, keys, values, nkeys * kvheads * dim, allowed,
                             mask_bytes, d, h0, (int64_t)(kh_end * group), h0, odst, nq, olen,
                             do_stride);
    if (ok && odst != out)
        for (size_t i = 0; i < nq; ++i)
            std::memcpy(out + i * o_stride, &obuf[i * do_stride], olen * sizeof(float));
    return ok;
}

// attention_with (src/kernels/quantized/int8.rs:596-663) for this backend.
int pcl_attention_heads(const float *query, size_t query_len, const float *keys,
                        size_t keys_len, const float *values, size_t values_len,
                        size_t kv_heads, size_t head_dim, const uint8_t *allowed,
                        size_t mask_len, int has_mask, size_t h_first, size_t h_end,
                        int has_heads, float *out)
{
    if (kv_heads == 0 || head_dim == 0 || kv_heads > SIZE_MAX / head_dim)
        return PCL_INVALID_SHAPE;
    const size_t width = kv_heads * head_dim;
    if (query_len == 0 || head_dim % 16 != 0 || query_len % head_dim != 0 || keys_len == 0 ||
        keys_len % width != 0 || values_len != keys_len)
        return PCL_INVALID_SHAPE;
    const size_t qheads = query_len / head_dim;
    const size_t nkeys = keys_len / width;
    if (qheads % kv_heads != 0)
        return PCL_INVALID_SHAPE;
    std::vector<uint8_t> mask;
    if (has_mask) {
        if (mask_len != nkeys)
            return PCL_INVALID_SHAPE;
        mask.resize(nkeys);
        bool any = false;
        for (size_t t = 0; t < nkeys; ++t) {
            mask[t] = allowed[t] != 0;
            any |= mask[t] != 0;
        }
        if (!any)
            return PCL_INVALID_PARAMETER;
    }
    if (!has_heads) {
        h_first = 0;
        h_end = qheads;
    }
    if (h_first > h_end || h_end > qheads)
        return PCL_INVALID_SHAPE;
    if (!all_finite(query, query_len))
        return PCL_NON_FINITE_VALUE;
    const bool ok = pcl_hip_attention_f32_heads(query, keys, values, qheads, kv_heads, head_dim,
                                                nkeys, has_mask ? mask.data() : nullptr,
                                                nullptr, out, h_first, h_end);
    return ok ? PCL_OK : PCL_NON_FINITE_VALUE;
}

// attention_multi_with (src/kernels/quantized/int8.rs:489-573) for this backend.
int pcl_attention_multi_kv(const float *const *queries, size_t nq, size_t query_len,
                           const float *keys, size_t keys_len, const float *values,
                           size_t values_len, size_t kv_heads, size_t head_dim,
                           const uint8_t *const *masks, size_t mask_len, size_t kv_first,
                           size_t kv_end, float *out)
{
    if (nq == 0)
        return PCL_OK;
    if (kv_first >= kv_end || kv_end > kv_heads)
        return PCL_INVALID_SHAPE;
    if (kv_heads == 0 || head_dim == 0 || kv_heads > SIZE_MAX / head_dim)
        return PCL_INVALID_SHAPE;
    const size_t width = kv_heads * head_dim;
    if (query_len == 0 || head_dim % 16 != 0 || query_len % head_dim != 0 || keys_len == 0 ||
        keys_len % width != 0 || values_len != keys_len ||
        (query_len / head_dim) % kv_heads != 0)
        return PCL_INVALID_SHAPE;
    const size_t nkeys = keys_len / width;
    std::vector<uint8_t> mask;
    if (masks) {
        if (mask_len != nkeys)
            return PCL_INVALID_SHAPE;
        mask.resize(nq * nkeys);
        for (size_t i = 0; i < nq; ++i) {
            bool any = false;
            for (size_t t = 0; t < nkeys; ++t) {
                mask[i * nkeys + t] = masks[i][t] != 0;
                any |= mask[i * nkeys + t] != 0;
            }
            if (!any)
                return PCL_INVALID_PARAMETER;
        }
    }
    for (size_t i = 0; i < nq; ++i)
        if (!all_finite(queries[i], query_len))
            return PCL_NON_FINITE_VALUE;
    std::vector<float> flat(nq * query_len);
    for (size_t i = 0; i < nq; ++i)
        std::memcpy(&flat[i * query_len], queries[i], query_len * sizeof(float));
    const size_t group = query_len / head_dim / kv_heads;
    const size_t olen = (kv_end - kv_first) * group * head_dim;
    const bool ok = pcl_hip_attention_f32_multi_kv(
        flat.data(), nq, query_len, keys, values, query_len / head_dim, kv_heads, head_dim, nkeys,
        masks ? mask.data() : nullptr, nkeys, nullptr, out, olen, kv_first, kv_end);
    return ok ? PCL_OK : PCL_NON_FINITE_VALUE;
}

} // extern "C"
