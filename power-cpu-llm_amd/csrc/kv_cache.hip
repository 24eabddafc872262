// Device-resident layer cache: the engine's LayerCache
// (src/engine/attention.rs:244-311) with its K/V rows in HBM.
//
// Rows [start, len) of the two token-major buffers are retained; an
// uncommitted step appends rows after them. The buffers grow like a Vec: a
// step that does not fit moves the retained rows into a new allocation sized
// for at least twice what the step needs (bounded by the cache's byte limit).
// commit() drops window-evicted rows by moving `start`, and compacts once the
// dead prefix is at least half the rows, as the engine does; with
// start >= len - start the compacting copy never overlaps itself.
#include "context.hpp"
#include "pcl_attention.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>

namespace pcl {

// Caller rows of K and V that are device memory of the cache's device are
// copied by one launch of this kernel (blockIdx.y picks K or V) rather than
// two runtime copies: a decode step's one-row append is then one dispatch.
// n 16-byte pieces per array when `wide`, else n floats.
__global__ __launch_bounds__(256) void append_rows_kernel(const float *sk, const float *sv,
                                                         float *dk, float *dv, int64_t n,
                                                         int wide)
{
    const float *src = blockIdx.y ? sv : sk;
    float *dst = blockIdx.y ? dv : dk;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        if (wide)
            reinterpret_cast<float4 *>(dst)[i] = reinterpret_cast<const float4 *>(src)[i];
        else
            dst[i] = src[i];
    }
}

} // namespace pcl

namespace {

void report(const char *what, hipError_t e)
{
    std::fprintf(stderr, "pcl_kv_cache: %s: %s\n", what, hipGetErrorString(e));
}

// retained_count (attention.rs:1166-1168).
int64_t retained_count(int64_t count, int64_t window)
{
    if (window == 0)
        return count;
    return std::min(count, window - 1);
}

// Rows of K and V on the context's stream; `kind` is hipMemcpyDefault for
// caller rows (device or host memory) and device-to-device inside the cache.
hipError_t copy_rows(pcl_kv_cache *c, float *dk, float *dv, const float *sk, const float *sv,
                     int64_t rows, hipMemcpyKind kind = hipMemcpyDeviceToDevice)
{
    if (rows == 0)
        return hipSuccess;
    const size_t bytes = (size_t)rows * c->width * sizeof(float);
    hipError_t e = hipMemcpyAsync(dk, sk, bytes, kind, c->ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dv, sv, bytes, kind, c->ctx->stream);
    return e;
}

// True when p is device memory of `device`. An unregistered host pointer
// makes the query fail; that failure is cleared here so that it is not
// reported by a later launch check.
bool device_memory(const void *p, int device)
{
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice && a.device == device;
}

// Appended caller rows: one kernel launch for device rows on the cache's
// device, runtime copies otherwise (host or peer memory).
hipError_t append_rows(pcl_kv_cache *c, float *dk, float *dv, const float *sk, const float *sv,
                       int64_t rows)
{
    const int dev = c->ctx->device;
    if (!device_memory(sk, dev) || !device_memory(sv, dev))
        return copy_rows(c, dk, dv, sk, sv, rows, hipMemcpyDefault);
    const int64_t floats = rows * c->width;
    const bool wide = floats % 4 == 0 && ((uintptr_t)sk | (uintptr_t)sv | (uintptr_t)dk |
                                          (uintptr_t)dv) % 16 == 0;
    const int64_t n = wide ? floats / 4 : floats;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 2048);
    pcl::append_rows_kernel<<<dim3((unsigned)blocks, 2), 256, 0, c->ctx->stream>>>(
        sk, sv, dk, dv, n, wide ? 1 : 0);
    return hipGetLastError();
}

// A pending record of the current step: its rows start within the retained
// rows and its position is not past the total. (A shared-K/V layer's step
// advances the total without rows, so the two need not move together.)
bool valid_pending(const pcl_kv_cache *c, const pcl_kv_pending *p)
{
    return p && p->old_len >= c->start && p->old_len <= c->len && p->old_total >= 0 &&
           p->old_total <= c->total;
}

} // namespace

namespace pcl {

// Rows the cache's byte limit allows in its buffers.
int64_t row_limit(const pcl_kv_cache *c)
{
    return (int64_t)(c->max_bytes / ((size_t)c->width * 2 * sizeof(float)));
}

// New buffers of `cap` rows (at least the retained rows), the retained rows
// moved to their start and the old buffers freed.
int move_to_buffers(pcl_kv_cache *c, int64_t cap)
{
    const int64_t retained = c->len - c->start;
    float *nk = nullptr, *nv = nullptr;
    hipError_t e = hipMalloc(&nk, (size_t)cap * c->width * sizeof(float));
    if (e == hipSuccess)
        e = hipMalloc(&nv, (size_t)cap * c->width * sizeof(float));
    if (e == hipSuccess && retained)
        e = copy_rows(c, nk, nv, c->k + c->start * c->width, c->v + c->start * c->width,
                      retained);
    if (e == hipSuccess)
        e = hipStreamSynchronize(c->ctx->stream); // the old buffers are read
    if (e != hipSuccess) {
        report("growing the cache", e);
        if (nk)
            (void)hipFree(nk);
        if (nv)
            (void)hipFree(nv);
        return PCL_RESOURCE_LIMIT;
    }
    if (c->k)
        (void)hipFree(c->k);
    if (c->v)
        (void)hipFree(c->v);
    c->k = nk;
    c->v = nv;
    c->cap = cap;
    c->len = retained;
    c->start = 0;
    return PCL_OK;
}

int kv_cache_reserve(pcl_kv_cache *c, int64_t n)
{
    // check_stage (attention.rs:543-558): the next position within the
    // context, the retained plus appended K+V within the byte limit
    if (n > c->context - c->total)
        return PCL_RESOURCE_LIMIT;
    const int64_t retained = c->len - c->start;
    const double bytes = (double)(retained + n) * (double)c->width * 2.0 * sizeof(float);
    if (bytes > (double)c->max_bytes)
        return PCL_RESOURCE_LIMIT;
    (void)hipSetDevice(c->ctx->device);
    if (c->len + n <= c->cap)
        return PCL_OK;
    // new buffers for at least twice the step's rows (a Vec's growth),
    // holding at most what the byte limit allows, retained rows first
    const int64_t limit = row_limit(c);
    const int64_t need = retained + n;
    return move_to_buffers(c, std::max(need, std::min(2 * need, limit)));
}

void kv_cache_advance_rows(pcl_kv_cache *c, int64_t n, pcl_kv_pending *pending)
{
    pending->old_len = c->len;
    pending->old_total = c->total;
    c->len += n;
    c->total += n;
}

} // namespace pcl

extern "C" {

int pcl_kv_cache_create(pcl_context *ctx, int64_t kvheads, int64_t dim, int64_t context,
                        int64_t window, size_t max_bytes, pcl_kv_cache **out)
{
    if (!out)
        return PCL_INVALID_SHAPE;
    *out = nullptr;
    if (!ctx || kvheads <= 0 || dim <= 0 || context <= 0 || window < 0 ||
        kvheads > ((int64_t)1 << 20) || dim > ((int64_t)1 << 20))
        return PCL_INVALID_SHAPE;
    const size_t one_token = (size_t)kvheads * dim * 2 * sizeof(float);
    if (max_bytes < one_token) // new_cache (attention.rs:487-492)
        return PCL_RESOURCE_LIMIT;
    auto *c = new pcl_kv_cache;
    c->ctx = ctx;
    c->kvheads = kvheads;
    c->dim = dim;
    c->width = kvheads * dim;
    c->context = context;
    c->window = window;
    c->max_bytes = max_bytes;
    *out = c;
    return PCL_OK;
}

int pcl_kv_cache_reserve_rows(pcl_kv_cache *c, int64_t rows)
{
    if (!c || rows < 0)
        return PCL_INVALID_SHAPE;
    const int64_t cap = std::min(rows, pcl::row_limit(c));
    if (cap <= c->cap)
        return PCL_OK;
    (void)hipSetDevice(c->ctx->device);
    return pcl::move_to_buffers(c, cap);
}

void pcl_kv_cache_destroy(pcl_kv_cache *c)
{
    if (!c)
        return;
    (void)hipSetDevice(c->ctx->device);
    (void)hipStreamSynchronize(c->ctx->stream);
    if (c->k)
        (void)hipFree(c->k);
    if (c->v)
        (void)hipFree(c->v);
    delete c;
}

int64_t pcl_kv_cache_total_tokens(const pcl_kv_cache *c)
{
    return c ? c->total : -1;
}

int64_t pcl_kv_cache_retained_tokens(const pcl_kv_cache *c)
{
    return c ? c->len - c->start : -1;
}

int pcl_kv_cache_view(const pcl_kv_cache *c, const float **keys, const float **values,
                      int64_t *rows, int64_t *first_position)
{
    if (!c)
        return PCL_INVALID_SHAPE;
    const int64_t retained = c->len - c->start;
    if (keys)
        *keys = c->k ? c->k + c->start * c->width : nullptr;
    if (values)
        *values = c->v ? c->v + c->start * c->width : nullptr;
    if (rows)
        *rows = retained;
    if (first_position)
        *first_position = c->total - retained;
    return PCL_OK;
}

int pcl_kv_cache_read(const pcl_kv_cache *c, int64_t first, int64_t rows, float *keys,
                      float *values)
{
    if (!c || first < 0 || rows < 0 || rows > c->len - c->start - first ||
        (rows > 0 && (!keys || !values)))
        return PCL_INVALID_SHAPE;
    if (rows == 0)
        return PCL_OK;
    (void)hipSetDevice(c->ctx->device);
    const int64_t at = (c->start + first) * c->width;
    auto *self = const_cast<pcl_kv_cache *>(c);
    hipError_t e = copy_rows(self, keys, values, c->k + at, c->v + at, rows, hipMemcpyDefault);
    if (e == hipSuccess)
        e = hipStreamSynchronize(c->ctx->stream);
    if (e != hipSuccess) {
        report("reading rows", e);
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

int pcl_kv_cache_append(pcl_kv_cache *c, const float *keys, const float *values, int64_t n,
                        pcl_kv_pending *pending)
{
    if (!c || !pending || n <= 0 || !keys || !values)
        return PCL_INVALID_SHAPE;
    const int rc = pcl::kv_cache_reserve(c, n);
    if (rc != PCL_OK)
        return rc;
    const hipError_t e =
        append_rows(c, c->k + c->len * c->width, c->v + c->len * c->width, keys, values, n);
    if (e != hipSuccess) {
        report("appending rows", e);
        return PCL_NON_FINITE_VALUE;
    }
    pcl::kv_cache_advance_rows(c, n, pending);
    return PCL_OK;
}

int pcl_kv_cache_rollback(pcl_kv_cache *c, const pcl_kv_pending *pending)
{
    if (!c || !valid_pending(c, pending))
        return PCL_INVALID_PARAMETER;
    c->len = pending->old_len;
    c->total = pending->old_total;
    return PCL_OK;
}

int pcl_kv_cache_keep(pcl_kv_cache *c, const pcl_kv_pending *pending, int64_t tokens)
{
    if (!c || !valid_pending(c, pending) || tokens < 0)
        return PCL_INVALID_PARAMETER;
    const int64_t len = pending->old_len + tokens;
    if (len < c->len)
        c->len = len;
    c->total = pending->old_total + tokens;
    return PCL_OK;
}

int pcl_kv_cache_commit(pcl_kv_cache *c)
{
    if (!c)
        return PCL_INVALID_SHAPE;
    const int64_t count = c->len - c->start;
    const int64_t keep = retained_count(count, c->window);
    c->start += count - keep;
    if (c->start > 0 && c->start * 2 >= c->len) {
        // drop the dead prefix: rows [start, len) to the front; with
        // start >= len - start the two ranges are disjoint
        (void)hipSetDevice(c->ctx->device);
        const hipError_t e = copy_rows(c, c->k, c->v, c->k + c->start * c->width,
                                       c->v + c->start * c->width, c->len - c->start);
        if (e != hipSuccess) {
            report("compacting", e);
            return PCL_NON_FINITE_VALUE;
        }
        c->len -= c->start;
        c->start = 0;
    }
    return PCL_OK;
}

int pcl_kv_cache_encoder_desc(const pcl_kv_cache *c, const pcl_kv_pending *pending,
                              pcl_attention_desc *d)
{
    if (!c || !d || !valid_pending(c, pending))
        return PCL_INVALID_PARAMETER;
    const int64_t retained = c->len - c->start;
    d->k0 = c->k + c->start * c->width;
    d->v0 = c->v + c->start * c->width;
    d->n0 = retained;
    d->k1 = d->v1 = nullptr;
    d->n1 = 0;
    d->kvheads = c->kvheads;
    d->dim = c->dim;
    d->mask = nullptr;
    d->causal = 1;
    d->window = c->window;
    d->first_key = c->total - retained;
    d->first_query = pending->old_total;
    return PCL_OK;
}

int pcl_kv_cache_decoder_desc(const pcl_kv_cache *c, const float *canvas_keys,
                              const float *canvas_values, int64_t n, pcl_attention_desc *d)
{
    if (!c || !d || n < 0 || (n > 0 && (!canvas_keys || !canvas_values)))
        return PCL_INVALID_PARAMETER;
    const int64_t retained = c->len - c->start;
    d->k0 = retained ? c->k + c->start * c->width : nullptr;
    d->v0 = retained ? c->v + c->start * c->width : nullptr;
    d->n0 = retained;
    d->k1 = canvas_keys;
    d->v1 = canvas_values;
    d->n1 = n;
    d->kvheads = c->kvheads;
    d->dim = c->dim;
    d->mask = nullptr;
    d->causal = 0;
    d->window = 0;
    d->first_key = c->total - retained;
    d->first_query = c->total;
    return PCL_OK;
}

int pcl_kv_cache_shared_desc(const pcl_kv_cache *c, const pcl_kv_cache *src,
                             const pcl_kv_pending *sp, int64_t n, pcl_attention_desc *d)
{
    if (!c || !src || !d || n <= 0 || !valid_pending(src, sp))
        return PCL_INVALID_PARAMETER;
    if (c->kvheads != src->kvheads || c->dim != src->dim || c->total != sp->old_total ||
        src->total != c->total + n)
        return PCL_INVALID_SHAPE;
    const int64_t retained = src->len - src->start;
    d->k0 = src->k + src->start * src->width;
    d->v0 = src->v + src->start * src->width;
    d->n0 = retained;
    d->k1 = d->v1 = nullptr;
    d->n1 = 0;
    d->kvheads = c->kvheads;
    d->dim = c->dim;
    d->mask = nullptr;
    d->causal = 1;
    d->window = c->window;
    d->first_key = sp->old_total - (sp->old_len - src->start);
    d->first_query = c->total;
    return PCL_OK;
}

int pcl_kv_cache_advance(pcl_kv_cache *c, int64_t n, pcl_kv_pending *pending)
{
    if (!c || !pending || n <= 0)
        return PCL_INVALID_SHAPE;
    if (n > c->context - c->total)
        return PCL_RESOURCE_LIMIT;
    pending->old_len = c->len;
    pending->old_total = c->total;
    c->total += n;
    return PCL_OK;
}

} // extern "C"
