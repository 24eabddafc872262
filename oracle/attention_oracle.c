/*
 * CPU oracle for the attention hot path of power-cpu-llm: a restatement in C
 * of the reference's portable attention, for checking and timing only.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg; never by the product library.
 *
 * Build with -O2 -ffp-contract=off (oracle/Makefile): the reference is Rust,
 * which never contracts a*b+c, and uses an FMA only where it writes mul_add.
 * The reference links bit-exact ports of glibc 2.28's libm (src/libm.rs).
 * The binary32 twin's expf and the rotation's sincosf are restated here from
 * the same glibc 2.28 algorithms and reproduce the reference's libm digests
 * (src/libm/tests.rs:70-92); powf is the host's, which reproduces its digest
 * too. The exact path's f64 exp is the host's; the reference's (glibc 2.28's
 * table-driven IBM exp) differs from it in the last bit on some inputs, so
 * the exact path matches the reference to the last bit except where such an
 * ulp decides a rounding.
 *
 * Licence notice for the two libm restatements (power8_expf and
 * glibc228_sincosf, with their helpers and constants): they restate
 * algorithms of the GNU C Library 2.28, sysdeps/powerpc/powerpc64/power8/
 * fpu/e_expf.S (Copyright (C) 2016-2018 Free Software Foundation, Inc.) and
 * sysdeps/ieee754/flt-32/s_sincosf.c and s_sincosf.h (Copyright (C)
 * 2017-2018 Free Software Foundation, Inc.), which are licensed under the
 * GNU Lesser General Public License version 2.1 or (at your option) any
 * later version, as are the reference's own ports of them (src/libm.rs;
 * the reference's LICENSE and THIRD-PARTY-NOTICES). Those parts of this file
 * are distributed under the same licence. They are test infrastructure: no
 * product code includes or links them.
 */
#include "attention_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* glibc 2.28's POWER8 expf, restated below (the binary32 twin's softmax). */
static float power8_expf(float x);

/* p9_ref_attention_heads (src/kernels/portable/reference.rs:327-393); with
 * cap > 0, every score s first becomes f32(cap * tanh(f64(s) / cap)), the
 * reference's p9_ref_softcap (reference.rs:226-235) applied to the scores. */
static bool ref_heads(const float *query, const float *keys, const float *values,
                      size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                      const uint8_t *allowed, float *scratch, float *out, size_t h_first,
                      size_t h_end, double cap)
{
    if (h_first > h_end || h_end > qheads) /* reference.rs:341-343 */
        return false;
    if (kvheads == 0 || qheads < kvheads) /* the wrapper's shape checks (reference.rs:421-437) */
        return false;
    const size_t group = qheads / kvheads;
    const size_t stride = kvheads * dim;
    for (size_t h = h_first; h < h_end; ++h) {
        const size_t kh = h / group; /* reference.rs:358 */
        float max = -INFINITY;
        for (size_t t = 0; t < nkeys; ++t) { /* reference.rs:360-376 */
            scratch[t] = -INFINITY;
            if (allowed && allowed[t] == 0)
                continue;
            double score = 0.0;
            for (size_t d = 0; d < dim; ++d)
                score += (double)query[h * dim + d] * (double)keys[t * stride + kh * dim + d];
            scratch[t] = (float)score;
            if (cap > 0.0)
                scratch[t] = (float)(cap * tanh((double)scratch[t] / cap));
            if (!isfinite(scratch[t]))
                return false;
            if (scratch[t] > max)
                max = scratch[t];
        }
        double sum = 0.0; /* reference.rs:377-380: every key, masked ones add exp(-inf) */
        for (size_t t = 0; t < nkeys; ++t)
            sum += exp((double)scratch[t] - (double)max);
        for (size_t t = 0; t < nkeys; ++t) /* reference.rs:381-383 */
            scratch[t] = (float)(exp((double)scratch[t] - (double)max) / sum);
        for (size_t d = 0; d < dim; ++d) { /* reference.rs:384-390: d outer, t inner */
            double result = 0.0;
            for (size_t t = 0; t < nkeys; ++t)
                result += (double)scratch[t] * (double)values[t * stride + kh * dim + d];
            out[(h - h_first) * dim + d] = (float)result;
        }
    }
    return true;
}

bool oracle_ref_attention_heads(const float *query, const float *keys, const float *values,
                                size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                const uint8_t *allowed, float *scratch, float *out,
                                size_t h_first, size_t h_end)
{
    return ref_heads(query, keys, values, qheads, kvheads, dim, nkeys, allowed, scratch, out,
                     h_first, h_end, 0.0);
}

bool oracle_ref_attention_heads_softcap(const float *query, const float *keys,
                                        const float *values, size_t qheads, size_t kvheads,
                                        size_t dim, size_t nkeys, const uint8_t *allowed,
                                        float *scratch, float *out, size_t h_first,
                                        size_t h_end, float softcap)
{
    if (!(softcap > 0.0f))
        return false;
    return ref_heads(query, keys, values, qheads, kvheads, dim, nkeys, allowed, scratch, out,
                     h_first, h_end, (double)softcap);
}

/* oracle_ref_attention_heads restructured for speed where that cannot
 * change a bit, for checking full-size outputs (the CPU baseline times the
 * straightforward form above): masked keys, whose probability is exactly 0,
 * are left out of the sums (adding exp(-inf) = 0, or 0 * v for a finite v,
 * leaves an f64 sum unchanged); four keys' score sums run interleaved, each
 * still over ascending d; and the P.V sums run key-outer over a row of f64
 * accumulators, each output's sum still over ascending t. Equal to the
 * straightforward form bit for bit whenever the value rows of masked keys
 * are finite (the reference's 0 * inf makes its output NaN there). */
bool oracle_ref_attention_heads_checker(const float *query, const float *keys,
                                        const float *values, size_t qheads, size_t kvheads,
                                        size_t dim, size_t nkeys, const uint8_t *allowed,
                                        float *scratch, float *out, size_t h_first,
                                        size_t h_end)
{
    if (h_first > h_end || h_end > qheads)
        return false;
    if (kvheads == 0 || qheads < kvheads)
        return false;
    const size_t group = qheads / kvheads;
    const size_t stride = kvheads * dim;
    double *acc = (double *)malloc(dim * sizeof(double));
    size_t *live = (size_t *)malloc((nkeys ? nkeys : 1) * sizeof(size_t));
    if (!acc || !live) {
        free(acc);
        free(live);
        return false;
    }
    bool ok = true;
    for (size_t h = h_first; h < h_end && ok; ++h) {
        const size_t kh = h / group;
        const float *q = query + h * dim;
        size_t n = 0;
        for (size_t t = 0; t < nkeys; ++t)
            if (!allowed || allowed[t] != 0)
                live[n++] = t;
        float max = -INFINITY;
        size_t i = 0;
        for (; i + 4 <= n && ok; i += 4) {
            const float *k0 = keys + live[i] * stride + kh * dim;
            const float *k1 = keys + live[i + 1] * stride + kh * dim;
            const float *k2 = keys + live[i + 2] * stride + kh * dim;
            const float *k3 = keys + live[i + 3] * stride + kh * dim;
            double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
            for (size_t d = 0; d < dim; ++d) {
                const double qd = (double)q[d];
                s0 += qd * (double)k0[d];
                s1 += qd * (double)k1[d];
                s2 += qd * (double)k2[d];
                s3 += qd * (double)k3[d];
            }
            const double s[4] = {s0, s1, s2, s3};
            for (int j = 0; j < 4; ++j) {
                const float f = (float)s[j];
                scratch[i + j] = f;
                if (!isfinite(f))
                    ok = false;
                if (f > max)
                    max = f;
            }
        }
        for (; i < n && ok; ++i) {
            const float *k = keys + live[i] * stride + kh * dim;
            double score = 0.0;
            for (size_t d = 0; d < dim; ++d)
                score += (double)q[d] * (double)k[d];
            scratch[i] = (float)score;
            if (!isfinite(scratch[i]))
                ok = false;
            if (scratch[i] > max)
                max = scratch[i];
        }
        if (!ok)
            break;
        double sum = 0.0;
        for (i = 0; i < n; ++i)
            sum += exp((double)scratch[i] - (double)max);
        for (size_t d = 0; d < dim; ++d)
            acc[d] = 0.0;
        for (i = 0; i < n; ++i) {
            const double p = (double)(float)(exp((double)scratch[i] - (double)max) / sum);
            const float *v = values + live[i] * stride + kh * dim;
            for (size_t d = 0; d < dim; ++d)
                acc[d] += p * (double)v[d];
        }
        for (size_t d = 0; d < dim; ++d)
            out[(h - h_first) * dim + d] = (float)acc[d];
    }
    free(live);
    free(acc);
    return ok;
}

/* softmax (src/kernels/portable/attention.rs:15-43). */
static bool oracle_softmax_f32(float *scores, size_t n, const uint8_t *allowed)
{
    float max = -INFINITY;
    for (size_t t = 0; t < n; ++t) {
        if (allowed && allowed[t] == 0)
            continue;
        if (!isfinite(scores[t]))
            return false;
        if (scores[t] > max)
            max = scores[t];
    }
    float sum = 0.0f;
    for (size_t t = 0; t < n; ++t) {
        const float e = (allowed && allowed[t] == 0) ? 0.0f : power8_expf(scores[t] - max);
        scores[t] = e;
        sum += e;
    }
    for (size_t t = 0; t < n; ++t)
        scores[t] /= sum;
    return true;
}

/* pa_attention_f32_heads (src/kernels/portable/attention.rs:51-112). */
bool oracle_pa_attention_f32_heads(const float *query, const float *keys, const float *values,
                                   size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                   const uint8_t *allowed, float *scratch, float *out,
                                   size_t h_first, size_t h_end)
{
    if (h_first > h_end || h_end > qheads)
        return false;
    if (dim % 16 != 0 || kvheads == 0 || qheads % kvheads != 0) /* attention.rs:68-70 */
        return false;
    const size_t group = qheads / kvheads;
    const size_t stride = kvheads * dim;
    for (size_t h = h_first; h < h_end; ++h) {
        const float *q = query + h * dim;
        const size_t kh = h / group;
        for (size_t t = 0; t < nkeys; ++t) { /* attention.rs:87-95 */
            const float *k = keys + t * stride + kh * dim;
            float p[16] = {0};
            for (size_t d = 0; d < dim; ++d)
                p[d % 16] = fmaf(q[d], k[d], p[d % 16]);
            float v[4];
            for (int l = 0; l < 4; ++l)
                v[l] = (p[l] + p[4 + l]) + (p[8 + l] + p[12 + l]);
            scratch[t] = (v[0] + v[1]) + (v[2] + v[3]);
        }
        if (!oracle_softmax_f32(scratch, nkeys, allowed))
            return false;
        float *o = out + (h - h_first) * dim;
        for (size_t d = 0; d < dim; ++d) /* attention.rs:99-106 */
            o[d] = 0.0f;
        for (size_t t = 0; t < nkeys; ++t) {
            const float *vt = values + t * stride + kh * dim;
            for (size_t d = 0; d < dim; ++d)
                o[d] = fmaf(scratch[t], vt[d], o[d]);
        }
        for (size_t d = 0; d < dim; ++d) /* attention.rs:107-109 */
            if (!isfinite(o[d]))
                return false;
    }
    return true;
}

typedef bool (*heads_fn)(const float *, const float *, const float *, size_t, size_t, size_t,
                         size_t, const uint8_t *, float *, float *, size_t, size_t);

/* One single-query call per query over query heads kh_first*group ..
 * kh_end*group, output row i at out + i*o_stride. */
static bool oracle_multi_kv(heads_fn kernel, const float *query, size_t nq, size_t q_stride,
                            const float *keys, const float *values, size_t qheads,
                            size_t kvheads, size_t dim, size_t nkeys, const uint8_t *allowed,
                            size_t mask_stride, float *scratch, float *out, size_t o_stride,
                            size_t kh_first, size_t kh_end)
{
    if (kvheads == 0 || kh_first > kh_end || kh_end > kvheads || qheads % kvheads != 0)
        return false;
    const size_t group = qheads / kvheads;
    for (size_t i = 0; i < nq; ++i) {
        const uint8_t *mask = allowed ? allowed + i * mask_stride : NULL;
        if (!kernel(query + i * q_stride, keys, values, qheads, kvheads, dim, nkeys, mask,
                    scratch, out + i * o_stride, kh_first * group, kh_end * group))
            return false;
    }
    return true;
}

bool oracle_pa_attention_f32_multi_kv(const float *query, size_t nq, size_t q_stride,
                                      const float *keys, const float *values, size_t qheads,
                                      size_t kvheads, size_t dim, size_t nkeys,
                                      const uint8_t *allowed, size_t mask_stride,
                                      float *scratch, float *out, size_t o_stride,
                                      size_t kh_first, size_t kh_end)
{
    return oracle_multi_kv(oracle_pa_attention_f32_heads, query, nq, q_stride, keys, values,
                           qheads, kvheads, dim, nkeys, allowed, mask_stride, scratch, out,
                           o_stride, kh_first, kh_end);
}

bool oracle_ref_attention_multi_kv(const float *query, size_t nq, size_t q_stride,
                                   const float *keys, const float *values, size_t qheads,
                                   size_t kvheads, size_t dim, size_t nkeys,
                                   const uint8_t *allowed, size_t mask_stride, float *scratch,
                                   float *out, size_t o_stride, size_t kh_first, size_t kh_end)
{
    return oracle_multi_kv(oracle_ref_attention_heads, query, nq, q_stride, keys, values,
                           qheads, kvheads, dim, nkeys, allowed, mask_stride, scratch, out,
                           o_stride, kh_first, kh_end);
}

/* all_finite (src/kernels/reference.rs:88-94): no inf or NaN. */
static bool oracle_all_finite(const float *x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(x[i]))
            return false;
    return true;
}

/* kernels::reference::attention_heads (src/kernels/reference.rs:412-478). */
int oracle_attention_heads_checked(const float *query, size_t query_len, const float *keys,
                                   size_t keys_len, const float *values, size_t values_len,
                                   size_t kv_heads, size_t head_dim, const uint8_t *allowed,
                                   size_t mask_len, int has_mask, size_t h_first, size_t h_end,
                                   int has_heads, float *out)
{
    if (kv_heads == 0 || head_dim == 0 || kv_heads > SIZE_MAX / head_dim)
        return ORACLE_INVALID_SHAPE; /* reference.rs:421-424 */
    const size_t width = kv_heads * head_dim;
    if (query_len == 0 || query_len % head_dim != 0 || keys_len == 0 || keys_len % width != 0 ||
        values_len != keys_len)
        return ORACLE_INVALID_SHAPE; /* reference.rs:425-432 */
    const size_t qheads = query_len / head_dim;
    const size_t nkeys = keys_len / width;
    if (qheads % kv_heads != 0)
        return ORACLE_INVALID_SHAPE;
    if (has_mask) { /* reference.rs:438-445 */
        if (mask_len != nkeys)
            return ORACLE_INVALID_SHAPE;
        bool any = false;
        for (size_t t = 0; t < nkeys; ++t)
            any |= allowed[t] != 0;
        if (!any)
            return ORACLE_INVALID_PARAMETER;
    }
    if (!has_heads) {
        h_first = 0;
        h_end = qheads;
    }
    if (h_first > h_end || h_end > qheads)
        return ORACLE_INVALID_SHAPE;
    if (!oracle_all_finite(query, query_len) || !oracle_all_finite(keys, keys_len) ||
        !oracle_all_finite(values, values_len))
        return ORACLE_NON_FINITE_VALUE; /* reference.rs:450-452 */
    uint8_t *mask = NULL;
    if (has_mask) { /* bool -> u8 (reference.rs:453) */
        mask = (uint8_t *)malloc(nkeys ? nkeys : 1);
        for (size_t t = 0; t < nkeys; ++t)
            mask[t] = allowed[t] != 0;
    }
    float *scratch = (float *)malloc(nkeys * sizeof(float));
    const bool ok = oracle_ref_attention_heads(query, keys, values, qheads, kv_heads, head_dim,
                                               nkeys, mask, scratch, out, h_first, h_end);
    free(scratch);
    free(mask);
    if (!ok)
        return ORACLE_NON_FINITE_VALUE;
    return oracle_all_finite(out, (h_end - h_first) * head_dim) ? ORACLE_OK
                                                                : ORACLE_NON_FINITE_VALUE;
}

/* encoder_mask (src/engine/attention.rs:1170-1182). */
int oracle_encoder_mask(size_t first_key, size_t count, size_t query, size_t window,
                        int has_window, uint8_t *out)
{
    if (count == 0 || (has_window && window == 0) || first_key > SIZE_MAX - count)
        return ORACLE_INVALID_SHAPE;
    for (size_t i = 0; i < count; ++i) {
        const size_t k = first_key + i;
        out[i] = k <= query && (!has_window || query - k < window);
    }
    return ORACLE_OK;
}

/* retained_count (src/engine/attention.rs:1166-1168). */
size_t oracle_retained_count(size_t count, size_t window, int has_window)
{
    if (!has_window)
        return count;
    const size_t keep = window > 0 ? window - 1 : 0;
    return count < keep ? count : keep;
}

/* ---- layer cache ------------------------------------------------------- */

/* new_cache (src/engine/attention.rs:484-505). */
int oracle_cache_init(oracle_layer_cache *c, size_t kv_heads, size_t head_dim, size_t context,
                      size_t window, int has_window, size_t max_bytes)
{
    memset(c, 0, sizeof(*c));
    if (kv_heads == 0 || head_dim == 0 || kv_heads > SIZE_MAX / head_dim)
        return ORACLE_INVALID_SHAPE;
    const size_t width = kv_heads * head_dim;
    if (width > SIZE_MAX / (2 * sizeof(float)))
        return ORACLE_RESOURCE_LIMIT;
    if (max_bytes < width * 2 * sizeof(float))
        return ORACLE_RESOURCE_LIMIT;
    c->width = width;
    c->context = context;
    c->window = window;
    c->has_window = has_window;
    c->max_bytes = max_bytes;
    return ORACLE_OK;
}

void oracle_cache_free(oracle_layer_cache *c)
{
    free(c->keys);
    free(c->values);
    c->keys = c->values = NULL;
    c->len = c->cap = 0;
}

/* retained_tokens (attention.rs:271-273). */
size_t oracle_cache_retained(const oracle_layer_cache *c)
{
    return (c->len - c->start) / c->width;
}

/* try_reserve: room for `extra` more floats after len. */
static int oracle_cache_reserve(oracle_layer_cache *c, size_t extra)
{
    if (c->len + extra <= c->cap)
        return ORACLE_OK;
    const size_t cap = c->len + extra;
    float *k = realloc(c->keys, cap * sizeof(float));
    if (!k)
        return ORACLE_RESOURCE_LIMIT;
    c->keys = k;
    float *v = realloc(c->values, cap * sizeof(float));
    if (!v)
        return ORACLE_RESOURCE_LIMIT;
    c->values = v;
    c->cap = cap;
    return ORACLE_OK;
}

/* check_stage's limits (attention.rs:542-559) and encode_in_place's append
 * (attention.rs:956-980, 1070-1073). */
int oracle_cache_append(oracle_layer_cache *c, const float *keys, const float *values, size_t n,
                        size_t *old_len, size_t *old_total)
{
    if (n == 0)
        return ORACLE_INVALID_SHAPE; /* "hidden-state rows" */
    if (c->total > SIZE_MAX - n || c->total + n > c->context)
        return ORACLE_RESOURCE_LIMIT;
    const size_t next_position = c->total + n;
    const size_t count = oracle_cache_retained(c) + n;
    if (count > SIZE_MAX / c->width)
        return ORACLE_RESOURCE_LIMIT;
    const size_t cells = count * c->width;
    if (cells > SIZE_MAX / (2 * sizeof(float)) || cells * 2 * sizeof(float) > c->max_bytes)
        return ORACLE_RESOURCE_LIMIT;
    *old_len = c->len;
    *old_total = c->total;
    const size_t extra = cells - (c->len - c->start);
    if (oracle_cache_reserve(c, extra) != ORACLE_OK)
        return ORACLE_RESOURCE_LIMIT;
    memcpy(c->keys + c->len, keys, n * c->width * sizeof(float));
    memcpy(c->values + c->len, values, n * c->width * sizeof(float));
    c->len += n * c->width;
    c->total = next_position;
    return ORACLE_OK;
}

/* LayerCache::rollback (attention.rs:280-285). */
void oracle_cache_rollback(oracle_layer_cache *c, size_t old_len, size_t old_total)
{
    if (old_len < c->len)
        c->len = old_len;
    c->total = old_total;
}

/* LayerCache::keep (attention.rs:286-296). */
void oracle_cache_keep(oracle_layer_cache *c, size_t old_len, size_t old_total, size_t tokens)
{
    const size_t len = old_len + tokens * c->width;
    if (len < c->len)
        c->len = len;
    c->total = old_total + tokens;
}

/* LayerCache::commit (attention.rs:297-310): window retention, then the dead
 * prefix drained once it is at least half the buffer. */
void oracle_cache_commit(oracle_layer_cache *c)
{
    const size_t count = (c->len - c->start) / c->width;
    const size_t keep = oracle_retained_count(count, c->window, c->has_window);
    c->start += (count - keep) * c->width;
    if (c->start > 0 && c->start * 2 >= c->len) {
        memmove(c->keys, c->keys + c->start, (c->len - c->start) * sizeof(float));
        memmove(c->values, c->values + c->start, (c->len - c->start) * sizeof(float));
        c->len -= c->start;
        c->start = 0;
    }
}

/* ---- head transform primitives ----------------------------------------- */

/* p9_ref_rms_norm (src/kernels/portable/reference.rs:11-33). */
void oracle_rms_norm(const float *x, const float *scale, size_t n, float eps, float *out)
{
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i)
        sum += (double)x[i] * (double)x[i];
    const double inv = 1.0 / sqrt(sum / (double)n + (double)eps);
    for (size_t i = 0; i < n; ++i) {
        const float normed = (float)((double)x[i] * inv);
        out[i] = scale ? normed * scale[i] : normed;
    }
}

static float from_bits(uint32_t b);

/* expf of glibc 2.28 on POWER8 (sysdeps/powerpc/powerpc64/power8/fpu/e_expf.S),
 * which the reference ports bit for bit (libm::expf, src/libm.rs:292-345) for
 * the binary32 twin's softmax: x = (64n + j) ln2/64 + y, e^x = 2^n 2^(j/64)
 * (1 + P(y)) in f64 with the table 2^(j/64) (correctly rounded; generated
 * with 60-digit decimals), rounded once to binary32. The multiply-adds fuse
 * where the reference's mul_add calls do. */
static const double ex_t[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0,
    0x1.0874518759bc8p+0, 0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0,
    0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0, 0x1.172b83c7d517bp+0,
    0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0,
    0x1.2d285a6e4030bp+0, 0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0,
    0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, 0x1.3dea64c123422p+0,
    0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0,
    0x1.56f4736b527dap+0, 0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0,
    0x1.6247eb03a5585p+0, 0x1.6623882552225p+0, 0x1.6a09e667f3bcdp+0,
    0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0,
    0x1.868d99b4492edp+0, 0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0,
    0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0, 0x1.9c49182a3f090p+0,
    0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0,
    0x1.bcc1e904bc1d2p+0, 0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0,
    0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0, 0x1.d5818dcfba487p+0,
    0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0,
    0x1.fa7c1819e90d8p+0
};

static float ex_reduce(float x, int near_limit)
{
    const double xd = (double)x;
    const double kd = fma(xd, 0x1.71547652b82fep+6, 0x1.8p+23); /* 64/ln2, 2^23 + 2^22 */
    const float k = (float)kd;
    uint32_t kb;
    memcpy(&kb, &k, 4);
    const uint32_t j = kb & 63;
    const double y = fma((double)(k - 12582912.0f), -0x1.62e42fefa39efp-7, xd); /* -ln2/64 */
    const double z = y * y;
    const double p = fma(y, fma(0x1.55550da752d4fp-3, z, 0x1.fffffffffe7c6p-1),
                         fma(0x1.56420eb78fa85p-5, z, 0x1.00000008d6118p-1) * z);
    const double t = ex_t[j];
    const double r = fma(p, t, t);
    const uint32_t n = kb & ~63u;
    double scale;
    if (near_limit) {
        const uint64_t sb = ((uint64_t)(uint32_t)(n + 0xffc0u) & 0x1ffffu) << 46;
        memcpy(&scale, &sb, 8);
    } else {
        const uint32_t sb = ((n + 0x1fc0u) & 0x3fffu) << 17;
        float sf;
        memcpy(&sf, &sb, 4);
        scale = (double)sf;
    }
    return (float)(scale * r);
}

static float power8_expf(float x)
{
    uint32_t bits;
    memcpy(&bits, &x, 4);
    const uint32_t a = bits & 0x7fffffffu;
    if (a >= 0x42ad496bu) { /* |x| >= 125 ln 2 */
        const int negative = (bits >> 31) != 0;
        if (a <= (negative ? 0x42cff1b4u : 0x42b17217u))
            return ex_reduce(x, 1);
        if (a >= 0x7f800000u) {
            if (a != 0x7f800000u)
                return (float)((double)x + (double)x); /* NaN */
            return negative ? 0.0f : INFINITY;
        }
        const float s = from_bits(negative ? 0x0d800000u : 0x71800000u);
        return s * s; /* underflow or overflow, rounded once */
    }
    if (a < 0x31800000u) /* |x| < 2^-28 */
        return x + 1.0f;
    return ex_reduce(x, 0);
}

/* sincosf of glibc 2.28's generic s_sincosf.c / s_sincosf.h, which the
 * reference ports bit for bit (libm::sincosf, src/libm.rs:350-497): |x| is
 * reduced by k*pi/2 (a table below 9pi/4, two pi/2 pieces below 2^23, 28-bit
 * pieces of 4/pi above) and evaluated in f64 with Chebyshev forms on
 * [-pi/4, pi/4], then rounded to binary32. The multiply-adds are fused
 * exactly where the reference fuses them (its mul_add calls; glibc built with
 * FMA contraction); every other operation is unfused. The newer glibc of
 * this host differs from it in the last bit on some inputs. */
static const double sc_cos[5] = {-0x1.ffffffffe98aep-2, 0x1.55555545c50c7p-5,
                                 -0x1.6c16b348b6874p-10, 0x1.a00eb9ac43ccp-16,
                                 -0x1.23c97dd8844d7p-22};
static const double sc_sin[5] = {-0x1.5555555551cd9p-3, 0x1.1111110c2688bp-7,
                                 -0x1.a019f8b4bd1f9p-13, 0x1.71d7264e6b5b4p-19,
                                 -0x1.a947e1674b58ap-26};
static const double sc_pio2[6] = {0.0, 0x1.921fb54442d18p+0, 0x1.921fb54442d18p+1,
                                  0x1.2d97c7f3321d2p+2, 0x1.921fb54442d18p+2,
                                  0x1.f6a7a2955385ep+2};
static const double sc_invpio4[8] = {0.0,           0x1.45f306cp+0,  0x1.c9c882ap-28,
                                     0x1.4fe13a8p-58, 0x1.f47d4d0p-85, 0x1.bb81b6cp-112,
                                     0x1.4acc9e0p-142, 0x1.0e4107cp-169};

static double sc_sin_poly(double t, double t2)
{
    double p = fma(sc_sin[4], t2, sc_sin[3]);
    for (int k = 2; k >= 0; --k)
        p = fma(t2, p, sc_sin[k]);
    return fma(t * t2, p, t);
}

static double sc_cos_poly(double t2)
{
    double p = fma(sc_cos[4], t2, sc_cos[3]);
    for (int k = 2; k >= 0; --k)
        p = fma(t2, p, sc_cos[k]);
    return fma(t2, p, 1.0);
}

/* t: reduced |x|; n = trunc(|x| / (pi/4)) + 1 selects the form and sign. */
static void sc_reduced(double t, uint32_t n, unsigned negative, float *s, float *c)
{
    const double t2 = t * t;
    const double sv = (n & 2) == 0 ? sc_sin_poly(t, t2) : sc_cos_poly(t2);
    const uint32_t m = n + 2;
    const double cv = (m & 2) == 0 ? sc_sin_poly(t, t2) : sc_cos_poly(t2);
    *s = (float)((((n >> 2) & 1) ^ negative) ? -sv : sv);
    *c = (float)(((m >> 2) & 1) ? -cv : cv);
}

static void glibc228_sincosf(float x, float *s, float *c)
{
    const double pi_4 = 0x1.921fb54442d18p-1, inv_pi_4 = 0x1.45f306dc9c883p+0;
    const double t = (double)x, at = fabs(t);
    if (at < pi_4) {
        if (at >= 0x1p-5) {
            const double t2 = t * t;
            *s = (float)sc_sin_poly(t, t2);
            *c = (float)sc_cos_poly(t2);
            return;
        }
        if (at >= 0x1p-27) {
            const double t2 = t * t, t3 = t * t2;
            *c = (float)fma(t2, fma(t3, 0x1.55514b178dac5p-5, -0x1.fffffff5cc6fdp-2), 1.0);
            *s = (float)fma(t3, fma(t2, 0x1.110f475cec8c5p-7, -0x1.555555543d49dp-3), t);
            return;
        }
        *s = (float)(t != 0.0 ? fma(-t, 0x1p-50, t) : t);
        *c = (float)(1.0 - at);
        return;
    }
    const unsigned negative = x < 0.0f;
    if (at < 0x1.c463abeccb2bbp+2) { /* 9 pi/4 */
        const uint32_t n = (uint32_t)fma(at, inv_pi_4, 1.0);
        sc_reduced(at - sc_pio2[n / 2], n, negative, s, c);
        return;
    }
    if (!isfinite(at)) {
        *s = *c = x - x;
        return;
    }
    if (at < 0x1p23) {
        const uint32_t n = (uint32_t)(at * inv_pi_4) + 1;
        const double k = (double)(n / 2);
        const double r = fma(-k, 0x1.0b4611a626332p-34, fma(-k, 0x1.921fb544p+0, at));
        sc_reduced(r, n, negative, s, c);
        return;
    }
    /* |x| >= 2^23: the product of |x| with four 28-bit pieces of 4/pi from
     * the piece that keeps the integer part below 2^53 */
    uint32_t bits;
    const float ax = fabsf(x);
    memcpy(&bits, &ax, 4);
    const int e = ((int)(bits >> 23) - 127 + 3) / 28;
    double a = sc_invpio4[e] * at;
    const double b = sc_invpio4[e + 1] * at, cc = sc_invpio4[e + 2] * at,
                 d = sc_invpio4[e + 3] * at;
    uint64_t l = (uint64_t)a;
    l &= ~(uint64_t)7;
    a -= (double)l;
    double f = a + b;
    l = (uint64_t)f;
    f = a - (double)l;
    if (l & 1) {
        f -= 1.0;
        f = d + (cc + (b + f));
    } else {
        f = d + (cc + (b + f));
        if (f > 1.0) {
            l += 1;
            f -= 2.0;
        }
    }
    sc_reduced(f * pi_4, (uint32_t)l + 1, negative, s, c);
}

/* p9_ref_rope (reference.rs:277-318). */
bool oracle_rope(const float *x, size_t heads, size_t dim, size_t position, float base,
                 const float *factors, float *out)
{
    const size_t half = dim / 2;
    for (size_t i = 0; i < half; ++i) {
        float inv = 1.0f / powf(base, (2.0f * (float)i) / (float)dim);
        if (factors)
            inv /= factors[i];
        const float angle = (float)position * inv;
        if (!isfinite(angle))
            return false;
        float s, c;
        glibc228_sincosf(angle, &s, &c);
        for (size_t h = 0; h < heads; ++h) {
            const size_t a = h * dim + i, b = h * dim + i + half;
            const float xa = x[a], xb = x[b];
            out[a] = xa * c - xb * s;
            out[b] = xb * c + xa * s;
        }
    }
    return true;
}

static uint64_t fnv(uint64_t h, uint64_t v)
{
    return (h ^ v) * 0x100000001b3ULL;
}

static float from_bits(uint32_t b)
{
    float x;
    memcpy(&x, &b, 4);
    return x;
}

/* bits of r; a NaN generated from non-NaN inputs as the positive default NaN */
static uint32_t digest_bits(float r, int inputs_nan)
{
    uint32_t b;
    memcpy(&b, &r, 4);
    return (!inputs_nan && isnan(r)) ? 0x7fc00000u : b;
}

/* The reference's digest inputs (src/libm/tests.rs:20-62): every 61st
 * binary32 pattern for sincosf; for powf, xorshift64 pairs from seed
 * 0x2545f4914f6cdd1d, random patterns at even steps and x in (0, 1e6],
 * y in [-2, 2] at odd steps. */
void oracle_sincosf(float x, float *s, float *c)
{
    glibc228_sincosf(x, s, c);
}

uint64_t oracle_libm_digest(int which)
{
    uint64_t h = 0xcbf29ce484222325ULL;
    if (which == 2) {
        for (uint64_t k = 0; k <= 0xffffffffULL / 61; ++k) {
            const float x = from_bits((uint32_t)(k * 61));
            h = fnv(h, digest_bits(power8_expf(x), isnan(x)));
        }
        return h;
    }
    if (which == 1) {
        for (uint64_t k = 0; k <= 0xffffffffULL / 61; ++k) {
            const float x = from_bits((uint32_t)(k * 61));
            float s, c;
            glibc228_sincosf(x, &s, &c);
            h = fnv(fnv(h, digest_bits(s, isnan(x))), digest_bits(c, isnan(x)));
        }
        return h;
    }
    uint64_t r = 0x2545f4914f6cdd1dULL;
    for (uint32_t k = 0; k < (1u << 22); ++k) {
        r ^= r << 13;
        r ^= r >> 7;
        r ^= r << 17;
        float x, y;
        if (k % 2 == 0) {
            x = from_bits((uint32_t)r);
            y = from_bits((uint32_t)(r >> 32));
        } else {
            const float u1 = (float)(r >> 40) / (float)(1u << 24);
            const float u2 = (float)((r << 24) >> 40) / (float)(1u << 24);
            x = 1e6f * u1;
            const float t = 4.0f * u2;
            y = t - 2.0f;
        }
        h = fnv(h, digest_bits(powf(x, y), isnan(x) || isnan(y)));
    }
    return h;
}

/* ---- output block primitives -------------------------------------------- */

/* p9_ref_matvec (src/kernels/portable/reference.rs:36-78); its eight-row
 * interleave does not change any row's sum. */
void oracle_matvec(const float *matrix, const float *x, size_t rows, size_t cols, float *out)
{
    for (size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c)
            sum += (double)matrix[r * cols + c] * (double)x[c];
        out[r] = (float)sum;
    }
}

/* p9_ref_add. */
void oracle_add(const float *a, const float *b, size_t n, float *out)
{
    for (size_t i = 0; i < n; ++i)
        out[i] = a[i] + b[i];
}

/* ---- threaded CPU baseline (the engine's decomposition) ---------------- */

struct job {
    heads_fn kernel;
    const float *query, *keys, *values;
    size_t nq, qheads, kvheads, dim, nkeys;
    int causal;
    size_t first_key, first_query, window;
    size_t query_step; /* query i is at position first_query + i * query_step */
    float *out;
    /* head-split decode: items (query, head range) */
    size_t per;
    size_t parts;
    /* this worker's contiguous range of items or queries */
    size_t first, end;
    bool heads_mode;
    bool ok;
};

static void *oracle_worker(void *arg)
{
    struct job *j = (struct job *)arg;
    float *scratch = (float *)malloc(j->nkeys * sizeof(float));
    uint8_t *mask = (uint8_t *)malloc(j->nkeys);
    const size_t width = j->qheads * j->dim;
    j->ok = true;
    if (j->heads_mode) {
        for (size_t item = j->first; item < j->end && j->ok; ++item) {
            const size_t i = item / j->parts;
            const size_t a = (item % j->parts) * j->per;
            const size_t b = a + j->per < j->qheads ? a + j->per : j->qheads;
            const uint8_t *m = NULL;
            if (j->causal) {
                oracle_encoder_mask(j->first_key, j->nkeys, j->first_query + i * j->query_step,
                                    j->window, j->window != 0, mask);
                m = mask;
            }
            j->ok = j->kernel(j->query + i * width, j->keys, j->values, j->qheads, j->kvheads,
                              j->dim, j->nkeys, m, scratch, j->out + i * width + a * j->dim,
                              a, b);
        }
    } else {
        /* attention.rs:783-785: blocks of 8 queries; the exact and portable
         * backends run each block's queries one by one (power9_fma.rs:211-230). */
        for (size_t i = j->first; i < j->end && j->ok; ++i) {
            const uint8_t *m = NULL;
            if (j->causal) {
                oracle_encoder_mask(j->first_key, j->nkeys, j->first_query + i * j->query_step,
                                    j->window, j->window != 0, mask);
                m = mask;
            }
            j->ok = j->kernel(j->query + i * width, j->keys, j->values, j->qheads, j->kvheads,
                              j->dim, j->nkeys, m, scratch, j->out + i * width, 0, j->qheads);
        }
    }
    free(mask);
    free(scratch);
    return NULL;
}

bool oracle_threaded_attention(int variant, int threads, const float *query, size_t nq,
                               const float *keys, const float *values, size_t qheads,
                               size_t kvheads, size_t dim, size_t nkeys, int causal,
                               size_t first_key, size_t first_query, size_t window,
                               float *out)
{
    return oracle_threaded_attention_sample(variant, threads, query, nq, 1, keys, values, qheads,
                                            kvheads, dim, nkeys, causal, first_key, first_query,
                                            window, out);
}

bool oracle_threaded_attention_sample(int variant, int threads, const float *query, size_t nq,
                                      size_t query_step, const float *keys, const float *values,
                                      size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                      int causal, size_t first_key, size_t first_query,
                                      size_t window, float *out)
{
    if (threads < 1)
        threads = 1;
    struct job base;
    memset(&base, 0, sizeof base);
    base.kernel = variant == 1   ? oracle_pa_attention_f32_heads
                  : variant == 2 ? oracle_ref_attention_heads_checker
                                 : oracle_ref_attention_heads;
    base.query = query;
    base.keys = keys;
    base.values = values;
    base.nq = nq;
    base.qheads = qheads;
    base.kvheads = kvheads;
    base.dim = dim;
    base.nkeys = nkeys;
    base.causal = causal;
    base.first_key = first_key;
    base.first_query = first_query;
    base.query_step = query_step ? query_step : 1;
    base.window = window;
    base.out = out;
    size_t length;
    if (nq < (size_t)threads) { /* attention.rs:755-765 */
        size_t split = (size_t)threads / nq;
        if (split < 1)
            split = 1;
        if (split > qheads)
            split = qheads;
        base.per = (qheads + split - 1) / split;
        base.parts = (qheads + base.per - 1) / base.per;
        base.heads_mode = true;
        length = nq * base.parts;
    } else {
        base.heads_mode = false;
        length = nq;
    }
    /* Workers::ranges (src/engine/execution.rs:583-597). */
    size_t n = (size_t)threads < length ? (size_t)threads : length;
    if (n == 0)
        return true;
    struct job *jobs = (struct job *)calloc(n, sizeof *jobs);
    pthread_t *tid = (pthread_t *)calloc(n, sizeof *tid);
    const size_t per = length / n, rem = length % n;
    for (size_t i = 0; i < n; ++i) {
        jobs[i] = base;
        jobs[i].first = i * per + (i < rem ? i : rem);
        jobs[i].end = jobs[i].first + per + (i < rem ? 1 : 0);
    }
    for (size_t i = 1; i < n; ++i)
        pthread_create(&tid[i], NULL, oracle_worker, &jobs[i]);
    oracle_worker(&jobs[0]);
    bool ok = jobs[0].ok;
    for (size_t i = 1; i < n; ++i) {
        pthread_join(tid[i], NULL);
        ok = ok && jobs[i].ok;
    }
    free(tid);
    free(jobs);
    return ok;
}

void oracle_xorshift_units(uint64_t *state, float scale, size_t n, float *out)
{
    uint64_t x = *state;
    for (size_t i = 0; i < n; ++i) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        float u = (float)(x % 20001) / 10000.0f - 1.0f;
        if (scale != 1.0f)
            u = u * scale;
        out[i] = u;
    }
    *state = x;
}
