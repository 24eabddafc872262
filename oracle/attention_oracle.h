/*
 * CPU oracle for the attention hot path of power-cpu-llm.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path (power-cpu-llm_amd/) never links, loads or calls it.
 *
 * Every function restates a reference function; the citation is next to each
 * declaration (paths relative to the reference checkout).
 */
#ifndef PCL_ATTENTION_ORACLE_H
#define PCL_ATTENTION_ORACLE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes of kernels::reference::Error (src/kernels/reference.rs:6-11). */
enum oracle_status {
    ORACLE_OK = 0,
    ORACLE_INVALID_SHAPE = 1,
    ORACLE_INVALID_PARAMETER = 2,
    ORACLE_NON_FINITE_VALUE = 3,
};

/* a1 — exact attention: p9_ref_attention_heads
 * (src/kernels/portable/reference.rs:320-393). F64 score and value sums,
 * F32 scores and probabilities, f64 softmax, scale one. scratch [nkeys]. */
bool oracle_ref_attention_heads(const float *query, const float *keys, const float *values,
                                size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                const uint8_t *allowed, float *scratch, float *out,
                                size_t h_first, size_t h_end);

/* The exact path with a logit soft-cap (softcap > 0): each score s becomes
 * f32(softcap * tanh(f64(s) / softcap)) before the softmax, the form of
 * p9_ref_softcap (src/kernels/portable/reference.rs:226-235). The reference
 * applies no cap inside attention; this is the checker of the descriptor's
 * optional softcap field. */
bool oracle_ref_attention_heads_softcap(const float *query, const float *keys,
                                        const float *values, size_t qheads, size_t kvheads,
                                        size_t dim, size_t nkeys, const uint8_t *allowed,
                                        float *scratch, float *out, size_t h_first,
                                        size_t h_end, float softcap);
/* a1 restructured for speed without changing a bit (masked keys left out of
 * the sums, interleaved score sums, key-outer P.V), for checking full-size
 * outputs; equal to oracle_ref_attention_heads whenever masked keys' value
 * rows are finite. */
bool oracle_ref_attention_heads_checker(const float *query, const float *keys,
                                        const float *values, size_t qheads, size_t kvheads,
                                        size_t dim, size_t nkeys, const uint8_t *allowed,
                                        float *scratch, float *out, size_t h_first,
                                        size_t h_end);

/* a3/a4 — binary32 attention: pa_attention_f32_heads + softmax
 * (src/kernels/portable/attention.rs:14-112). 16 FMA score lanes reduced as a
 * fixed tree, f32 softmax (glibc 2.28's POWER8 expf, the reference's
 * libm::expf), FMA PV chain from +0. scratch [nkeys]. */
bool oracle_pa_attention_f32_heads(const float *query, const float *keys, const float *values,
                                   size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                   const uint8_t *allowed, float *scratch, float *out,
                                   size_t h_first, size_t h_end);

/* a7 contract — several queries, KV heads [kh_first, kh_end): one a3 call
 * per query over that head range (the AttentionMulti ABI of
 * src/kernels/quantized/int8.rs:446-484, pinned bitwise to single-query
 * calls by src/kernels/quantized/int8/tests.rs:661-768). */
bool oracle_pa_attention_f32_multi_kv(const float *query, size_t nq, size_t q_stride,
                                      const float *keys, const float *values, size_t qheads,
                                      size_t kvheads, size_t dim, size_t nkeys,
                                      const uint8_t *allowed, size_t mask_stride,
                                      float *scratch, float *out, size_t o_stride,
                                      size_t kh_first, size_t kh_end);

/* The exact backends' multi-query fallback: per query a1 over query heads
 * kv.start*group..kv.end*group (src/kernels/quantized/power9_fma.rs:211-230).
 * scratch [nkeys]. */
bool oracle_ref_attention_multi_kv(const float *query, size_t nq, size_t q_stride,
                                   const float *keys, const float *values, size_t qheads,
                                   size_t kvheads, size_t dim, size_t nkeys,
                                   const uint8_t *allowed, size_t mask_stride, float *scratch,
                                   float *out, size_t o_stride, size_t kh_first, size_t kh_end);

/* a2 — checked exact attention: kernels::reference::attention_heads
 * (src/kernels/reference.rs:412-478). Lengths are element counts; has_mask /
 * has_heads select Option::Some. out holds (h_end-h_first)*head_dim. */
int oracle_attention_heads_checked(const float *query, size_t query_len, const float *keys,
                                   size_t keys_len, const float *values, size_t values_len,
                                   size_t kv_heads, size_t head_dim, const uint8_t *allowed,
                                   size_t mask_len, int has_mask, size_t h_first, size_t h_end,
                                   int has_heads, float *out);

/* a10 — encoder_mask (src/engine/attention.rs:1170-1182): allowed(k) =
 * k <= query && (no window || query - k < window) for k in
 * [first_key, first_key+count). Returns ORACLE_INVALID_SHAPE on count 0,
 * window 0 or overflow. */
int oracle_encoder_mask(size_t first_key, size_t count, size_t query, size_t window,
                        int has_window, uint8_t *out);

/* a10 — retained_count (src/engine/attention.rs:1166-1168). */
size_t oracle_retained_count(size_t count, size_t window, int has_window);

/* Layer cache — LayerCache (src/engine/attention.rs:244-311) with the
 * K/V half of encode_in_place (attention.rs:949-1080): token-major f32
 * rows, lengths and `start` in floats as the engine keeps them. */
enum { ORACLE_RESOURCE_LIMIT = 4 }; /* engine::Error::ResourceLimit */
typedef struct oracle_layer_cache {
    size_t width;      /* kv_heads * head_dim */
    size_t context;    /* ModelSpec::context */
    size_t window;     /* sliding window when has_window */
    int has_window;
    size_t max_bytes;  /* bound of one staged K+V pair */
    size_t total;      /* positions processed */
    size_t start;      /* first retained float */
    size_t len;        /* floats in keys / values */
    size_t cap;        /* floats allocated */
    float *keys, *values;
} oracle_layer_cache;

/* new_cache (attention.rs:484-505). ORACLE_RESOURCE_LIMIT when max_bytes is
 * below one token's K+V. */
int oracle_cache_init(oracle_layer_cache *c, size_t kv_heads, size_t head_dim, size_t context,
                      size_t window, int has_window, size_t max_bytes);
void oracle_cache_free(oracle_layer_cache *c);
/* retained_tokens (attention.rs:271-273). */
size_t oracle_cache_retained(const oracle_layer_cache *c);
/* encode_in_place's K/V step: check_stage's position and byte limits
 * (attention.rs:542-559), then the rows appended after the retained ones and
 * total = next position; fills the PendingKv record (old_len in floats). On
 * an error the cache is unchanged. */
int oracle_cache_append(oracle_layer_cache *c, const float *keys, const float *values, size_t n,
                        size_t *old_len, size_t *old_total);
/* rollback / keep / commit (attention.rs:280-310). */
void oracle_cache_rollback(oracle_layer_cache *c, size_t old_len, size_t old_total);
void oracle_cache_keep(oracle_layer_cache *c, size_t old_len, size_t old_total, size_t tokens);
void oracle_cache_commit(oracle_layer_cache *c);

/* Head transform primitives. p9_ref_rms_norm
 * (src/kernels/portable/reference.rs:11-33): sequential f64 sum of squares,
 * inv = 1 / sqrt(sum / n + eps) in f64, out = f32(x * inv) [* scale in f32]. */
void oracle_rms_norm(const float *x, const float *scale, size_t n, float eps, float *out);
/* p9_ref_rope (reference.rs:277-318): NeoX pairs (i, i + dim/2), f32
 * frequencies 1 / powf(base, 2i/dim) [/ factor_i], f32 angles, glibc 2.28's
 * sincosf (the reference's libm::sincosf, src/libm.rs:350); false on a
 * non-finite angle. */
bool oracle_rope(const float *x, size_t heads, size_t dim, size_t position, float base,
                 const float *factors, float *out);
/* FNV-1a digests of the C library's powf (which = 0), the glibc 2.28
 * sincosf of oracle_rope (which = 1) or the glibc 2.28 POWER8 expf of the
 * binary32 twin (which = 2) over the inputs of the reference's libm digest
 * tests
 * (src/libm/tests.rs:20-62, 87-136); NaNs that an invalid operation
 * generates are counted with the positive default-NaN bits of the
 * reference's platform. */
uint64_t oracle_libm_digest(int which);
/* The rotation's sine and cosine of one angle: glibc 2.28's sincosf as
 * oracle_rope uses it (the reference's libm::sincosf, src/libm.rs:350-497). */
void oracle_sincosf(float x, float *s, float *c);

/* Test input generator, not on the attention path: the reference tests'
 * xorshift64 stream (src/kernels/quantized/int8/tests.rs:15-33). Writes
 * out[i] = (f32(next % 20001) / 10000 - 1) * scale, every operation in
 * binary32 (the multiply skipped when scale == 1), and advances *state. */
void oracle_xorshift_units(uint64_t *state, float scale, size_t n, float *out);

/* Output block primitives. p9_ref_matvec (src/kernels/portable/
 * reference.rs:36-78): out[r] = f32(sequential f64 sum over c ascending of
 * f64(m[r][c]) * f64(x[c])); p9_ref_add: out = a + b in f32. */
void oracle_matvec(const float *matrix, const float *x, size_t rows, size_t cols, float *out);
void oracle_add(const float *a, const float *b, size_t n, float *out);

/* CPU baseline: the exact (a1, variant 0) or binary32 (a3, variant 1) path,
 * or the exact path's checker form (variant 2), threaded as the engine
 * threads it (src/engine/attention.rs:755-836): one query's heads split
 * into ceil(qheads/split) ranges with split = clamp(workers/queries, 1,
 * qheads) when queries < workers, else contiguous query ranges
 * (src/engine/execution.rs:571-599) walked in blocks of 8 queries.
 * Masks come from encoder_mask(first_key, nkeys, first_query+i, window),
 * or none when causal == 0 (decoder mode). Queries [nq][qheads*dim];
 * out [nq][qheads*dim]. Returns false on a kernel error. */
bool oracle_threaded_attention(int variant, int threads, const float *query, size_t nq,
                               const float *keys, const float *values, size_t qheads,
                               size_t kvheads, size_t dim, size_t nkeys, int causal,
                               size_t first_key, size_t first_query, size_t window,
                               float *out);
/* The same over a sample of a prompt's queries: query i of the nq given
 * rows is at position first_query + i * query_step (every query_step-th
 * row of the prompt), so a bounded share of a long prefill is timed with
 * the masks, threading and per-row work of the whole. */
bool oracle_threaded_attention_sample(int variant, int threads, const float *query, size_t nq,
                                      size_t query_step, const float *keys, const float *values,
                                      size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                      int causal, size_t first_key, size_t first_query,
                                      size_t window, float *out);

#ifdef __cplusplus
}
#endif

#endif
