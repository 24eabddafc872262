/*
 * pcl_attention.h — C ABI of the MI355X (gfx950) attention backend for the
 * power-cpu-llm engine.
 *
 * Layouts are the engine's (src/kernels/portable/reference.rs:320-326):
 *   query  [qheads][dim] per query position,
 *   keys   [nkeys][kvheads][dim], values the same (token-major f32 cache),
 *   GQA    query head h reads KV head h / (qheads / kvheads),
 *   scale  exactly one (callers pre-scale the query).
 * Results match the reference's exact f32 attention within 1e-4 max-abs and
 * do not depend on the head range, the query batch, the KV-head range or the
 * kernel chosen: every (query, head) row is computed by the same arithmetic.
 *
 * Three layers, all plain C types:
 *   1. kernel entry points with the engine's function-pointer signatures
 *      (host pointers, bool result, false = error);
 *   2. checked wrappers with the reference wrappers' validation and error
 *      codes;
 *   3. a device-resident entry (device pointers, descriptor masks, two KV
 *      segments, asynchronous on a caller-visible stream).
 */
#ifndef PCL_ATTENTION_H
#define PCL_ATTENTION_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 1. kernel entry points (host pointers) ------------------------------ */

/* One query position, query heads [h_first, h_end).
 * Replaces the AttentionF32 function pointer type
 * (src/kernels/quantized/int8.rs:576-589), i.e. pa_attention_f32_heads
 * (src/kernels/portable/attention.rs:51-64) and pa_attention_f32_power9_heads
 * (src/kernels/quantized/int8.rs:155-168); the exact p9_ref_attention_heads
 * (src/kernels/portable/reference.rs:327-340) has the same arguments.
 * query [qheads*dim], keys/values [nkeys*kvheads*dim], allowed NULL or
 * [nkeys] 0/1, scratch is the caller's host scratch (unused here),
 * out [(h_end-h_first)*dim]. False on bad geometry (dim % 16, kvheads 0,
 * qheads % kvheads, head range, dim > 512), a non-finite allowed score, a
 * non-finite output, or a device failure. */
bool pcl_hip_attention_f32_heads(const float *query, const float *keys, const float *values,
                                 size_t qheads, size_t kvheads, size_t dim, size_t nkeys,
                                 const uint8_t *allowed, float *scratch, float *out,
                                 size_t h_first, size_t h_end);

/* Several query positions over the same K/V, KV heads [kh_first, kh_end).
 * Replaces the AttentionMulti function pointer type
 * (src/kernels/quantized/int8.rs:446-484), i.e.
 * pa_attention_f32_power9_multi_kv. query [nq][q_stride] (qheads*dim used),
 * allowed NULL or [nq][mask_stride], out [nq][o_stride] holding the query
 * heads kh_first*group .. kh_end*group. Every row equals the single-query
 * entry's result bitwise. */
bool pcl_hip_attention_f32_multi_kv(const float *query, size_t nq, size_t q_stride,
                                    const float *keys, const float *values, size_t qheads,
                                    size_t kvheads, size_t dim, size_t nkeys,
                                    const uint8_t *allowed, size_t mask_stride, float *scratch,
                                    float *out, size_t o_stride, size_t kh_first, size_t kh_end);

/* ---- 2. checked wrappers (reference wrapper semantics) ------------------- */

/* Error codes of kernels::reference::Error (src/kernels/reference.rs:6-11). */
enum pcl_status {
    PCL_OK = 0,
    PCL_INVALID_SHAPE = 1,
    PCL_INVALID_PARAMETER = 2,
    PCL_NON_FINITE_VALUE = 3,
};

/* attention_with (src/kernels/quantized/int8.rs:596-663) over this backend:
 * FmaKernels::attention_heads for the HIP backend
 * (src/kernels/quantized/power9_fma.rs:237-255). Lengths are element
 * counts; has_mask / has_heads stand for Option::Some. A mask entry is a
 * bool (0 or 1). out holds (h_end-h_first)*head_dim floats. */
int pcl_attention_heads(const float *query, size_t query_len, const float *keys,
                        size_t keys_len, const float *values, size_t values_len,
                        size_t kv_heads, size_t head_dim, const uint8_t *allowed,
                        size_t mask_len, int has_mask, size_t h_first, size_t h_end,
                        int has_heads, float *out);

/* attention_multi_with (src/kernels/quantized/int8.rs:489-573):
 * FmaKernels::attention_multi_kv (power9_fma.rs:197-232). queries: nq
 * pointers to query_len floats; masks: NULL or nq pointers to mask_len
 * bools; out: nq rows of (kv_end-kv_first)*group*head_dim floats. */
int pcl_attention_multi_kv(const float *const *queries, size_t nq, size_t query_len,
                           const float *keys, size_t keys_len, const float *values,
                           size_t values_len, size_t kv_heads, size_t head_dim,
                           const uint8_t *const *masks, size_t mask_len, size_t kv_first,
                           size_t kv_end, float *out);

/* ---- 3. device-resident entry -------------------------------------------- */

typedef struct pcl_context pcl_context;

/* Kernel choice; every choice gives bitwise-identical results. */
enum pcl_kernel {
    PCL_KERNEL_AUTO = 0,
    PCL_KERNEL_SPLIT_KV = 1,    /* split-KV flash decode + ordered combine */
    PCL_KERNEL_TILED = 2,       /* LDS-tiled prefill, one pass over the keys */
    PCL_KERNEL_TILED_SPLIT = 3, /* LDS-tiled prefill, one key chunk per block */
    PCL_KERNEL_PIPE_KV = 4,     /* pipelined split-KV decode (score/value wave
                                   pairs, head dim <= 256) + ordered combine */
    PCL_KERNEL_TWO_PASS = 5,    /* split-KV decode as a K-streaming pass and a
                                   V-streaming pass + ordered combine */
};

/* Attention of nq query positions over keys [0, n0+n1): keys 0..n0-1 come
 * from segment 0 (k0/v0) and the rest from segment 1 (k1/v1), both
 * [n][kvheads][dim] device arrays. All pointers are device pointers.
 *
 * Mask, per query i and key t (absolute key position first_key+t, query
 * position first_query+i):
 *   mask != NULL : allowed = mask[i*mask_stride + t] != 0;
 *   causal != 0  : allowed = kp <= qp && (window == 0 || qp - kp < window)
 *                  (encoder_mask, src/engine/attention.rs:1170-1182);
 *   otherwise    : every key (decoder/canvas mode, attention.rs:696-698).
 * The query is scaled by q_scale in f32 before the dot products, as the
 * engine's pre-scale (src/engine/nemotron/forward.rs:336-346); 1 = none.
 * Output: query i, head h (kh_first*group <= h < kh_end*group) at
 * out + i*o_stride + (h - kh_first*group)*dim. */
typedef struct pcl_attention_desc {
    const float *q;
    int64_t q_stride;
    int64_t nq;
    const float *k0, *v0;
    int64_t n0;
    const float *k1, *v1;
    int64_t n1;
    int64_t qheads, kvheads, dim;
    int64_t kh_first, kh_end;
    const uint8_t *mask;
    int64_t mask_stride;
    int32_t causal;
    int64_t window;
    int64_t first_key, first_query;
    float q_scale;
    float *out;
    int64_t o_stride;
    int32_t kernel; /* enum pcl_kernel */
} pcl_attention_desc;

/* Create a context on a device that owns a new non-blocking stream. */
int pcl_context_create(int device, pcl_context **out);
/* Create a context that launches on the caller's hipStream_t `stream`
 * (NULL = the device's null stream); the caller keeps ownership. */
int pcl_context_create_on_stream(int device, void *stream, pcl_context **out);
void pcl_context_destroy(pcl_context *ctx);
/* The stream launches go to (a hipStream_t). */
void *pcl_context_stream(pcl_context *ctx);
/* Launch asynchronously. Returns PCL_OK, PCL_INVALID_SHAPE for a descriptor
 * that fails validation, or PCL_NON_FINITE_VALUE for a launch failure. Data
 * errors (non-finite allowed score or output) are recorded in the context's
 * device error flag. Grows the context's workspace when needed (a device
 * allocation); pcl_context_reserve avoids that inside timed regions. */
int pcl_attention_launch(pcl_context *ctx, const pcl_attention_desc *desc);
/* Workspace bytes a descriptor needs with the kernel it would run. */
size_t pcl_attention_workspace_bytes(const pcl_attention_desc *desc);
int pcl_context_reserve(pcl_context *ctx, size_t bytes);
/* Wait for the stream; *device_error receives the error flag (bit 0: a
 * non-finite allowed score, bit 1: a non-finite output) and is cleared. */
int pcl_context_sync(pcl_context *ctx, int *device_error);
/* Kernel the descriptor resolves to under PCL_KERNEL_AUTO. */
int pcl_attention_resolve_kernel(const pcl_attention_desc *desc);

/* Per-kernel timing, the device-side counterpart of the engine's stage
 * timers (stats::Span, src/engine/stats.rs:9-64). While enabled, every launch
 * records HIP events on the context's stream around the kernels that stream
 * K/V (role 0: split-KV, pipelined, two-pass or tiled kernels) and around the
 * ordered combine (role 1). pcl_context_timing waits for the stream, adds the
 * elapsed times of the recorded launches to ms[role] and their number to
 * launches[role], and forgets them. Enabling costs two event records per role
 * per launch; leave it off in production. */
int pcl_context_set_timing(pcl_context *ctx, int enable);
int pcl_context_timing(pcl_context *ctx, double *ms, int64_t *launches);

/* Library identification (for loaders). */
const char *pcl_version(void);

#ifdef __cplusplus
}
#endif

#endif
