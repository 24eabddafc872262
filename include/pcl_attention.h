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
 *      segments, asynchronous on a caller-visible stream);
 *   4. a device-resident layer cache whose rows the entry of 3 reads in
 *      place;
 *   5. the head transform that prepares Q, K and V rows for 3 and 4;
 *   6. the attention output block (projection, post-norm, residual).
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
    /* engine::Error::ResourceLimit: a cache's position or byte limit */
    PCL_RESOURCE_LIMIT = 4,
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
    /* 5 is retired (a two-launch decode that no choice selected) and is
       refused with PCL_INVALID_PARAMETER */
    PCL_KERNEL_SPREAD_KV = 6,   /* split-KV decode with each key chunk spread
                                   over head_dim/32 slices that exchange raw
                                   scores (two-wave slices up to head dim
                                   256, one-wave slices at 512; short
                                   launches); the launch's own merge
                                   workgroups run the ordered combine */
    PCL_KERNEL_FAN_KV = 7,      /* split-KV decode with each (key chunk,
                                   16-row unit, KV head) item fanned over the
                                   eight waves of one workgroup (head dims
                                   above 64, launches of two or more chunks;
                                   otherwise the pipelined kernel runs) +
                                   ordered combine */
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
 * softcap: logit soft-cap, off when 0 (a zero-initialised descriptor). When
 * > 0 every allowed score s becomes softcap * tanh(s / softcap) in f32 before
 * the softmax (the form of p9_ref_softcap, src/kernels/portable/reference.rs:
 * 226-235; the engine itself caps only its final logits, src/engine/text.rs:
 * 963,979, so it leaves this off). An infinite score then becomes
 * +-softcap; a NaN one is still an error. Negative, subnormal or non-finite
 * values, and values above 2^126 (whose f32 reciprocal is subnormal), are
 * PCL_INVALID_PARAMETER.
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
    float softcap;  /* 0 = off */
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
 * that fails validation (including the size limits: at most 2^30 keys, and
 * nq * (qheads / kvheads) * (kh_end - kh_first) at most 2^22; larger calls
 * are split by query range or KV-head range, which leaves every result bit
 * unchanged), PCL_RESOURCE_LIMIT when the workspace cannot be allocated,
 * or PCL_NON_FINITE_VALUE for a launch failure. Data errors (non-finite
 * allowed score or output) are recorded in the context's device error flag.
 * Grows the context's workspace when needed (a device allocation);
 * pcl_context_reserve avoids that inside timed regions and before a graph
 * capture. On a stream that is capturing a graph, AUTO does not take the
 * spread decode (its workgroups accept a published word by the launch's
 * epoch, which every replay would repeat) but the pipelined kernel, with the
 * same bits; an explicit PCL_KERNEL_SPREAD_KV is refused there with
 * PCL_INVALID_PARAMETER. No counterpart in the reference (host calls only). */
int pcl_attention_launch(pcl_context *ctx, const pcl_attention_desc *desc);
/* Workspace bytes a descriptor needs with the kernel it would run (under
 * AUTO, also enough for the kernel a graph capture of it takes). */
size_t pcl_attention_workspace_bytes(const pcl_attention_desc *desc);

/* Bytes of the per-GPU scratch array of pcl_attention_launch_noalloc. */
#define PCL_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* pcl_attention_launch without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The same kernels and results as pcl_attention_launch, bit for
 * bit, but the chunk and span partials live in a file-scope device array of
 * PCL_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends; its
 * address is looked up once per device when the first context on that
 * device is created) instead of the context's workspace. A descriptor whose
 * pcl_attention_workspace_bytes exceeds that size returns
 * PCL_RESOURCE_LIMIT (for example a prefill of more than 4096 keys with
 * more than 64 Mi floats of running totals; the 32K and 128K decodes, the
 * 4K prefills and the 256 x 2304 canvas fit). Calls no hipMalloc, hipFree
 * or other allocating routine and records no timing spans. Every call on
 * one GPU shares that GPU's array, which keeps the last call's contents.
 * The partials need no clearing (each launch writes every partial before
 * its combine reads it); the region of published words at the array's
 * start must hold no word of the current epoch, which the array's zero
 * contents at load give and the library restores (a fill kernel on the
 * call's stream) whenever the device's epoch counter has wrapped since.
 * Calls that overlap on one GPU, on different streams or contexts, race
 * and must be serialised by the caller. PCL_NON_FINITE_VALUE if the scratch
 * address could not be taken for this context's device. */
int pcl_attention_launch_noalloc(pcl_context *ctx, const pcl_attention_desc *desc);
int pcl_context_reserve(pcl_context *ctx, size_t bytes);
/* Wait for the stream; *device_error receives the error flag (bit 0: a
 * non-finite allowed score, bit 1: a non-finite output, bit 2: a non-finite
 * head-transform value, bit 3: a non-finite output-block value, bit 4: a
 * wait between workgroups ran out, pcl_context_set_wait_limit) and is
 * cleared. */
int pcl_context_sync(pcl_context *ctx, int *device_error);
/* Kernel the descriptor resolves to under PCL_KERNEL_AUTO. */
int pcl_attention_resolve_kernel(const pcl_attention_desc *desc);

/* Bound of the spread decode's waits for the scores of the other
 * workgroups of a key chunk, in polls of a few hundred cycles each; 0
 * restores the default (65536, some tens of milliseconds). A wave whose wait
 * runs out forms the missing score blocks itself by the same chain (the
 * same bits), so the launch's result stays valid: a GPU shared with other
 * work, on which some of a launch's workgroups may not run alongside the
 * others, costs time, not correctness. Tests use a tiny limit to exercise
 * that path. The launch's merge workgroups wait only for workgroups
 * dispatched before them, under a fixed guard of about a second; bit 4 (16)
 * of the device error flag reports a guard that ran out (then the output is
 * not valid; the host-pointer entries of section 1 rerun such a launch with
 * the pipelined kernel, which never waits). ctx NULL sets the limit of the
 * context the host-pointer entries use. No counterpart in the reference
 * (its CPU threads do not wait on each other inside an attention call).
 * PCL_INVALID_PARAMETER for a negative limit. */
int pcl_context_set_wait_limit(pcl_context *ctx, int polls);
/* Testing hook, no counterpart in the reference: sets the device's epoch
 * counter (the spread decode's launches each take the next value; its low
 * 32 bits are the epoch its published words carry, its high bits count
 * wraps) so that a test can run launches across a wrap. PCL_INVALID_SHAPE
 * for a device index outside the library's table. */
int pcl_debug_set_epoch_counter(int device, uint64_t value);

/* Per-kernel timing, the device-side counterpart of the engine's stage
 * timers (stats::Span, src/engine/stats.rs:9-64). While enabled, every launch
 * records HIP events on the context's stream around the kernels that stream
 * K/V (role 0: split-KV, pipelined, two-pass, spread or tiled kernels; the
 * spread kernel includes its own merge) and around the
 * ordered combine (role 1). pcl_context_timing waits for the stream, adds the
 * elapsed times of the recorded launches to ms[role] and their number to
 * launches[role], and forgets them. Enabling costs two event records per role
 * per launch; leave it off in production. */
int pcl_context_set_timing(pcl_context *ctx, int enable);
int pcl_context_timing(pcl_context *ctx, double *ms, int64_t *launches);

/* ---- 4. device-resident layer cache ----------------------------------------
 *
 * The engine's LayerCache (src/engine/attention.rs:244-311) with its K/V rows
 * in HBM: token-major [tokens][kvheads][dim] f32, the retained rows
 * contiguous, so attention reads them in place (no staging copy, unlike
 * stage(), attention.rs:562-581). All copies run on the context's stream. */
typedef struct pcl_kv_cache pcl_kv_cache;

/* Undo record of one uncommitted step (PendingKv, attention.rs:263-266);
 * lengths in tokens. */
typedef struct pcl_kv_pending {
    int64_t old_len;
    int64_t old_total;
} pcl_kv_pending;

/* new_cache (attention.rs:484-505): rows of kvheads x dim floats, positions
 * up to `context`, window 0 for a global layer (a sliding layer keeps
 * window - 1 tokens, retained_count, attention.rs:1166-1168), max_bytes
 * bounding the retained plus appended K+V bytes of a step. PCL_RESOURCE_LIMIT
 * when max_bytes is below one token's K+V. */
int pcl_kv_cache_create(pcl_context *ctx, int64_t kvheads, int64_t dim, int64_t context,
                        int64_t window, size_t max_bytes, pcl_kv_cache **out);
/* Destroy caches (and head transforms) before the context they were made on. */
void pcl_kv_cache_destroy(pcl_kv_cache *cache);
/* Room for `rows` rows in the cache's buffers now (at most what max_bytes
 * allows), so that appends up to that many retained plus appended rows do not
 * reallocate (growth frees the old buffers, and on MI355X a process that
 * frees device memory streams more slowly afterwards). Grow-only; call it
 * between steps (moving the rows invalidates a pending record).
 * PCL_RESOURCE_LIMIT if the buffers cannot be allocated. No counterpart in
 * the reference (its caches are host vectors). */
int pcl_kv_cache_reserve_rows(pcl_kv_cache *cache, int64_t rows);
/* LayerCache::total_tokens / retained_tokens (attention.rs:268-273). */
int64_t pcl_kv_cache_total_tokens(const pcl_kv_cache *cache);
int64_t pcl_kv_cache_retained_tokens(const pcl_kv_cache *cache);
/* The retained rows (LayerCache::keys / values, attention.rs:274-279) as device
 * pointers, their count and the absolute position of the first. Valid until
 * the next append, keep, rollback or commit. */
int pcl_kv_cache_view(const pcl_kv_cache *cache, const float **keys, const float **values,
                      int64_t *rows, int64_t *first_position);
/* Copy retained rows [first, first + rows) of K and V into keys / values
 * (host or device memory, [rows][kvheads][dim] each) and wait for the copy:
 * the host-side read of LayerCache::keys / values. */
int pcl_kv_cache_read(const pcl_kv_cache *cache, int64_t first, int64_t rows, float *keys,
                      float *values);
/* One uncommitted step of n tokens (encode_in_place's append,
 * attention.rs:949-1080): checks total + n <= context and the byte limit
 * (check_stage, attention.rs:545-558), copies the rows keys/values
 * ([n][kvheads][dim]; device memory of the cache's device in one launch, host
 * memory by runtime copies) after the retained rows, advances the total and
 * fills *pending. On an error the cache is unchanged. */
int pcl_kv_cache_append(pcl_kv_cache *cache, const float *keys, const float *values, int64_t n,
                        pcl_kv_pending *pending);
/* LayerCache::rollback / keep / commit (attention.rs:280-310): undo the step;
 * keep only its first `tokens` positions; apply window retention (the dead
 * prefix is dropped once it is at least half the rows). */
int pcl_kv_cache_rollback(pcl_kv_cache *cache, const pcl_kv_pending *pending);
int pcl_kv_cache_keep(pcl_kv_cache *cache, const pcl_kv_pending *pending, int64_t tokens);
int pcl_kv_cache_commit(pcl_kv_cache *cache);
/* Key/value fields of an attention descriptor over the cache; the caller sets
 * the query, output and head fields. Encoder pass (after append, before
 * commit): the retained rows including the step, causal with the cache's
 * window, first_key = position of the first retained row, first_query =
 * pending->old_total (encode_in_place's view, attention.rs:978-987). Decoder
 * pass (DiffusionGemma canvas, decode_routed, attention.rs:1156-1163): the
 * retained rows then n canvas rows as a second segment, no mask, first_query =
 * the cache total; the cache is not changed. */
int pcl_kv_cache_encoder_desc(const pcl_kv_cache *cache, const pcl_kv_pending *pending,
                              pcl_attention_desc *desc);
int pcl_kv_cache_decoder_desc(const pcl_kv_cache *cache, const float *canvas_keys,
                              const float *canvas_values, int64_t n, pcl_attention_desc *desc);
/* Shared-K/V layer step (encode_shared_in_place, attention.rs:1086-1145): the
 * layer stores no K/V and attends over its source layer's rows of the same
 * uncommitted step. shared_desc checks cache total == source_pending->old_total
 * and source total == cache total + n, and fills the key/value fields: the
 * source's retained rows, causal with this cache's window, first_key =
 * source_pending->old_total - the rows the source retained before its step,
 * first_query = the cache total. advance records *pending and moves the
 * total to total + n (keep / rollback / commit apply as for any step). */
int pcl_kv_cache_shared_desc(const pcl_kv_cache *cache, const pcl_kv_cache *source,
                             const pcl_kv_pending *source_pending, int64_t n,
                             pcl_attention_desc *desc);
int pcl_kv_cache_advance(pcl_kv_cache *cache, int64_t n, pcl_kv_pending *pending);

/* ---- 5. head transform (the attention prologue) ----------------------------
 *
 * HeadTransform (src/engine/attention.rs:51-243) on the device: per head an
 * RMS norm with a sequential f64 sum of squares (p9_ref_rms_norm,
 * src/kernels/portable/reference.rs:11-33), the learned scale for Q and K,
 * then NeoX rotation of pairs (j, j + dim/2) by f32 angles
 * position * (1 / powf(base, 2j/dim)) / factor_j (p9_ref_rope,
 * reference.rs:277-318); V is normalised without scale and not rotated.
 * Row layouts: raw and prepared Q [n][qheads][dim], K and V [n][kvheads][dim],
 * device pointers; token i is at position `position + i`. Launches are
 * asynchronous on the context's stream; a non-finite input or output sets
 * bit 2 of the context's device error flag (pcl_context_sync). */
typedef struct pcl_head_transform pcl_head_transform;

/* HeadTransform::new (attention.rs:65-101): scales [dim] and factors NULL or
 * [dim/2] are host arrays, copied. sliding != 0: the layer needs a V
 * projection; otherwise raw_v NULL means V = the raw K (global K-as-V,
 * attention.rs:121-129). PCL_INVALID_SHAPE for a head geometry this backend
 * does not run (dim 16, 32, 64, 128, 256 or 512); PCL_INVALID_PARAMETER for a
 * non-finite or non-positive epsilon, base or factor, or a non-finite scale. */
int pcl_head_transform_create(pcl_context *ctx, int64_t qheads, int64_t kvheads, int64_t dim,
                              int sliding, const float *query_scale, const float *key_scale,
                              float epsilon, float base, const float *factors,
                              pcl_head_transform **out);
void pcl_head_transform_destroy(pcl_head_transform *transform);
/* HeadTransform::prepare (attention.rs:102-156) for n tokens. The rotation
 * table is built on the host (the C library's powf; the C library's double
 * sin and cos of each f32 angle, rounded once to f32: within an f32 ulp of
 * the reference's libm::sincosf, src/libm.rs:350, and equal to it for all
 * but about 0.1 % of angles) for positions up to the largest seen so far and
 * kept on the device; PCL_NON_FINITE_VALUE for a non-finite angle,
 * PCL_RESOURCE_LIMIT beyond 2^24 positions. A rotated Q or K value y_j
 * (pair j, j + dim/2) is therefore within 2^-20 * (|y_j| + |y_{j+dim/2}|)
 * of the reference's, and almost always equal to it; V rows are bit for
 * bit. */
int pcl_head_transform_prepare(pcl_head_transform *transform, const float *raw_q,
                               const float *raw_k, const float *raw_v, int64_t n,
                               int64_t position, float *q_out, float *k_out, float *v_out);
/* prepare_query (attention.rs:223-242): the query half, for shared-K/V
 * layers. */
int pcl_head_transform_query(pcl_head_transform *transform, const float *raw_q, int64_t n,
                             int64_t position, float *q_out);
/* encode_in_place's projection tail (project_tokens, attention.rs:584-666)
 * fused with the cache append: prepared K and V go straight into the cache's
 * rows after the retained ones, at positions total .. total+n-1, and the
 * prepared queries into q_out. Limits and *pending as pcl_kv_cache_append. */
int pcl_kv_cache_append_transformed(pcl_kv_cache *cache, pcl_head_transform *transform,
                                    const float *raw_q, const float *raw_k, const float *raw_v,
                                    int64_t n, float *q_out, pcl_kv_pending *pending);

/* One decode token of a layer in one call: pcl_kv_cache_append_transformed
 * for n = 1 (the token's raw rows prepared, K and V written after the
 * retained rows, the prepared queries to q_out [qheads][dim]), then the
 * attention of the prepared queries over the cache's rows with the step's
 * new key (pcl_kv_cache_encoder_desc of the step, every KV head, q_scale as
 * the descriptor's, kernel an enum pcl_kernel) into out [qheads][dim]: the
 * one-position decode of encode_in_place (src/engine/attention.rs:949-1080,
 * prepare 102-156 then the attention pass 755-777). Where the kernel that
 * runs is the pipelined decode at head dim 64, 128, 256 or 512, the
 * transform is folded into its launch: every workgroup prepares its own
 * query rows and the workgroups of the new key's chunk write that key's K
 * and V rows before reading them (one launch fewer, the same bits);
 * otherwise the transform's own launch runs first. Limits, errors and
 * *pending as pcl_kv_cache_append_transformed and pcl_attention_launch; on
 * an error nothing was launched and the cache is unchanged. */
int pcl_kv_cache_attend_token(pcl_kv_cache *cache, pcl_head_transform *transform,
                              const float *raw_q, const float *raw_k, const float *raw_v,
                              float q_scale, int kernel, float *q_out, float *out,
                              pcl_kv_pending *pending);

/* ---- 6. attention output block ---------------------------------------------
 *
 * The step after attention (src/engine/attention.rs:866-884): projected =
 * W . attended with f32 weights [out][in] (Matrix::project / p9_ref_matvec,
 * src/kernels/portable/reference.rs:36-78: f64 sums of exact f32 products),
 * then result = residual + rms_norm(projected, post_scale, epsilon) in the
 * engine's rounding (f64 norm, f32 scale and add). attended [n][in],
 * residual, projected and result [n][out], post_scale [out]: device pointers;
 * result may be the residual buffer. Asynchronous on the context's stream; a
 * non-finite projected or result value sets bit 3 of the device error flag.
 * The sums are f64 in the kernels' own order, so a value equals the engine's
 * unless the two f64 sums fall on opposite sides of an f32 rounding
 * boundary. PCL_INVALID_SHAPE beyond n = 2^22 tokens or in, out = 2^20. */
int pcl_attention_output(pcl_context *ctx, const float *attended, int64_t n, int64_t in,
                         const float *weights, int64_t out, const float *post_scale,
                         float epsilon, const float *residual, float *projected, float *result);

/* Library identification (for loaders). */
const char *pcl_version(void);

#ifdef __cplusplus
}
#endif

#endif
