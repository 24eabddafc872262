/*
 * Host self-check of the oracle under the address and undefined-behaviour
 * sanitizers (make -C oracle sanitize). TEST INFRASTRUCTURE ONLY.
 *
 * Known answers from the reference's own tests: the grouped-attention case
 * of src/kernels/reference/tests.rs:115-135 and the layer-cache window and
 * byte-limit cases of src/engine/attention/tests.rs:5-47.
 */
#include "attention_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int failures;

#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                          \
        }                                                                        \
    } while (0)

static void grouped_attention(void)
{
    const float query[8] = {1, 0, 2, 0, 0, 1, 0, 2};
    const float keys[8] = {1, 0, 0, 1, -1, 0, 0, -1};
    const float values[8] = {10, 11, 20, 21, 30, 31, 40, 41};
    float out[8];
    CHECK(oracle_attention_heads_checked(query, 8, keys, 8, values, 8, 2, 2, NULL, 0, 0, 0, 0, 0,
                                         out) == ORACLE_OK);
    for (int h = 0; h < 4; ++h) {
        const double s = h % 2 == 0 ? 1.0 : 2.0;
        const double p = exp(s) / (exp(s) + exp(-s));
        const int kh = h / 2;
        for (int d = 0; d < 2; ++d) {
            const double want = p * values[kh * 2 + d] + (1 - p) * values[4 + kh * 2 + d];
            CHECK(fabs(out[h * 2 + d] - want) < 3e-6);
        }
    }
}

static void cache_window_and_limits(void)
{
    float rows[5 * 8];
    for (int i = 0; i < 5 * 8; ++i)
        rows[i] = (float)i;
    size_t old_len, old_total;
    oracle_layer_cache c;
    /* window 3 keeps the last 2 of 5 tokens, whole or in chunks 1+2+2 */
    CHECK(oracle_cache_init(&c, 2, 4, 64, 3, 1, 1 << 20) == ORACLE_OK);
    CHECK(oracle_cache_append(&c, rows, rows, 5, &old_len, &old_total) == ORACLE_OK);
    oracle_cache_commit(&c);
    CHECK(c.total == 5 && oracle_cache_retained(&c) == 2);
    CHECK(c.keys[c.start] == 24.0f && c.values[c.len - 1] == 39.0f);
    oracle_cache_free(&c);
    CHECK(oracle_cache_init(&c, 2, 4, 64, 3, 1, 1 << 20) == ORACLE_OK);
    const size_t chunks[3] = {1, 2, 2};
    size_t at = 0;
    for (int i = 0; i < 3; ++i) {
        CHECK(oracle_cache_append(&c, rows + at * 8, rows + at * 8, chunks[i], &old_len,
                                  &old_total) == ORACLE_OK);
        oracle_cache_commit(&c);
        at += chunks[i];
    }
    CHECK(c.total == 5 && oracle_cache_retained(&c) == 2);
    CHECK(c.keys[c.start] == 24.0f && c.values[c.len - 1] == 39.0f);
    oracle_cache_free(&c);
    /* one token of width 2 in 16 bytes: two tokens are a resource limit */
    CHECK(oracle_cache_init(&c, 1, 2, 64, 3, 1, 16) == ORACLE_OK);
    CHECK(oracle_cache_append(&c, rows, rows, 2, &old_len, &old_total) == ORACLE_RESOURCE_LIMIT);
    CHECK(c.total == 0 && oracle_cache_retained(&c) == 0);
    CHECK(oracle_cache_append(&c, rows, rows, 1, &old_len, &old_total) == ORACLE_OK);
    oracle_cache_rollback(&c, old_len, old_total);
    CHECK(c.total == 0 && oracle_cache_retained(&c) == 0);
    oracle_cache_free(&c);
    CHECK(oracle_cache_init(&c, 1, 2, 64, 3, 1, 15) == ORACLE_RESOURCE_LIMIT);
}

/* The checker form and the sampled threaded path under the sanitizers:
 * both must give the straightforward form's bits. */
static void checker_and_sample(void)
{
    enum { QH = 4, KVH = 2, DIM = 48, N = 37, STEP = 5 };
    static float q[N * QH * DIM], k[N * KVH * DIM], v[N * KVH * DIM];
    static float full[N * QH * DIM], part[N * QH * DIM], a[QH * DIM], b[QH * DIM];
    static float scratch[N];
    static uint8_t mask[N];
    uint64_t r = 0x9e3779b97f4a7c15ULL;
    float *all[3] = {q, k, v};
    const size_t len[3] = {N * QH * DIM, N * KVH * DIM, N * KVH * DIM};
    for (int x = 0; x < 3; ++x)
        for (size_t i = 0; i < len[x]; ++i) {
            r = r * 6364136223846793005ULL + 1442695040888963407ULL;
            all[x][i] = (float)((double)(r >> 40) / (double)(1 << 24) - 0.5);
        }
    for (int t = 0; t < N; ++t)
        mask[t] = (uint8_t)(t % 3 != 1);
    for (int h0 = 0; h0 < QH; ++h0) {
        CHECK(oracle_ref_attention_heads(q, k, v, QH, KVH, DIM, N, mask, scratch, a, h0, QH));
        CHECK(oracle_ref_attention_heads_checker(q, k, v, QH, KVH, DIM, N, mask, scratch, b, h0,
                                                 QH));
        CHECK(memcmp(a, b, (size_t)(QH - h0) * DIM * sizeof(float)) == 0);
    }
    CHECK(oracle_threaded_attention(0, 3, q, N, k, v, QH, KVH, DIM, N, 1, 0, 0, 11, full));
    float rows[((N + STEP - 1) / STEP) * QH * DIM];
    size_t nr = 0;
    for (int i = 0; i < N; i += STEP, ++nr)
        memcpy(rows + nr * QH * DIM, q + (size_t)i * QH * DIM, QH * DIM * sizeof(float));
    for (int variant = 0; variant < 3; variant += 2) {
        CHECK(oracle_threaded_attention_sample(variant, 2, rows, nr, STEP, k, v, QH, KVH, DIM, N,
                                               1, 0, 0, 11, part));
        for (size_t i = 0; i < nr; ++i)
            CHECK(memcmp(part + i * QH * DIM, full + i * STEP * QH * DIM,
                         QH * DIM * sizeof(float)) == 0);
    }
}

int main(void)
{
    grouped_attention();
    cache_window_and_limits();
    checker_and_sample();
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    puts("oracle selftest: ok");
    return 0;
}
