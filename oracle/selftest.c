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

int main(void)
{
    grouped_attention();
    cache_window_and_limits();
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    puts("oracle selftest: ok");
    return 0;
}
