/* Drives the CPU oracle (oracle/vrt_oracle.c) under AddressSanitizer and UndefinedBehavior-
 * Sanitizer: the quantisers and dequantiser on ragged and special-value rows, the matvec
 * orders, the norms, RoPE and attention at small shapes, then a whole-model generation over
 * the GGUF file named on the command line (fp32 and fp16 KV cache) and the error paths of the
 * loader. Prints "ok" and exits 0 when every check holds; a sanitizer report aborts the run.
 * usage: oracle_sanitize MODEL.gguf BAD.gguf */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vrt_oracle.h"

static int fails = 0;
#define CHECK(c)                                                               \
    do {                                                                       \
        if (!(c)) {                                                            \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c);    \
            ++fails;                                                           \
        }                                                                      \
    } while (0)

static uint32_t rng_state = 12345u;
static float frand(void) {   /* xorshift32, uniform in [-1, 1) */
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 17;
    rng_state ^= rng_state << 5;
    return (float)((double)rng_state / 2147483648.0 - 1.0);
}

static void kernels(void) {
    const uint32_t K = 96, rows = 5;
    float* w = malloc(sizeof(float) * K * rows);
    for (uint32_t i = 0; i < K * rows; ++i) w[i] = frand() * 3.0f;
    /* special values in row 1: zero block, tiny, huge and a tie case */
    for (uint32_t i = 0; i < 32; ++i) w[K + i] = 0.0f;
    w[K + 32] = 1e-30f;
    w[K + 33] = 65504.0f;
    w[K + 34] = -65504.0f;
    w[K + 64] = 0.5f;
    const uint64_t nb = (uint64_t)rows * (K / 32);
    uint8_t* qa = malloc(nb * 34);
    uint8_t* qb = malloc(nb * 34);
    or_q8_quantize_a(w, rows, K, qa);
    or_q8_quantize_b(w, rows, K, qb);
    float* dq = malloc(sizeof(float) * K * rows);
    or_q8_dequant(qa, nb, dq);
    for (uint32_t i = 0; i < K * rows; ++i) CHECK(isfinite(dq[i]));
    for (uint32_t i = 0; i < 32; ++i) CHECK(dq[K + i] == 0.0f);

    float x[96], y8[5];
    double yd[5];
    for (uint32_t i = 0; i < K; ++i) x[i] = frand();
    or_q8_matvec_lanes(qa, x, y8, K, rows, 8);
    or_q8_matvec_f64(qa, x, yd, K, rows);
    for (uint32_t r = 0; r < rows; ++r) CHECK(fabs((double)y8[r] - yd[r]) <= 1e-3 * (1.0 + fabs(yd[r])));

    uint32_t idx;
    float val;
    or_argmax(y8, rows, &idx, &val);
    CHECK(idx < rows);

    float g[7] = {-3.0f, -1.0f, -0.5f, 0.0f, 0.5f, 1.0f, 3.0f}, u[7] = {1, 1, 1, 1, 1, 1, 1};
    or_gelu_mul(g, u, 7);
    CHECK(g[3] == 0.0f && g[6] > 2.9f);

    float v[64], nw[64], out[64];
    for (uint32_t i = 0; i < 64; ++i) {
        v[i] = frand();
        nw[i] = 1.0f + 0.1f * frand();
    }
    or_rms_norm_into(v, nw, out, 64, 1e-6f);
    or_rms_norm_inplace(v, nw, 64, 1e-6f);
    for (uint32_t i = 0; i < 64; ++i) CHECK(isfinite(out[i]) && isfinite(v[i]));
    or_rms_norm_heads(v, nw, 2, 32, 1e-6f);

    float inv[16], c[16], s[16];
    or_rope_inv_freq(32, 10000.0f, inv);
    or_rope_table(inv, 16, 7, c, s);
    or_apply_rope(v, 2, 32, c, s);

    /* attention: 2 heads x 32 dims over a history of 5 positions */
    float q[64], keys[5 * 32], vals[5 * 32], att[64];
    for (uint32_t i = 0; i < 64; ++i) q[i] = frand();
    for (uint32_t i = 0; i < 5 * 32; ++i) {
        keys[i] = frand();
        vals[i] = frand();
    }
    CHECK(or_attention(q, keys, vals, 5, 2, 32, 0.17677669f, att) == 0);
    for (uint32_t i = 0; i < 64; ++i) CHECK(isfinite(att[i]));

    uint16_t h = or_f32_to_f16(1.0f);
    CHECK(or_f16_to_f32(h) == 1.0f);
    CHECK(or_f16_to_f32(or_f32_to_f16_rne(-2.5f)) == -2.5f);
    free(w);
    free(qa);
    free(qb);
    free(dq);
}

static void model(const char* path, const char* bad) {
    char err[256];
    or_g3* m = or_g3_open(path, 8, err, sizeof err);
    CHECK(m != NULL);
    if (!m) {
        fprintf(stderr, "open: %s\n", err);
        return;
    }
    or_g3_info info;
    or_g3_get_info(m, &info);
    const uint32_t prompt[4] = {2u, 5u % info.vocab_size, 7u % info.vocab_size, 11u % info.vocab_size};
    uint32_t out[24], n = 0;
    for (int kv16 = 0; kv16 < 2; ++kv16) {
        or_g3_set_kv_f16(m, kv16);
        or_g3_reset(m);
        CHECK(or_g3_generate(m, prompt, 4, 12, out, &n) == 0);
        CHECK(n >= 4 && n <= 16);
        for (uint32_t i = 0; i < n; ++i) CHECK(out[i] < info.vocab_size);
    }
    float* hidden = malloc(sizeof(float) * info.embedding_length);
    float* logits = malloc(sizeof(float) * info.vocab_size);
    uint32_t ai;
    float av;
    or_g3_reset(m);
    CHECK(or_g3_decode(m, prompt[0], 0, 1, hidden, logits, &ai, &av) == 0);
    CHECK(ai < info.vocab_size && logits[ai] == av);
    /* a position that does not follow the cache is an error, not a crash */
    CHECK(or_g3_decode(m, prompt[1], 5, 0, NULL, NULL, NULL, NULL) != 0);
    CHECK(strlen(or_g3_error(m)) > 0);
    free(hidden);
    free(logits);
    or_g3_close(m);

    or_g3* b = or_g3_open(bad, 8, err, sizeof err);
    CHECK(b == NULL && strlen(err) > 0);
    if (b) or_g3_close(b);
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    kernels();
    model(argv[1], argv[2]);
    if (fails) {
        fprintf(stderr, "%d checks failed\n", fails);
        return 1;
    }
    printf("ok\n");
    return 0;
}
