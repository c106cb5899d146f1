/*
 * TEST INFRASTRUCTURE ONLY: a driver that runs the C oracle's entry points
 * on small inputs that walk every path (Laya tile/GEMM and scalar paths,
 * windows, empty rows, NaN/inf values, short storage; Jeff GQA expansion,
 * partial RoPE, masked and empty rows) so that an AddressSanitizer +
 * UndefinedBehaviorSanitizer build of tfd_oracle.c (`make -C oracle
 * sanitize`) can check them for out-of-bounds accesses, leaks and undefined
 * behaviour. Exit status 0 when every call returned as expected; the
 * sanitizers abort the process on the first finding.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void oracle_set_threads(int threads);
void oracle_rope_table(size_t length, size_t hd, float base, float *cos_out, float *sin_out);
int oracle_laya_attention_block(const float *qkv, size_t qkv_len, const uint8_t *keep,
                                size_t keep_len, size_t d, size_t heads, size_t length,
                                size_t batch, float rope_base, float *out, size_t out_len,
                                int scalar_only);
void oracle_laya_build_mask(const uint8_t *valid, size_t length, size_t batch, long window,
                            uint8_t *keep);
int oracle_jeff_full_attention(const float *q, const float *k, const float *v,
                               const float *gate, const float *q_norm, const float *k_norm,
                               const float *mask, size_t length, size_t heads,
                               size_t head_dim, size_t rotary_dim, float theta, float eps,
                               float *out);
void oracle_expand_kv(const float *src, size_t length, size_t heads, size_t kv_heads,
                      size_t head_dim, float *dst);

static uint64_t g_state = 12345;
static float uniform(void) {
    g_state = g_state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)((g_state >> 40) & 0xffffff) / 16777216.0f;
}
static float *randn(size_t n) {
    float *x = malloc(sizeof(float) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) x[i] = 2.0f * uniform() - 1.0f;
    return x;
}

static int laya_case(size_t d, size_t heads, size_t L, size_t B, long window, float base,
                     int scalar_only, int poison) {
    size_t n = d * L * B;
    float *qkv = randn(3 * n);
    uint8_t *valid = malloc(L * B), *keep = malloc(L * L * B);
    for (size_t b = 0; b < B; ++b)
        for (size_t l = 0; l < L; ++l) valid[l + L * b] = l < L - b * (L / 3);
    oracle_laya_build_mask(valid, L, B, window, keep);
    if (poison && L > 2) {
        qkv[2 * d + 0] = NAN;                 /* a value of key 0 */
        qkv[2 * d + 3 * d * 1 + 1] = INFINITY; /* a value of key 1 */
    }
    float *out = malloc(sizeof(float) * (n ? n : 1));
    int rc = oracle_laya_attention_block(qkv, 3 * n, keep, L * L * B, d, heads, L, B, base, out,
                                         n, scalar_only);
    int bad = rc != 0;
    /* short storage is rejected before any access */
    if (n && oracle_laya_attention_block(qkv, 3 * n - 1, keep, L * L * B, d, heads, L, B, base,
                                         out, n, scalar_only) != -1)
        bad = 1;
    free(qkv);
    free(valid);
    free(keep);
    free(out);
    return bad;
}

static int jeff_case(size_t L, size_t heads, size_t kv, size_t hd, size_t rot, int empty_row) {
    size_t W = heads * hd, KW = kv * hd;
    float *q = randn(L * W), *gate = randn(L * W), *kk = randn(L * KW), *vv = randn(L * KW);
    float *k = malloc(sizeof(float) * L * W), *v = malloc(sizeof(float) * L * W);
    oracle_expand_kv(kk, L, heads, kv, hd, k);
    oracle_expand_kv(vv, L, heads, kv, hd, v);
    float *qn = randn(hd), *kn = randn(hd), *mask = malloc(sizeof(float) * L);
    for (size_t t = 0; t < L; ++t) mask[t] = empty_row ? 0.0f : (t >= L / 4 && t != L / 2);
    float *out = malloc(sizeof(float) * L * W);
    int rc = oracle_jeff_full_attention(q, k, v, gate, qn, kn, mask, L, heads, hd, rot, 1e7f,
                                        1e-6f, out);
    free(q); free(gate); free(kk); free(vv); free(k); free(v); free(qn); free(kn); free(mask);
    free(out);
    return rc != 0;
}

int main(void) {
    int bad = 0;
    for (int threads = 1; threads <= 3; threads += 2) {
        oracle_set_threads(threads);
        float c[64 * 8], s[64 * 8];
        oracle_rope_table(64, 16, 160000.0f, c, s);
        bad |= laya_case(64, 4, 32, 1, -1, 160000.0f, 0, 0);   /* C1 shape, tile path */
        bad |= laya_case(64, 4, 32, 1, -1, 160000.0f, 1, 0);   /* scalar path */
        bad |= laya_case(48, 3, 70, 2, 5, 10000.0f, 0, 0);     /* window, ragged tiles */
        bad |= laya_case(48, 3, 70, 2, -1, 0.0f, 0, 1);        /* RoPE off, NaN/inf values */
        bad |= laya_case(32, 2, 1, 3, -1, 10000.0f, 0, 0);     /* L = 1 */
        bad |= laya_case(30, 4, 9, 1, -1, 10000.0f, 0, 0);     /* heads do not divide d */
        bad |= laya_case(0, 1, 0, 0, -1, 0.0f, 0, 0);          /* empty */
        bad |= jeff_case(40, 8, 2, 16, 8, 0);                   /* GQA, partial RoPE */
        bad |= jeff_case(33, 4, 4, 32, 32, 0);                  /* full RoPE */
        bad |= jeff_case(17, 2, 1, 8, 0, 1);                    /* RoPE off, empty row */
    }
    oracle_set_threads(1);
    printf(bad ? "oracle sanitize driver: FAILED\n" : "oracle sanitize driver: ok\n");
    return bad;
}
