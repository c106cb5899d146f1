/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the fused attention path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline. The
 * product (libtfd_attention.so) never calls into it.
 *
 * A plain-C restatement of the reference's CPU kernels:
 *   - laya_attention_block_with_workspace  crates/cpu-kernels/src/lib.rs:843-1156
 *   - jeff_full_attention_into             crates/cpu-kernels/src/lib.rs:609-763
 *   - build_mask (Laya keep tensor)        crates/laya-infer/src/model.rs:465-490
 *   - GQA K/V expansion                    crates/jeff-infer/src/checkpoint.rs:307-319
 *   - Jeff row trim / RoPE rebase policy   crates/jeff-infer/src/engine.rs:317-329
 *
 * Arithmetic follows the reference's f32 operation order. The scalar paths
 * (Laya's scalar path, all of Jeff) are compiled without FP contraction and
 * so reproduce the reference bit for bit on the same libm. The Laya tile path
 * replaces matrixmultiply 0.3.11 sgemm with a local sgemm whose summation
 * order differs (the reference pins that path only by tolerance: micro.json
 * max_abs_error <= 5.6e-9 and laya-infer tests/model.rs:338-373 <= 3e-5).
 *
 * Parallelism mirrors rayon's decomposition: one task per (batch, head) for
 * Laya (lib.rs:954-961), one per head for Jeff (lib.rs:653), on a persistent
 * pthread pool.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ pool */

typedef void (*task_fn)(void *ctx, size_t index);

typedef struct {
    pthread_mutex_t lock;
    pthread_cond_t start;
    pthread_cond_t done;
    pthread_t *workers;
    int nworkers;          /* helper threads; the caller is one more */
    unsigned generation;
    int active;            /* helpers still inside the current job */
    int quit;
    task_fn fn;
    void *ctx;
    size_t count;
    atomic_size_t next;
} pool_t;

static pool_t g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
                        PTHREAD_COND_INITIALIZER, NULL, 0, 0, 0, 0, NULL, NULL, 0, 0};
static int g_threads = 1;

static void run_tasks(pool_t *p) {
    for (;;) {
        size_t i = atomic_fetch_add(&p->next, 1);
        if (i >= p->count) break;
        p->fn(p->ctx, i);
    }
}

static void *worker_main(void *arg) {
    pool_t *p = (pool_t *)arg;
    unsigned seen = 0;
    pthread_mutex_lock(&p->lock);
    for (;;) {
        while (p->generation == seen && !p->quit) pthread_cond_wait(&p->start, &p->lock);
        if (p->quit) break;
        seen = p->generation;
        pthread_mutex_unlock(&p->lock);
        run_tasks(p);
        pthread_mutex_lock(&p->lock);
        if (--p->active == 0) pthread_cond_signal(&p->done);
    }
    pthread_mutex_unlock(&p->lock);
    return NULL;
}

static void pool_stop(void) {
    pool_t *p = &g_pool;
    if (!p->workers) return;
    pthread_mutex_lock(&p->lock);
    p->quit = 1;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->lock);
    for (int i = 0; i < p->nworkers; ++i) pthread_join(p->workers[i], NULL);
    free(p->workers);
    p->workers = NULL;
    p->nworkers = 0;
    p->quit = 0;
}

/* Number of threads used by every parallel oracle call (>= 1). */
void oracle_set_threads(int threads) {
    if (threads < 1) threads = 1;
    if (threads == g_threads && (threads == 1 || g_pool.workers)) return;
    pool_stop();
    g_threads = threads;
    if (threads > 1) {
        g_pool.workers = (pthread_t *)calloc((size_t)threads - 1, sizeof(pthread_t));
        g_pool.nworkers = threads - 1;
        for (int i = 0; i < threads - 1; ++i)
            pthread_create(&g_pool.workers[i], NULL, worker_main, &g_pool);
    }
}

int oracle_get_threads(void) { return g_threads; }

static void parallel_for(size_t count, task_fn fn, void *ctx) {
    pool_t *p = &g_pool;
    if (count == 0) return;
    if (g_threads <= 1 || count == 1 || !p->workers) {
        for (size_t i = 0; i < count; ++i) fn(ctx, i);
        return;
    }
    pthread_mutex_lock(&p->lock);
    p->fn = fn;
    p->ctx = ctx;
    p->count = count;
    atomic_store(&p->next, 0);
    p->active = p->nworkers;
    p->generation++;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->lock);
    run_tasks(p);
    pthread_mutex_lock(&p->lock);
    while (p->active > 0) pthread_cond_wait(&p->done, &p->lock);
    pthread_mutex_unlock(&p->lock);
}

/* ---------------------------------------------------------------- RoPE */

/* RoPE tables `(length, half)`: lib.rs:874-888. theta is computed in f32 as
 * (l as f32) * base.powf(-2 i / hd). */
void oracle_rope_table(size_t length, size_t hd, float base, float *cos_out, float *sin_out) {
    size_t half = hd / 2;
    for (size_t l = 0; l < length; ++l) {
        for (size_t i = 0; i < half; ++i) {
            float expo = -2.0f * (float)i / (float)hd;
            float theta = (float)l * powf(base, expo);
            cos_out[l * half + i] = cosf(theta);
            sin_out[l * half + i] = sinf(theta);
        }
    }
}

/* ---------------------------------------------------------------- sgemm */

/* The two products of the Laya tile path, in the row-major shapes the
 * reference passes to matrixmultiply::sgemm (lib.rs:1037-1052, 1081-1096).
 * Every output is accumulated over k in order, acc = fma(a, b, acc) from 0,
 * so the blocked kernel below and the plain loop give the same bits.
 *
 * This is an in-order FMA restatement of the two products, not a copy of
 * matrixmultiply 0.3.11's summation order: that crate blocks k by its kc
 * and its source is not vendored with the reference, so the two agree to
 * f32 rounding, not bit for bit (the reference itself pins this path only
 * by tolerance). For speed it is a packed, register-tiled kernel: B is
 * packed into panels of 16 columns (k x 16, contiguous), and a 6 x 16
 * block of C lives in twelve 8-wide registers for the whole k loop (two B
 * loads and six A broadcasts per twelve FMAs). k is never split (at most
 * the span length or the head dim), which keeps the in-order summation
 * above. Edge rows and columns run the same FMA chain one element at a
 * time. */
#if defined(__x86_64__)
#include <immintrin.h>

__attribute__((target("avx2,fma")))
static void gemm_block_6x16(size_t rows, size_t k, const float *a, size_t lda, const float *bp,
                            float *c, size_t ldc) {
    __m256 acc[6][2];
    for (int r = 0; r < 6; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
    if (rows == 6) {
        for (size_t p = 0; p < k; ++p) {
            const __m256 b0 = _mm256_loadu_ps(bp + 16 * p), b1 = _mm256_loadu_ps(bp + 16 * p + 8);
            for (int r = 0; r < 6; ++r) {
                const __m256 av = _mm256_broadcast_ss(a + r * lda + p);
                acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
                acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
            }
        }
    } else {
        for (size_t p = 0; p < k; ++p) {
            const __m256 b0 = _mm256_loadu_ps(bp + 16 * p), b1 = _mm256_loadu_ps(bp + 16 * p + 8);
            for (size_t r = 0; r < rows; ++r) {
                const __m256 av = _mm256_broadcast_ss(a + r * lda + p);
                acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
                acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
            }
        }
    }
    for (size_t r = 0; r < rows; ++r) {
        _mm256_storeu_ps(c + r * ldc, acc[r][0]);
        _mm256_storeu_ps(c + r * ldc + 8, acc[r][1]);
    }
}

__attribute__((target("avx2,fma")))
static void gemm_packed_fma(size_t m, size_t k, size_t n, const float *a, size_t lda,
                            const float *b, size_t ldb, float *c, size_t ldc) {
    const size_t full = n / 16 * 16;
    float *bp = (float *)aligned_alloc(64, sizeof(float) * 16 * (k ? k : 1));
    for (size_t j = 0; j < full; j += 16) {
        for (size_t p = 0; p < k; ++p) memcpy(bp + 16 * p, b + p * ldb + j, sizeof(float) * 16);
        for (size_t i = 0; i < m; i += 6)
            gemm_block_6x16(m - i < 6 ? m - i : 6, k, a + i * lda, lda, bp, c + i * ldc + j, ldc);
    }
    free(bp);
    for (size_t i = 0; i < m; ++i)
        for (size_t j = full; j < n; ++j) {
            float acc = 0.0f;
            for (size_t p = 0; p < k; ++p) acc = fmaf(a[i * lda + p], b[p * ldb + j], acc);
            c[i * ldc + j] = acc;
        }
}
#endif

static void axpy_rows_plain(size_t m, size_t k, size_t n, const float *a, size_t lda,
                            const float *b, size_t ldb, float *c, size_t ldc) {
    for (size_t i = 0; i < m; ++i) {
        float *ci = c + i * ldc;
        for (size_t j = 0; j < n; ++j) ci[j] = 0.0f;
        for (size_t p = 0; p < k; ++p) {
            float av = a[i * lda + p];
            const float *bp = b + p * ldb;
            for (size_t j = 0; j < n; ++j) ci[j] += av * bp[j];
        }
    }
}

static int g_have_fma = -1;

/* C (m x n, row stride ldc) = A (m x k, row stride lda) * B (k x n, row stride ldb) */
static void sgemm_rows(size_t m, size_t k, size_t n, const float *a, size_t lda,
                       const float *b, size_t ldb, float *c, size_t ldc) {
#if defined(__x86_64__)
    if (g_have_fma < 0) {
        __builtin_cpu_init();
        g_have_fma = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    if (g_have_fma) {
        gemm_packed_fma(m, k, n, a, lda, b, ldb, c, ldc);
        return;
    }
#endif
    axpy_rows_plain(m, k, n, a, lda, b, ldb, c, ldc);
}

/* ----------------------------------------------------------------- Laya */

typedef struct {
    const float *qkv;
    const uint8_t *keep;
    float *out;
    size_t d, heads, length, batch, hd, half;
    float scale;
    int use_rope;
    const float *cos, *sin;
    int use_gemm;
    int scalar_only;
    size_t tile, tiles, max_keys;
    const size_t *ranges; /* (first, last, allowed) per (batch, tile) */
    const uint8_t *dense;  /* per batch */
} laya_job_t;

/* One (batch, head) task: lib.rs:964-1153. */
static void laya_task(void *vctx, size_t bh) {
    const laya_job_t *J = (const laya_job_t *)vctx;
    const size_t d = J->d, L = J->length, hd = J->hd, half = J->half;
    const size_t b = bh / J->heads, head = bh % J->heads, feat = head * hd;
    const float *qkv = J->qkv;
    const uint8_t *keep = J->keep;
    float *out = J->out;
    float *q = (float *)malloc(sizeof(float) * L * hd);
    float *k = (float *)malloc(sizeof(float) * L * hd);
    float *v = (float *)malloc(sizeof(float) * L * hd);
    /* split qkv -> q/k/v head band (981-990) */
    for (size_t l = 0; l < L; ++l) {
        size_t src = 3 * d * (l + L * b) + feat, dst = l * hd;
        for (size_t i = 0; i < hd; ++i) {
            q[dst + i] = qkv[src + i];
            k[dst + i] = qkv[src + d + i];
            v[dst + i] = qkv[src + 2 * d + i];
        }
    }
    if (J->use_rope) { /* 991-1010 */
        for (size_t l = 0; l < L; ++l) {
            size_t row = l * hd, table = l * half;
            for (size_t i = 0; i < half; ++i) {
                float c = J->cos[table + i], s = J->sin[table + i];
                float a = q[row + i], bb = q[row + i + half];
                q[row + i] = a * c - bb * s;
                q[row + i + half] = a * s + bb * c;
                a = k[row + i];
                bb = k[row + i + half];
                k[row + i] = a * c - bb * s;
                k[row + i + half] = a * s + bb * c;
            }
        }
    }
    int v_finite = 1;
    for (size_t i = 0; i < L * hd; ++i)
        if (!isfinite(v[i])) { v_finite = 0; break; }

    if (!J->scalar_only && J->use_gemm && J->dense[b] && v_finite) { /* 1015-1107 */
        const size_t tile = J->tile;
        float *probs = (float *)malloc(sizeof(float) * (tile * J->max_keys + 1));
        float *mixed = (float *)malloc(sizeof(float) * tile * hd);
        float *kt = (float *)malloc(sizeof(float) * (hd * J->max_keys + 1));
        for (size_t index = 0, start = 0; start < L; ++index, start += tile) {
            size_t queries = (L - start) < tile ? (L - start) : tile;
            const size_t *r = J->ranges + 3 * (b * J->tiles + index);
            size_t key_start = r[0], keys = r[1] - r[0];
            if (keys == 0) { /* 1025-1033: all-masked tile gives NaN rows */
                for (size_t local = 0; local < queries; ++local) {
                    size_t dst = feat + d * (start + local + L * b);
                    for (size_t i = 0; i < hd; ++i) out[dst + i] = NAN;
                }
                continue;
            }
            /* scores = Q_tile (queries x hd) * K_span^T (hd x keys) (1037-1052) */
            for (size_t p = 0; p < hd; ++p)
                for (size_t j = 0; j < keys; ++j) kt[p * keys + j] = k[(key_start + j) * hd + p];
            sgemm_rows(queries, hd, keys, q + start * hd, hd, kt, keys, probs, keys);
            for (size_t local = 0; local < queries; ++local) { /* 1053-1080 */
                size_t query = start + local;
                float *row = probs + local * keys;
                float max = -INFINITY;
                for (size_t key = 0; key < keys; ++key) {
                    if (keep[query + L * (key_start + key + L * b)])
                        row[key] = row[key] * J->scale;
                    else
                        row[key] = -INFINITY;
                    if (row[key] > max) max = row[key];
                }
                float sum = 0.0f;
                for (size_t key = 0; key < keys; ++key) {
                    row[key] = isfinite(row[key]) ? expf(row[key] - max) : 0.0f;
                    sum += row[key];
                }
                for (size_t key = 0; key < keys; ++key) row[key] /= sum;
            }
            /* mixed = P (queries x keys) * V_span (keys x hd) (1081-1096) */
            sgemm_rows(queries, keys, hd, probs, keys, v + key_start * hd, hd, mixed, hd);
            for (size_t local = 0; local < queries; ++local) {
                size_t dst = feat + d * (start + local + L * b);
                memcpy(out + dst, mixed + local * hd, sizeof(float) * hd);
            }
        }
        free(kt);
        free(mixed);
        free(probs);
    } else { /* scalar path 1108-1153 */
        float *probs = (float *)malloc(sizeof(float) * L);
        for (size_t query = 0; query < L; ++query) {
            size_t qo = query * hd;
            float max = -INFINITY;
            for (size_t key = 0; key < L; ++key) {
                if (!keep[query + L * (key + L * b)]) {
                    probs[key] = -INFINITY;
                    continue;
                }
                size_t ko = key * hd;
                float acc = 0.0f;
                for (size_t i = 0; i < hd; ++i) acc += q[qo + i] * k[ko + i];
                float score = acc * J->scale;
                probs[key] = score;
                if (score > max) max = score;
            }
            float sum = 0.0f;
            for (size_t key = 0; key < L; ++key) {
                probs[key] = isfinite(probs[key]) ? expf(probs[key] - max) : 0.0f;
                sum += probs[key];
            }
            size_t o_base = feat + d * (query + L * b);
            for (size_t i = 0; i < hd; ++i) out[o_base + i] = 0.0f;
            for (size_t key = 0; key < L; ++key) {
                float prob = probs[key] / sum;
                if (prob == 0.0f) continue;
                size_t vo = key * hd;
                for (size_t i = 0; i < hd; ++i) out[o_base + i] += v[vo + i] * prob;
            }
        }
        free(probs);
    }
    free(v);
    free(k);
    free(q);
}

/*
 * laya_attention_block_into (lib.rs:809-840, 843-1156). `keep` holds one byte
 * per (query, key, batch) at query + L*(key + L*batch). `out` must hold d*L*B
 * floats; like the kernel it is left untouched when heads == 0 or d % heads != 0
 * (the extension op zero-fills it first, laya_attention.rs:141).
 * scalar_only = 1 forces the scalar path for every (batch, head), as the
 * reference micro-benchmark's scalar twin does.
 * Returns 0, or -1 on a storage-length mismatch (the reference panics there).
 */
int oracle_laya_attention_block(const float *qkv, size_t qkv_len, const uint8_t *keep,
                                size_t keep_len, size_t d, size_t heads, size_t length,
                                size_t batch, float rope_base, float *out, size_t out_len,
                                int scalar_only) {
    size_t n = d * length * batch;
    if (qkv_len != 3 * n) return -1;          /* "qkv length" */
    if (out_len != n) return -2;              /* "output length" */
    if (keep_len != length * length * batch) return -3; /* "mask length" */
    if (n == 0 || heads == 0 || d % heads != 0) return 0;
    laya_job_t J;
    memset(&J, 0, sizeof J);
    J.qkv = qkv;
    J.keep = keep;
    J.out = out;
    J.d = d;
    J.heads = heads;
    J.length = length;
    J.batch = batch;
    J.hd = d / heads;
    J.half = J.hd / 2;
    J.scale = 1.0f / sqrtf((float)J.hd);
    J.scalar_only = scalar_only;
    J.use_rope = rope_base != 0.0f;
    float *cos_t = NULL, *sin_t = NULL;
    if (J.use_rope) {
        cos_t = (float *)malloc(sizeof(float) * (length * J.half + 1));
        sin_t = (float *)malloc(sizeof(float) * (length * J.half + 1));
        oracle_rope_table(length, J.hd, rope_base, cos_t, sin_t);
        J.cos = cos_t;
        J.sin = sin_t;
    }
    /* per-tile key spans (890-947) */
    J.tile = length < 64 ? length : 64;
    J.tiles = (length + J.tile - 1) / J.tile;
    J.use_gemm = length >= 32;
    size_t *ranges = NULL;
    uint8_t *dense = NULL;
    if (J.use_gemm) {
        ranges = (size_t *)calloc(3 * batch * J.tiles, sizeof(size_t));
        dense = (uint8_t *)calloc(batch, 1);
        for (size_t b = 0; b < batch; ++b) {
            for (size_t t = 0; t < J.tiles; ++t) {
                size_t start = t * J.tile;
                size_t end = start + J.tile < length ? start + J.tile : length;
                size_t first = length, last = 0, allowed = 0;
                for (size_t key = 0; key < length; ++key) {
                    const uint8_t *column = keep + length * (key + length * b);
                    size_t active = 0;
                    for (size_t qq = start; qq < end; ++qq) active += column[qq] != 0;
                    if (active > 0) {
                        if (key < first) first = key;
                        last = key + 1;
                        allowed += active;
                    }
                }
                size_t *r = ranges + 3 * (b * J.tiles + t);
                if (first == length) {
                    r[0] = r[1] = r[2] = 0;
                } else {
                    r[0] = first;
                    r[1] = last;
                    r[2] = allowed;
                }
                if (r[1] - r[0] > J.max_keys) J.max_keys = r[1] - r[0];
            }
            int all = 1;
            for (size_t t = 0; t < J.tiles; ++t) {
                const size_t *r = ranges + 3 * (b * J.tiles + t);
                size_t queries = (length - t * J.tile) < J.tile ? (length - t * J.tile) : J.tile;
                size_t need = (queries * (r[1] - r[0]) + 1) / 2;
                if (r[2] < need) { all = 0; break; }
            }
            dense[b] = (uint8_t)all;
        }
    }
    J.ranges = ranges;
    J.dense = dense;
    parallel_for(batch * heads, laya_task, &J);
    free(dense);
    free(ranges);
    free(sin_t);
    free(cos_t);
    return 0;
}

/* build_mask (laya-infer model.rs:465-490): valid is (L, B) at l + L*b,
 * window < 0 selects FullAttention, otherwise SlidingAttention with
 * |q - k| <= window. keep[q + L*(k + L*b)] = valid_k && (inside || !valid_q). */
void oracle_laya_build_mask(const uint8_t *valid, size_t length, size_t batch,
                            long window, uint8_t *keep) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t q = 0; q < length; ++q)
            for (size_t k = 0; k < length; ++k) {
                int valid_k = valid[k + length * b] != 0;
                int valid_q = valid[q + length * b] != 0;
                size_t diff = q > k ? q - k : k - q;
                int inside = window < 0 ? 1 : ((long)diff <= window || !valid_q);
                keep[q + length * (k + length * b)] = (uint8_t)(valid_k && inside);
            }
}

/* ----------------------------------------------------------------- Jeff */

typedef struct {
    const float *q, *k, *v, *gate, *q_norm, *k_norm, *mask;
    float *out;
    size_t length, heads, hd, rot, half;
    float theta, eps, attn_scale;
} jeff_job_t;

static void jeff_norm(float *data, const float *weight, size_t length, size_t hd, float eps) {
    for (size_t t = 0; t < length; ++t) { /* lib.rs:676-689 */
        size_t row = t * hd;
        float mean_sq = 0.0f;
        for (size_t i = 0; i < hd; ++i) mean_sq += data[row + i] * data[row + i];
        mean_sq /= (float)hd;
        float scale = 1.0f / sqrtf(mean_sq + eps);
        for (size_t i = 0; i < hd; ++i) data[row + i] *= scale * (1.0f + weight[i]);
    }
}

/* One head: lib.rs:653-761. */
static void jeff_task(void *vctx, size_t head) {
    const jeff_job_t *J = (const jeff_job_t *)vctx;
    const size_t L = J->length, hd = J->hd, half = J->half, feat = head * hd;
    float *qh = (float *)malloc(sizeof(float) * L * hd);
    float *kh = (float *)malloc(sizeof(float) * L * hd);
    float *vh = (float *)malloc(sizeof(float) * L * hd);
    for (size_t t = 0; t < L; ++t) { /* 664-675 */
        size_t src = t + L * feat, dst = t * hd;
        for (size_t i = 0; i < hd; ++i) {
            qh[dst + i] = J->q[src + L * i];
            kh[dst + i] = J->k[src + L * i];
            vh[dst + i] = J->v[src + L * i];
        }
    }
    jeff_norm(qh, J->q_norm, L, hd, J->eps);
    jeff_norm(kh, J->k_norm, L, hd, J->eps);
    if (half > 0) { /* 692-709 */
        for (size_t t = 0; t < L; ++t) {
            size_t row = t * hd;
            for (size_t i = 0; i < half; ++i) {
                float expo = -2.0f * (float)i / (float)J->rot;
                float angle = (float)t * powf(J->theta, expo);
                float c = cosf(angle), s = sinf(angle);
                float a = qh[row + i], b = qh[row + i + half];
                qh[row + i] = a * c - b * s;
                qh[row + i + half] = a * s + b * c;
                a = kh[row + i];
                b = kh[row + i + half];
                kh[row + i] = a * c - b * s;
                kh[row + i + half] = a * s + b * c;
            }
        }
    }
    float *probs = (float *)malloc(sizeof(float) * L);
    float *oh = (float *)malloc(sizeof(float) * hd);
    for (size_t query = 0; query < L; ++query) { /* 710-760 */
        size_t qo = query * hd;
        float max = -INFINITY;
        for (size_t key = 0; key < L; ++key) {
            if (key > query || J->mask[key] == 0.0f) {
                probs[key] = -INFINITY;
                continue;
            }
            size_t ko = key * hd;
            float acc = 0.0f;
            for (size_t i = 0; i < hd; ++i) acc += qh[qo + i] * kh[ko + i];
            float score = acc * J->attn_scale;
            probs[key] = score;
            if (score > max) max = score;
        }
        float sum = 0.0f;
        for (size_t key = 0; key < L; ++key) {
            probs[key] = isfinite(probs[key]) ? expf(probs[key] - max) : 0.0f;
            sum += probs[key];
        }
        for (size_t i = 0; i < hd; ++i) oh[i] = 0.0f;
        if (sum > 0.0f) {
            for (size_t key = 0; key < L; ++key) {
                float p = probs[key] / sum;
                if (p == 0.0f) continue;
                size_t vo = key * hd;
                for (size_t i = 0; i < hd; ++i) oh[i] += vh[vo + i] * p;
            }
        }
        for (size_t i = 0; i < hd; ++i) {
            size_t at = query + L * (feat + i);
            float g = J->gate[at];
            float sigmoid = 1.0f / (1.0f + expf(-g));
            J->out[at] = oh[i] * sigmoid;
        }
    }
    free(oh);
    free(probs);
    free(vh);
    free(kh);
    free(qh);
}

/*
 * jeff_full_attention_into (lib.rs:618-763). q, k, v, gate and out are
 * column-major (length, width) with width = heads * head_dim, element
 * t + length*f; q_norm/k_norm hold head_dim weights; mask holds length values,
 * a key is active when mask != 0. Returns 0 (or -1 on a length mismatch,
 * which the reference only debug-asserts).
 */
int oracle_jeff_full_attention(const float *q, const float *k, const float *v,
                               const float *gate, const float *q_norm, const float *k_norm,
                               const float *mask, size_t length, size_t heads,
                               size_t head_dim, size_t rotary_dim, float theta, float eps,
                               float *out) {
    size_t width = heads * head_dim;
    if (length == 0 || width == 0 || head_dim == 0) return 0;
    jeff_job_t J;
    J.q = q;
    J.k = k;
    J.v = v;
    J.gate = gate;
    J.q_norm = q_norm;
    J.k_norm = k_norm;
    J.mask = mask;
    J.out = out;
    J.length = length;
    J.heads = heads;
    J.hd = head_dim;
    J.rot = rotary_dim;
    J.half = rotary_dim / 2;
    J.theta = theta;
    J.eps = eps;
    J.attn_scale = 1.0f / sqrtf((float)head_dim);
    parallel_for(heads, jeff_task, &J);
    return 0;
}

/*
 * GQA expansion (jeff-infer checkpoint.rs:307-319): head h reads kv head
 * min(h / (heads / kv_heads), kv_heads - 1). src is (length, kv_heads*hd),
 * dst is (length, heads*hd), both column-major.
 */
void oracle_expand_kv(const float *src, size_t length, size_t heads, size_t kv_heads,
                      size_t head_dim, float *dst) {
    size_t groups = heads / kv_heads;
    for (size_t h = 0; h < heads; ++h) {
        size_t kvh = h / groups;
        if (kvh > kv_heads - 1) kvh = kv_heads - 1;
        for (size_t dd = 0; dd < head_dim; ++dd)
            memcpy(dst + length * (h * head_dim + dd), src + length * (kvh * head_dim + dd),
                   sizeof(float) * length);
    }
}
