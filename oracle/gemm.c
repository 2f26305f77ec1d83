/*
 * CPU oracle: the reference GEMM.  TEST INFRASTRUCTURE ONLY; see oracle.h.
 * Built with -ffp-contract=off (separate multiply and add roundings).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <pthread.h>
#include <stdlib.h>

/* Reference::matmul_nt, crates/raya-kernels/src/gemm.rs:22-37: out = a * b^T
 * with one sequential f32 sum per output element; out is overwritten. */
void oracle_matmul_nt(float *out, const float *a, const float *b, uint64_t m, uint64_t n,
                      uint64_t k) {
    for (uint64_t i = 0; i < m; ++i) {
        const float *arow = a + i * k;
        for (uint64_t j = 0; j < n; ++j) {
            const float *brow = b + j * k;
            float sum = 0.0f;
            for (uint64_t t = 0; t < k; ++t) sum += arow[t] * brow[t];
            out[i * n + j] = sum;
        }
    }
}

typedef struct {
    float *out;
    const float *a, *b;
    uint64_t m, n, k, r0, r1;
} gemm_part;

static void *gemm_worker(void *arg) {
    gemm_part *p = (gemm_part *)arg;
    oracle_matmul_nt(p->out + p->r0 * p->n, p->a + p->r0 * p->k, p->b, p->r1 - p->r0, p->n, p->k);
    return NULL;
}

void oracle_matmul_nt_threaded(float *out, const float *a, const float *b, uint64_t m,
                               uint64_t n, uint64_t k, int threads) {
    uint64_t w = threads < 1 ? 1 : (uint64_t)threads;
    if (w > m) w = m ? m : 1;
    if (w == 1) {
        oracle_matmul_nt(out, a, b, m, n, k);
        return;
    }
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * w);
    gemm_part *parts = (gemm_part *)malloc(sizeof(gemm_part) * w);
    for (uint64_t t = 0; t < w; ++t) {
        parts[t] = (gemm_part){out, a, b, m, n, k, m * t / w, m * (t + 1) / w};
        pthread_create(&tid[t], NULL, gemm_worker, &parts[t]);
    }
    for (uint64_t t = 0; t < w; ++t) pthread_join(tid[t], NULL);
    free(parts);
    free(tid);
}
