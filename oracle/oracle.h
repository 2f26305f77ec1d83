/*
 * CPU oracle for the block-local attention hot path and the encoder GEMMs.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only the test suite,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * to check or to time the CPU baseline.  The product (raya_amd, libraya_hip)
 * never links it and never falls back to it.
 *
 * Every function restates the reference's algorithm (joaoajmatos/raya, Rust)
 * and cites the file:line it follows.  How each function is pinned:
 *
 *   oracle_key_range / oracle_allows   Block3/Window64/Full/Sliding: pinned by the
 *       reference's own key_range test values (masks_dense.rs:93-98) and by the
 *       golden block_local_L256 vectors through oracle_naive_attend.
 *       BlockDiag (not in the reference): pinned by brute force over (i, j)
 *       against its definition and by torch SDPA with a boolean mask.
 *   oracle_naive_attend   pinned by the golden block_local_L256 tensors
 *       ("reference" and "kernel", 1e-5), by the dense brute force below at
 *       1e-6, and, for every mask, by torch's scaled_dot_product_attention in
 *       float64 with an explicit boolean mask (an independent library routine).
 *   oracle_dense_attend   restates crates/raya-kernels/tests/common/mod.rs:39-84;
 *       pinned by the same torch SDPA check.
 *   oracle_tiled_attend   pinned against oracle_naive_attend (1e-5) and the
 *       golden tensors; bit-identical across thread counts.
 *   oracle_matmul_nt      pinned by the hand values of gemm_reference.rs:5-12,
 *       the NaN/Inf cases of gemm_edges.rs:26-51 and by numpy float64 matmul
 *       within the reordered-accumulation bound 2*k*2^-24*sum|a*b|.
 *   oracle_rand_vec / oracle_lcg_fill   test-input generators; pinned by their
 *       first outputs recomputed from the recurrence with Python integers.
 */
#ifndef RAYA_ORACLE_H
#define RAYA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORACLE_MASK_BLOCK3 = 0,
    ORACLE_MASK_WINDOW64 = 1,
    ORACLE_MASK_FULL = 2,
    ORACLE_MASK_SLIDING = 3,
    ORACLE_MASK_BLOCKDIAG = 4,
};

/* Allowed keys of query row i, clipped to valid_len: [*lo, *hi). */
void oracle_key_range(int kind, uint64_t block, uint64_t window, uint64_t i,
                      uint64_t valid_len, uint64_t *lo, uint64_t *hi);
/* Whether query i may attend key j, ignoring valid_len. */
int oracle_allows(int kind, uint64_t block, uint64_t window, uint64_t i, uint64_t j);

/* Naive scalar attention of one sequence, [heads][seq][head_dim]. */
void oracle_naive_attend(uint64_t heads, uint64_t seq, uint64_t head_dim, int kind,
                         uint64_t block, uint64_t window, uint64_t valid_len, float scale,
                         const float *q, const float *k, const float *v, float *out);

/* Dense brute force: full score matrix with -inf for masked keys. */
void oracle_dense_attend(uint64_t heads, uint64_t seq, uint64_t head_dim, int kind,
                         uint64_t block, uint64_t window, uint64_t valid_len, float scale,
                         const float *q, const float *k, const float *v, float *out);

/* Batched naive: batch sequences of [heads][seq][head_dim], valid_len[batch]. */
void oracle_naive_attend_batched(uint64_t batch, uint64_t heads, uint64_t seq,
                                 uint64_t head_dim, int kind, uint64_t block, uint64_t window,
                                 const int32_t *valid_len, float scale, const float *q,
                                 const float *k, const float *v, float *out);

/* Tiled (online softmax, 8-row micro tiles, 64-key tiles, threads over
 * (sequence, head, 128-row block)).  backend: 0 portable, 1 avx2+fma (falls
 * back to portable when the CPU lacks it).  Returns the backend used. */
int oracle_tiled_attend_batched(uint64_t batch, uint64_t heads, uint64_t seq,
                                uint64_t head_dim, int kind, uint64_t block, uint64_t window,
                                const int32_t *valid_len, float scale, const float *q,
                                const float *k, const float *v, float *out, int threads,
                                int backend);
int oracle_cpu_has_avx2_fma(void);

/* out[m][n] = sum_t a[m][t] * b[n][t], sequential f32 accumulation. */
void oracle_matmul_nt(float *out, const float *a, const float *b, uint64_t m, uint64_t n,
                      uint64_t k);
/* Same contraction, threaded over rows (identical results, used to time). */
void oracle_matmul_nt_threaded(float *out, const float *a, const float *b, uint64_t m,
                               uint64_t n, uint64_t k, int threads);

/* Scalar ops of the reference forward (crates/raya-core/src/ops.rs). */
double oracle_erf(double x);
float oracle_gelu(float x);
void oracle_gelu_vec(float *out, const float *x, uint64_t n);
void oracle_layer_norm(float *out, const float *x, const float *weight, const float *bias,
                       float eps, uint64_t rows, uint64_t d);
void oracle_softmax(float *x, uint64_t n);
void oracle_rope(float *x, uint64_t heads, uint64_t seq, uint64_t head_dim, float theta);

/* Input generators of the reference's tests. */
void oracle_rand_vec(uint64_t n, uint64_t seed, float *out);
void oracle_lcg_fill(uint64_t n, uint32_t seed, float *out);

#ifdef __cplusplus
}
#endif

#endif
