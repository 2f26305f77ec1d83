/*
 * CPU oracle: masks, naive attention, dense brute force and the tiled
 * (online-softmax) CPU baseline.  TEST INFRASTRUCTURE ONLY; see oracle.h.
 *
 * Built with -ffp-contract=off so that `s += a * b` rounds the product and the
 * sum separately, as the reference's Rust loops do (Rust never contracts to FMA).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* crates/raya-kernels/src/attention.rs:4 and :6 */
#define REF_BLOCK 128u
#define REF_WINDOW 64u
/* crates/raya-kernels/src/tiled/tile.rs:7 and simd/mod.rs:13 */
#define MR 8
#define NC 64

static uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }
static uint64_t sat_add(uint64_t a, uint64_t b) { return a + b < a ? UINT64_MAX : a + b; }
static uint64_t umin(uint64_t a, uint64_t b) { return a < b ? a : b; }
static uint64_t umax(uint64_t a, uint64_t b) { return a > b ? a : b; }
static uint64_t absdiff(uint64_t a, uint64_t b) { return a > b ? a - b : b - a; }

/* Mask::key_range, crates/raya-kernels/src/attention.rs:48-59.  BlockDiag(b)
 * (query block i/b sees only its own key block) is this build's extension. */
void oracle_key_range(int kind, uint64_t block, uint64_t window, uint64_t i,
                      uint64_t valid_len, uint64_t *lo, uint64_t *hi) {
    uint64_t a = 0, z = 0;
    switch (kind) {
    case ORACLE_MASK_BLOCK3: {
        uint64_t b = i / REF_BLOCK;
        a = sat_sub(b, 1) * REF_BLOCK;
        z = (b + 2) * REF_BLOCK;
        break;
    }
    case ORACLE_MASK_WINDOW64:
        a = sat_sub(i, REF_WINDOW);
        z = i + REF_WINDOW + 1;
        break;
    case ORACLE_MASK_FULL:
        a = 0;
        z = valid_len;
        break;
    case ORACLE_MASK_SLIDING:
        a = sat_sub(i, window);
        z = sat_add(sat_add(i, window), 1);
        break;
    case ORACLE_MASK_BLOCKDIAG: {
        uint64_t b = i / block;
        a = b * block;
        z = (b + 1) * block;
        break;
    }
    default:
        break;
    }
    *lo = umin(a, valid_len);
    *hi = umin(z, valid_len);
}

/* Mask::allows, crates/raya-kernels/src/attention.rs:62-69 (+ BlockDiag). */
int oracle_allows(int kind, uint64_t block, uint64_t window, uint64_t i, uint64_t j) {
    switch (kind) {
    case ORACLE_MASK_BLOCK3: return absdiff(i / REF_BLOCK, j / REF_BLOCK) <= 1;
    case ORACLE_MASK_WINDOW64: return absdiff(i, j) <= REF_WINDOW;
    case ORACLE_MASK_FULL: return 1;
    case ORACLE_MASK_SLIDING: return absdiff(i, j) <= window;
    case ORACLE_MASK_BLOCKDIAG: return i / block == j / block;
    default: return 0;
    }
}

/* Naive::attend, crates/raya-kernels/src/naive.rs:13-65: per row, sequential f32
 * dot products over key_range, scale, max, exp(s - max) with libm expf, sum,
 * then out += (p / sum) * v.  Rows >= valid_len and empty ranges stay zero. */
void oracle_naive_attend(uint64_t heads, uint64_t seq, uint64_t d, int kind,
                         uint64_t block, uint64_t window, uint64_t valid_len, float scale,
                         const float *q, const float *k, const float *v, float *out) {
    float *scores = (float *)malloc(sizeof(float) * (seq ? seq : 1));
    for (uint64_t h = 0; h < heads; ++h) {
        const uint64_t base = h * seq * d;
        for (uint64_t i = 0; i < seq; ++i) {
            float *orow = out + base + i * d;
            for (uint64_t c = 0; c < d; ++c) orow[c] = 0.0f;
            if (i >= valid_len) continue;
            uint64_t lo, hi;
            oracle_key_range(kind, block, window, i, valid_len, &lo, &hi);
            if (lo >= hi) continue;
            const float *qrow = q + base + i * d;
            float mx = -INFINITY;
            for (uint64_t j = lo; j < hi; ++j) {
                const float *krow = k + base + j * d;
                float s = 0.0f;
                for (uint64_t c = 0; c < d; ++c) s += qrow[c] * krow[c];
                s = s * scale;
                mx = fmaxf(mx, s);
                scores[j - lo] = s;
            }
            float sum = 0.0f;
            for (uint64_t j = lo; j < hi; ++j) {
                scores[j - lo] = expf(scores[j - lo] - mx);
                sum += scores[j - lo];
            }
            for (uint64_t j = lo; j < hi; ++j) {
                const float *vrow = v + base + j * d;
                const float w = scores[j - lo] / sum;
                for (uint64_t c = 0; c < d; ++c) orow[c] += w * vrow[c];
            }
        }
    }
    free(scores);
}

void oracle_naive_attend_batched(uint64_t batch, uint64_t heads, uint64_t seq, uint64_t d,
                                 int kind, uint64_t block, uint64_t window,
                                 const int32_t *valid_len, float scale, const float *q,
                                 const float *k, const float *v, float *out) {
    const uint64_t per = heads * seq * d;
    for (uint64_t b = 0; b < batch; ++b)
        oracle_naive_attend(heads, seq, d, kind, block, window, (uint64_t)valid_len[b], scale,
                            q + b * per, k + b * per, v + b * per, out + b * per);
}

/* dense_reference, crates/raya-kernels/tests/common/mod.rs:39-84: the full
 * [seq][seq] score row with -inf where (i, j) is not allowed (boolean mask from
 * Mask::allows, not key_range), softmax over the whole row, zero rows when
 * nothing is allowed. */
void oracle_dense_attend(uint64_t heads, uint64_t seq, uint64_t d, int kind,
                         uint64_t block, uint64_t window, uint64_t valid_len, float scale,
                         const float *q, const float *k, const float *v, float *out) {
    float *scores = (float *)malloc(sizeof(float) * (seq ? seq : 1));
    memset(out, 0, sizeof(float) * heads * seq * d);
    for (uint64_t h = 0; h < heads; ++h) {
        const uint64_t base = h * seq * d;
        for (uint64_t i = 0; i < seq; ++i) {
            float mx = -INFINITY;
            for (uint64_t j = 0; j < seq; ++j) {
                scores[j] = -INFINITY;
                if (j < valid_len && i < valid_len && oracle_allows(kind, block, window, i, j)) {
                    float dot = 0.0f;
                    for (uint64_t c = 0; c < d; ++c) dot += q[base + i * d + c] * k[base + j * d + c];
                    scores[j] = dot * scale;
                }
                mx = fmaxf(mx, scores[j]);
            }
            if (mx == -INFINITY) continue;
            float sum = 0.0f;
            for (uint64_t j = 0; j < seq; ++j) {
                scores[j] = expf(scores[j] - mx);
                sum += scores[j];
            }
            for (uint64_t j = 0; j < seq; ++j) {
                const float w = scores[j] / sum;
                for (uint64_t c = 0; c < d; ++c) out[base + i * d + c] += w * v[base + j * d + c];
            }
        }
    }
    free(scores);
}

/* ---------------------------------------------------------------------------
 * Tiled CPU baseline: crates/raya-kernels/src/tiled/{mod.rs,tile.rs} and the
 * micro-kernels of simd/{portable.rs,avx2.rs}.
 * ------------------------------------------------------------------------- */

int oracle_cpu_has_avx2_fma(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* simd/portable.rs:55-74 (dot_tile) in plain C: out[r*NC + j] = q_r . k_j. */
static void dot_tile_portable(const float *q, const float *k, uint64_t d, int mr, int nk,
                              float *out) {
    for (int r = 0; r < mr; ++r) {
        const float *qr = q + (uint64_t)r * d;
        for (int j = 0; j < nk; ++j) {
            const float *kj = k + (uint64_t)j * d;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (uint64_t c = 0; c < d; c += 8)
                for (int t = 0; t < 8; ++t) acc[t] += qr[c + t] * kj[c + t];
            out[r * NC + j] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                              ((acc[4] + acc[5]) + (acc[6] + acc[7]));
        }
    }
}

/* simd/portable.rs:76-109 (axpy_rows): acc[0..d] += sum_j p[j] * v_j. */
static void axpy_rows_portable(float *acc, const float *p, int n, const float *v, uint64_t d) {
    for (int j = 0; j < n; ++j) {
        const float pj = p[j];
        const float *vj = v + (uint64_t)j * d;
        for (uint64_t c = 0; c < d; ++c) acc[c] += pj * vj[c];
    }
}

/* simd/portable.rs:112-127 (exp_shifted_sum), scalar libm exp. */
static float exp_shifted_sum_portable(float *x, int n, float shift) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        x[i] = expf(x[i] - shift);
        sum += x[i];
    }
    return sum;
}

__attribute__((target("avx2,fma"))) static inline float hsum256(__m256 x) {
    __m128 lo = _mm256_castps256_ps128(x);
    __m128 hi = _mm256_extractf128_ps(x, 1);
    __m128 s = _mm_add_ps(lo, hi);
    __m128 sh = _mm_movehdup_ps(s);
    __m128 s2 = _mm_add_ps(s, sh);
    __m128 hi2 = _mm_movehl_ps(sh, s2);
    return _mm_cvtss_f32(_mm_add_ss(s2, hi2));
}

/* simd/avx2.rs:22-47 (dot_tile): two 8-lane FMA accumulators per score. */
__attribute__((target("avx2,fma"))) static void dot_tile_avx2(const float *q, const float *k,
                                                              uint64_t d, int mr, int nk,
                                                              float *out) {
    for (int j = 0; j < nk; ++j) {
        const float *kj = k + (uint64_t)j * d;
        for (int r = 0; r < mr; ++r) {
            const float *qr = q + (uint64_t)r * d;
            __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
            uint64_t c = 0;
            for (; c + 16 <= d; c += 16) {
                a0 = _mm256_fmadd_ps(_mm256_loadu_ps(qr + c), _mm256_loadu_ps(kj + c), a0);
                a1 = _mm256_fmadd_ps(_mm256_loadu_ps(qr + c + 8), _mm256_loadu_ps(kj + c + 8), a1);
            }
            if (c < d) a0 = _mm256_fmadd_ps(_mm256_loadu_ps(qr + c), _mm256_loadu_ps(kj + c), a0);
            out[r * NC + j] = hsum256(_mm256_add_ps(a0, a1));
        }
    }
}

/* simd/avx2.rs:51-74 (axpy_rows): 64 output lanes held in eight registers. */
__attribute__((target("avx2,fma"))) static void axpy_rows_avx2(float *acc, const float *p, int n,
                                                               const float *v, uint64_t d) {
    for (uint64_t c0 = 0; c0 < d; c0 += 64) {
        const uint64_t w = d - c0 < 64 ? d - c0 : 64;
        const int nv = (int)(w / 8);
        __m256 r[8];
        for (int t = 0; t < nv; ++t) r[t] = _mm256_loadu_ps(acc + c0 + 8 * t);
        for (int j = 0; j < n; ++j) {
            const float *vj = v + (uint64_t)j * d + c0;
            const __m256 ps = _mm256_set1_ps(p[j]);
            for (int t = 0; t < nv; ++t) r[t] = _mm256_fmadd_ps(ps, _mm256_loadu_ps(vj + 8 * t), r[t]);
        }
        for (int t = 0; t < nv; ++t) _mm256_storeu_ps(acc + c0 + 8 * t, r[t]);
    }
}

/* 8-lane exp for the AVX2 path (this build's own; the reference uses the
 * `wide` crate's f32x8::exp, which is not vendored).  Cody-Waite reduction
 * x = n ln2 + r, |r| <= ln2/2, degree-7 Taylor polynomial (remainder < 6e-9
 * relative), scaled by 2^n built in the exponent field; x below ln(FLT_MIN)
 * (including -inf) gives 0. */
__attribute__((target("avx2,fma"))) static inline __m256 exp256(__m256 x) {
    const __m256 lo = _mm256_set1_ps(-87.33654475f);
    const __m256 hi = _mm256_set1_ps(88.0f);
    const __m256 under = _mm256_cmp_ps(x, lo, _CMP_LT_OQ);
    x = _mm256_min_ps(_mm256_max_ps(x, lo), hi);
    const __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f)),
                                     _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.693359375f), x);
    r = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.12194440e-4f), r);
    __m256 p = _mm256_set1_ps(1.0f / 5040.0f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 720.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
    const __m256 y = _mm256_mul_ps(p, _mm256_castsi256_ps(e));
    return _mm256_andnot_ps(under, y);
}

__attribute__((target("avx2,fma"))) static float exp_shifted_sum_avx2(float *x, int n, float shift) {
    const __m256 sh = _mm256_set1_ps(shift);
    __m256 acc = _mm256_setzero_ps();
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 e = exp256(_mm256_sub_ps(_mm256_loadu_ps(x + i), sh));
        _mm256_storeu_ps(x + i, e);
        acc = _mm256_add_ps(acc, e);
    }
    float sum = hsum256(acc);
    for (; i < n; ++i) {
        x[i] = expf(x[i] - shift);
        sum += x[i];
    }
    return sum;
}

typedef struct {
    uint64_t batch, heads, seq, d, block, window;
    int kind, backend;
    float scale;
    const int32_t *valid;
    const float *q, *k, *v;
    float *out;
    atomic_ulong next;
    uint64_t ntasks, blocks_per_head;
} tiled_job;

/* tile.rs:65-151 (micro_tile): online softmax over 64-key tiles for mr rows. */
static void micro_tile(const tiled_job *J, const float *q, const float *k, const float *v,
                       uint64_t valid_len, uint64_t gi0, int mr, float *out, float *scores,
                       float *acc) {
    const uint64_t d = J->d;
    uint64_t rlo[MR], rhi[MR];
    for (int r = 0; r < MR; ++r)
        oracle_key_range(J->kind, J->block, J->window, gi0 + (uint64_t)(r < mr - 1 ? r : mr - 1),
                         valid_len, &rlo[r], &rhi[r]);
    const uint64_t ks = rlo[0], ke = rhi[mr - 1];
    float m[MR], l[MR];
    for (int r = 0; r < MR; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }
    memset(acc, 0, sizeof(float) * (uint64_t)mr * d);
    const float *qt = q + gi0 * d;
    for (uint64_t kt = ks; kt < ke;) {
        const uint64_t kend = umin(kt + NC, ke);
        const int nk = (int)(kend - kt);
        if (J->backend == 1)
            dot_tile_avx2(qt, k + kt * d, d, mr, nk, scores);
        else
            dot_tile_portable(qt, k + kt * d, d, mr, nk, scores);
        int ba[MR], bz[MR];
        for (int r = 0; r < mr; ++r) {
            ba[r] = bz[r] = 0;
            const uint64_t lo = umax(rlo[r], kt), hi = umin(rhi[r], kend);
            if (lo >= hi) continue;
            const int a = (int)(lo - kt), z = (int)(hi - kt);
            ba[r] = a;
            bz[r] = z;
            float *row = scores + r * NC;
            float tmax = -INFINITY;
            for (int j = a; j < z; ++j) {
                row[j] *= J->scale;
                tmax = fmaxf(tmax, row[j]);
            }
            const float new_m = fmaxf(m[r], tmax);
            const float alpha = m[r] == -INFINITY ? 0.0f : expf(m[r] - new_m);
            const float sum = J->backend == 1 ? exp_shifted_sum_avx2(row + a, z - a, new_m)
                                              : exp_shifted_sum_portable(row + a, z - a, new_m);
            l[r] = l[r] * alpha + sum;
            const int raised = new_m > m[r];
            m[r] = new_m;
            if (raised)
                for (uint64_t c = 0; c < d; ++c) acc[(uint64_t)r * d + c] *= alpha;
        }
        for (int r = 0; r < mr; ++r) {
            if (ba[r] >= bz[r]) continue;
            const float *p = scores + r * NC + ba[r];
            const float *vv = v + (kt + (uint64_t)ba[r]) * d;
            if (J->backend == 1)
                axpy_rows_avx2(acc + (uint64_t)r * d, p, bz[r] - ba[r], vv, d);
            else
                axpy_rows_portable(acc + (uint64_t)r * d, p, bz[r] - ba[r], vv, d);
        }
        kt = kend;
    }
    for (int r = 0; r < mr; ++r) {
        const float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
        for (uint64_t c = 0; c < d; ++c) out[(uint64_t)r * d + c] = acc[(uint64_t)r * d + c] * inv;
    }
}

/* tile.rs:27-62 (run_block) within the worker loop of tiled/mod.rs:96-115. */
static void *tiled_worker(void *arg) {
    tiled_job *J = (tiled_job *)arg;
    const uint64_t d = J->d;
    float scores[MR * NC];
    float *acc = (float *)malloc(sizeof(float) * MR * d);
    for (;;) {
        const uint64_t t = atomic_fetch_add(&J->next, 1);
        if (t >= J->ntasks) break;
        const uint64_t blk = t % J->blocks_per_head;
        const uint64_t hb = t / J->blocks_per_head; /* sequence * heads + head */
        const uint64_t b = hb / J->heads;
        const uint64_t head_off = hb * J->seq * d;
        const float *q = J->q + head_off, *k = J->k + head_off, *v = J->v + head_off;
        float *out = J->out + head_off;
        const uint64_t valid_len = (uint64_t)J->valid[b];
        const uint64_t row0 = blk * REF_BLOCK;
        const uint64_t rows = umin(REF_BLOCK, J->seq - row0);
        for (uint64_t i0 = 0; i0 < rows; i0 += MR) {
            const int mr = (int)umin(MR, rows - i0);
            const uint64_t gi0 = row0 + i0;
            const int valid = (int)umin(sat_sub(valid_len, gi0), (uint64_t)mr);
            float *o = out + gi0 * d;
            memset(o + (uint64_t)valid * d, 0, sizeof(float) * (uint64_t)(mr - valid) * d);
            if (valid > 0) micro_tile(J, q, k, v, valid_len, gi0, valid, o, scores, acc);
        }
    }
    free(acc);
    return NULL;
}

/* Tiled::attend_with_stages, tiled/mod.rs:61-126, batched over sequences. */
int oracle_tiled_attend_batched(uint64_t batch, uint64_t heads, uint64_t seq, uint64_t d,
                                int kind, uint64_t block, uint64_t window,
                                const int32_t *valid_len, float scale, const float *q,
                                const float *k, const float *v, float *out, int threads,
                                int backend) {
    if (backend == 1 && !oracle_cpu_has_avx2_fma()) backend = 0;
    tiled_job J;
    J.batch = batch;
    J.heads = heads;
    J.seq = seq;
    J.d = d;
    J.block = block;
    J.window = window;
    J.kind = kind;
    J.backend = backend;
    J.scale = scale;
    J.valid = valid_len;
    J.q = q;
    J.k = k;
    J.v = v;
    J.out = out;
    J.blocks_per_head = (seq + REF_BLOCK - 1) / REF_BLOCK;
    J.ntasks = batch * heads * J.blocks_per_head;
    atomic_init(&J.next, 0);
    if (J.ntasks == 0) return backend;
    uint64_t workers = threads < 1 ? 1 : (uint64_t)threads;
    if (workers > J.ntasks) workers = J.ntasks;
    if (workers == 1) {
        tiled_worker(&J);
        return backend;
    }
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * workers);
    for (uint64_t w = 0; w < workers; ++w) pthread_create(&tid[w], NULL, tiled_worker, &J);
    for (uint64_t w = 0; w < workers; ++w) pthread_join(tid[w], NULL);
    free(tid);
    return backend;
}

/* rand_vec, crates/raya-kernels/tests/common/mod.rs:6-18: xorshift64 values
 * uniform in [-1, 1]. */
void oracle_rand_vec(uint64_t n, uint64_t seed, float *out) {
    uint64_t s = (seed * 0x9E3779B97F4A7C15ull) | 1ull;
    for (uint64_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        const float u = (float)(s >> 40) / (float)(1ull << 24);
        out[i] = 2.0f * u - 1.0f;
    }
}

/* fill, crates/raya-kernels/tests/masks_dense.rs:5-13: LCG values in [-0.5, 0.5). */
void oracle_lcg_fill(uint64_t n, uint32_t seed, float *out) {
    uint32_t s = seed;
    for (uint64_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        out[i] = (float)(s >> 8) / (float)(1u << 24) - 0.5f;
    }
}
