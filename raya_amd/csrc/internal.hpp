// Internal interfaces between the C ABI (capi.cpp) and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "raya_hip.h"

namespace raya {

// Launch description of the fused attention kernel (all validated by the caller).
struct AttnLaunch {
    const float *q, *k, *v;
    float *out;
    const int32_t *valid_len;  // device [batch]; nullptr => valid_scalar for every sequence
    int32_t valid_scalar;
    int64_t q_bs, q_hs, q_rs;  // strides in floats: batch, head, row
    int64_t k_bs, k_hs, k_rs;
    int64_t v_bs, v_hs, v_rs;
    int64_t o_bs, o_hs, o_rs;
    int32_t batch, heads, seq, head_dim;
    int32_t mask_kind;
    int32_t mask_arg;  // Sliding half-width / BlockDiag width, clamped to seq
    float scale;
    // Packed sequences: when set, sequence b's rows start at row seq_start[b] of
    // each operand (batch strides unused), only its valid rows exist and rows at
    // or beyond valid_len are neither read nor written.
    const int32_t *seq_start;
    // Non-null selects the instrumented kernel, which adds its per-stage clock
    // totals to this device struct.
    raya_stage_cycles *stage_cycles;
};

// Largest head_dim the fused attention kernel is instantiated for.
constexpr int kMaxHeadDim = 256;

hipError_t launch_attention(const AttnLaunch &a, hipStream_t stream);

// Launch description of the NT GEMM (all validated by the caller).
struct GemmLaunch {
    float *out;
    int64_t ldo;
    const float *a;
    int64_t lda;
    const float *b;
    int64_t ldb;
    int32_t m, n, k;
    int32_t n_rows_b;  // rows of b: n, or 2n for GeGLU
    int32_t act;       // RAYA_EPI_*
    const float *bias;
    const float *residual;
    int64_t ldr;
    // Rotary embedding fused into a plain (RAYA_EPI_NONE) epilogue: columns below
    // rope_cols (the q and k sections of a packed QKV projection, head_dim 64)
    // are rotated in pairs (c, c + 32) at position positions[row], with
    // cos/sin tables [position][32].  rope_cos == nullptr disables it.
    const float *rope_cos, *rope_sin;
    const int32_t *positions;
    int32_t rope_cols;
    // A pre-LN LayerNorm of the input rows folded into the product (the ring
    // kernel only): b holds the weight with the norm's gain folded into its
    // columns, colsum[j] = sum_t b[j][t] (f64, rounded), and in_stats each row's
    // (mean_hi, mean_lo, rstd, 0) ([m], from launch_ln_stats; mean = mean_hi +
    // mean_lo, rstd = 1 / sqrt(var + eps)).  A row whose mean is more than one
    // standard deviation from zero has its A operands centred by mean_hi as they
    // leave LDS, so that its mean is removed before the contraction as
    // ops::layer_norm removes it before scaling; the rest of the mean comes out
    // as mean colsum.  Then y = rstd (acc - mean' colsum) before bias, activation
    // and RoPE: LayerNorm(a) W^T.  Null: off.
    const float4 *in_stats;
    const float *colsum;
    // Per output row and 64-column chunk, after the residual add ([m][n / 64]; n a
    // multiple of 64): (c, sum (x - c), sum (x - c)^2, 0) with c the chunk's f32
    // mean, the same c in every lane, so that launch_ln_stats recovers the chunk's
    // mean as c + sum (x - c) / 64 to the precision of the deviations rather than
    // of |x|.  Null: off.
    float4 *out_stats;
    // Split-K (the ring kernel only), for launches whose output tiles alone leave
    // compute units idle: each tile's K loop is divided among `splits` workgroups,
    // which store their partial tiles to `partials` ([tiles][splits][128 x 128]);
    // a second launch of the same kernel (reduce = 1, set by launch_gemm) sums each
    // tile's partials in split order and runs the epilogue.  splits <= 1: off.
    float *partials;
    int32_t splits;
    int32_t reduce;
};

// Split-K for the ring kernel: the split count gemm_splits chooses for an
// m x n output (GeGLU: n output columns from 2n weight rows) of depth k (1: no
// split; never past kGemmSplitMaxTiles output tiles), and the partials' floats.
constexpr int kGemmSplitMaxTiles = 256;
int gemm_splits(int m, int n, int k, int act);
size_t gemm_split_floats(int m, int n, int act, int splits);

// Head dim of the fused RoPE epilogue (other head dims use launch_rope).
constexpr int kRopeHeadDim = 64;

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t stream);
hipError_t launch_fill_zero(float *out, int64_t ldo, int m, int n, hipStream_t stream);

// Row-wise LayerNorm over `rows` rows of width d (see encoder.hip).
struct LayerNormLaunch {
    const float *x;
    int64_t ldx;
    const int32_t *gather;  // nullptr, or the source row of each output row (embedding ids)
    const float *w, *b;     // b may be nullptr
    float eps;
    int32_t rows, d;
    float *out;  // may be nullptr when out_add is set
    int64_t ldo;
    const float *add;          // nullptr, or a table whose row seq_index[row_seq[row]] is added
    const int32_t *row_seq;    // sequence of each row
    const int32_t *seq_index;  // table row of each sequence
    float *out_add;
};

hipError_t launch_layer_norm(const LayerNormLaunch &l, hipStream_t stream);
// Each row's (mean_hi, mean_lo, 1 / sqrt(var + eps), 0) from its 64-column chunk
// statistics (GemmLaunch::out_stats, [rows][n_chunks]) into out ([rows]).
hipError_t launch_ln_stats(const float4 *chunks, int rows, int n_chunks, float eps, float4 *out, hipStream_t stream);
// sums[j] = sum over t < k of b[j][t] in f64, rounded to f32 ([rows]).
hipError_t launch_row_sums(const float *b, int64_t ldb, int rows, int k, float *sums, hipStream_t stream);
hipError_t launch_rope(float *qkv, int64_t ld, const int32_t *positions, const float *cos_t,
                       const float *sin_t, int rows, int d, int head_dim, hipStream_t stream);
hipError_t launch_gather_rows(const float *h, int64_t ldh, const int32_t *rows, int n, int d,
                              float *out, hipStream_t stream);
hipError_t launch_head_finish(const float *raw_logits, const uint8_t *mask, int batch, int markers,
                              const float *h, int64_t ldh, const int32_t *seq_start, int d,
                              float *logits, float *probs, float *features, float *pooled,
                              float *act_in, int ld_act, hipStream_t stream);

// Thread-local error state of the C ABI (capi.cpp).
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail_device(hipError_t e, const char *what);
int ok();

}  // namespace raya
