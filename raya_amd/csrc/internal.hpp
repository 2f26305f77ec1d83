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
};

// Largest head_dim the fused attention kernel is instantiated for.
constexpr int kMaxHeadDim = 128;

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
};

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t stream);
hipError_t launch_fill_zero(float *out, int64_t ldo, int m, int n, hipStream_t stream);

}  // namespace raya
