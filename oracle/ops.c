/*
 * CPU oracle: scalar building blocks of the reference forward pass.
 * TEST INFRASTRUCTURE ONLY; see oracle.h.  Pinned by the known answers of
 * crates/raya-core/tests/ops.rs:9-92 (erf at seven points, exact GELU, biased
 * LayerNorm variance, softmax shift invariance, RoPE rotation values).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <stdint.h>

/* ops::erf, crates/raya-core/src/ops.rs:7-30: Taylor series below 2.5,
 * continued fraction for erfc above, saturated at 6. */
double oracle_erf(double x) {
    const double ax = fabs(x);
    double value;
    if (ax >= 6.0) {
        value = 1.0;
    } else if (ax < 2.5) {
        double term = ax, sum = ax;
        const double x2 = ax * ax;
        uint32_t n = 0;
        for (;;) {
            double floor_ = fabs(sum) > 1e-300 ? fabs(sum) : 1e-300;
            if (!(fabs(term) > 1e-18 * floor_)) break;
            n += 1;
            term *= -x2 / (double)n;
            sum += term / (double)(2 * n + 1);
        }
        value = sum * 1.12837916709551257390; /* 2/sqrt(pi) */
    } else {
        double t = ax;
        for (uint32_t n = 120; n >= 1; --n) t = ax + (double)n / 2.0 / t;
        value = 1.0 - exp(-ax * ax) / sqrt(3.14159265358979323846) / t;
    }
    return copysign(value, x);
}

/* ops::gelu, ops.rs:35-38: exact GELU evaluated in f64. */
float oracle_gelu(float x) {
    const double xd = (double)x;
    return (float)(0.5 * xd * (1.0 + oracle_erf(xd * 0.70710678118654752440)));
}

/* ops::gelu over an array. */
void oracle_gelu_vec(float *out, const float *x, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_gelu(x[i]);
}

/* ops::layer_norm, ops.rs:51-74: f64 mean and biased variance per row. */
void oracle_layer_norm(float *out, const float *x, const float *weight, const float *bias,
                       float eps, uint64_t rows, uint64_t d) {
    for (uint64_t r = 0; r < rows; ++r) {
        const float *row = x + r * d;
        float *dst = out + r * d;
        double mean = 0.0;
        for (uint64_t i = 0; i < d; ++i) mean += (double)row[i];
        mean /= (double)d;
        double var = 0.0;
        for (uint64_t i = 0; i < d; ++i) {
            const double c = (double)row[i] - mean;
            var += c * c;
        }
        var /= (double)d;
        const double inv = 1.0 / sqrt(var + (double)eps);
        for (uint64_t i = 0; i < d; ++i) {
            const float y = (float)(((double)row[i] - mean) * inv) * weight[i];
            dst[i] = bias ? y + bias[i] : y;
        }
    }
}

/* ops::softmax_in_place, ops.rs:77-87. */
void oracle_softmax(float *x, uint64_t n) {
    float mx = -INFINITY;
    for (uint64_t i = 0; i < n; ++i) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (uint64_t i = 0; i < n; ++i) x[i] /= sum;
}

/* ops::rope_in_place, ops.rs:118-141: rotate-half RoPE on [heads][seq][head_dim]
 * with f32 inv_freq = 1/theta^(2i/D) and f32 angles pos * inv_freq. */
void oracle_rope(float *x, uint64_t heads, uint64_t seq, uint64_t head_dim, float theta) {
    const uint64_t half = head_dim / 2;
    float inv_freq[512], cs[512], sn[512];
    for (uint64_t i = 0; i < half; ++i)
        inv_freq[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
    for (uint64_t pos = 0; pos < seq; ++pos) {
        for (uint64_t i = 0; i < half; ++i) {
            const float angle = (float)pos * inv_freq[i];
            cs[i] = cosf(angle);
            sn[i] = sinf(angle);
        }
        for (uint64_t h = 0; h < heads; ++h) {
            float *row = x + (h * seq + pos) * head_dim;
            for (uint64_t i = 0; i < half; ++i) {
                const float a = row[i], b = row[i + half];
                row[i] = a * cs[i] - b * sn[i];
                row[i + half] = b * cs[i] + a * sn[i];
            }
        }
    }
}
