// Row-wise kernels of the device-resident decision-model forward: embedding
// gather + LayerNorm, LayerNorm (+ per-sequence vector add), rotary embedding on
// the packed QKV projection, marker-row gather, and the per-sequence tail of the
// head (marker mask, softmax, score features, act-head input).
//
// Rows are tokens of a packed batch: sequence b owns rows
// [seq_start[b], seq_start[b] + valid_len[b]) and padded positions are never
// materialised.  Every kernel is HBM-bound; one wave handles one row so that
// loads are coalesced along the hidden dimension.
#include <cmath>

#include "internal.hpp"

namespace raya {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row, four waves per workgroup

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
}

// ops::layer_norm (crates/raya-core/src/ops.rs:51-74): mean and biased variance
// in f64, y = f32((x - mean) * inv) * w (+ b).  The statistics are reduced in a
// different order than the reference's sequential sums, which moves them by a
// few f64 ulps and the f32 result by at most one ulp in rare rounding ties.
// When `add` is given, out_add = y + add[add_row(row)] (the type embedding of
// the row's sequence, model.rs:297-303).
__global__ void __launch_bounds__(64 * kRowsPerBlock)
    layer_norm_kernel(const float *x, int64_t ldx, const int32_t *gather, const float *w,
                      const float *b, float eps, int rows, int d, float *out, int64_t ldo,
                      const float *add, const int32_t *row_seq, const int32_t *seq_index,
                      float *out_add) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int64_t src = gather ? (int64_t)gather[row] : (int64_t)row;
    const float *xr = x + src * ldx;
    double s = 0.0;
    for (int c = lane; c < d; c += 64) s += (double)xr[c];
    const double mean = wave_sum(s) / (double)d;
    double v = 0.0;
    for (int c = lane; c < d; c += 64) {
        const double t = (double)xr[c] - mean;
        v += t * t;
    }
    const double var = wave_sum(v) / (double)d;
    const double inv = 1.0 / sqrt(var + (double)eps);
    const float *addr = nullptr;
    if (add) addr = add + (int64_t)seq_index[row_seq[row]] * d;
    for (int c = lane; c < d; c += 64) {
        float y = __fmul_rn((float)(((double)xr[c] - mean) * inv), w[c]);
        if (b) y = __fadd_rn(y, b[c]);
        if (out) out[(int64_t)row * ldo + c] = y;
        if (out_add) out_add[(int64_t)row * ldo + c] = __fadd_rn(y, addr[c]);
    }
}

// The same LayerNorm for rows of NC * 256 floats (16-byte aligned rows): each lane
// holds NC float4 of the row in registers, so the row is read once.
template <int NC>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
    layer_norm_vec_kernel(const float *x, int64_t ldx, const int32_t *gather, const float *w,
                          const float *b, float eps, int rows, float *out, int64_t ldo,
                          const float *add, const int32_t *row_seq, const int32_t *seq_index,
                          float *out_add) {
    constexpr int d = NC * 256;
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int64_t src = gather ? (int64_t)gather[row] : (int64_t)row;
    const float *xr = x + src * ldx;
    float4 v[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) v[i] = *(const float4 *)(xr + 256 * i + 4 * lane);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < NC; ++i) s += ((double)v[i].x + (double)v[i].y) + ((double)v[i].z + (double)v[i].w);
    const double mean = wave_sum(s) / (double)d;
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const double a = (double)v[i].x - mean, bb = (double)v[i].y - mean;
        const double c = (double)v[i].z - mean, e = (double)v[i].w - mean;
        q += (a * a + bb * bb) + (c * c + e * e);
    }
    const double var = wave_sum(q) / (double)d;
    const double inv = 1.0 / sqrt(var + (double)eps);
    const float *addr = add ? add + (int64_t)seq_index[row_seq[row]] * d : nullptr;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = 256 * i + 4 * lane;
        const float4 wv = *(const float4 *)(w + c);
        float4 y;
        y.x = __fmul_rn((float)(((double)v[i].x - mean) * inv), wv.x);
        y.y = __fmul_rn((float)(((double)v[i].y - mean) * inv), wv.y);
        y.z = __fmul_rn((float)(((double)v[i].z - mean) * inv), wv.z);
        y.w = __fmul_rn((float)(((double)v[i].w - mean) * inv), wv.w);
        if (b) {
            const float4 bv = *(const float4 *)(b + c);
            y.x = __fadd_rn(y.x, bv.x);
            y.y = __fadd_rn(y.y, bv.y);
            y.z = __fadd_rn(y.z, bv.z);
            y.w = __fadd_rn(y.w, bv.w);
        }
        if (out) *(float4 *)(out + (int64_t)row * ldo + c) = y;
        if (out_add) {
            const float4 av = *(const float4 *)(addr + c);
            *(float4 *)(out_add + (int64_t)row * ldo + c) =
                make_float4(__fadd_rn(y.x, av.x), __fadd_rn(y.y, av.y), __fadd_rn(y.z, av.z), __fadd_rn(y.w, av.w));
        }
    }
}

// ops::rope_in_place (ops.rs:118-141) on the q and k sections of a packed
// [rows][3 d] projection: for head h and i < half, (a, b) = (x[i], x[i + half])
// becomes (a cos - b sin, b cos + a sin) at the row's position.  Each product
// and the sum are rounded separately, as the reference's scalar code does.
__global__ void rope_kernel(float *qkv, int64_t ld, const int32_t *positions, const float *cos_t,
                            const float *sin_t, int rows, int d, int head_dim) {
    const int half = head_dim / 2;
    const int per_row = d / head_dim * half * 2;  // (q, k) x heads x half
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * per_row) return;
    const int row = (int)(idx / per_row);
    int rem = (int)(idx % per_row);
    const int sec = rem / (d / 2);  // 0: q, 1: k
    rem %= d / 2;
    const int h = rem / half, i = rem % half;
    float *p = qkv + (int64_t)row * ld + sec * d + h * head_dim;
    const int64_t t = (int64_t)positions[row] * half + i;
    const float c = cos_t[t], s = sin_t[t];
    const float a = p[i], bb = p[i + half];
    p[i] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(bb, s));
    p[i + half] = __fadd_rn(__fmul_rn(bb, c), __fmul_rn(a, s));
}

// out[j] = h[rows[j]] (zeros where rows[j] < 0).
__global__ void gather_rows_kernel(const float *h, int64_t ldh, const int32_t *rows, int n, int d,
                                   float *out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)n * d) return;
    const int j = (int)(idx / d), c = (int)(idx % d);
    const int r = rows[j];
    out[idx] = r >= 0 ? h[(int64_t)r * ldh + c] : 0.0f;
}

// The tail of Network::forward (model.rs:310-334) and head::features
// (head.rs:70-92) for one sequence per thread, in the reference's sequential
// f32 order: invalid markers' logits become -1e4, softmax_in_place
// (ops.rs:77-87), [top1, top1 - top2, entropy / ln k, k / 255] with
// k = max(valid markers, 2), pooled = row 0, act_in = [pooled, features] in rows of
// ld_act floats whose columns past d + 4 are zero (the act head's padded depth).
__global__ void head_finish_kernel(const float *raw_logits, const uint8_t *mask, int batch,
                                   int markers, const float *h, int64_t ldh,
                                   const int32_t *seq_start, int d, float *logits, float *probs,
                                   float *features, float *pooled, float *act_in, int ld_act) {
    // One workgroup per sequence: every thread copies part of the CLS row; thread 0
    // runs the marker softmax and the features in the reference's sequential order.
    const int b = blockIdx.x;
    if (b >= batch) return;
    const float *row0 = h + (int64_t)seq_start[b] * ldh;
    float *ai = act_in + (int64_t)b * ld_act;
    for (int c = threadIdx.x; c < d; c += blockDim.x) {
        const float x = row0[c];
        pooled[(int64_t)b * d + c] = x;
        ai[c] = x;
    }
    for (int c = d + 4 + threadIdx.x; c < ld_act; c += blockDim.x) ai[c] = 0.0f;
    if (threadIdx.x != 0) return;
    const float *raw = raw_logits + (int64_t)b * markers;
    const uint8_t *mk = mask + (int64_t)b * markers;
    float *lg = logits + (int64_t)b * markers;
    float *pr = probs + (int64_t)b * markers;
    float mx = -INFINITY;
    int valid = 0;
    for (int j = 0; j < markers; ++j) {
        lg[j] = mk[j] ? raw[j] : -1e4f;
        valid += mk[j] ? 1 : 0;
        mx = fmaxf(mx, lg[j]);
    }
    float sum = 0.0f;
    for (int j = 0; j < markers; ++j) {
        pr[j] = expf(__fsub_rn(lg[j], mx));
        sum = __fadd_rn(sum, pr[j]);
    }
    for (int j = 0; j < markers; ++j) pr[j] = __fdiv_rn(pr[j], sum);
    const float k = (float)(valid > 2 ? valid : 2);
    float ent = 0.0f, top1 = -INFINITY, top2 = -INFINITY;
    for (int j = 0; j < markers; ++j) {
        const float x = pr[j];
        ent = __fadd_rn(ent, __fmul_rn(x, logf(fmaxf(x, 1e-9f))));
        if (x > top1) {
            top2 = top1;
            top1 = x;
        } else if (x > top2) {
            top2 = x;
        }
    }
    if (markers < 2) top2 = 0.0f;
    float f[4] = {top1, __fsub_rn(top1, top2), __fdiv_rn(-ent, logf(k)), __fdiv_rn(k, 255.0f)};
    for (int c = 0; c < 4; ++c) {
        features[b * 4 + c] = f[c];
        ai[d + c] = f[c];
    }
}

unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

namespace {

// The pre-LN LayerNorm statistics of each row from its 64-column chunks'
// (c, r = sum (x - c), s = sum (x - c)^2), in f64 as ops::layer_norm keeps its
// statistics (crates/raya-core/src/ops.rs:51-74): a chunk's mean is c + r / 64 and
// its sum of squared deviations s - r^2 / 64; the chunks combine as Chan et al.'s
// pairwise update.  Out: (mean_hi, mean_lo, 1 / sqrt(var + eps), 0) with var the
// biased variance and mean_hi + mean_lo the f64 mean to 48 bits.
__global__ void ln_stats_kernel(const float4 *chunks_in, int rows, int chunks, float eps, float4 *out) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const float4 *st = chunks_in + (int64_t)row * chunks;
    double mean = 0.0;
    for (int c = 0; c < chunks; ++c) mean += (double)st[c].x + (double)st[c].y * (1.0 / 64.0);
    mean /= chunks;
    double m2 = 0.0;
    for (int c = 0; c < chunks; ++c) {
        const double r = st[c].y, cm = (double)st[c].x + r * (1.0 / 64.0);
        const double dm = cm - mean;
        m2 += ((double)st[c].z - r * r * (1.0 / 64.0)) + 64.0 * dm * dm;
    }
    const double var = fmax(m2, 0.0) / (64.0 * chunks);
    const float hi = (float)mean;
    out[row] = make_float4(hi, (float)(mean - (double)hi), (float)(1.0 / sqrt(var + (double)eps)), 0.0f);
}

// One wave per row: each lane sums a strided share of the row in f64, then the
// lanes' sums are combined by a fixed butterfly (the same order every call).
__global__ void row_sums_kernel(const float *b, int64_t ldb, int rows, int k, float *sums) {
    const int row = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *p = b + (int64_t)row * ldb;
    double s = 0.0;
    for (int t = lane; t < k; t += 64) s += (double)p[t];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) sums[row] = (float)s;
}

}  // namespace

hipError_t launch_row_sums(const float *b, int64_t ldb, int rows, int k, float *sums, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(row_sums_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, b, ldb, rows, k, sums);
    return hipGetLastError();
}

hipError_t launch_ln_stats(const float4 *chunks, int rows, int n_chunks, float eps, float4 *out, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(ln_stats_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, chunks, rows,
                       n_chunks, eps, out);
    return hipGetLastError();
}


hipError_t launch_layer_norm(const LayerNormLaunch &l, hipStream_t stream) {
    if (l.rows == 0) return hipSuccess;
    const auto aligned = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool vec = l.d % 256 == 0 && l.d <= 1024 && l.ldx % 4 == 0 && l.ldo % 4 == 0 && aligned(l.x) &&
                     aligned(l.w) && aligned(l.b) && aligned(l.out) && aligned(l.add) && aligned(l.out_add);
    if (vec) {
        const dim3 grid(blocks_for(l.rows, kRowsPerBlock)), block(64 * kRowsPerBlock);
        switch (l.d / 256) {
        case 1: hipLaunchKernelGGL(layer_norm_vec_kernel<1>, grid, block, 0, stream, l.x, l.ldx, l.gather, l.w,
                                   l.b, l.eps, l.rows, l.out, l.ldo, l.add, l.row_seq, l.seq_index, l.out_add);
                break;
        case 2: hipLaunchKernelGGL(layer_norm_vec_kernel<2>, grid, block, 0, stream, l.x, l.ldx, l.gather, l.w,
                                   l.b, l.eps, l.rows, l.out, l.ldo, l.add, l.row_seq, l.seq_index, l.out_add);
                break;
        case 3: hipLaunchKernelGGL(layer_norm_vec_kernel<3>, grid, block, 0, stream, l.x, l.ldx, l.gather, l.w,
                                   l.b, l.eps, l.rows, l.out, l.ldo, l.add, l.row_seq, l.seq_index, l.out_add);
                break;
        default: hipLaunchKernelGGL(layer_norm_vec_kernel<4>, grid, block, 0, stream, l.x, l.ldx, l.gather, l.w,
                                    l.b, l.eps, l.rows, l.out, l.ldo, l.add, l.row_seq, l.seq_index, l.out_add);
                 break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(layer_norm_kernel, dim3(blocks_for(l.rows, kRowsPerBlock)),
                       dim3(64 * kRowsPerBlock), 0, stream, l.x, l.ldx, l.gather, l.w, l.b, l.eps,
                       l.rows, l.d, l.out, l.ldo, l.add, l.row_seq, l.seq_index, l.out_add);
    return hipGetLastError();
}

hipError_t launch_rope(float *qkv, int64_t ld, const int32_t *positions, const float *cos_t,
                       const float *sin_t, int rows, int d, int head_dim, hipStream_t stream) {
    const int64_t n = (int64_t)rows * d;  // (q, k) x d / 2 pairs per row
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, qkv, ld,
                       positions, cos_t, sin_t, rows, d, head_dim);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float *h, int64_t ldh, const int32_t *rows, int n, int d,
                              float *out, hipStream_t stream) {
    const int64_t total = (int64_t)n * d;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, h, ldh,
                       rows, n, d, out);
    return hipGetLastError();
}

hipError_t launch_head_finish(const float *raw_logits, const uint8_t *mask, int batch, int markers,
                              const float *h, int64_t ldh, const int32_t *seq_start, int d,
                              float *logits, float *probs, float *features, float *pooled,
                              float *act_in, int ld_act, hipStream_t stream) {
    if (batch == 0) return hipSuccess;
    if (ld_act < d + 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(head_finish_kernel, dim3((unsigned)batch), dim3(256), 0, stream,
                       raw_logits, mask, batch, markers, h, ldh, seq_start, d, logits, probs,
                       features, pooled, act_in, ld_act);
    return hipGetLastError();
}

}  // namespace raya
