// One post-LN Transformer encoder layer (BERT's layer: LayerNorm after each
// residual add, a GELU feed-forward, biases on every projection) on a dense
// batch, composed from the library's kernels:
//
//   qkv = x Wqkv^T + bqkv                          (GEMM, bias epilogue)
//   ctx = attention(q, k, v; mask, valid_len)      (strided reads of the packed qkv)
//   y1  = LayerNorm1(x + ctx Wo^T + bo)            (GEMM, bias + residual; LayerNorm)
//   f   = gelu(y1 W1^T + b1)                       (GEMM, bias + GELU epilogue)
//   out = LayerNorm2(y1 + f W2^T + b2)             (GEMM, bias + residual; LayerNorm)
//
// Weights are nn.Linear's [out_features][in_features]; Wqkv stacks the q, k and
// v projections (each [hidden][hidden]) and a head is a contiguous slice of
// head_dim columns of each, as nn.MultiheadAttention's in_proj_weight.  GELU is
// the exact (erf) one and LayerNorm keeps its statistics in f64, as
// crates/raya-core/src/ops.rs:7-74 computes them.
#include <hip/hip_runtime.h>

#include <cinttypes>
#include <climits>
#include <cmath>
#include <cstdint>

#include "internal.hpp"
#include "raya_hip.h"

namespace raya {
namespace {

// Workspace layout in floats: qkv [T][3d], ctx [T][d], sum [T][d], y1 [T][d], f [T][F].
struct PostLNPlan {
    uint64_t tokens, qkv, ctx, sum, y1, f, total;  // offsets and total, in floats
};

PostLNPlan plan_of(const raya_postln_layer &L) {
    const auto up = [](uint64_t n) { return (n + 63) / 64 * 64; };  // 256-byte aligned parts
    PostLNPlan p{};
    p.tokens = L.batch * L.seq;
    const uint64_t T = p.tokens, d = L.hidden;
    p.qkv = 0;
    p.ctx = p.qkv + up(T * 3 * d);
    p.sum = p.ctx + up(T * d);
    p.y1 = p.sum + up(T * d);
    p.f = p.y1 + up(T * d);
    p.total = p.f + up(T * L.ffn);
    return p;
}

int check_postln(const raya_postln_layer *L) {
    if (!L) return fail(RAYA_ERR_SHAPE, "invalid shape: null layer");
    if (L->batch == 0 || L->seq == 0 || L->hidden == 0 || L->heads == 0 || L->ffn == 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: batch, seq, hidden, heads and ffn must be at least 1");
    if (L->hidden % L->heads != 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: hidden %" PRIu64 " is not a multiple of heads %" PRIu64,
                    L->hidden, L->heads);
    const uint64_t hd = L->hidden / L->heads;
    if (hd % 8 != 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: head_dim %" PRIu64 " is not a multiple of 8", hd);
    if (hd > (uint64_t)kMaxHeadDim)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: head_dim %" PRIu64 " (the HIP kernel handles up to %d)", hd,
                    kMaxHeadDim);
    if (L->ffn % 4 != 0) return fail(RAYA_ERR_UNSUPPORTED, "unsupported: ffn %" PRIu64 " is not a multiple of 4", L->ffn);
    if (L->mask_kind < RAYA_MASK_BLOCK3 || L->mask_kind > RAYA_MASK_BLOCKDIAG || L->reserved != 0)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: mask kind %d", L->mask_kind);
    if (L->mask_kind == RAYA_MASK_BLOCKDIAG && L->mask_arg == 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: block_diag width must be at least 1");
    if (L->seq >= (uint64_t(1) << 30) || L->batch > 0x7fffffffu || L->batch * L->seq > 0x7fffffffu ||
        3 * L->hidden > 0x3fffffffu || L->ffn > 0x3fffffffu)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: layer dimensions past the kernels' 32-bit indexing");
    // The workspace in bytes (6 hidden + ffn floats per token, plus 256-byte padding of
    // its five parts) must fit 64 bits.
    if (6 * L->hidden + L->ffn + 5 * 64 > (UINT64_MAX / sizeof(float)) / (L->batch * L->seq))
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: a layer workspace past 64-bit sizes");
    if (!(L->ln_eps >= 0.f) || !std::isfinite(L->ln_eps))
        return fail(RAYA_ERR_SHAPE, "invalid shape: ln_eps must be finite and non-negative");
    if (!L->wqkv || !L->wo || !L->w1 || !L->w2 || !L->ln1_w || !L->ln2_w)
        return fail(RAYA_ERR_SHAPE, "invalid shape: null weight");
    return RAYA_OK;
}

}  // namespace
}  // namespace raya

using namespace raya;

extern "C" {

uint64_t raya_postln_workspace_bytes(const raya_postln_layer *L) {
    if (check_postln(L)) return 0;
    return plan_of(*L).total * sizeof(float);
}

int raya_postln_layer_forward(const raya_postln_layer *L, const int32_t *valid_len, const float *x, float *out,
                              void *workspace, uint64_t workspace_bytes, void *stream_ptr) {
    int rc = check_postln(L);
    if (rc) return rc;
    const PostLNPlan p = plan_of(*L);
    if (workspace_bytes < p.total * sizeof(float))
        return fail(RAYA_ERR_SHAPE, "invalid shape: workspace of %" PRIu64 " bytes, the layer needs %" PRIu64,
                    workspace_bytes, p.total * sizeof(float));
    if (!valid_len || !x || !out || !workspace) return fail(RAYA_ERR_SHAPE, "invalid shape: null device pointer");
    hipStream_t stream = (hipStream_t)stream_ptr;
    const uint64_t T = p.tokens, d = L->hidden, F = L->ffn, H = L->heads, hd = d / H;
    float *ws = (float *)workspace;
    float *qkv = ws + p.qkv, *ctx = ws + p.ctx, *sum = ws + p.sum, *y1 = ws + p.y1, *f = ws + p.f;

    const auto gemm = [&](float *o, const float *a, uint64_t k, const float *w, uint64_t n, int act, const float *bias,
                          const float *res) -> hipError_t {
        GemmLaunch g{};
        g.out = o;
        g.ldo = (int64_t)n;
        g.a = a;
        g.lda = (int64_t)k;
        g.b = w;
        g.ldb = (int64_t)k;
        g.m = (int32_t)T;
        g.n = (int32_t)n;
        g.k = (int32_t)k;
        g.n_rows_b = (int32_t)n;
        g.act = act;
        g.bias = bias;
        g.residual = res;
        g.ldr = (int64_t)n;
        return launch_gemm(g, stream);
    };
    const auto layer_norm = [&](const float *in, const float *w, const float *b, float *o) -> hipError_t {
        LayerNormLaunch l{};
        l.x = in;
        l.ldx = (int64_t)d;
        l.w = w;
        l.b = b;
        l.eps = L->ln_eps;
        l.rows = (int32_t)T;
        l.d = (int32_t)d;
        l.out = o;
        l.ldo = (int64_t)d;
        return launch_layer_norm(l, stream);
    };
    hipError_t e;
    if ((e = gemm(qkv, x, d, L->wqkv, 3 * d, RAYA_EPI_NONE, L->bqkv, nullptr)) != hipSuccess)
        return fail_device(e, "qkv gemm");
    AttnLaunch a{};
    a.q = qkv;
    a.k = qkv + d;
    a.v = qkv + 2 * d;
    a.out = ctx;
    a.valid_len = valid_len;
    a.q_bs = a.k_bs = a.v_bs = (int64_t)(L->seq * 3 * d);
    a.q_hs = a.k_hs = a.v_hs = a.o_hs = (int64_t)hd;
    a.q_rs = a.k_rs = a.v_rs = (int64_t)(3 * d);
    a.o_bs = (int64_t)(L->seq * d);
    a.o_rs = (int64_t)d;
    a.batch = (int32_t)L->batch;
    a.heads = (int32_t)H;
    a.seq = (int32_t)L->seq;
    a.head_dim = (int32_t)hd;
    a.mask_kind = L->mask_kind;
    a.mask_arg = (L->mask_kind == RAYA_MASK_SLIDING || L->mask_kind == RAYA_MASK_BLOCKDIAG)
                     ? (int32_t)(L->mask_arg < L->seq ? L->mask_arg : L->seq)
                     : 0;
    a.scale = 1.0f / sqrtf((float)hd);  // nn.MultiheadAttention's 1/sqrt(head_dim), AttnParams::new's default
    if ((e = launch_attention(a, stream)) != hipSuccess) return fail_device(e, "attention");
    if ((e = gemm(sum, ctx, d, L->wo, d, RAYA_EPI_NONE, L->bo, x)) != hipSuccess) return fail_device(e, "wo gemm");
    if ((e = layer_norm(sum, L->ln1_w, L->ln1_b, y1)) != hipSuccess) return fail_device(e, "layer norm 1");
    if ((e = gemm(f, y1, d, L->w1, F, RAYA_EPI_GELU, L->b1, nullptr)) != hipSuccess) return fail_device(e, "ffn in gemm");
    if ((e = gemm(sum, f, F, L->w2, d, RAYA_EPI_NONE, L->b2, y1)) != hipSuccess) return fail_device(e, "ffn out gemm");
    if ((e = layer_norm(sum, L->ln2_w, L->ln2_b, out)) != hipSuccess) return fail_device(e, "layer norm 2");
    return ok();
}

}  // extern "C"
