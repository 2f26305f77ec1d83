// C ABI of libraya_hip.so: argument validation with the reference's error
// semantics, the host-slice entry points that mirror the Rust traits, and the
// device-pointer entry points.
#include <hip/hip_runtime.h>

#include <cinttypes>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "internal.hpp"
#include "raya_hip.h"

namespace raya {

thread_local raya_error g_err = {RAYA_OK, {0}, 0, 0, {0}};

int fail(int code, const char *fmt, ...) {
    g_err.code = code;
    g_err.buffer[0] = 0;
    g_err.got = g_err.expected = 0;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err.message, sizeof g_err.message, fmt, ap);
    va_end(ap);
    return code;
}

// KernelError::Length, attention.rs:12-17: "buffer `q` has length 3, expected 32".
int fail_length(const char *name, uint64_t got, uint64_t expected) {
    fail(RAYA_ERR_LENGTH, "buffer `%s` has length %" PRIu64 ", expected %" PRIu64, name, got,
         expected);
    snprintf(g_err.buffer, sizeof g_err.buffer, "%s", name);
    g_err.got = got;
    g_err.expected = expected;
    return RAYA_ERR_LENGTH;
}

int fail_device(hipError_t e, const char *what) {
    return fail(RAYA_ERR_DEVICE, "device error: %s: %s", what, hipGetErrorString(e));
}

int ok() {
    g_err.code = RAYA_OK;
    g_err.buffer[0] = 0;
    g_err.got = g_err.expected = 0;
    g_err.message[0] = 0;
    return RAYA_OK;
}

namespace {

// validate() (attention.rs:128-158) in its order: shape, head_dim, valid_len,
// block.  The buffer lengths (attention.rs:159-168) come next, checked by the
// host-slice entry points, and only then the limits of the HIP kernel
// (check_hip_limits), which the reference has no counterpart for.
int check_attn(uint64_t heads, uint64_t head_dim, uint64_t seq, uint64_t block,
               const uint64_t *valid_len) {
    if (heads == 0 || head_dim == 0) return fail(RAYA_ERR_SHAPE, "invalid shape: heads and head_dim must be at least 1");
    if (head_dim % 8 != 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: head_dim %" PRIu64 " is not a multiple of 8", head_dim);
    if (valid_len && *valid_len > seq)
        return fail(RAYA_ERR_SHAPE, "invalid shape: valid_len %" PRIu64 " exceeds seq %" PRIu64, *valid_len, seq);
    if (block != RAYA_BLOCK)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: block %" PRIu64 " (only %d is supported)", block,
                    RAYA_BLOCK);
    return RAYA_OK;
}

// The mask extension and the kernel's instantiated limits.
int check_hip_limits(uint64_t heads, uint64_t seq, uint64_t head_dim, int32_t kind, uint64_t mask_arg) {
    if (kind < RAYA_MASK_BLOCK3 || kind > RAYA_MASK_BLOCKDIAG)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: mask kind %d", kind);
    if (kind == RAYA_MASK_BLOCKDIAG && mask_arg == 0)
        return fail(RAYA_ERR_SHAPE, "invalid shape: block_diag width must be at least 1");
    if (head_dim > (uint64_t)kMaxHeadDim)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: head_dim %" PRIu64 " (the HIP kernel handles up to %d)",
                    head_dim, kMaxHeadDim);
    if (seq >= (uint64_t(1) << 30))
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: seq %" PRIu64 " (the HIP kernel handles below 2^30)", seq);
    if (heads > 0x7fffffffu)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: %" PRIu64 " heads", heads);
    return RAYA_OK;
}

int32_t clamp_arg(int32_t kind, uint64_t mask_arg, uint64_t seq) {
    if (kind != RAYA_MASK_SLIDING && kind != RAYA_MASK_BLOCKDIAG) return 0;
    // Sliding(w >= seq) and BlockDiag(b >= seq) select the same keys as w = b = seq.
    const uint64_t c = mask_arg < seq ? mask_arg : (seq ? seq : 1);
    return (int32_t)c;
}

// One grow-only device workspace per device for the host-slice entry points.
struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
    hipStream_t stream = nullptr;
};
std::mutex g_ws_mutex;
std::unordered_map<int, Workspace> g_ws;

int workspace(size_t bytes, void **ptr, hipStream_t *stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_device(e, "hipGetDevice");
    Workspace &w = g_ws[dev];
    if (!w.stream) {
        e = hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking);
        if (e != hipSuccess) return fail_device(e, "hipStreamCreate");
    }
    if (w.bytes < bytes) {
        if (w.ptr) {
            e = hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
            if (e != hipSuccess) return fail_device(e, "hipFree");
        }
        e = hipMalloc(&w.ptr, bytes);
        if (e != hipSuccess) return fail_device(e, "hipMalloc");
        w.bytes = bytes;
    }
    *ptr = w.ptr;
    *stream = w.stream;
    return RAYA_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// The allocation-free host-slice entry point's staging area: four slots of
// RAYA_STATIC_ATTEND_MAX_NUMEL floats (q, k, v, out; 64 MiB in all) that each
// device holds from the library's load until the process ends.  Host code never
// uses the array's name as an address (on the host it is a stand-in symbol):
// the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kStaticSlotFloats = RAYA_STATIC_ATTEND_MAX_NUMEL;
static __device__ __align__(256) float scratch[4 * kStaticSlotFloats];

// One lock per device, held for a whole call: calls on one device run one at a time, calls on
// different devices (each with its own copy of the array) do not wait for each other.
constexpr int kMaxStaticDevices = 64;
std::mutex g_static_mutex[kMaxStaticDevices];
std::mutex g_static_ptr_mutex;  // guards g_static_ptr
std::unordered_map<int, float *> g_static_ptr;

// The current device, checked against the stream's (a stream of another device would stage
// into this device's array from that device's queue).
int static_device(hipStream_t stream, int *out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_device(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxStaticDevices)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: device %d is past the static array's %d devices", dev,
                    kMaxStaticDevices);
    if (stream) {
        hipDevice_t sdev = 0;
        e = hipStreamGetDevice(stream, &sdev);
        if (e != hipSuccess) return fail_device(e, "hipStreamGetDevice");
        if ((int)sdev != dev)
            return fail(RAYA_ERR_UNSUPPORTED, "unsupported: the stream belongs to device %d, the current device is %d",
                        (int)sdev, dev);
    }
    *out = dev;
    return RAYA_OK;
}

// The array's address on device `dev` (current), looked up once per device.
int static_scratch(int dev, float **ptr) {
    std::lock_guard<std::mutex> lock(g_static_ptr_mutex);
    auto it = g_static_ptr.find(dev);
    if (it == g_static_ptr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) return fail_device(e, "hipGetSymbolAddress(scratch)");
        it = g_static_ptr.emplace(dev, (float *)p).first;
    }
    *ptr = it->second;
    return RAYA_OK;
}

}  // namespace
}  // namespace raya

using namespace raya;

// raya_attend, and with `stages` (host) set raya_attend_with_stages: the
// device totals live in a 256-byte slot after the four operand slots.  With
// `fixed` set, raya_attend_static: the operands are staged in the static
// scratch array instead of the grow-only workspace, on the caller's stream.
static int attend_host(const raya_attn_shape *shape, const raya_attn_params *params, const float *q,
                       size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len,
                       float *out, size_t out_len, raya_stage_cycles *stages, bool fixed = false,
                       void *user_stream = nullptr) {
    if (!shape || !params) return fail(RAYA_ERR_SHAPE, "invalid shape: null shape or params");
    int rc = check_attn(shape->heads, shape->head_dim, shape->seq, params->block, &params->valid_len);
    if (rc) return rc;
    // AttnShape::numel (attention.rs:81-83); a product past 2^64 matches no buffer.
    uint64_t numel = 0;
    if (__builtin_mul_overflow(shape->heads, shape->seq, &numel) ||
        __builtin_mul_overflow(numel, shape->head_dim, &numel))
        return fail(RAYA_ERR_SHAPE, "invalid shape: heads x seq x head_dim overflows 64 bits");
    const struct {
        const char *name;
        size_t len;
    } bufs[4] = {{"q", q_len}, {"k", k_len}, {"v", v_len}, {"out", out_len}};
    for (const auto &bf : bufs)
        if (bf.len != numel) return fail_length(bf.name, bf.len, numel);
    rc = check_hip_limits(shape->heads, shape->seq, shape->head_dim, params->mask_kind, params->mask_arg);
    if (rc) return rc;
    if (fixed && numel > kStaticSlotFloats)
        return fail(RAYA_ERR_UNSUPPORTED,
                    "unsupported: heads x seq x head_dim = %" PRIu64 " exceeds the static workspace (%d floats per buffer)",
                    numel, RAYA_STATIC_ATTEND_MAX_NUMEL);
    if (stages) *stages = raya_stage_cycles{};
    if (numel == 0) return ok();
    if (!q || !k || !v || !out) return fail(RAYA_ERR_SHAPE, "invalid shape: null buffer");

    int static_dev = 0;
    if (fixed && (rc = static_device((hipStream_t)user_stream, &static_dev))) return rc;
    std::lock_guard<std::mutex> lock(fixed ? g_static_mutex[static_dev] : g_ws_mutex);
    void *base = nullptr;
    hipStream_t stream = nullptr;
    const size_t bytes = numel * sizeof(float);
    size_t slot = (bytes + 255) / 256 * 256;
    if (fixed) {
        float *sp = nullptr;
        rc = static_scratch(static_dev, &sp);
        if (rc) return rc;
        base = sp;
        slot = kStaticSlotFloats * sizeof(float);
        stream = (hipStream_t)user_stream;
    } else {
        rc = workspace(4 * slot + (stages ? 256 : 0), &base, &stream);
        if (rc) return rc;
    }
    char *p = (char *)base;
    float *dq = (float *)p, *dk = (float *)(p + slot), *dv = (float *)(p + 2 * slot),
          *dout = (float *)(p + 3 * slot);
    hipError_t e;
    if ((e = hipMemcpyAsync(dq, q, bytes, hipMemcpyHostToDevice, stream)) != hipSuccess ||
        (e = hipMemcpyAsync(dk, k, bytes, hipMemcpyHostToDevice, stream)) != hipSuccess ||
        (e = hipMemcpyAsync(dv, v, bytes, hipMemcpyHostToDevice, stream)) != hipSuccess)
        return fail_device(e, "hipMemcpy host to device");

    AttnLaunch a{};
    a.q = dq;
    a.k = dk;
    a.v = dv;
    a.out = dout;
    a.valid_len = nullptr;
    a.valid_scalar = (int32_t)params->valid_len;
    const int64_t hs = (int64_t)(shape->seq * shape->head_dim), rs = (int64_t)shape->head_dim;
    a.q_bs = a.k_bs = a.v_bs = a.o_bs = 0;
    a.q_hs = a.k_hs = a.v_hs = a.o_hs = hs;
    a.q_rs = a.k_rs = a.v_rs = a.o_rs = rs;
    a.batch = 1;
    a.heads = (int32_t)shape->heads;
    a.seq = (int32_t)shape->seq;
    a.head_dim = (int32_t)shape->head_dim;
    a.mask_kind = params->mask_kind;
    a.mask_arg = clamp_arg(params->mask_kind, params->mask_arg, shape->seq);
    a.scale = params->scale;
    if (stages) {
        a.stage_cycles = (raya_stage_cycles *)(p + 4 * slot);
        if ((e = hipMemsetAsync(a.stage_cycles, 0, sizeof(raya_stage_cycles), stream)) != hipSuccess)
            return fail_device(e, "hipMemsetAsync");
    }
    if ((e = launch_attention(a, stream)) != hipSuccess) return fail_device(e, "attention launch");
    if ((e = hipMemcpyAsync(out, dout, bytes, hipMemcpyDeviceToHost, stream)) != hipSuccess)
        return fail_device(e, "hipMemcpy device to host");
    if (stages && (e = hipMemcpyAsync(stages, a.stage_cycles, sizeof(raya_stage_cycles),
                                      hipMemcpyDeviceToHost, stream)) != hipSuccess)
        return fail_device(e, "hipMemcpy device to host");
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return fail_device(e, "hipStreamSynchronize");
    return ok();
}

extern "C" {

const raya_error *raya_last_error(void) { return &g_err; }

const char *raya_attention_name(void) { return "hip-gfx950"; }

const char *raya_gemm_name(void) { return "hip-gfx950-mfma"; }

#ifndef RAYA_BUILD_COMPILER
#define RAYA_BUILD_COMPILER "unknown"
#endif
#ifndef RAYA_BUILD_COMMIT
#define RAYA_BUILD_COMMIT "unknown"
#endif
#ifndef RAYA_BUILD_FLAGS
#define RAYA_BUILD_FLAGS "unknown"
#endif

const char *raya_build_info(void) {
    return "arch=gfx950\ncompiler=" RAYA_BUILD_COMPILER "\ncommit=" RAYA_BUILD_COMMIT "\nflags=" RAYA_BUILD_FLAGS;
}

int raya_attend(const raya_attn_shape *shape, const raya_attn_params *params, const float *q,
                size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len,
                float *out, size_t out_len) {
    return attend_host(shape, params, q, q_len, k, k_len, v, v_len, out, out_len, nullptr);
}

int raya_attend_static(const raya_attn_shape *shape, const raya_attn_params *params, const float *q,
                       size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len, float *out,
                       size_t out_len, void *stream) {
    return attend_host(shape, params, q, q_len, k, k_len, v, v_len, out, out_len, nullptr, true, stream);
}

int raya_attend_with_stages(const raya_attn_shape *shape, const raya_attn_params *params,
                            const float *q, size_t q_len, const float *k, size_t k_len,
                            const float *v, size_t v_len, float *out, size_t out_len,
                            raya_stage_cycles *stages) {
    if (!stages) return fail(RAYA_ERR_SHAPE, "invalid shape: null stages");
    return attend_host(shape, params, q, q_len, k, k_len, v, v_len, out, out_len, stages);
}

namespace {

int attend_batched(const raya_attn_batch *d, const int32_t *valid_len, const float *q, const float *k,
                   const float *v, float *out, raya_stage_cycles *stages, void *stream) {
    if (!d) return fail(RAYA_ERR_SHAPE, "invalid shape: null descriptor");
    int rc = check_attn(d->heads, d->head_dim, d->seq, d->block, nullptr);
    if (!rc) rc = check_hip_limits(d->heads, d->seq, d->head_dim, d->mask_kind, d->mask_arg);
    if (rc) return rc;
    if (d->batch > 0x7fffffffu) return fail(RAYA_ERR_UNSUPPORTED, "unsupported: batch %" PRIu64, d->batch);
    if (d->batch == 0 || d->seq == 0) return ok();
    if (!valid_len || !q || !k || !v || !out)
        return fail(RAYA_ERR_SHAPE, "invalid shape: null device pointer");
    const raya_attn_layout *lay[4] = {&d->q, &d->k, &d->v, &d->out};
    const void *ptrs[4] = {q, k, v, out};
    const char *names[4] = {"q", "k", "v", "out"};
    int64_t st[4][3];
    for (int i = 0; i < 4; ++i) {
        const raya_attn_layout &L = *lay[i];
        if (L.batch_stride == 0 && L.head_stride == 0 && L.row_stride == 0) {
            st[i][2] = (int64_t)d->head_dim;
            st[i][1] = (int64_t)(d->seq * d->head_dim);
            st[i][0] = (int64_t)(d->heads * d->seq * d->head_dim);
        } else {
            st[i][0] = L.batch_stride;
            st[i][1] = L.head_stride;
            st[i][2] = L.row_stride;
        }
        if (!aligned16(ptrs[i]) || (st[i][0] & 3) || (st[i][1] & 3) || (st[i][2] & 3) ||
            st[i][0] < 0 || st[i][1] < 0 || st[i][2] < 0)
            return fail(RAYA_ERR_UNSUPPORTED,
                        "unsupported: `%s` needs a 16-byte aligned pointer and non-negative strides that are "
                        "multiples of 4 floats",
                        names[i]);
    }
    AttnLaunch a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.valid_len = valid_len;
    a.valid_scalar = 0;
    a.q_bs = st[0][0], a.q_hs = st[0][1], a.q_rs = st[0][2];
    a.k_bs = st[1][0], a.k_hs = st[1][1], a.k_rs = st[1][2];
    a.v_bs = st[2][0], a.v_hs = st[2][1], a.v_rs = st[2][2];
    a.o_bs = st[3][0], a.o_hs = st[3][1], a.o_rs = st[3][2];
    a.batch = (int32_t)d->batch;
    a.heads = (int32_t)d->heads;
    a.seq = (int32_t)d->seq;
    a.head_dim = (int32_t)d->head_dim;
    a.mask_kind = d->mask_kind;
    a.mask_arg = clamp_arg(d->mask_kind, d->mask_arg, d->seq);
    a.scale = d->scale;
    a.stage_cycles = stages;
    const hipError_t e = launch_attention(a, (hipStream_t)stream);
    if (e != hipSuccess) return fail_device(e, "attention launch");
    return ok();
}

}  // namespace

int raya_attend_batched(const raya_attn_batch *d, const int32_t *valid_len, const float *q,
                        const float *k, const float *v, float *out, void *stream) {
    return attend_batched(d, valid_len, q, k, v, out, nullptr, stream);
}

int raya_attend_batched_stages(const raya_attn_batch *d, const int32_t *valid_len, const float *q,
                               const float *k, const float *v, float *out, raya_stage_cycles *stages,
                               void *stream) {
    if (!stages || ((uintptr_t)stages & 7))
        return fail(RAYA_ERR_SHAPE, "invalid shape: `stages` must be an 8-byte aligned device pointer");
    return attend_batched(d, valid_len, q, k, v, out, stages, stream);
}

int raya_matmul_nt(float *out, size_t out_len, const float *a, size_t a_len, const float *b,
                   size_t b_len, uint64_t m, uint64_t n, uint64_t k) {
    // The reference asserts these three lengths in this order (gemm.rs:23-25).
    if (a_len != m * k) {
        fail_length("a", a_len, m * k);
        snprintf(g_err.message, sizeof g_err.message, "a must be [m, k]");
        return RAYA_ERR_LENGTH;
    }
    if (b_len != n * k) {
        fail_length("b", b_len, n * k);
        snprintf(g_err.message, sizeof g_err.message, "b must be [n, k]");
        return RAYA_ERR_LENGTH;
    }
    if (out_len != m * n) {
        fail_length("out", out_len, m * n);
        snprintf(g_err.message, sizeof g_err.message, "out must be [m, n]");
        return RAYA_ERR_LENGTH;
    }
    if (m == 0 || n == 0) return ok();
    if (k == 0) {  // an empty sum: out is overwritten with zeros (gemm_reference.rs:19-22)
        memset(out, 0, sizeof(float) * m * n);
        return ok();
    }
    if (m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: gemm dimension above 2^31");
    if (!out || !a || !b) return fail(RAYA_ERR_SHAPE, "invalid shape: null buffer");

    std::lock_guard<std::mutex> lock(g_ws_mutex);
    const size_t sa = (m * k * sizeof(float) + 255) / 256 * 256;
    const size_t sb = (n * k * sizeof(float) + 255) / 256 * 256;
    const size_t so = m * n * sizeof(float);
    void *base = nullptr;
    hipStream_t stream = nullptr;
    int rc = workspace(sa + sb + so, &base, &stream);
    if (rc) return rc;
    char *p = (char *)base;
    float *da = (float *)p, *db = (float *)(p + sa), *dout = (float *)(p + sa + sb);
    hipError_t e;
    if ((e = hipMemcpyAsync(da, a, m * k * sizeof(float), hipMemcpyHostToDevice, stream)) != hipSuccess ||
        (e = hipMemcpyAsync(db, b, n * k * sizeof(float), hipMemcpyHostToDevice, stream)) != hipSuccess)
        return fail_device(e, "hipMemcpy host to device");
    GemmLaunch g{};
    g.out = dout;
    g.ldo = (int64_t)n;
    g.a = da;
    g.lda = (int64_t)k;
    g.b = db;
    g.ldb = (int64_t)k;
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.n_rows_b = (int32_t)n;
    g.act = RAYA_EPI_NONE;
    if ((e = launch_gemm(g, stream)) != hipSuccess) return fail_device(e, "gemm launch");
    if ((e = hipMemcpyAsync(out, dout, so, hipMemcpyDeviceToHost, stream)) != hipSuccess)
        return fail_device(e, "hipMemcpy device to host");
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return fail_device(e, "hipStreamSynchronize");
    return ok();
}

int raya_matmul_nt_device(float *out, int64_t ldo, const float *a, int64_t lda, const float *b,
                          int64_t ldb, uint64_t m, uint64_t n, uint64_t k,
                          const raya_gemm_epilogue *ep, void *stream) {
    const int act = ep ? ep->activation : RAYA_EPI_NONE;
    if (act < RAYA_EPI_NONE || act > RAYA_EPI_GEGLU || (ep && ep->reserved != 0))
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: epilogue activation %d", act);
    if (m > 0x7fffffffu || n > 0x3fffffffu || k > 0x7fffffffu)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: gemm dimension above 2^31");
    if (m == 0 || n == 0) return ok();
    const int64_t kk = (int64_t)k, nn = (int64_t)n;
    if (lda < kk || ldb < kk || ldo < nn || (ep && ep->residual && ep->ldr < nn))
        return fail(RAYA_ERR_SHAPE, "invalid shape: a leading dimension is smaller than the row length");
    if (!out || (k > 0 && (!a || !b))) return fail(RAYA_ERR_SHAPE, "invalid shape: null device pointer");
    GemmLaunch g{};
    g.out = out;
    g.ldo = ldo;
    g.a = a;
    g.lda = lda;
    g.b = b;
    g.ldb = ldb;
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.n_rows_b = act == RAYA_EPI_GEGLU ? (int32_t)(2 * n) : (int32_t)n;
    g.act = act;
    g.bias = ep ? ep->bias : nullptr;
    g.residual = ep ? ep->residual : nullptr;
    g.ldr = ep ? ep->ldr : 0;
    g.out_stats = ep ? (float4 *)ep->out_row_stats : nullptr;
    g.in_stats = ep ? (const float4 *)ep->in_row_stats : nullptr;
    g.colsum = ep ? ep->in_weight_sums : nullptr;
    if (g.in_stats && !g.colsum)
        return fail(RAYA_ERR_SHAPE, "invalid shape: in_row_stats needs in_weight_sums (raya_weight_row_sums)");
    if (g.out_stats || g.in_stats) {
        const auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
        const bool ring = k > 0 && k % 16 == 0 && lda % 4 == 0 && ldb % 4 == 0 && ldo % 4 == 0 && al(a) &&
                          al(b) && al(out) && (!g.residual || (g.ldr % 4 == 0 && al(g.residual)));
        if (!ring)
            return fail(RAYA_ERR_UNSUPPORTED,
                        "unsupported: row statistics need k a multiple of 16 and 16-byte aligned rows");
        if (g.out_stats && (act == RAYA_EPI_GEGLU || n % 64 != 0))
            return fail(RAYA_ERR_UNSUPPORTED,
                        "unsupported: out_row_stats needs n a multiple of 64 and no GEGLU epilogue");
        if (!al(g.out_stats) || !al(g.in_stats) || ((uintptr_t)g.colsum & 3))
            return fail(RAYA_ERR_SHAPE, "invalid shape: row statistics must be 16-byte aligned");
    }
    const hipError_t e = launch_gemm(g, (hipStream_t)stream);
    if (e != hipSuccess) return fail_device(e, "gemm launch");
    return ok();
}

int raya_weight_row_sums(const float *b, int64_t ldb, uint64_t rows, uint64_t k, float *sums, void *stream) {
    if (rows > 0x7fffffffu || k > 0x7fffffffu) return fail(RAYA_ERR_UNSUPPORTED, "unsupported: dimension above 2^31");
    if (ldb < (int64_t)k) return fail(RAYA_ERR_SHAPE, "invalid shape: ldb is smaller than k");
    if (rows == 0) return ok();
    if (!sums || (k > 0 && !b)) return fail(RAYA_ERR_SHAPE, "invalid shape: null device pointer");
    const hipError_t e = launch_row_sums(b, ldb, (int)rows, (int)k, sums, (hipStream_t)stream);
    if (e != hipSuccess) return fail_device(e, "row sums launch");
    return ok();
}

int raya_row_norm_stats(const float *chunk_stats, uint64_t rows, uint64_t n, float eps, float *row_stats,
                        void *stream) {
    if (n == 0 || n % 64 != 0) return fail(RAYA_ERR_UNSUPPORTED, "unsupported: row width %llu is not a multiple of 64",
                                           (unsigned long long)n);
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(RAYA_ERR_SHAPE, "invalid shape: eps must be finite and >= 0");
    if (rows > 0x7fffffffu || n / 64 > 0x7fffffffu)
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: row statistics above 2^31 rows");
    if (rows == 0) return ok();
    if (!chunk_stats || !row_stats) return fail(RAYA_ERR_SHAPE, "invalid shape: null device pointer");
    const hipError_t e = launch_ln_stats((const float4 *)chunk_stats, (int)rows, (int)(n / 64), eps,
                                         (float4 *)row_stats, (hipStream_t)stream);
    if (e != hipSuccess) return fail_device(e, "row statistics launch");
    return ok();
}

}  // extern "C"
