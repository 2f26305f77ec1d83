// Fused fp32 block-local attention for gfx950 (CDNA4).
//
// One workgroup computes 64 query rows of one (sequence, head): four waves of
// 16 rows each.  The keys the 64 rows may attend (the union of their
// key_range intervals, crates/raya-kernels/src/attention.rs:48-59) are walked
// in tiles of 64 keys.  Each K/V tile is read from HBM once per workgroup with
// 16-byte coalesced loads and staged in LDS; every wave then computes
//
//   S^T = K Q^T   on v_mfma_f32_16x16x4_f32  (16 keys x 16 queries per tile)
//   online softmax in registers (running max m and partial sums l, natural
//   units, exp(s - m) evaluated as exp2((s - m) log2 e))
//   O^T += V^T P^T on the same MFMA, P^T taken straight from the S^T registers
//
// Computing the transposed products puts each query in one lane column
// (lane % 16) of every accumulator, so the softmax statistics of a query live
// in the four lanes {q, q+16, q+32, q+48}: a row maximum needs two xor
// shuffles and the row sum is reduced once at the end.  Keys outside a row's
// interval (mask edges, key padding) are set to -inf in registers.  Rows at or
// beyond valid_len are written as exact zeros, as Naive::attend does
// (crates/raya-kernels/src/naive.rs:28-31).
//
// Register layouts of v_mfma_f32_16x16x4_f32 (lane l, group g = l / 16):
//   A[i][k] in lane i + 16 k, B[k][j] in lane j + 16 k,
//   D[i][j] in lane j + 16 (i / 4), register i % 4.
// The contraction index assigned to (lane group, step) is free as long as A
// and B agree; it is chosen so that every operand is a contiguous LDS or HBM
// read.
#include "internal.hpp"
#include "raya_hip.h"

namespace raya {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQRows = 16 * kWaves;  // query rows per workgroup
constexpr int kKeys = 64;            // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

struct Range {
    int lo, hi;
};

// Mask::key_range (attention.rs:48-59) plus BlockDiag, clipped to valid.
// mask_arg was clamped to seq by the host, so no sum below overflows int32
// for seq < 2^30.
__device__ __forceinline__ Range key_range(int kind, int arg, int i, int valid) {
    int lo, hi;
    switch (kind) {
    case RAYA_MASK_BLOCK3: {
        const int b = i >> 7;
        lo = (b > 0 ? b - 1 : 0) << 7;
        hi = (b + 2) << 7;
        break;
    }
    case RAYA_MASK_WINDOW64:
        lo = i > RAYA_WINDOW ? i - RAYA_WINDOW : 0;
        hi = i + RAYA_WINDOW + 1;
        break;
    case RAYA_MASK_FULL:
        lo = 0;
        hi = valid;
        break;
    case RAYA_MASK_SLIDING:
        lo = i > arg ? i - arg : 0;
        hi = i + arg + 1;
        break;
    default: {  // RAYA_MASK_BLOCKDIAG
        const int b = i / arg;
        lo = b * arg;
        hi = lo + arg;
        break;
    }
    }
    return {min(lo, valid), min(hi, valid)};
}

__device__ __forceinline__ floatx4 mfma(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int DP>  // head_dim padded to a multiple of 16
__global__ void __launch_bounds__(kThreads) attend_kernel(const AttnLaunch a, int wg_offset) {
    constexpr int DQ = DP / 4;   // head-dim slice owned by one lane group
    constexpr int NT = DP / 16;  // 16-dim output tiles
    constexpr int SK = DP + 4;   // K row stride in LDS: 16 rows hit 16 distinct bank quads
    constexpr int SV = DP;       // V rows are read 16 lanes x NT floats contiguous
    __shared__ __attribute__((aligned(16))) float ks[kKeys * SK];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * SV];

    const int n_qt = (a.seq + kQRows - 1) / kQRows;
    int wg = blockIdx.x + wg_offset;
    const int tile = wg % n_qt;
    wg /= n_qt;
    const int h = wg % a.heads;
    const int b = wg / a.heads;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int li = lane & 15;
    const int D = a.head_dim;
    const int kind = a.mask_kind, arg = a.mask_arg;

    int valid = a.valid_len ? a.valid_len[b] : a.valid_scalar;
    valid = min(max(valid, 0), a.seq);

    const float *qb = a.q + (int64_t)b * a.q_bs + (int64_t)h * a.q_hs;
    const float *kb = a.k + (int64_t)b * a.k_bs + (int64_t)h * a.k_hs;
    const float *vb = a.v + (int64_t)b * a.v_bs + (int64_t)h * a.v_hs;
    float *ob = a.out + (int64_t)b * a.o_bs + (int64_t)h * a.o_hs;

    const int q0 = tile * kQRows;
    const int qw = q0 + wave * 16;
    const int qi = qw + li;

    floatx4 oacc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) oacc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;
    float l = 0.f;

    if (q0 < valid) {  // workgroup-uniform: fully padded tiles only write zeros
        const int qlast = min(q0 + kQRows, valid) - 1;
        const int k_lo = key_range(kind, arg, q0, valid).lo;
        const int k_hi = key_range(kind, arg, qlast, valid).hi;

        const Range rr = qi < valid ? key_range(kind, arg, qi, valid) : Range{0, 0};
        const bool wave_live = qw < valid;
        const bool wave_full_rows = qw + 15 < valid;
        const Range w_first = key_range(kind, arg, min(qw, valid - 1), valid);
        const Range w_last = key_range(kind, arg, min(qw + 15, valid - 1), valid);

        // Q slice of this lane: row qi, dims [g*DQ, g*DQ + DQ).
        float qreg[DQ];
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            const int col = g * DQ + 4 * c;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (qi < valid && col < D) x = *(const float4 *)(qb + (int64_t)qi * a.q_rs + col);
            qreg[4 * c + 0] = x.x;
            qreg[4 * c + 1] = x.y;
            qreg[4 * c + 2] = x.z;
            qreg[4 * c + 3] = x.w;
        }

        for (int kt = k_lo; kt < k_hi; kt += kKeys) {
            __syncthreads();  // the previous tile's LDS reads are done
            const int kend = min(kt + kKeys, k_hi);
            constexpr int CH = DP / 4;
            for (int c = tid; c < kKeys * CH; c += kThreads) {
                const int row = c / CH, c4 = c % CH;
                const int j = kt + row;
                float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
                if (j < kend && 4 * c4 < D) {
                    kx = *(const float4 *)(kb + (int64_t)j * a.k_rs + 4 * c4);
                    vx = *(const float4 *)(vb + (int64_t)j * a.v_rs + 4 * c4);
                }
                *(float4 *)&ks[row * SK + 4 * c4] = kx;
                *(float4 *)&vs[row * SV + 4 * c4] = vx;
            }
            __syncthreads();

            if (!wave_live || kt >= w_last.hi || kt + kKeys <= w_first.lo) continue;
            const bool full = wave_full_rows && kt >= w_last.lo && kt + kKeys <= w_first.hi;

            // S^T tile t: rows are keys 16t + 4(i%4) + i/4 for A-row i.
            floatx4 sacc[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) sacc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int krow = 16 * t + 4 * (li & 3) + (li >> 2);
                const float *kp = &ks[krow * SK + g * DQ];
                float kop[DQ];
#pragma unroll
                for (int c = 0; c < DQ / 4; ++c) {
                    const float4 x = *(const float4 *)(kp + 4 * c);
                    kop[4 * c + 0] = x.x;
                    kop[4 * c + 1] = x.y;
                    kop[4 * c + 2] = x.z;
                    kop[4 * c + 3] = x.w;
                }
#pragma unroll
                for (int kk = 0; kk < DQ; ++kk) sacc[t] = mfma(kop[kk], qreg[kk], sacc[t]);
            }

            // Register (t, r) of lane (g, li) holds the score of key
            // kt + 16t + 4r + g for query qi.
            float p[4][4];
            float tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = kt + 16 * t + 4 * r + g;
                    float x = sacc[t][r] * a.scale;
                    if (!full && (j < rr.lo || j >= rr.hi)) x = -INFINITY;
                    p[t][r] = x;
                    tmax = fmaxf(tmax, x);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m, tmax);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            // exp(s - m) as exp2((s - m) log2 e): the difference is formed first, so
            // the terms that carry the weight (s near m) see no rounding from |s|.
            const float alpha = exp2f((m - m_use) * kLog2e);
            float psum = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[t][r] = exp2f((p[t][r] - m_use) * kLog2e);
                    psum += p[t][r];
                }
            }
            l = l * alpha + psum;
            m = m_new;
#pragma unroll
            for (int n = 0; n < NT; ++n) oacc[n] *= alpha;

            // O^T tile n: A-row i is dim NT*i + n, so one lane reads NT
            // contiguous floats of a V row for all n at once.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float *vp = &vs[(16 * t + 4 * r + g) * SV + NT * li];
                    float vop[NT];
#pragma unroll
                    for (int n = 0; n < NT; ++n) vop[n] = vp[n];
#pragma unroll
                    for (int n = 0; n < NT; ++n) oacc[n] = mfma(vop[n], p[t][r], oacc[n]);
                }
            }
        }
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
    }

    // Register r of oacc[n] holds dim g*DQ + NT*r + n of row qi.
    if (qi < a.seq) {
        const float inv = (qi < valid && l > 0.f) ? 1.f / l : 0.f;
        float *orow = ob + (int64_t)qi * a.o_rs + g * DQ;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            if (g * DQ + 4 * c < D) {
                float4 y;
                y.x = oacc[(4 * c + 0) % NT][(4 * c + 0) / NT] * inv;
                y.y = oacc[(4 * c + 1) % NT][(4 * c + 1) / NT] * inv;
                y.z = oacc[(4 * c + 2) % NT][(4 * c + 2) / NT] * inv;
                y.w = oacc[(4 * c + 3) % NT][(4 * c + 3) / NT] * inv;
                *(float4 *)(orow + 4 * c) = y;
            }
        }
    }
}

template <int DP>
hipError_t launch_dp(const AttnLaunch &a, hipStream_t stream) {
    const int64_t n_qt = (a.seq + kQRows - 1) / kQRows;
    const int64_t total = n_qt * a.heads * a.batch;
    constexpr int64_t kMaxGrid = int64_t(1) << 22;  // keep grid * 256 within 32 bits
    for (int64_t off = 0; off < total; off += kMaxGrid) {
        const int64_t n = total - off < kMaxGrid ? total - off : kMaxGrid;
        hipLaunchKernelGGL(attend_kernel<DP>, dim3((unsigned)n), dim3(kThreads), 0, stream, a,
                           (int)off);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_attention(const AttnLaunch &a, hipStream_t stream) {
    const int dp = (a.head_dim + 15) / 16 * 16;
    switch (dp) {
    case 16: return launch_dp<16>(a, stream);
    case 32: return launch_dp<32>(a, stream);
    case 48: return launch_dp<48>(a, stream);
    case 64: return launch_dp<64>(a, stream);
    case 80: return launch_dp<80>(a, stream);
    case 96: return launch_dp<96>(a, stream);
    case 112: return launch_dp<112>(a, stream);
    case 128: return launch_dp<128>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace raya
