// fp32 NT GEMM on gfx950 MFMA: out[m][n] = epilogue(sum_t a[m][t] * b[n][t]).
//
// The contraction is GemmBackend::matmul_nt (crates/raya-kernels/src/gemm.rs:2-11):
// a is [m, k] row-major, b is a Linear weight [n, k] row-major, so both
// operands are contiguous along k.  A workgroup of four waves owns a 128 x 128
// tile of out; each wave a 64 x 64 quadrant made of 2 x 2
// v_mfma_f32_32x32x2_f32 tiles.  K is walked in slabs of 32: the next slab is
// fetched from HBM into registers (16-byte loads) while the current one is
// multiplied out of LDS.
//
// Register layouts of v_mfma_f32_32x32x2_f32 (lane l, half h = l / 32):
//   A[i][k] in lane i + 32 k, B[k][j] in lane j + 32 k,
//   D[i][j] in lane j + 32 ((i / 4) % 2), register 4 (i / 8) + i % 4.
// Within each 8-wide chunk of k, half h takes k = 4h .. 4h + 3 over four
// consecutive MFMAs, so one 16-byte LDS read feeds four instructions.
//
// Epilogues (ops.rs:91-109 bias add, encoder.rs:139-146 GeGLU, head.rs:392
// ReLU, encoder.rs:132-134 residual add): y = acc + bias; y = act(y);
// out = y + residual.  For GeGLU the weight has 2n rows; a workgroup loads the
// "input" rows j and the "gate" rows n + j side by side so that both halves of
// an output element land in the same lane and register.  The plain epilogue can
// also apply rotary embedding (ops.rs:118-141) to the q and k sections of a
// packed QKV projection, so encoder::attend's split_qkv + rope_in_place pass
// (encoder.rs:36-71) is not needed.
#include "internal.hpp"

namespace raya {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int SA = BK + 4;  // LDS row stride: 16 rows x 16 B reads hit distinct bank quads
constexpr int kThreads = 256;

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

template <int ACT>
__device__ __forceinline__ float activate(float x) {
    if constexpr (ACT == RAYA_EPI_GELU) return gelu_erf(x);
    else if constexpr (ACT == RAYA_EPI_RELU) return fmaxf(x, 0.0f);
    else return x;
}

// Loads 4 consecutive k values of row `row` (zero outside [0, rows) x [0, k)).
template <bool VEC>
__device__ __forceinline__ float4 load4(const float *base, int64_t ld, int row, int rows, int kcol,
                                        int kdim) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row >= rows) return x;
    const float *p = base + (int64_t)row * ld + kcol;
    if constexpr (VEC) {
        if (kcol + 4 <= kdim) return *(const float4 *)p;
    }
    if (kcol + 0 < kdim) x.x = p[0];
    if (kcol + 1 < kdim) x.y = p[1];
    if (kcol + 2 < kdim) x.z = p[2];
    if (kcol + 3 < kdim) x.w = p[3];
    return x;
}

template <int ACT, bool VEC, bool ROPE>
__global__ void __launch_bounds__(kThreads) gemm_nt_kernel(const GemmLaunch g) {
    __shared__ __attribute__((aligned(16))) float As[BM * SA];
    __shared__ __attribute__((aligned(16))) float Bs[BN * SA];

    constexpr bool GEGLU = ACT == RAYA_EPI_GEGLU;
    constexpr int OUT_BN = GEGLU ? BN / 2 : BN;  // output columns per workgroup

    const int tiles_n = (g.n + OUT_BN - 1) / OUT_BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * BM;
    const int n0 = tn * OUT_BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 31, h = lane >> 5;

    // Global -> register staging: each thread moves 4 float4 of A and 4 of B
    // per slab; 8 threads cover one 32-float row.
    const int ld_row = tid >> 3, ld_col = (tid & 7) * 4;
    int brow[4];  // b row feeding LDS row ld_row + 32 i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = ld_row + 32 * i;  // LDS row of the B tile
        if constexpr (GEGLU) {
            // LDS rows [64c, 64c + 32) are input columns, [64c + 32, 64c + 64) the gates.
            const int c = r >> 6, within = r & 63;
            const int col = n0 + 32 * c + (within & 31);
            brow[i] = col < g.n ? ((within < 32) ? col : col + g.n) : g.n_rows_b;
        } else {
            brow[i] = n0 + r;
        }
    }

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float4 ra[4], rb[4];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] = load4<VEC>(g.a, g.lda, m0 + ld_row + 32 * i, g.m, k0 + ld_col, g.k);
            rb[i] = load4<VEC>(g.b, g.ldb, brow[i], g.n_rows_b, k0 + ld_col, g.k);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *(float4 *)&As[(ld_row + 32 * i) * SA + ld_col] = ra[i];
            *(float4 *)&Bs[(ld_row + 32 * i) * SA + ld_col] = rb[i];
        }
    };

    const int nk = (g.k + BK - 1) / BK;
    fetch(0);
    stash();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) fetch((kt + 1) * BK);
#pragma unroll
        for (int kc = 0; kc < BK; kc += 8) {
            float4 av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                av[i] = *(const float4 *)&As[(wm + 32 * i + li) * SA + kc + 4 * h];
                bv[i] = *(const float4 *)&Bs[(wn + 32 * i + li) * SA + kc + 4 * h];
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(av[i][s], bv[j][s], acc[i][j]);
            }
        }
        __syncthreads();
        if (kt + 1 < nk) {
            stash();
            __syncthreads();
        }
    }

    // Epilogue.  Register r of acc[i][j] is row wm + 32 i + 8 (r / 4) + 4 h + r % 4
    // and column wn + 32 j + li of the workgroup tile.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row >= g.m) continue;
            if constexpr (GEGLU) {
                const int col = n0 + (wn >> 1) + li;
                if (col >= g.n) continue;
                float x = acc[i][0][r], gate = acc[i][1][r];
                if (g.bias) {
                    x += g.bias[col];
                    gate += g.bias[g.n + col];
                }
                float y = gelu_erf(x) * gate;
                if (g.residual) y += g.residual[(int64_t)row * g.ldr + col];
                g.out[(int64_t)row * g.ldo + col] = y;
            } else {
                float y[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn + 32 * j + li;
                    y[j] = acc[i][j][r];
                    if (g.bias && col < g.n) y[j] += g.bias[col];
                    y[j] = activate<ACT>(y[j]);
                }
                if constexpr (ROPE) {
                    // Columns c and c + 32 of one 64-wide head sit in the same lane
                    // and register of acc[i][0] and acc[i][1].
                    const int col0 = n0 + wn + li;
                    if (col0 < g.rope_cols) {
                        const int64_t t = (int64_t)g.positions[row] * (kRopeHeadDim / 2) + li;
                        const float c = g.rope_cos[t], sn = g.rope_sin[t];
                        const float x0 = y[0], x1 = y[1];
                        y[0] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
                        y[1] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, sn));
                    }
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn + 32 * j + li;
                    if (col >= g.n) continue;
                    float v = y[j];
                    if (g.residual) v += g.residual[(int64_t)row * g.ldr + col];
                    g.out[(int64_t)row * g.ldo + col] = v;
                }
            }
        }
    }
}

template <int ACT>
hipError_t launch_act(const GemmLaunch &g, hipStream_t stream) {
    constexpr int OUT_BN = ACT == RAYA_EPI_GEGLU ? BN / 2 : BN;
    const int64_t tiles = (int64_t)((g.m + BM - 1) / BM) * ((g.n + OUT_BN - 1) / OUT_BN);
    if (tiles > 0x7fffffff / kThreads) return hipErrorInvalidValue;
    const bool vec = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && (((uintptr_t)g.a & 15) == 0) &&
                     (((uintptr_t)g.b & 15) == 0) && (g.k % 4 == 0);
    const dim3 grid((unsigned)tiles), block(kThreads);
    if constexpr (ACT == RAYA_EPI_NONE) {
        if (g.rope_cos) {
            // The pairing (c, c + 32) needs 64-wide heads aligned to the 64-column wave tiles.
            if (g.rope_cols % kRopeHeadDim != 0 || g.rope_cols > g.n) return hipErrorInvalidValue;
            if (vec)
                hipLaunchKernelGGL((gemm_nt_kernel<ACT, true, true>), grid, block, 0, stream, g);
            else
                hipLaunchKernelGGL((gemm_nt_kernel<ACT, false, true>), grid, block, 0, stream, g);
            return hipGetLastError();
        }
    } else if (g.rope_cos) {
        return hipErrorInvalidValue;
    }
    if (vec)
        hipLaunchKernelGGL((gemm_nt_kernel<ACT, true, false>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((gemm_nt_kernel<ACT, false, false>), grid, block, 0, stream, g);
    return hipGetLastError();
}

__global__ void fill_zero_kernel(float *out, int64_t ldo, int m, int n) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)m * n) return;
    out[(idx / n) * ldo + idx % n] = 0.f;
}

}  // namespace

hipError_t launch_gemm(const GemmLaunch &g, hipStream_t stream) {
    if (g.m == 0 || g.n == 0) return hipSuccess;
    switch (g.act) {
    case RAYA_EPI_NONE: return launch_act<RAYA_EPI_NONE>(g, stream);
    case RAYA_EPI_GELU: return launch_act<RAYA_EPI_GELU>(g, stream);
    case RAYA_EPI_RELU: return launch_act<RAYA_EPI_RELU>(g, stream);
    case RAYA_EPI_GEGLU: return launch_act<RAYA_EPI_GEGLU>(g, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_fill_zero(float *out, int64_t ldo, int m, int n, hipStream_t stream) {
    const int64_t total = (int64_t)m * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, out,
                       ldo, m, n);
    return hipGetLastError();
}

}  // namespace raya
