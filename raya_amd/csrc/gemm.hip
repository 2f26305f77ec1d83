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
#include <algorithm>
#include <type_traits>

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

constexpr int kXcds = 8;     // workgroup i runs on XCD i mod 8, each with its own L2
constexpr int kGroupM = 8;   // row blocks walked together by the tile order

// Output tile of workgroup `bid`.  Each XCD takes a contiguous range of the
// tile sequence, and the sequence walks GROUP_M row blocks at a time, column
// by column, so a B column tile is reused GROUP_M times and the A row blocks of
// a group stay in that XCD's L2 while all of B streams past them.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = bid % kXcds, slot = bid / kXcds;
    const int t = xcd * per + min(xcd, rem) + slot;
    const int width = kGroupM * tiles_n;
    const int group = t / width, first = group * kGroupM;
    const int size = min(tiles_m - first, kGroupM);
    const int r = t - group * width;
    tm = first + r % size;
    tn = r / size;
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

// Epilogue shared by both kernels.  Register r of acc[i][j] is row
// wm + 32 i + 8 (r / 4) + 4 h + r % 4 and column wn + 32 j + li of the workgroup tile.
template <int ACT, bool ROPE>
__device__ __forceinline__ void epilogue(const GemmLaunch &g, const floatx16 (&acc)[2][2], int m0, int n0,
                                         int wm, int wn, int li, int h) {
    constexpr bool GEGLU = ACT == RAYA_EPI_GEGLU;
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

template <int ACT, bool VEC, bool ROPE>
__global__ void __launch_bounds__(kThreads) gemm_nt_kernel(const GemmLaunch g) {
    __shared__ __attribute__((aligned(16))) float As[BM * SA];
    __shared__ __attribute__((aligned(16))) float Bs[BN * SA];

    constexpr bool GEGLU = ACT == RAYA_EPI_GEGLU;
    constexpr int OUT_BN = GEGLU ? BN / 2 : BN;  // output columns per workgroup

    const int tiles_n = (g.n + OUT_BN - 1) / OUT_BN;
    const int tiles_m = (g.m + BM - 1) / BM;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
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

    epilogue<ACT, ROPE>(g, acc, m0, n0, wm, wn, li, h);
}


// The ring kernel: k a multiple of 16, 16-byte aligned operands with row
// strides a multiple of 4 floats.  Slabs of 16 k go from HBM straight into an
// LDS ring (global_load_lds_dwordx4, no staging registers) with one barrier per
// slab.  Two ring depths: 2 stages, one slab ahead of the MFMAs, 37 KB of LDS and
// at most 128 VGPRs, so 4 workgroups share a CU; or 3 stages, two slabs ahead,
// 48 KB and 3 workgroups per CU, for the split-K launches (short K loops on small
// grids) and the folded LayerNorm (whose centring needs more registers).  The DMA
// is issued from asm with explicit vmcnt waits: the compiler cannot tell the
// ring's stages apart and would otherwise wait for every DMA before each LDS read.
// Rows past m (or past b's rows) load a clamped in-range row; the epilogue drops them.
constexpr int RBK = 16;       // k per slab
constexpr int kTileFloats = BM * RBK;  // one operand tile of one stage (8 KB)

// 16-byte chunk c (0..3) of tile row r sits at chunk c ^ rswz(r) of the row:
// the rows of any 8 or 16 consecutive lanes then cover every bank group.
__device__ __forceinline__ int rswz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

typedef __attribute__((address_space(3))) void lds_ptr_t;

__device__ __forceinline__ void dma16(const float *src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(src) : "memory", "m0");
}

__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Sum over each 16-lane row of the wave with DPP moves (no LDS crossbar): lane
// pairs (quad_perm [1,0,3,2]), quads ([2,3,0,1]), then the row's halves of 8
// (row_half_mirror pairs quad 0 with 1 and 2 with 3) and the row (row_mirror
// pairs quad 0 with 3 and 1 with 2).  Every step adds the same two values in
// each lane of a pair, in the other order, and addition commutes, so all 16
// lanes hold the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    x += dpp<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp<0x141>(x);  // row_half_mirror
    x += dpp<0x140>(x);  // row_mirror
    return x;
}

// Epilogue through LDS, for out (and residual) with row strides a multiple of 4
// floats and 16-byte aligned bases.  Bias, activation and GeGLU are applied in the
// accumulator layout, as in epilogue(); each wave then writes its y rows to its own
// LDS area and reads them back row-major, so that RoPE reads its tables as float4,
// and the residual reads and the stores are float4 with 256-byte (GeGLU: 128-byte)
// row segments: a quarter of the store instructions of the accumulator layout.
// Staged row strides: lanes i and i + 32 of a write are 4 rows apart, and
// 4 * stride = 32 (mod 64) puts them on disjoint banks.
constexpr int kStageStride = 72;      // 64 columns per wave
constexpr int kStageStrideGlu = 40;   // 32 GeGLU output columns per wave
constexpr int kStageFloats = 32 * kStageStride;  // per wave: 32 rows at a time

//
// With g.in_stats, rownorm holds (rest, rstd) of the workgroup's 128 input rows,
// rest = (mean_hi - centre) + mean_lo the part of the mean the centring left (see
// norm_centre), and the accumulators are normalised first: y = rstd (acc - rest
// colsum).  With g.out_stats, each
// wave's 64 output columns are one chunk: the 16 lanes that hold a row reduce
// its sum to the chunk mean c (the same bits in every lane), then the deviations
// from c and their squares.
template <int ACT, bool ROPE, bool NORM, bool STATS>
__device__ __forceinline__ void epilogue_staged(const GemmLaunch &g, floatx16 (&acc)[2][2], int m0, int n0,
                                                int wm, int wn, int li, int h, int lane, float *stg,
                                                const float2 *rownorm, const float (&cs)[2]) {
    constexpr bool GEGLU = ACT == RAYA_EPI_GEGLU;
    static_assert(!(ROPE && STATS), "RoPE outputs carry no row statistics");
    constexpr int COLS = GEGLU ? 32 : 64;  // output columns of this wave
    constexpr int S = GEGLU ? kStageStrideGlu : kStageStride;
    constexpr int C4 = COLS / 4;           // float4 per staged row
    const int c0 = n0 + (GEGLU ? (wn >> 1) : wn);  // first output column of this wave
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float2 st = rownorm[wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3)];
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j][r] = st.y * (acc[i][j][r] - st.x * cs[j]);
            }
    }
    float bias[2] = {0.f, 0.f};
    if (g.bias) {
        if constexpr (GEGLU) {
            const int col = min(c0 + li, g.n - 1);
            bias[0] = g.bias[col];
            bias[1] = g.bias[g.n + col];
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) bias[j] = g.bias[min(c0 + 32 * j + li, g.n - 1)];
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int rr = 8 * (r >> 2) + 4 * h + (r & 3);
            // Without a bias the accumulator is used as it is (x + 0 would turn -0 into +0).
            if constexpr (GEGLU) {
                const float x = g.bias ? acc[i][0][r] + bias[0] : acc[i][0][r];
                const float gate = g.bias ? acc[i][1][r] + bias[1] : acc[i][1][r];
                stg[rr * S + li] = gelu_erf(x) * gate;
            } else {
                float y[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) y[j] = activate<ACT>(g.bias ? acc[i][j][r] + bias[j] : acc[i][j][r]);
                stg[rr * S + li] = y[0];
                stg[rr * S + 32 + li] = y[1];
            }
        }
        // LDS accesses of one wave complete in order: the reads below see the
        // writes above, and the next half's writes follow these reads.
        if constexpr (ROPE && !GEGLU) {
            // RoPE on row-major data: this wave's 64 columns are one head (n0 and wn are
            // multiples of 64), so a lane takes the 16-byte chunks c4 and c4 + 8 of a row,
            // columns c .. c + 3 and c + 32 .. c + 35 with c = 4 c4, and rotates each pair
            // at frequencies c .. c + 3: one float4 of each table per 8 outputs.  Bias and
            // activation came first, the residual comes after, as in epilogue().
            const bool rot = c0 < g.rope_cols;  // the q and k sections: whole heads
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int idx = t * 64 + lane, rr = idx >> 3, c4 = idx & 7;
                const int row = m0 + wm + 32 * i + rr;
                if (row >= g.m) continue;
                float4 x0 = *(const float4 *)&stg[rr * S + 4 * c4];
                float4 x1 = *(const float4 *)&stg[rr * S + 32 + 4 * c4];
                if (rot) {
                    const int64_t tb = (int64_t)g.positions[row] * (kRopeHeadDim / 2) + 4 * c4;
                    const float4 cs4 = *(const float4 *)(g.rope_cos + tb), sn4 = *(const float4 *)(g.rope_sin + tb);
                    const auto turn = [](float &a, float &b, float c, float sn) {
                        const float a0 = a, b0 = b;
                        a = __fsub_rn(__fmul_rn(a0, c), __fmul_rn(b0, sn));
                        b = __fadd_rn(__fmul_rn(b0, c), __fmul_rn(a0, sn));
                    };
                    turn(x0.x, x1.x, cs4.x, sn4.x);
                    turn(x0.y, x1.y, cs4.y, sn4.y);
                    turn(x0.z, x1.z, cs4.z, sn4.z);
                    turn(x0.w, x1.w, cs4.w, sn4.w);
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int col = c0 + 32 * half + 4 * c4;
                    if (col >= g.n) continue;
                    float4 v = half ? x1 : x0;
                    float *o = g.out + (int64_t)row * g.ldo + col;
                    const float *res = g.residual ? g.residual + (int64_t)row * g.ldr + col : nullptr;
                    if (col + 4 <= g.n) {
                        if (res) {
                            const float4 x = *(const float4 *)res;
                            v.x += x.x;
                            v.y += x.y;
                            v.z += x.z;
                            v.w += x.w;
                        }
                        *(float4 *)o = v;
                    } else {
                        const float e[4] = {v.x, v.y, v.z, v.w};
                        for (int q = 0; q < 4 && col + q < g.n; ++q) o[q] = res ? e[q] + res[q] : e[q];
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (int t = 0; t < 32 * C4 / 64; ++t) {
            const int idx = t * 64 + lane, rr = idx / C4, c4 = idx % C4;
            const int row = m0 + wm + 32 * i + rr, col = c0 + 4 * c4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < g.m && col < g.n) {
                v = *(const float4 *)&stg[rr * S + 4 * c4];
                float *o = g.out + (int64_t)row * g.ldo + col;
                const float *res = g.residual ? g.residual + (int64_t)row * g.ldr + col : nullptr;
                if (col + 4 <= g.n) {
                    if (res) {
                        const float4 x = *(const float4 *)res;
                        v.x += x.x;
                        v.y += x.y;
                        v.z += x.z;
                        v.w += x.w;
                    }
                    *(float4 *)o = v;
                } else {
                    const float e[4] = {v.x, v.y, v.z, v.w};
                    for (int q = 0; q < 4 && col + q < g.n; ++q) o[q] = res ? e[q] + res[q] : e[q];
                }
            }
            if constexpr (STATS && !GEGLU) {
                // n is a multiple of 64, so this wave's 64 columns are either all in range
                // (a chunk of the row) or all past n (a tile wider than the matrix: no chunk).
                if (c0 < g.n) {
                    const float c = row16_sum((v.x + v.y) + (v.z + v.w)) * (1.0f / 64.0f);
                    const float dx = v.x - c, dy = v.y - c, dz = v.z - c, dw = v.w - c;
                    const float r1 = row16_sum((dx + dy) + (dz + dw));
                    const float r2 = row16_sum((dx * dx + dy * dy) + (dz * dz + dw * dw));
                    if (c4 == 0 && row < g.m)
                        g.out_stats[(int64_t)row * (g.n / 64) + (c0 >> 6)] = make_float4(c, r1, r2, 0.0f);
                }
            }
        }
    }
}

// The folded LayerNorm's centre of an input row with statistics st = (mean_hi,
// mean_lo, rstd, 0): the row's A operands enter the product as x - centre.  A row
// within one standard deviation of zero (|mean| rstd <= 1) is not centred: the
// mean comes out afterwards as mean colsum, whose cancellation then costs at most
// about as much as the product's own rounding (mean_lo, below half a unit of
// mean_hi, is dropped there).  Rows further out are centred by mean_hi (exact for
// x within a factor 2 of it), so that only mean_lo colsum is subtracted
// afterwards.  A function of the row alone: a row's result does not depend on the
// rows it shares a workgroup with.
__device__ __forceinline__ float norm_centre(float4 st) { return fabsf(st.x) * st.z > 1.0f ? st.x : 0.0f; }

// NORM: the input rows' LayerNorm is folded in (GemmLaunch::in_stats); STATS:
// the output rows' chunk statistics are written (GemmLaunch::out_stats); DEEP: the
// 3-stage ring (taken with NORM too).
template <int ACT, bool ROPE, bool NORM = false, bool STATS = false, bool DEEP = false>
__global__ void __launch_bounds__(kThreads, NORM || DEEP ? 3 : 4) gemm_ring_kernel(const GemmLaunch g) {
    constexpr int RSTAGES = NORM || DEEP ? 3 : 2;
    // The ring, also the epilogue's staging and row statistics once the K loop is done.
    constexpr int kRingFloats = std::max(RSTAGES * 2 * kTileFloats, 4 * kStageFloats + 2 * BM);
    __shared__ __attribute__((aligned(16))) float ring[kRingFloats];  // 48 KB or 37 KB

    constexpr bool GEGLU = ACT == RAYA_EPI_GEGLU;
    constexpr int OUT_BN = GEGLU ? BN / 2 : BN;
    const int tiles_n = (g.n + OUT_BN - 1) / OUT_BN;
    const int tiles_m = (g.m + BM - 1) / BM;
    // Split-K: workgroups tile * S .. tile * S + S - 1 share one output tile (the
    // reducing launch: one workgroup per tile).
    const int S = g.splits > 1 ? g.splits : 1;
    const int tile = g.reduce ? (int)blockIdx.x : (int)blockIdx.x / S;
    const int split = (int)blockIdx.x - tile * S;
    int tm, tn;
    tile_of(tile, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * OUT_BN;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int li = lane & 31, h = lane >> 5;

    // This thread's DMA sources: slot q = (2 wave + j) 64 + lane holds stored
    // chunk q % 4 of tile row q / 4, i.e. data chunk (q % 4) ^ rswz(row).
    // Folded LayerNorm: the centres of the two A rows this lane reads out of LDS
    // (rows wm + li and wm + 32 + li of the tile).  The subtraction runs only in
    // workgroups where some row is centred (subtracting a centre of 0 is exact, so
    // the other rows are unchanged).
    float cen[2] = {0.f, 0.f};
    bool centre = false;
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < 2; ++i) cen[i] = norm_centre(g.in_stats[min(m0 + wm + 32 * i + li, g.m - 1)]);
        centre = __builtin_amdgcn_readfirstlane(__syncthreads_or(cen[0] != 0.f || cen[1] != 0.f)) != 0;
    }

    const float *asrc[2], *bsrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int q = (2 * wave + j) * 64 + lane;
        const int row = q >> 2, c = (q & 3) ^ rswz(q >> 2);
        asrc[j] = g.a + (int64_t)min(m0 + row, g.m - 1) * g.lda + 4 * c;
        int brow;
        if constexpr (GEGLU) {
            // Tile rows [64t, 64t + 32) are input columns, [64t + 32, 64t + 64) their gates.
            const int t = row >> 6, within = row & 63;
            const int col = min(n0 + 32 * t + (within & 31), g.n - 1);
            brow = within < 32 ? col : col + g.n;
        } else {
            brow = min(n0 + row, g.n_rows_b - 1);
        }
        bsrc[j] = g.b + (int64_t)brow * g.ldb + 4 * c;
    }
    const uint32_t ring_base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t *)ring);
    const int nk = g.k / RBK / S;  // this workgroup's slabs: split * nk .. split * nk + nk - 1
    const int slab0 = split * nk;
    const auto issue = [&](int slab, int stage) {
        const int k0 = (slab0 + slab) * RBK;
        const uint32_t sa = ring_base + (uint32_t)(stage * 2 * kTileFloats * 4);
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16(asrc[j] + k0, sa + (2 * wave + j) * 1024);
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16(bsrc[j] + k0, sa + kTileFloats * 4 + (2 * wave + j) * 1024);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    constexpr int kTile4 = BM * BN / 4, kWave4 = kTile4 / 4;
    if (g.reduce) {
        // The partials of this tile, summed in split order, a whole partial's 16 loads per
        // lane in flight at a time.
        const float4 *all = (const float4 *)g.partials + (int64_t)tile * S * kTile4 + wave * kWave4;
        float4 t[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) t[q] = all[q * 64 + lane];
        for (int s2 = 1; s2 < S; ++s2) {
            float4 u[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) u[q] = all[(int64_t)s2 * kTile4 + q * 64 + lane];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                t[q].x += u[q].x;
                t[q].y += u[q].y;
                t[q].z += u[q].z;
                t[q].w += u[q].w;
            }
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            floatx16 &x = acc[q >> 3][(q >> 2) & 1];
            const int r = 4 * (q & 3);
            x[r] = t[q].x;
            x[r + 1] = t[q].y;
            x[r + 2] = t[q].z;
            x[r + 3] = t[q].w;
        }
    } else {
      // The K loop, with (C) or without the A operands' centring: two copies, so that
      // the one without runs the plain kernel's schedule.
      const auto kloop = [&](auto centre_tag) {
        constexpr bool C = decltype(centre_tag)::value;
        issue(0, 0);
        if (RSTAGES == 3 && nk > 1) issue(1, 1);
        int stage = 0;
        for (int kt = 0; kt < nk; ++kt) {
            // Each wave issues 4 DMAs per slab.  3 stages: with slab kt + 1 in flight,
            // vmcnt(4) means slab kt has landed; 2 stages: slab kt is the only one in
            // flight.  The barrier makes that hold for every wave and retires the reads
            // of the stage the next issue goes into (slab kt - 1's).
            if (RSTAGES == 3 && kt + 1 < nk)
                asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            barrier_only();
            if constexpr (RSTAGES == 3) {
                if (kt + 2 < nk) issue(kt + 2, stage == 0 ? 2 : stage - 1);
            } else {
                if (kt + 1 < nk) issue(kt + 1, stage ^ 1);
            }
            // The slab's operand reads and MFMAs run at raised wave priority, so a
            // wave that has passed its barrier keeps the matrix core busy while the
            // other workgroups' waves wait at theirs: the workgroups of a CU
            // drift out of step instead of stalling together (+2-5% on the encoder
            // shapes against equal priority).
            __builtin_amdgcn_s_setprio(1);
            const float *As = ring + stage * 2 * kTileFloats, *Bs = As + kTileFloats;
#pragma unroll
            for (int kc = 0; kc < RBK / 4; kc += 2) {
                float4 av[2], bv[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int ra = wm + 32 * i + li, rb = wn + 32 * i + li;
                    av[i] = *(const float4 *)&As[ra * RBK + 4 * ((kc + h) ^ rswz(ra))];
                    bv[i] = *(const float4 *)&Bs[rb * RBK + 4 * ((kc + h) ^ rswz(rb))];
                    if constexpr (C) {
                        av[i].x -= cen[i];
                        av[i].y -= cen[i];
                        av[i].z -= cen[i];
                        av[i].w -= cen[i];
                    }
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(av[i][s], bv[j][s], acc[i][j]);
            }
            __builtin_amdgcn_s_setprio(0);
            stage = stage == RSTAGES - 1 ? 0 : stage + 1;
        }
      };
        if constexpr (NORM) {
            if (centre)
                kloop(std::true_type{});
            else
                kloop(std::false_type{});
        } else {
            kloop(std::false_type{});
        }
        if (S > 1) {
            // The partial tile goes out in the accumulator layout (each wave's 64 x 64 quadrant
            // as 16 lane-contiguous float4 rows); the reducing launch reads it back.
            float4 *mine = (float4 *)g.partials + ((int64_t)tile * S + split) * kTile4 + wave * kWave4;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const floatx16 &x = acc[q >> 3][(q >> 2) & 1];
                const int r = 4 * (q & 3);
                mine[q * 64 + lane] = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
            }
            return;
        }
    }
    const bool vec_out = (g.ldo & 3) == 0 && ((uintptr_t)g.out & 15) == 0 &&
                         (!g.residual || ((g.ldr & 3) == 0 && ((uintptr_t)g.residual & 15) == 0));
    if (vec_out) {
        __syncthreads();  // every wave's reads of the last slab are done: the ring is free
        // Folded LayerNorm: one row's (rest, rstd) per thread of the first half and the
        // weight rows' sums this lane's columns need (GemmLaunch::colsum), read after the
        // K loop so that they hold no registers there.
        float2 *rownorm = (float2 *)(ring + 4 * kStageFloats);
        float cs[2] = {0.f, 0.f};
        if constexpr (NORM) {
            if (tid < BM) {
                const float4 st = g.in_stats[min(m0 + tid, g.m - 1)];
                rownorm[tid] = make_float2((st.x - norm_centre(st)) + st.y, st.z);
            }
            const int c0 = n0 + (GEGLU ? (wn >> 1) : wn);
            if constexpr (GEGLU) {
                const int col = min(c0 + li, g.n - 1);
                cs[0] = g.colsum[col];
                cs[1] = g.colsum[g.n + col];
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) cs[j] = g.colsum[min(c0 + 32 * j + li, g.n - 1)];
            }
            __syncthreads();
        }
        epilogue_staged<ACT, ROPE, NORM, STATS>(g, acc, m0, n0, wm, wn, li, h, lane, ring + wave * kStageFloats,
                                                rownorm, cs);
    } else {
        epilogue<ACT, ROPE>(g, acc, m0, n0, wm, wn, li, h);
    }
}

template <int ACT>
hipError_t launch_act(const GemmLaunch &g, hipStream_t stream) {
    constexpr int OUT_BN = ACT == RAYA_EPI_GEGLU ? BN / 2 : BN;
    const int64_t tiles = (int64_t)((g.m + BM - 1) / BM) * ((g.n + OUT_BN - 1) / OUT_BN);
    if (tiles > 0x7fffffff / kThreads) return hipErrorInvalidValue;
    const bool vec = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && (((uintptr_t)g.a & 15) == 0) &&
                     (((uintptr_t)g.b & 15) == 0) && (g.k % 4 == 0);
    const bool ring_ok = vec && g.k % RBK == 0 && g.k > 0;
    const int splits = g.splits > 1 ? g.splits : 1;
    if (g.reduce || (splits > 1 && (!ring_ok || !g.partials || tiles > kGemmSplitMaxTiles || splits > 16 ||
                                    (g.k / RBK) % splits != 0)))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(tiles * splits)), block(kThreads);
    if (g.in_stats || g.out_stats) {
        // Only the ring kernel's staged epilogue carries them (see GemmLaunch).
        const bool vec_out = (g.ldo & 3) == 0 && ((uintptr_t)g.out & 15) == 0 &&
                             (!g.residual || ((g.ldr & 3) == 0 && ((uintptr_t)g.residual & 15) == 0));
        if (!ring_ok || !vec_out) return hipErrorInvalidValue;
        if (g.in_stats && !g.colsum) return hipErrorInvalidValue;
        if (g.out_stats && (ACT == RAYA_EPI_GEGLU || g.n % 64 != 0)) return hipErrorInvalidValue;
    }
    if constexpr (ACT == RAYA_EPI_NONE) {
        if (g.rope_cos && (g.rope_cols % kRopeHeadDim != 0 || g.rope_cols > g.n)) return hipErrorInvalidValue;
    } else if (g.rope_cos) {
        return hipErrorInvalidValue;
    }
    if (ring_ok) {
        constexpr bool NONE = ACT == RAYA_EPI_NONE;
        // Split-K launches (small grids, short K loops) take the 3-stage ring.
        const auto ring_depth = [&](const GemmLaunch &gg, dim3 gr, auto deep_tag) -> hipError_t {
            constexpr bool D = decltype(deep_tag)::value;
            if (gg.in_stats) {  // folded LayerNorm: QKV (with or without RoPE) and GeGLU
                if (gg.rope_cos)
                    hipLaunchKernelGGL((gemm_ring_kernel<ACT, NONE, true>), gr, block, 0, stream, gg);
                else
                    hipLaunchKernelGGL((gemm_ring_kernel<ACT, false, true>), gr, block, 0, stream, gg);
            } else if (gg.out_stats) {  // the residual GEMMs
                if constexpr (NONE)
                    hipLaunchKernelGGL((gemm_ring_kernel<ACT, false, false, true, D>), gr, block, 0, stream, gg);
                else
                    return hipErrorInvalidValue;
            } else if (gg.rope_cos) {
                hipLaunchKernelGGL((gemm_ring_kernel<ACT, NONE, false, false, D>), gr, block, 0, stream, gg);
            } else {
                hipLaunchKernelGGL((gemm_ring_kernel<ACT, false, false, false, D>), gr, block, 0, stream, gg);
            }
            return hipGetLastError();
        };
        const auto ring = [&](const GemmLaunch &gg, dim3 gr) -> hipError_t {
            return splits > 1 ? ring_depth(gg, gr, std::true_type{}) : ring_depth(gg, gr, std::false_type{});
        };
        hipError_t e = ring(g, grid);
        if (e != hipSuccess || splits == 1) return e;
        // Split-K: the partial tiles are complete when the first launch ends; one workgroup
        // per tile sums them and runs the epilogue.
        GemmLaunch r = g;
        r.reduce = 1;
        return ring(r, dim3((unsigned)tiles));
    }
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

// MI355X: 256 compute units, 3 ring-kernel workgroups each.  A launch of few tiles (few
// rows: one short sequence) runs each tile's K loop on one workgroup, whose slabs then wait
// on HBM one after another; splitting K fills the units' slots and shortens those chains,
// keeping at least 4 slabs (64 k) per workgroup.
constexpr int kWorkgroupSlots = 3 * 256;
constexpr int kMaxSplits = 8;

int gemm_splits(int m, int n, int k, int act) {
    const int out_bn = act == RAYA_EPI_GEGLU ? BN / 2 : BN;
    const int64_t tiles = (int64_t)((m + BM - 1) / BM) * ((n + out_bn - 1) / out_bn);
    if (m <= 0 || n <= 0 || k <= 0 || k % RBK != 0 || tiles > kGemmSplitMaxTiles) return 1;
    const int nk = k / RBK;
    int s = (int)std::min<int64_t>(kMaxSplits, kWorkgroupSlots / tiles);
    while (s > 1 && (nk % s != 0 || nk / s < 4)) --s;
    return s > 1 ? s : 1;
}

size_t gemm_split_floats(int m, int n, int act, int splits) {
    if (splits <= 1) return 0;
    const int out_bn = act == RAYA_EPI_GEGLU ? BN / 2 : BN;
    const size_t tiles = (size_t)((m + BM - 1) / BM) * ((n + out_bn - 1) / out_bn);
    return tiles * (size_t)splits * BM * BN;
}

hipError_t launch_fill_zero(float *out, int64_t ldo, int m, int n, hipStream_t stream) {
    const int64_t total = (int64_t)m * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, out,
                       ldo, m, n);
    return hipGetLastError();
}

}  // namespace raya
