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
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

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

// One work item: 64 query rows [q0, q0 + 64) of one (sequence, head) and the
// key interval [k_lo, k_hi) they attend (empty when every row is padding).
struct Item {
    int b, h, q0, valid, k_lo, k_hi;
};

__device__ __forceinline__ int clamp_valid(const AttnLaunch &a, int b) {
    const int valid = a.valid_len ? a.valid_len[b] : a.valid_scalar;
    return min(max(valid, 0), a.seq);
}

__device__ __forceinline__ Item make_item(const AttnLaunch &a, int b, int h, int tile, int valid) {
    Item it;
    it.b = b;
    it.h = h;
    it.q0 = tile * kQRows;
    it.valid = valid;
    if (it.q0 < valid) {
        const int qlast = min(it.q0 + kQRows, valid) - 1;
        it.k_lo = key_range(a.mask_kind, a.mask_arg, it.q0, valid).lo;
        it.k_hi = key_range(a.mask_kind, a.mask_arg, qlast, valid).hi;
    } else {
        it.k_lo = it.k_hi = 0;
    }
    return it;
}

// Item `item` of the (sequence, head, tile) order.
__device__ __forceinline__ Item decode(const AttnLaunch &a, int item, int n_qt) {
    const int tile = item % n_qt;
    const int bh = item / n_qt;
    const int b = bh / a.heads;
    return make_item(a, b, bh % a.heads, tile, clamp_valid(a, b));
}

// Largest b in [0, n) with heads * prefix[b] <= x (prefix[0] == 0, non-decreasing).
__device__ __forceinline__ int find_seq(const int *prefix, int n, int heads, int x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (heads * prefix[mid] <= x) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Waves per SIMD each head-dim instantiation is built for: the largest
// occupancy whose register budget holds the kernel without scratch spills.
template <int DP>
constexpr int kMinWaves = DP <= 32 ? 4 : DP == 64 ? 3 : DP == 48 || DP == 128 ? 2 : 1;

// Sequences a workgroup can schedule from LDS; larger batches take the
// one-workgroup-per-item launch.
constexpr int kMaxSeqs = 512;
// Work queues per launch and the spacing of their counters (ints): each
// counter sits on its own 128-byte line so claims on different queues do not
// serialise on one line.
constexpr int kQueues = 8;
constexpr int kQueueStride = 32;
constexpr int kQueueInts = (kQueues + 1) * kQueueStride;

// Persistent, software-pipelined kernel.
//
// Tiles of padded rows (q0 >= valid) are only zero-filled; they are spread
// statically over the grid.  The tiles with work are numbered 0..A-1 through
// per-sequence prefix sums built in LDS, permuted, split into kQueues
// contiguous ranges, and claimed one ahead of use from per-queue counters;
// a workgroup whose queue runs dry steals from the next ones.  So every
// workgroup stays busy until the work runs out however uneven the valid
// lengths are, and the counters see few enough claims not to serialise.
// While one K/V tile is multiplied out of LDS the loads of the next are in
// flight: the next key tile of the item, or the next item's first tile; the
// next item's Q goes into the Q registers as soon as the last S^T product of
// the current item has consumed them.  The last workgroup to finish zeroes
// the counters for the next launch on the same stream.  With queue ==
// nullptr the grid is one workgroup per item instead (no counters).
template <int DP>  // head_dim padded to a multiple of 16
__global__ void __launch_bounds__(kThreads, kMinWaves<DP>)
    attend_kernel(const AttnLaunch a, int total_items, int perm, int *queue) {
    constexpr int DQ = DP / 4;                   // head-dim slice owned by one lane group
    constexpr int NT = DP / 16;                  // 16-dim output tiles
    constexpr int SK = DP + 4;                   // K row stride in LDS: 16 rows hit 16 distinct bank quads
    constexpr int SV = DP;                       // V rows are read 16 lanes x NT floats contiguous
    constexpr int CH = DP / 4;                   // float4 chunks per row
    constexpr int PER = kKeys * CH / kThreads;  // K (and V) chunks staged per thread
    constexpr int RPI = kThreads / CH;           // rows between a thread's consecutive chunks
    __shared__ __attribute__((aligned(16))) float ks[kKeys * SK];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * SV];

    const int n_qt = (a.seq + kQRows - 1) / kQRows;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int li = lane & 15;
    const int D = a.head_dim;
    const int kind = a.mask_kind, arg = a.mask_arg;
    // exp(scale * (x - y)) = exp2((x - y) * c) on raw dot products x, y; a
    // negative scale is carried by negating Q, so c > 0 and max commutes.
    const float c_exp = fabsf(a.scale) * kLog2e;
    const float q_sign = a.scale < 0.f ? -1.f : 1.f;

    // Staging chunk i of this thread: row st_row(i), float4 column st_c4(i).
    // When CH divides the thread count every chunk of a thread is in the same
    // column and RPI rows apart.
    constexpr bool kEven = kThreads % CH == 0;
    auto st_row = [&](int i) { return kEven ? tid / CH + i * RPI : (i * kThreads + tid) / CH; };
    auto st_c4 = [&](int i) { return kEven ? tid % CH : (i * kThreads + tid) % CH; };

    auto zero_rows = [&](const Item &it) {
        const float *ob = a.out + (int64_t)it.b * a.o_bs + (int64_t)it.h * a.o_hs;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int r = it.q0 + st_row(i), c4 = st_c4(i);
            if (r < a.seq && 4 * c4 < D)
                *(float4 *)(const_cast<float *>(ob) + (int64_t)r * a.o_rs + 4 * c4) =
                    make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // --- Schedule -----------------------------------------------------------
    // s_act[b] / s_pad[b]: tiles with work / padded tiles of sequences < b.
    __shared__ int s_act[kMaxSeqs + 1];
    __shared__ int s_pad[kMaxSeqs + 1];
    __shared__ int s_claim;
    const int B = a.batch;
    int n_act = 0, n_pad = 0;  // per head, over the batch
    if (queue) {
        // Chunked exclusive scan over the batch (the K LDS tile is scratch here).
        int *part = reinterpret_cast<int *>(ks);
        const int per = (B + kThreads - 1) / kThreads;
        int sa = 0, sp = 0;
        for (int i = 0; i < per; ++i) {
            const int b = tid * per + i;
            if (b < B) {
                const int na = (clamp_valid(a, b) + kQRows - 1) / kQRows;
                sa += na;
                sp += n_qt - na;
            }
        }
        part[tid] = sa;
        part[kThreads + tid] = sp;
        __syncthreads();
        for (int off = 1; off < kThreads; off <<= 1) {
            const int xa = tid >= off ? part[tid - off] : 0;
            const int xp = tid >= off ? part[kThreads + tid - off] : 0;
            __syncthreads();
            part[tid] += xa;
            part[kThreads + tid] += xp;
            __syncthreads();
        }
        sa = part[tid] - sa;  // exclusive prefix of this thread's chunk
        sp = part[kThreads + tid] - sp;
        for (int i = 0; i < per; ++i) {
            const int b = tid * per + i;
            if (b < B) {
                s_act[b] = sa;
                s_pad[b] = sp;
                const int na = (clamp_valid(a, b) + kQRows - 1) / kQRows;
                sa += na;
                sp += n_qt - na;
            }
        }
        n_act = part[kThreads - 1];
        n_pad = part[2 * kThreads - 1];
        if (tid == 0) {
            s_act[B] = n_act;
            s_pad[B] = n_pad;
        }
        __syncthreads();
    }
    const int H = a.heads;
    const int total_act = H * n_act;
    // Permutation of the work indices (multiplier coprime to total_act near
    // total_act / golden ratio): consecutive claims get tiles far apart, so
    // every queue holds a fair mix of sequences and tile positions.
    int perm_act = 1;
    if (queue && total_act > 2) {
        perm_act = (int)(total_act * 0.6180339887498949f) | 1;
        for (;; perm_act += 2) {
            int x = perm_act, y = total_act;
            while (y) {
                const int t = x % y;
                x = y;
                y = t;
            }
            if (x == 1) break;
        }
    }

    // Padded tiles: zero-filled by a static share of the grid.
    if (queue) {
        for (int z = blockIdx.x; z < H * n_pad; z += gridDim.x) {
            const int b = find_seq(s_pad, B, H, z);
            const int np = s_pad[b + 1] - s_pad[b];
            const int r = z - H * s_pad[b];
            const int valid = clamp_valid(a, b);
            const int tile = (valid + kQRows - 1) / kQRows + r % np;
            zero_rows(make_item(a, b, r / np, tile, valid));
        }
    }

    // Tiles with work: queue q owns permuted indices [lo(q), lo(q + 1)).
    auto q_lo = [&](int q) { return (int)((int64_t)total_act * q / kQueues); };
    int cq = blockIdx.x % kQueues;  // thread 0: queue being drained
    int tried = 0;                  // thread 0: queues found empty
    int pending = 0;                // thread 0: claim in flight on queue cq
    if (queue && tid == 0) pending = atomicAdd(&queue[cq * kQueueStride], 1);
    bool first = true;              // one-workgroup-per-item mode: one item only
    // Next item with work, or -1.  All threads call it together.
    auto next_active = [&](Item &it) {
        if (!queue) {
            if (!first) return -1;
            first = false;
            it = decode(a, (int)((int64_t)blockIdx.x * perm % total_items), n_qt);
            if (it.k_lo < it.k_hi) return 0;
            zero_rows(it);
            return -1;
        }
        __syncthreads();  // every thread has read the previous claim
        if (tid == 0) {
            int res = -1;
            while (tried < kQueues) {
                const int x = q_lo(cq) + pending;
                if (x < q_lo(cq + 1)) {
                    res = x;
                    pending = atomicAdd(&queue[cq * kQueueStride], 1);
                    break;
                }
                cq = (cq + 1) % kQueues;
                ++tried;
                pending = atomicAdd(&queue[cq * kQueueStride], 1);
            }
            s_claim = res;
        }
        __syncthreads();
        const int x = s_claim;
        if (x < 0) return -1;
        const int t = (int)((int64_t)x * perm_act % total_act);
        const int b = find_seq(s_act, B, H, t);
        const int na = s_act[b + 1] - s_act[b];
        const int r = t - H * s_act[b];
        it = make_item(a, b, r / na, r % na, clamp_valid(a, b));
        return x;
    };

    float qreg[DQ];
    float4 kx[PER], vx[PER];
    // Q slice of this lane: row q0 + 16 wave + li, dims [g DQ, g DQ + DQ).
    auto fetch_q = [&](const Item &it) {
        const int qi = it.q0 + wave * 16 + li;
        const float *qp = a.q + (int64_t)it.b * a.q_bs + (int64_t)it.h * a.q_hs +
                          (int64_t)qi * a.q_rs + g * DQ;
        const bool row_ok = qi < it.valid;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row_ok && g * DQ + 4 * c < D) x = *(const float4 *)(qp + 4 * c);
            qreg[4 * c + 0] = x.x * q_sign;
            qreg[4 * c + 1] = x.y * q_sign;
            qreg[4 * c + 2] = x.z * q_sign;
            qreg[4 * c + 3] = x.w * q_sign;
        }
    };
    auto fetch_kv = [&](const Item &it, int kt) {
        const float *kb = a.k + (int64_t)it.b * a.k_bs + (int64_t)it.h * a.k_hs;
        const float *vb = a.v + (int64_t)it.b * a.v_bs + (int64_t)it.h * a.v_hs;
        const int kend = min(kt + kKeys, it.k_hi);
        if constexpr (kEven) {
            // One column per thread: walk the rows with pointer increments.
            const int c4 = tid % CH;
            const bool col_ok = 4 * c4 < D;
            const int j0 = kt + tid / CH;
            const float *kp = kb + (int64_t)j0 * a.k_rs + 4 * c4;
            const float *vp = vb + (int64_t)j0 * a.v_rs + 4 * c4;
            const int64_t ks_step = (int64_t)RPI * a.k_rs, vs_step = (int64_t)RPI * a.v_rs;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                if (j0 + i * RPI < kend && col_ok) {
                    kx[i] = *(const float4 *)(kp + i * ks_step);
                    vx[i] = *(const float4 *)(vp + i * vs_step);
                } else {
                    kx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    vx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int j = kt + st_row(i), c4 = st_c4(i);
                if (j < kend && 4 * c4 < D) {
                    kx[i] = *(const float4 *)(kb + (int64_t)j * a.k_rs + 4 * c4);
                    vx[i] = *(const float4 *)(vb + (int64_t)j * a.v_rs + 4 * c4);
                } else {
                    kx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    vx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
    };

    Item cur;
    int cur_item = next_active(cur);
    if (cur_item >= 0) {
        fetch_q(cur);
        fetch_kv(cur, cur.k_lo);
    }

    // LDS addresses of this lane's operands.
    const float *const k_op = &ks[(4 * (li & 3) + (li >> 2)) * SK + g * DQ];
    const float *const v_op = &vs[g * SV + NT * li];

    while (cur_item >= 0) {
        const int qw = cur.q0 + wave * 16;
        const int qi = qw + li;
        const int valid = cur.valid;
        const Range rr = qi < valid ? key_range(kind, arg, qi, valid) : Range{0, 0};
        const bool wave_live = qw < valid;
        const bool wave_full_rows = qw + 15 < valid;
        const Range w_first = key_range(kind, arg, min(qw, valid - 1), valid);
        const Range w_last = key_range(kind, arg, min(qw + 15, valid - 1), valid);

        floatx4 oacc[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) oacc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
        float m = -INFINITY;  // running max of raw dot products
        float l = 0.f;        // this lane's partial sum of weights

        Item nxt;
        int nxt_item = -1;
        for (int kt = cur.k_lo; kt < cur.k_hi; kt += kKeys) {
            __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                *(float4 *)&ks[st_row(i) * SK + 4 * st_c4(i)] = kx[i];
                *(float4 *)&vs[st_row(i) * SV + 4 * st_c4(i)] = vx[i];
            }
            __syncthreads();
            const bool last = kt + kKeys >= cur.k_hi;
            if (!last) {
                fetch_kv(cur, kt + kKeys);
            } else {
                nxt_item = next_active(nxt);
                if (nxt_item >= 0) fetch_kv(nxt, nxt.k_lo);
            }

            const bool work = wave_live && kt < w_last.hi && kt + kKeys > w_first.lo;
            floatx4 sacc[4];
            if (work) {
                // S^T tile t: A-row i is key kt + 16t + 4(i%4) + i/4.
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    sacc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
                    float kop[DQ];
#pragma unroll
                    for (int c = 0; c < DQ / 4; ++c) {
                        const float4 x = *(const float4 *)(k_op + 16 * t * SK + 4 * c);
                        kop[4 * c + 0] = x.x;
                        kop[4 * c + 1] = x.y;
                        kop[4 * c + 2] = x.z;
                        kop[4 * c + 3] = x.w;
                    }
#pragma unroll
                    for (int kk = 0; kk < DQ; ++kk) sacc[t] = mfma(kop[kk], qreg[kk], sacc[t]);
                }
            }
            if (last && nxt_item >= 0) fetch_q(nxt);  // Q registers are free from here on
            if (!work) continue;

            // Register (t, r) of lane (g, li) is the raw score of key
            // kt + 16t + 4r + g for query qi.
            if (!(wave_full_rows && kt >= w_last.lo && kt + kKeys <= w_first.hi)) {
                const int lo = rr.lo - kt - g, hi = rr.hi - kt - g;
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int j = 16 * t + 4 * r;
                        if (j < lo || j >= hi) sacc[t][r] = -INFINITY;
                    }
            }
            float tmax = sacc[0][0];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[t][r]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m, tmax);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            if (kt != cur.k_lo) {  // rescale what earlier tiles accumulated
                const float alpha = fast_exp2((m - m_use) * c_exp);
                l *= alpha;
#pragma unroll
                for (int n = 0; n < NT; ++n) oacc[n] *= alpha;
            }
            m = m_new;
            // The difference is formed before scaling, so the terms that carry
            // the weight (x near m) see no rounding from |x|.
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sacc[t][r] = fast_exp2((sacc[t][r] - m_use) * c_exp);
                    l += sacc[t][r];
                }

            // O^T tile n: A-row i is dim NT i + n, so one lane reads NT
            // contiguous floats of a V row for all n at once.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float *vp = v_op + (16 * t + 4 * r) * SV;
                    float vop[NT];
#pragma unroll
                    for (int n = 0; n < NT; ++n) vop[n] = vp[n];
#pragma unroll
                    for (int n = 0; n < NT; ++n) oacc[n] = mfma(vop[n], sacc[t][r], oacc[n]);
                }
            }
        }
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);

        // Register r of oacc[n] holds dim g DQ + NT r + n of row qi; rows at or
        // beyond valid hold zeros (every key was masked) and are stored as such.
        if (qi < a.seq) {
            const float inv = (qi < valid && l > 0.f) ? 1.f / l : 0.f;
            float *orow = a.out + (int64_t)cur.b * a.o_bs + (int64_t)cur.h * a.o_hs +
                          (int64_t)qi * a.o_rs + g * DQ;
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
        cur_item = nxt_item;
        cur = nxt;
    }

    // Sign off; the last workgroup resets the counter pair.  The fence waits
    // for this workgroup's outstanding claim, so once every workgroup has
    // signed off no claim can race with the reset.
    if (queue && tid == 0) {
        __threadfence();
        if (atomicAdd(&queue[kQueues * kQueueStride], 1) == (int)gridDim.x - 1) {
            for (int q = 0; q <= kQueues; ++q) atomicExch(&queue[q * kQueueStride], 0);
        }
    }
}

int gcd(int x, int y) {
    while (y) {
        const int t = x % y;
        x = y;
        y = t;
    }
    return x;
}

// Multiplier of the item permutation: near total / golden ratio and coprime
// to total, so consecutive claims get items far apart.
int item_permutation(int total) {
    int p = (int)(total * 0.6180339887498949) | 1;
    while (p > 1 && gcd(p, total) != 1) p += 2;
    return p < 1 ? 1 : p;
}

// Work-queue counters: one set (kQueues claim counters and a sign-off
// counter) per stream that launches the kernel, zero at module load and left
// at zero by every launch.  Launches on
// one stream are ordered, so they can share a pair; streams beyond
// kQueueSlots fall back to one workgroup per item.
constexpr int kQueueSlots = 64;
__device__ int g_queue[kQueueInts * kQueueSlots];

struct QueueSlots {
    std::mutex mu;
    std::map<int, int *> base;                           // device -> g_queue address
    std::map<std::pair<int, hipStream_t>, int> slot;     // (device, stream) -> pair index
    std::map<int, int> used;                             // device -> pairs handed out
    std::map<std::pair<int, int>, int> resident;         // (device, DP) -> workgroups per CU
};
QueueSlots g_slots;

template <int DP>
hipError_t launch_dp(const AttnLaunch &a, hipStream_t stream) {
    const int64_t n_qt = (a.seq + kQRows - 1) / kQRows;
    const int64_t total = n_qt * a.heads * a.batch;
    if (total > 0x7fffffff) return hipErrorInvalidValue;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int *queue = nullptr;
    int grid = (int)total;
    {
        std::lock_guard<std::mutex> lock(g_slots.mu);
        auto b = g_slots.base.find(dev);
        if (b == g_slots.base.end()) {
            void *p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_queue));
            if (e != hipSuccess) return e;
            b = g_slots.base.emplace(dev, (int *)p).first;
        }
        auto r = g_slots.resident.find({dev, DP});
        if (r == g_slots.resident.end()) {
            int cus = 0, per_cu = 0;
            e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            if (e == hipSuccess)
                e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attend_kernel<DP>, kThreads, 0);
            if (e != hipSuccess) return e;
            r = g_slots.resident.emplace(std::make_pair(dev, DP), std::max(1, cus * per_cu)).first;
        }
        auto sl = g_slots.slot.find({dev, stream});
        if (sl == g_slots.slot.end() && g_slots.used[dev] < kQueueSlots)
            sl = g_slots.slot.emplace(std::make_pair(dev, stream), g_slots.used[dev]++).first;
        if (sl != g_slots.slot.end() && a.batch <= kMaxSeqs) {
            queue = b->second + kQueueInts * sl->second;
            grid = (int)std::min<int64_t>(total, r->second);
        }
    }
    hipLaunchKernelGGL(attend_kernel<DP>, dim3(grid), dim3(kThreads), 0, stream, a, (int)total,
                       item_permutation((int)total), queue);
    return hipGetLastError();
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
