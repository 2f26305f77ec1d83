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
// in the four lanes {q, q+16, q+32, q+48}: a row maximum needs two cross-lane
// steps (lanes i ^ 16, i ^ 32) and the row sum is reduced once at the end.  Keys outside a row's
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
#include <cstdlib>
#include <cstring>

#include "internal.hpp"
#include "raya_hip.h"

namespace raya {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQRows = 16 * kWaves;  // query rows per workgroup
constexpr int kSplitRows = 16;       // query rows per workgroup of the split kernel
constexpr int kKeys = 64;            // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

struct Range {
    int lo, hi;
};

// Exact division of n in [0, 2^31) by a divisor d fixed per launch:
// floor(n / d) = (n * m) >> s with s = 31 + ceil(log2 d), m = ceil(2^s / d),
// which fits 32 bits (the error n (m d - 2^s) / (d 2^s) stays below 1 / d).
struct FastDiv {
    uint32_t m, s;
};

FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint32_t s = 31 + l;
    return {(uint32_t)(((1ull << s) + d - 1) / d), s};
}

__device__ __forceinline__ int fdiv(int n, FastDiv f) {
    return (int)(((uint64_t)(uint32_t)n * f.m) >> f.s);
}

// Per-launch constants of the item decomposition.
struct Plan {
    int total, half_bits, n_qt;
    FastDiv by_qt, by_heads, by_arg;  // by_arg: the BlockDiag width (1 otherwise)
    int pairs_per_xcd;                 // > 0: whole (sequence, head) pairs per XCD
    int quads;                         // split kernel: each 4 consecutive items on one XCD (2: rotated)
    int rot_units, rot_shift;          // > 0: units of 2^rot_shift tiles dealt round the XCDs
    FastDiv by_rot;                    // by rot_units << rot_shift (items of a pair per XCD)
};

constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroup i runs on XCD i mod 8

// Row strides (floats) below which the balanced Window64 steps form their
// K/V offsets (up to 191 rows plus a row's last chunk) in 31 bits.
constexpr int64_t kMaxBalancedRowStride = (int64_t(1) << 31) / (4 * 3 * 64) - 64;

// Mask::key_range (attention.rs:48-59) plus BlockDiag, clipped to valid.
// mask_arg was clamped to seq by the host, so no sum below overflows int32
// for seq < 2^30.
__device__ __forceinline__ Range key_range(int kind, int arg, FastDiv by_arg, int i, int valid) {
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
        const int b = fdiv(i, by_arg);
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

// b is uniform, so the valid length comes through the scalar cache.
__device__ __forceinline__ int clamp_valid(const AttnLaunch &a, int b) {
    const int valid = a.valid_len ? a.valid_len[__builtin_amdgcn_readfirstlane(b)] : a.valid_scalar;
    return min(max(valid, 0), a.seq);
}

// Item `item` of the (sequence, head, tile) order, tiles of ROWS query rows.
// MK >= 0 fixes the mask kind at compile time (the launch has checked a.mask_kind).
template <int ROWS, int MK = -1>
__device__ __forceinline__ Item decode(const AttnLaunch &a, const Plan &p, int item) {
    const int kind = MK >= 0 ? MK : a.mask_kind;
    Item it;
    const int bh = fdiv(item, p.by_qt);
    const int tile = item - bh * p.n_qt;
    it.b = fdiv(bh, p.by_heads);
    it.h = bh - it.b * a.heads;
    it.q0 = tile * ROWS;
    it.valid = clamp_valid(a, it.b);
    if (it.q0 < it.valid) {
        const int qlast = min(it.q0 + ROWS, it.valid) - 1;
        it.k_lo = key_range(kind, a.mask_arg, p.by_arg, it.q0, it.valid).lo;
        it.k_hi = key_range(kind, a.mask_arg, p.by_arg, qlast, it.valid).hi;
    } else {
        it.k_lo = it.k_hi = 0;
    }
    return it;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane reductions over lanes i, i ^ 16 (resp. i ^ 32) without the LDS
// crossbar: v_permlane16_swap with both operands x swaps the odd 16-lane rows
// of one copy with the even rows of the other, so lane i of the two results
// holds x[i] and x[i ^ 16] in some order (likewise for 32-lane halves).
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int scatter(int i, int total, int half_bits);

// The item workgroup `bid` computes.  With rot_units > 0 (the 64-row kernels
// under Block3 and BlockDiag wider than a tile), each (sequence, head) pair's tiles
// form units of 2^rot_shift consecutive tiles dealt round the XCDs, rotated by
// the pair's index, and every XCD walks the pairs in order: each XCD holds an
// equal share of every pair's valid rows, and a unit's items share their key
// tiles in one L2.  Otherwise, when the number of pairs is a multiple of the
// XCD count, XCD x takes pairs x, x + 8, x + 16, ... and walks each one tile by
// tile: the workgroups running together on an XCD read neighbouring rows (DRAM
// pages stay open; overlapping key ranges of Block3 and Sliding hit in that
// XCD's L2), while the heads of each sequence, and with them its padding,
// spread over all XCDs.  Otherwise a scattered order.
//
// The split kernel's items are 16-row tiles: when the pairs do not divide
// among the XCDs, every four consecutive items (the 16-row tiles of one 64-row
// block, which share their key tiles) still go to one XCD, so that block's K/V
// is fetched into one L2 once rather than into four.  XCD x takes the k-th of
// each run of 8 such quads rotated by 2k (quads = 2): with 8 quads per
// (sequence, head) pair, XCD x would otherwise always take 64-row block x of
// every head, and under Block3 at L = 512 the blocks in the middle span 6 tiles
// and the outer ones 4, so XCDs 2-5 held 1.5 times the work of the others;
// rotated, every XCD takes all four even or all four odd blocks of every four
// heads.  (One sequence of 12 x 512 under Block3: 15.27 -> 15.13 us;
// RAYA_ATTN_QUADS=plain keeps the unrotated order.)
__device__ __forceinline__ int item_of(int bid, const Plan &p) {
    if (p.rot_units > 0) {  // n_qt = 8 rot_units 2^rot_shift
        const int x = bid % kXcds, s = bid / kXcds;
        const int pair = fdiv(s, p.by_rot);
        const int r = s - pair * (p.rot_units << p.rot_shift);
        const int unit = kXcds * (r >> p.rot_shift) + ((x - pair) & (kXcds - 1));
        return pair * p.n_qt + (unit << p.rot_shift) + (r & ((1 << p.rot_shift) - 1));
    }
    if (p.pairs_per_xcd > 0) {
        const int x = bid % kXcds, j = bid / kXcds;
        const int pj = fdiv(j, p.by_qt);
        return (pj * kXcds + x) * p.n_qt + (j - pj * p.n_qt);
    }
    if (p.quads) {  // total is a multiple of 4 * kXcds
        const int x = bid % kXcds, j = bid / kXcds, k = j >> 2;
        const int xr = p.quads > 1 ? (x + 2 * k) & (kXcds - 1) : x;
        return (k * kXcds + xr) * 4 + (j & 3);
    }
    return scatter(bid, p.total, p.half_bits);
}

// Bijection of [0, total), the fallback assignment of items to workgroups.
// The dispatcher places workgroup i on an XCD and shader engine by the low
// bits of i, so items taken in (sequence, head, tile) order, or through any
// affine map modulo total, would pin each tile position (and so each share of
// padding) to a fixed group of CUs.  A 4-round Feistel network over 2 *
// half_bits bits, cycle-walked back into [0, total), decorrelates them.
__device__ __forceinline__ int scatter(int i, int total, int half_bits) {
    const unsigned mask = (1u << half_bits) - 1u;
    unsigned x = (unsigned)i;
    do {
        unsigned lo = x & mask, hi = x >> half_bits;
#pragma unroll
        for (int round = 0; round < 4; ++round) {
            unsigned f = (lo + 0x9E3779B9u * (round + 1)) * 0x85EBCA6Bu;
            f ^= f >> 13;
            f *= 0xC2B2AE35u;
            f ^= f >> 16;
            const unsigned t = lo;
            lo = (hi ^ f) & mask;
            hi = t;
        }
        x = (hi << half_bits) | lo;
    } while (x >= (unsigned)total);
    return (int)x;
}

// Waves per SIMD each head-dim instantiation is built for: the largest
// occupancy whose register budget holds the kernel without scratch spills.
template <int DP>
constexpr int kMinWaves = DP <= 64 ? 4 : DP == 128 ? 2 : 1;
// The split kernel at head_dim 64 holds each tile's K/V subtile and the next one's in
// registers: 3 waves per SIMD (768 workgroup slots, more than the small grids it serves
// need at once).
template <int DP, bool SPLIT, bool FUSED>
constexpr int kMinWavesOf = SPLIT && FUSED ? 3 : kMinWaves<DP>;

typedef __attribute__((address_space(3))) void lds_ptr_t;

// The first tile's loads at head_dim 64, as one block the compiler cannot
// split: 4 K DMAs (16 bytes per lane each, LDS address in m0, source a scalar
// base plus a 32-bit per-lane byte offset), the lane's 4 Q chunks into
// registers, 4 V DMAs, then a wait until only the V DMAs may be outstanding
// (loads complete in issue order).  Written as one asm statement so
// that the compiler neither waits for the V DMA before reading the K tile (it
// cannot tell the two LDS tiles apart) nor touches q before the wait.
__device__ __forceinline__ void issue_kqv64(const float *kbase, const uint32_t ko[4], const uint32_t kl[4],
                                            const float *qa, floatx4 q[4], const float *vbase,
                                            const uint32_t vo[4], const uint32_t vl[4]) {
    asm volatile(
        "s_mov_b32 m0, %[kl0]\n\tglobal_load_lds_dwordx4 %[ko0], %[kb]\n\t"
        "s_mov_b32 m0, %[kl1]\n\tglobal_load_lds_dwordx4 %[ko1], %[kb]\n\t"
        "s_mov_b32 m0, %[kl2]\n\tglobal_load_lds_dwordx4 %[ko2], %[kb]\n\t"
        "s_mov_b32 m0, %[kl3]\n\tglobal_load_lds_dwordx4 %[ko3], %[kb]\n\t"
        "global_load_dwordx4 %[q0], %[qa], off\n\t"
        "global_load_dwordx4 %[q1], %[qa], off offset:16\n\t"
        "global_load_dwordx4 %[q2], %[qa], off offset:32\n\t"
        "global_load_dwordx4 %[q3], %[qa], off offset:48\n\t"
        "s_mov_b32 m0, %[vl0]\n\tglobal_load_lds_dwordx4 %[vo0], %[vb]\n\t"
        "s_mov_b32 m0, %[vl1]\n\tglobal_load_lds_dwordx4 %[vo1], %[vb]\n\t"
        "s_mov_b32 m0, %[vl2]\n\tglobal_load_lds_dwordx4 %[vo2], %[vb]\n\t"
        "s_mov_b32 m0, %[vl3]\n\tglobal_load_lds_dwordx4 %[vo3], %[vb]\n\t"
        "s_waitcnt vmcnt(4)"
        : [q0] "=&v"(q[0]), [q1] "=&v"(q[1]), [q2] "=&v"(q[2]), [q3] "=&v"(q[3])
        : [kb] "s"(kbase), [ko0] "v"(ko[0]), [ko1] "v"(ko[1]), [ko2] "v"(ko[2]), [ko3] "v"(ko[3]),
          [kl0] "s"(kl[0]), [kl1] "s"(kl[1]), [kl2] "s"(kl[2]), [kl3] "s"(kl[3]), [qa] "v"(qa),
          [vb] "s"(vbase), [vo0] "v"(vo[0]), [vo1] "v"(vo[1]), [vo2] "v"(vo[2]), [vo3] "v"(vo[3]),
          [vl0] "s"(vl[0]), [vl1] "s"(vl[1]), [vl2] "s"(vl[2]), [vl3] "s"(vl[3])
        : "memory", "m0");
}

// A later tile at head_dim 64: 4 K DMAs, 4 V DMAs, wait until only V may be
// outstanding.
__device__ __forceinline__ void issue_kv64(const float *kbase, const uint32_t ko[4], const uint32_t kl[4],
                                           const float *vbase, const uint32_t vo[4], const uint32_t vl[4]) {
    asm volatile(
        "s_mov_b32 m0, %[kl0]\n\tglobal_load_lds_dwordx4 %[ko0], %[kb]\n\t"
        "s_mov_b32 m0, %[kl1]\n\tglobal_load_lds_dwordx4 %[ko1], %[kb]\n\t"
        "s_mov_b32 m0, %[kl2]\n\tglobal_load_lds_dwordx4 %[ko2], %[kb]\n\t"
        "s_mov_b32 m0, %[kl3]\n\tglobal_load_lds_dwordx4 %[ko3], %[kb]\n\t"
        "s_mov_b32 m0, %[vl0]\n\tglobal_load_lds_dwordx4 %[vo0], %[vb]\n\t"
        "s_mov_b32 m0, %[vl1]\n\tglobal_load_lds_dwordx4 %[vo1], %[vb]\n\t"
        "s_mov_b32 m0, %[vl2]\n\tglobal_load_lds_dwordx4 %[vo2], %[vb]\n\t"
        "s_mov_b32 m0, %[vl3]\n\tglobal_load_lds_dwordx4 %[vo3], %[vb]\n\t"
        "s_waitcnt vmcnt(4)"
        :
        : [kb] "s"(kbase), [ko0] "v"(ko[0]), [ko1] "v"(ko[1]), [ko2] "v"(ko[2]), [ko3] "v"(ko[3]),
          [kl0] "s"(kl[0]), [kl1] "s"(kl[1]), [kl2] "s"(kl[2]), [kl3] "s"(kl[3]),
          [vb] "s"(vbase), [vo0] "v"(vo[0]), [vo1] "v"(vo[1]), [vo2] "v"(vo[2]), [vo3] "v"(vo[3]),
          [vl0] "s"(vl[0]), [vl1] "s"(vl[1]), [vl2] "s"(vl[2]), [vl3] "s"(vl[3])
        : "memory", "m0");
}

// Workgroup barrier without the memory fence of __syncthreads: the fence would
// wait for every outstanding LDS DMA (they count as LDS writes), including the
// V tile that is meant to stay in flight during QK^T.  Callers order memory
// themselves with explicit s_waitcnt; the clobber keeps the compiler from
// moving memory operations across.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// A non-temporal (streaming) 16-byte store: the output is not read again by this
// launch, and whole lines written this way bypass the allocate-and-merge path.
__device__ __forceinline__ void store_stream(float *p, float4 y) {
    __builtin_nontemporal_store(floatx4{y.x, y.y, y.z, y.w}, (floatx4 *)p);
}
// A barrier after which other waves' direct loads overwrite LDS this wave has
// read: its own LDS reads have returned first.
__device__ __forceinline__ void barrier_after_reads() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Chunk (16 bytes) c of K/V row r sits at chunk swz(c, r) of the row in LDS:
// an XOR swizzle within aligned groups of P chunks (P the largest power of two
// dividing the chunks per row, 16 at head_dim 64).  The 16 rows an S^T
// operand read touches and the 16 chunks a PV operand read touches then hit
// distinct bank groups without padding the rows.
template <int CH>
__device__ __forceinline__ int swz(int c, int r) {
    constexpr int P = (CH & -CH) < 16 ? (CH & -CH) : 16;
    return (c & ~(P - 1)) | ((c ^ r) & (P - 1));
}

// S^T of one 64-key tile against this lane's Q slice: register (t, r) of lane
// (g, li) becomes the raw score of key 16t + 4r + g of the tile (A-row i of
// subtile t is key 16t + 4(i%4) + i/4, so row k_row0 = 4(li%4) + li/4).
// Subtiles whose bit in `live` (wave-uniform) is clear are skipped and left at
// zero: the caller masks every key of them.
template <int DP>
__device__ __forceinline__ void qk_tile(const float *ks, const float (&qreg)[DP / 4], int g, int k_row0,
                                        floatx4 (&sacc)[4], int live = 0xF) {
    constexpr int DQ = DP / 4, CH = DP / 4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        sacc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (!((live >> t) & 1)) continue;
        const int row = 16 * t + k_row0;
        const float *kp = ks + row * DP;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            const float4 x = *(const float4 *)(kp + 4 * swz<CH>(g * (DQ / 4) + c, row));
            sacc[t] = mfma(x.x, qreg[4 * c + 0], sacc[t]);
            sacc[t] = mfma(x.y, qreg[4 * c + 1], sacc[t]);
            sacc[t] = mfma(x.z, qreg[4 * c + 2], sacc[t]);
            sacc[t] = mfma(x.w, qreg[4 * c + 3], sacc[t]);
        }
    }
}

// Masks scores outside [lo0, hi0) in the even subtiles and [lo1, hi1) in
// the odd ones (tile-relative, already offset by g) when need_mask, folds the
// tile into the running max m and partial sum l (rescaling oacc unless
// first), and turns the scores into weights.
template <int NT>
__device__ __forceinline__ void softmax_tile(floatx4 (&sacc)[4], floatx4 (&oacc)[NT], float &m, float &l,
                                             bool first, bool need_mask, int lo0, int hi0, int lo1, int hi1,
                                             float c_exp) {
    if (need_mask) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = 16 * t + 4 * r;
                if (j < (t & 1 ? lo1 : lo0) || j >= (t & 1 ? hi1 : hi0)) sacc[t][r] = -INFINITY;
            }
    }
    float tmax = sacc[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[t][r]);
    tmax = max_xor32(max_xor16(tmax));
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    if (!first) {  // rescale what earlier tiles accumulated
        const float alpha = fast_exp2((m - m_use) * c_exp);
        l *= alpha;
#pragma unroll
        for (int n = 0; n < NT; ++n) oacc[n] *= alpha;
    }
    m = m_new;
    // The difference is formed before scaling, so the terms that carry the
    // weight (x near m) see no rounding from |x|.
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sacc[t][r] = fast_exp2((sacc[t][r] - m_use) * c_exp);
            l += sacc[t][r];
        }
}

// O^T += V^T P^T for one tile.  O^T tile n: A-row i is dim NT i + n, so one
// lane reads NT contiguous floats of a V row for all n at once.  Subtiles clear
// in `live` hold only zero weights and are skipped.
template <int DP>
__device__ __forceinline__ void pv_tile(const float *vs, const floatx4 (&sacc)[4], int g, int li,
                                        floatx4 (&oacc)[DP / 16], int live = 0xF) {
    constexpr int NT = DP / 16, CH = DP / 4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (!((live >> t) & 1)) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * t + 4 * r + g;
            const float *vp = vs + row * DP;
            float vop[NT];
            if constexpr (NT == 4) {
                const float4 x = *(const float4 *)(vp + 4 * swz<CH>(li, row));
                vop[0] = x.x;
                vop[1] = x.y;
                vop[2] = x.z;
                vop[3] = x.w;
            } else {
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const int d = NT * li + n;
                    vop[n] = vp[4 * swz<CH>(d >> 2, row) + (d & 3)];
                }
            }
#pragma unroll
            for (int n = 0; n < NT; ++n) oacc[n] = mfma(vop[n], sacc[t][r], oacc[n]);
        }
    }
}

// Non-finite V under masks whose key ranges differ between the rows of a wave
// (Window64, Sliding, BlockDiag of a width that 16 does not divide).  A 16-key
// subtile cut by some row's range gives that row weight 0 at the keys outside
// it, and the matrix core multiplies those zeros by V: 0 * Inf is NaN where
// Naive::attend sums each row over its own range only (naive.rs:13-65).  Such a
// NaN can only appear in a row whose output is not finite, so under these masks
// each non-finite output chunk is recomputed here, in Naive's order and over the
// row's own key range: 4 dims d0 .. d0 + 3 of the row with Q row qrow, from HBM
// (the path only runs on non-finite inputs).  Scores are the dot product in dim
// order times the scale; the maximum ignores NaN scores as the reference's
// f32::max does, and a NaN or +Inf score makes the row NaN through the sum.
__device__ __forceinline__ float4 exact_chunk(const float *qrow, const float *kb, int64_t k_rs, const float *vb,
                                              int64_t v_rs, int lo, int hi, int D, float scale, int d0) {
    float mx = -INFINITY;
#pragma unroll 1
    for (int j = lo; j < hi; ++j) {
        const float *krow = kb + (int64_t)j * k_rs;
        float s = 0.f;
#pragma unroll 1
        for (int d = 0; d < D; ++d) s = __fadd_rn(s, __fmul_rn(qrow[d], krow[d]));
        mx = fmaxf(mx, __fmul_rn(s, scale));
    }
    float sum = 0.f;
#pragma unroll 1
    for (int j = lo; j < hi; ++j) {
        const float *krow = kb + (int64_t)j * k_rs;
        float s = 0.f;
#pragma unroll 1
        for (int d = 0; d < D; ++d) s = __fadd_rn(s, __fmul_rn(qrow[d], krow[d]));
        sum = __fadd_rn(sum, expf(__fmul_rn(s, scale) - mx));
    }
    float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int j = lo; j < hi; ++j) {
        const float *krow = kb + (int64_t)j * k_rs;
        float s = 0.f;
#pragma unroll 1
        for (int d = 0; d < D; ++d) s = __fadd_rn(s, __fmul_rn(qrow[d], krow[d]));
        const float w = expf(__fmul_rn(s, scale) - mx) / sum;
        const float *vrow = vb + (int64_t)j * v_rs + d0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (d0 + e < D) o[e] = __fadd_rn(o[e], __fmul_rn(w, vrow[e]));
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ bool finite4(float4 x) {
    return (fabsf(x.x) <= 3.40282347e38f) & (fabsf(x.y) <= 3.40282347e38f) & (fabsf(x.z) <= 3.40282347e38f) &
           (fabsf(x.w) <= 3.40282347e38f);
}

// The split kernel's share of a tile: this wave's subtile t (keys 16t .. 16t + 15)
// only.  S^T of the subtile against the lane's Q slice, register r of lane
// (g, li) the raw score of key 16t + 4r + g.
template <int DP>
__device__ __forceinline__ floatx4 qk_sub(const float *ks, const float (&qreg)[DP / 4], int g, int k_row0, int t) {
    constexpr int DQ = DP / 4, CH = DP / 4;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * t + k_row0;
    const float *kp = ks + row * DP;
#pragma unroll
    for (int c = 0; c < DQ / 4; ++c) {
        const float4 x = *(const float4 *)(kp + 4 * swz<CH>(g * (DQ / 4) + c, row));
        acc = mfma(x.x, qreg[4 * c + 0], acc);
        acc = mfma(x.y, qreg[4 * c + 1], acc);
        acc = mfma(x.z, qreg[4 * c + 2], acc);
        acc = mfma(x.w, qreg[4 * c + 3], acc);
    }
    return acc;
}

// softmax_tile for one subtile's four scores per lane (keys 16t + 4r + g); the
// scores outside [lo, hi) (tile-relative, offset by g) are masked.
template <int NT>
__device__ __forceinline__ void softmax_sub(floatx4 &s, floatx4 (&oacc)[NT], float &m, float &l, int t, int lo, int hi,
                                            float c_exp) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 16 * t + 4 * r;
        if (j < lo || j >= hi) s[r] = -INFINITY;
    }
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tmax = max_xor32(max_xor16(tmax));
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2((m - m_use) * c_exp);
    l *= alpha;
#pragma unroll
    for (int n = 0; n < NT; ++n) oacc[n] *= alpha;
    m = m_new;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s[r] = fast_exp2((s[r] - m_use) * c_exp);
        l += s[r];
    }
}

// O^T += V^T P^T over this wave's subtile t.
template <int DP>
__device__ __forceinline__ void pv_sub(const float *vs, const floatx4 &s, int g, int li, floatx4 (&oacc)[DP / 16],
                                       int t) {
    constexpr int NT = DP / 16, CH = DP / 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 16 * t + 4 * r + g;
        const float *vp = vs + row * DP;
        float vop[NT];
        if constexpr (NT == 4) {
            const float4 x = *(const float4 *)(vp + 4 * swz<CH>(li, row));
            vop[0] = x.x;
            vop[1] = x.y;
            vop[2] = x.z;
            vop[3] = x.w;
        } else {
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const int d = NT * li + n;
                vop[n] = vp[4 * swz<CH>(d >> 2, row) + (d & 3)];
            }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) oacc[n] = mfma(vop[n], s[r], oacc[n]);
    }
}

// qk_sub and pv_sub with their operands already in registers (the split kernel's
// direct path at head_dim 64).  The contraction index of MFMA step (c, e) in lane
// group g is dim 16c + 4g + e here, so that the four lanes of a row read 64
// contiguous bytes per load: k[c] holds dims 16c + 4g .. 16c + 4g + 3 of this lane's
// Sᵀ key row and qreg[4c + e] the same dims of its query row; v[r] holds dims
// 4li .. 4li + 3 of the subtile's key 4r + g.
__device__ __forceinline__ floatx4 qk_regs(const float4 (&k)[4], const float (&qreg)[16]) {
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        acc = mfma(k[c].x, qreg[4 * c + 0], acc);
        acc = mfma(k[c].y, qreg[4 * c + 1], acc);
        acc = mfma(k[c].z, qreg[4 * c + 2], acc);
        acc = mfma(k[c].w, qreg[4 * c + 3], acc);
    }
    return acc;
}
// Zeroes the rows of a register subtile (v[r]: key k0 + 4r + g) at or past k_hi, which
// were loaded as copies of the item's last key: they weigh 0, and 0 * Inf would be NaN.
__device__ __forceinline__ void zero_past(float4 (&v)[4], int k0, int g, int k_hi) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (k0 + 4 * r + g >= k_hi) v[r] = make_float4(0.f, 0.f, 0.f, 0.f);
}
__device__ __forceinline__ void pv_regs(const float4 (&v)[4], const floatx4 &s, floatx4 (&oacc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        oacc[0] = mfma(v[r].x, s[r], oacc[0]);
        oacc[1] = mfma(v[r].y, s[r], oacc[1]);
        oacc[2] = mfma(v[r].z, s[r], oacc[2]);
        oacc[3] = mfma(v[r].w, s[r], oacc[3]);
    }
}

// Stage clock of the instrumented kernel (raya_attend_batched_stages): the
// shader clock (s_memtime) is read at each stage boundary of a tile and the
// difference added to that stage's total.  The scheduling barriers keep the
// compiler from moving work across a read; settle() makes the read wait until
// a stage's last result exists (a VALU op consumes it, so an MFMA result must
// have been written, and the asm keeps that op before the read).
struct StageClock {
    uint64_t last, qk, softmax, pv, load_wait;
    uint32_t tiles;
};

__device__ __forceinline__ uint64_t clock_now() {
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t t = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
    return t;
}

__device__ __forceinline__ void settle(float x) {
    const int s = __builtin_amdgcn_readfirstlane(__float_as_int(x));
    asm volatile("" ::"s"(s));
}

// Every accumulator chain of a stage (the MFMAs of different chains overlap).
template <int N>
__device__ __forceinline__ void settle(const floatx4 (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) settle(x[i][3]);
}

__device__ __forceinline__ void lap(StageClock *c, uint64_t &bucket) {
    const uint64_t t = clock_now();
    bucket += t - c->last;
    c->last = t;
}

// One workgroup computes one item.  Q goes straight to registers; each K/V
// tile goes straight from HBM to LDS (global_load_lds_dwordx4, no staging
// registers), so the kernel runs at high occupancy and other workgroups hide
// the load latency.  Rows or dims outside the tile's valid range load a
// clamped in-range address: their scores are masked, their V rows get weight
// zero, and Q is zero on the padded dims.
//
// For head dims other than 64 the loads are compiler builtins, and the
// compiler waits for every LDS DMA in flight before any LDS read, so a tile's V
// has landed before its QK^T starts.  FUSED (head_dim exactly 64): every tile's
// loads are issued by the asm blocks above with explicit waits, so V stays in
// flight during QK^T and the softmax.
//
// SPLIT: the item is 16 query rows and the four waves split every 64-key tile
// between them, wave w taking its 16-key subtile w (the grids too small to
// fill the chip: a quarter of the MFMA chain per wave).  Each wave keeps its
// own running max, sum and output over its keys; at the end the four partial
// states are combined through LDS, each wave finishing a quarter of the dims.
// At head_dim 64 (DIRECT) a wave's subtile of K and V goes straight into its
// registers, since no other wave reads it: no LDS staging and no barrier
// before the combine.
// MK >= 0: the mask kind is fixed at compile time; SINGLE: every item's keys fit one
// tile (BlockDiag(b) with b dividing 64).  Both only drop code the launch has ruled out.
//
// MAXT > 0 (the direct path, items of at most MAXT tiles): every tile's K/V subtile
// is loaded into registers before the first is computed, so the tile loads' latencies
// overlap each other rather than each one the previous tile's arithmetic.
template <int DP, bool FUSED, bool TIMED, bool SKIP = false, bool SPLIT = false, int MK = -1,
          bool SINGLE = false, int MAXT = 0, bool EXACTV = true>  // head_dim padded to a multiple of 16
__device__ __forceinline__ void attend_body(const AttnLaunch &a, const Plan &p, float *__restrict__ ks,
                                            float *__restrict__ vs, StageClock *clk) {
    static_assert(!FUSED || DP == 64, "the fused issue is written for head_dim 64");
    constexpr int ROWS = SPLIT ? kSplitRows : kQRows;
    constexpr int DQ = DP / 4;   // head-dim slice owned by one lane group
    constexpr int NT = DP / 16;  // 16-dim output tiles
    constexpr int CH = DP / 4;   // 16-byte chunks per row
    constexpr int LPW = CH / kWaves;  // direct loads per wave per tile (each 64 chunks)
    // SPLIT at head_dim 64: wave w only ever reads subtile w of each tile, so its K/V
    // go straight into registers (no LDS staging, no barrier before the combine), the
    // next tile's loaded while the current one is computed.
    constexpr bool DIRECT = SPLIT && FUSED;
    constexpr bool ALL = MAXT > 0;
    static_assert(!ALL || (DIRECT && !TIMED), "whole-item prefetch is a variant of the direct path");
    constexpr int kUnroll = ALL ? MAXT : 1;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int li = lane & 15;
    const int D = a.head_dim;
    const int dch = D / 4;  // valid chunks per row
    const int kind = MK >= 0 ? MK : a.mask_kind, arg = a.mask_arg;
    // Key ranges that differ between the rows of a 16-row wave (see exact_chunk).
    // (EXACTV false: the launch has checked that the mask has no such ranges.)
    const bool ragged = EXACTV && (kind == RAYA_MASK_WINDOW64 || kind == RAYA_MASK_SLIDING ||
                                   (kind == RAYA_MASK_BLOCKDIAG && arg % 16 != 0));
    // exp(scale * (x - y)) = exp2((x - y) * c) on raw dot products x, y; a
    // negative scale is carried by negating Q, so c > 0 and max commutes.  c is
    // kept at least FLT_MIN so that a masked key (x = -inf) weighs exactly 0
    // even at scale 0 (-inf * 0 would be NaN); every finite (x - y) * FLT_MIN
    // rounds to an exponent of 0, the uniform weights scale 0 asks for.
    const float c_exp = fmaxf(fabsf(a.scale) * kLog2e, 1.17549435e-38f);
    const float q_sign = a.scale < 0.f ? -1.f : 1.f;

    const Item it = decode<ROWS, MK>(a, p, item_of(blockIdx.x, p));
    // Packed sequences start at a row offset and have no padded rows in memory.
    const bool packed = a.seq_start != nullptr;
    const int64_t row0 = packed ? (int64_t)a.seq_start[it.b] : 0;
    const auto base = [&](int64_t bs, int64_t hs, int64_t rs) {
        return (packed ? row0 * rs : (int64_t)it.b * bs) + (int64_t)it.h * hs;
    };
    float *ob = a.out + base(a.o_bs, a.o_hs, a.o_rs);
    if (it.k_lo >= it.k_hi) {  // every row is padding: write zeros
        if (packed) return;
        for (int c = tid; c < ROWS * CH; c += kThreads) {
            const int r = it.q0 + c / CH, c4 = c % CH;
            if (r < a.seq && c4 < dch) {
                float *o = ob + (int64_t)r * a.o_rs + 4 * c4;
                // At head_dim 64 a store instruction covers four whole 256-byte rows.
                if constexpr (FUSED)
                    store_stream(o, make_float4(0.f, 0.f, 0.f, 0.f));
                else
                    *(float4 *)o = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        return;
    }

    const int qw = SPLIT ? it.q0 : it.q0 + wave * 16;
    const int qi = qw + li;
    const int valid = it.valid;
    const Range rr = qi < valid ? key_range(kind, arg, p.by_arg, qi, valid) : Range{0, 0};
    const bool wave_live = qw < valid;
    const bool wave_full_rows = qw + 15 < valid;
    const Range w_first = key_range(kind, arg, p.by_arg, min(qw, valid - 1), valid);
    const Range w_last = key_range(kind, arg, p.by_arg, min(qw + 15, valid - 1), valid);

    const float *kb = a.k + base(a.k_bs, a.k_hs, a.k_rs);
    const float *vb = a.v + base(a.v_bs, a.v_hs, a.v_rs);
    // Direct loads of this wave: LDS chunk slots (wave LPW + j) 64 + lane.
    auto stage = [&](const float *src, int64_t rs, float *lds, int kt) {
        const int kend = min(kt + kKeys, it.k_hi);
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            const int slot = (wave * LPW + j) * 64 + lane;
            const int r = slot / CH, p = slot % CH;
            const int c = min(swz<CH>(p, r), dch - 1);
            const int64_t row = min(kt + r, kend - 1);
            const int lds_off = (wave * LPW + j) * 64 * 16;
            __builtin_amdgcn_global_load_lds(src + row * rs + 4 * c, (lds_ptr_t *)((char *)lds + lds_off),
                                             16, 0, 0);
        }
    };
    // Loads return in issue order, so vmcnt(LPW) means everything but the LPW V
    // loads this wave issued last has landed.
    constexpr int kWaitAllButV = 0xF70 | (LPW & 0xF) | ((LPW >> 4) << 14);

    // K of the first tile goes out first, then Q (loaded unconditionally from a
    // clamped in-range address so all its loads are in flight together; the
    // out-of-range parts are zeroed after the wait), then V, which is only
    // waited for after QK^T and the softmax.
    float qreg[DQ];
    // Operands of one tile's asm issue: scalar bases at the tile's first row, 32-bit
    // byte offsets of this wave's chunks (rows past the item's keys clamped to its
    // last row) and the LDS slots.  The tile's even 16-key subtiles are keys
    // kx + 16t .., its odd ones ky + 16t .. (kx = ky but in the balanced steps
    // below).
    const auto tile_addrs = [&](int kx, int ky, const float *&kbase, uint32_t ko[4], uint32_t kl[4],
                                const float *&vbase, uint32_t vo[4], uint32_t vl[4]) {
        const int k0 = min(kx, ky);
        kbase = kb + (int64_t)k0 * a.k_rs;
        vbase = vb + (int64_t)k0 * a.v_rs;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int slot = (wave * LPW + j) * 64 + lane;
            const int lrow = slot / CH, c = swz<CH>(slot % CH, lrow);
            const int r = min(((lrow >> 4) & 1 ? ky : kx) + lrow, it.k_hi - 1) - k0;
            ko[j] = (uint32_t)(r * (int)a.k_rs * 4 + 16 * c);
            vo[j] = (uint32_t)(r * (int)a.v_rs * 4 + 16 * c);
            const int lds_off = (wave * LPW + j) * 64 * 16;
            kl[j] = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t *)((char *)ks + lds_off));
            vl[j] = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t *)((char *)vs + lds_off));
        }
    };
    // The item's n tiles are walked starting from the one whose global index
    // (k / 64) is a multiple of n, then on around.  The items running together
    // then touch, in each step, only the tiles of one residue mod n: an item's
    // neighbours share its tiles (Window64: 3, Block3: 6), so the first touches
    // of a tile, which go to HBM, spread over all n steps instead of all landing
    // in the first, and overlap the other steps' arithmetic.  The softmax is
    // independent of the order.
    const int n_tiles = SINGLE ? 1 : (it.k_hi - it.k_lo + kKeys - 1) / kKeys;
    int rot = 0;
    if (n_tiles > 1) {
        rot = (it.k_lo / kKeys) % n_tiles;
        rot = rot == 0 ? 0 : n_tiles - rot;
    }
    const auto tile_at = [&](int j) {
        j += rot;
        return it.k_lo + (j >= n_tiles ? j - n_tiles : j) * kKeys;
    };
    // Window64 and Sliding(64) items away from the sequence ends span exactly
    // three whole tiles, and wave w's rows meet 4 - w, 4 and w + 1 of their
    // subtiles: walked tile by tile, each step waits for its busiest wave (12
    // subtile steps per item for 9 subtiles of work per wave).  Balanced steps
    // pair the two edge tiles' halves instead: tile 0's even subtiles with tile
    // 2's odd ones, tile 1, then the other halves; every wave then meets 2, 4
    // and 3 subtiles.  Any mask stays exact: subtiles are scored at their own
    // keys.  The offsets of the paired step reach 191 rows of the row stride.
    const bool balanced = FUSED && SKIP && n_tiles == 3 && it.k_hi - it.k_lo == 3 * kKeys &&
                          a.k_rs < kMaxBalancedRowStride && a.v_rs < kMaxBalancedRowStride;
    const auto step_keys = [&](int kt, int &kx, int &ky) {
        kx = ky = kt;
        if (balanced && kt != it.k_lo + kKeys) {
            kx = kt == it.k_lo ? it.k_lo : it.k_lo + 2 * kKeys;
            ky = kt == it.k_lo ? it.k_lo + 2 * kKeys : it.k_lo;
        }
    };
    const int kt0 = tile_at(0);
    // Operand rows of this lane: S^T A-row i of subtile t is key 16t + 4(i%4) + i/4;
    // the PV operand of (t, r) is row 16t + 4r + g, dims NT li .. NT li + NT.
    const int k_row0 = 4 * (li & 3) + (li >> 2);
    // The direct path's operands of tile kt: this wave's subtile, rows past the
    // item's keys clamped to its last key.
    const auto load_sub = [&](int kt, float4 (&kr)[4], float4 (&vr)[4]) {
        const int key = min(kt + 16 * wave + k_row0, it.k_hi - 1);
        const float *kp = kb + (int64_t)key * a.k_rs + 4 * g;
#pragma unroll
        for (int c = 0; c < 4; ++c) kr[c] = *(const float4 *)(kp + 16 * c);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int vkey = min(kt + 16 * wave + 4 * r + g, it.k_hi - 1);
            vr[r] = *(const float4 *)(vb + (int64_t)vkey * a.v_rs + 4 * li);
        }
    };
    float4 kcur[4], vcur[4];
    float4 kall[kUnroll][4], vall[kUnroll][4];
    if constexpr (DIRECT) {
        const float *qp = a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)min(qi, valid - 1) * a.q_rs + 4 * g;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 x = *(const float4 *)(qp + 16 * c);
            qreg[4 * c + 0] = x.x;
            qreg[4 * c + 1] = x.y;
            qreg[4 * c + 2] = x.z;
            qreg[4 * c + 3] = x.w;
        }
        if constexpr (ALL) {
            // Steps past the item's last tile load that tile again (never computed).
#pragma unroll
            for (int j = 0; j < kUnroll; ++j) load_sub(tile_at(min(j, n_tiles - 1)), kall[j], vall[j]);
            __builtin_amdgcn_sched_barrier(0);
        } else {
            load_sub(kt0, kcur, vcur);
        }
        // A single tile's loads all leave here: the scheduler would otherwise sink each
        // one next to its first use and wait for it alone.
        if constexpr (SINGLE) __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (FUSED) {
        // K, Q and V in one asm block that ends waiting for K and Q only.
        const float *kbase, *vbase;
        uint32_t ko[4], kl[4], vo[4], vl[4];
        int kx, ky;
        step_keys(kt0, kx, ky);
        tile_addrs(kx, ky, kbase, ko, kl, vbase, vo, vl);
        const float *qa = a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)min(qi, valid - 1) * a.q_rs + g * DQ;
        floatx4 q4[4];
        issue_kqv64(kbase, ko, kl, qa, q4, vbase, vo, vl);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) qreg[4 * c + e] = q4[c][e];
    } else {
        stage(kb, a.k_rs, ks, kt0);
        const int qrow = min(qi, valid - 1);
        const float *qp = a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)qrow * a.q_rs;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            const float4 x = *(const float4 *)(qp + min(g * DQ + 4 * c, D - 4));
            qreg[4 * c + 0] = x.x;
            qreg[4 * c + 1] = x.y;
            qreg[4 * c + 2] = x.z;
            qreg[4 * c + 3] = x.w;
        }
        stage(vb, a.v_rs, vs, kt0);
    }

    floatx4 oacc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) oacc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;  // running max of raw dot products
    float l = 0.f;        // this lane's partial sum of weights

    if constexpr (TIMED) clk->last = clock_now();
    if constexpr (ALL) {
        // Every tile's operands are in registers: the scores of step j + 1 go to the
        // matrix core before the softmax of step j, which runs beside them.  The steps
        // run to MAXT, fully unrolled (the register sets are indexed by the step);
        // those past the item's tiles are neither scored nor accumulated.
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bool in = qi < valid;  // Q as below: zero past valid, negated for a negative scale
#pragma unroll
            for (int e = 0; e < 4; ++e) qreg[4 * c + e] = in ? qreg[4 * c + e] * q_sign : 0.f;
        }
        floatx4 s_cur = qk_regs(kall[0], qreg);
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
            floatx4 s_nxt;
            if (j + 1 < kUnroll && j + 1 < n_tiles) s_nxt = qk_regs(kall[j + 1], qreg);
            const int kt = tile_at(j);
            const int k16 = kt + 16 * wave;  // this wave's subtile, as `live` below
            const bool active = wave_live && j < n_tiles && kt < w_last.hi && kt + kKeys > w_first.lo &&
                                k16 < w_last.hi && k16 + 16 > w_first.lo;
            if (active) {
                const int m_lo = max(rr.lo, k16), m_hi = min(rr.hi, k16 + 16);
                softmax_sub<NT>(s_cur, oacc, m, l, wave, m_lo - kt - g, m_hi - kt - g, c_exp);
                if (kt + kKeys > it.k_hi) zero_past(vall[j], k16, g, it.k_hi);
                pv_regs(vall[j], s_cur, oacc);
            }
            if (j + 1 < kUnroll) s_cur = s_nxt;
        }
    } else {
#pragma unroll 1
    for (int j = 0; j < n_tiles; ++j) {
        const int kt = tile_at(j);
        int kx, ky;
        step_keys(kt, kx, ky);
        float4 knext[4], vnext[4];
        if constexpr (DIRECT) {
            if (j + 1 < n_tiles) load_sub(tile_at(j + 1), knext, vnext);
        }
        if (!DIRECT && j != 0) {
            // Every wave's LDS reads of the previous tile have returned.
            barrier_after_reads();
            if constexpr (FUSED) {
                const float *kbase, *vbase;
                uint32_t ko[4], kl[4], vo[4], vl[4];
                tile_addrs(kx, ky, kbase, ko, kl, vbase, vo, vl);
                issue_kv64(kbase, ko, kl, vbase, vo, vl);
            } else {
                stage(kb, a.k_rs, ks, kt);
                stage(vb, a.v_rs, vs, kt);
            }
        }
        // This wave's K (and Q) loads have landed (the fused issue waited already) ...
        if constexpr (!FUSED) __builtin_amdgcn_s_waitcnt(kWaitAllButV);
        if constexpr (!DIRECT) barrier_only();  // ... and every other wave's
        if (j == 0) {
            // Q is zero on rows at or beyond valid and on dims at or beyond D; a
            // negative scale is carried by negating Q.
#pragma unroll
            for (int c = 0; c < DQ / 4; ++c) {
                const bool in = qi < valid && g * DQ + 4 * c < D;
#pragma unroll
                for (int e = 0; e < 4; ++e) qreg[4 * c + e] = in ? qreg[4 * c + e] * q_sign : 0.f;
            }
        }
        bool rows_active = wave_live && kt < w_last.hi && kt + kKeys > w_first.lo;
        // Sliding windows: the 16-key subtiles outside the union of the wave's
        // key intervals [w_first.lo, w_last.hi) hold no live key for any of its
        // rows (about a quarter of an item's subtiles at Window64); such a tile
        // always takes the masked softmax, which sets those scores to -inf.
        // SPLIT keeps only the wave's own subtile.
        int live = 0xF;
        if constexpr (SKIP || SPLIT) {
            live = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int k16 = (t & 1 ? ky : kx) + 16 * t;
                if (k16 < w_last.hi && k16 + 16 > w_first.lo) live |= 1 << t;
            }
            live = __builtin_amdgcn_readfirstlane(live);
            // A tile meets the rows' keys exactly when one of its subtiles does.
            if constexpr (SKIP) rows_active = wave_live && live != 0;
            if constexpr (SPLIT) live &= 1 << wave;
        }
        const bool active = SPLIT ? rows_active && live != 0 : rows_active;
        // The keys this wave may score in this tile: the row's interval, and
        // under SPLIT only its own subtile.
        int m_lo = rr.lo, m_hi = rr.hi;
        if constexpr (SPLIT) {
            m_lo = max(m_lo, kt + 16 * wave);
            m_hi = min(m_hi, kt + 16 * wave + 16);
        }
        floatx4 sacc[4];
        floatx4 ssub;
        if constexpr (TIMED) {
            lap(clk, clk->load_wait);
            // A split tile (16 rows x 64 keys) is computed by the four waves together.
            if constexpr (SPLIT) clk->tiles += wave == 0 && rows_active;
        }
        if (active) {
            if constexpr (DIRECT) {
                ssub = qk_regs(kcur, qreg);
            } else if constexpr (SPLIT) {
                ssub = qk_sub<DP>(ks, qreg, g, k_row0, wave);
            } else {
                qk_tile<DP>(ks, qreg, g, k_row0, sacc, live);
            }
            if constexpr (TIMED) {
                if constexpr (SPLIT) {
                    settle(ssub[3]);
                } else {
                    settle(sacc);
                    ++clk->tiles;
                }
                lap(clk, clk->qk);
            }
            if constexpr (SPLIT) {
                softmax_sub<NT>(ssub, oacc, m, l, wave, m_lo - kt - g, m_hi - kt - g, c_exp);
            } else {
                softmax_tile<NT>(sacc, oacc, m, l, j == 0,
                                 kx != ky || !(wave_full_rows && kt >= w_last.lo && kt + kKeys <= w_first.hi),
                                 m_lo - kx - g, m_hi - kx - g, m_lo - ky - g, m_hi - ky - g, c_exp);
            }
            if constexpr (TIMED) {
                settle(l);
                settle(oacc);
                lap(clk, clk->softmax);
            }
        }
        if constexpr (!DIRECT) {
            __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): this wave's V loads have landed
            // Rows past the item's last key were loaded as copies of it: they weigh 0, but
            // 0 * Inf is NaN, so a non-finite V at that key would reach rows that do not
            // see the copies.  This wave zeroes its own chunks of them before PV.  (Under
            // the sliding masks keys inside a scored subtile but outside a row's window
            // weigh 0 the same way; there the copies change nothing.)
            if ((!SKIP || MK == RAYA_MASK_BLOCKDIAG) && max(kx, ky) + kKeys > it.k_hi) {
                int ln = lane;
                asm volatile("" : "+v"(ln));  // keeps this rare path's arithmetic inside it
#pragma unroll
                for (int jj = 0; jj < LPW; ++jj) {
                    const int lrow = ((wave * LPW + jj) * 64 + ln) / CH;
                    if (((lrow >> 4) & 1 ? ky : kx) + lrow >= it.k_hi)
                        *(float4 *)((char *)vs + (wave * LPW + jj) * 1024 + ln * 16) = make_float4(0.f, 0.f, 0.f, 0.f);
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zeros are in LDS
            }
            barrier_only();
        }
        if constexpr (TIMED) lap(clk, clk->load_wait);
        if (active) {
            if constexpr (DIRECT) {
                if (kt + kKeys > it.k_hi) zero_past(vcur, kt + 16 * wave, g, it.k_hi);
                pv_regs(vcur, ssub, oacc);
            } else if constexpr (SPLIT) {
                pv_sub<DP>(vs, ssub, g, li, oacc, wave);
            } else {
                pv_tile<DP>(vs, sacc, g, li, oacc, live);
            }
            if constexpr (TIMED) {
                settle(oacc);
                lap(clk, clk->pv);
            }
        }
        if constexpr (DIRECT) {
            if (j + 1 < n_tiles) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    kcur[c] = knext[c];
                    vcur[c] = vnext[c];
                }
            }
        }
    }
    }
    l = sum_xor32(sum_xor16(l));

    if constexpr (SPLIT) {
        // Partial states to LDS (the K tile holds the outputs [wave][n][r][lane],
        // the V tile the max and sum of each wave's lanes), then wave w finishes
        // the 16-byte chunks c = w, w + 4, ... of its lane's row.
        barrier_after_reads();
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) ks[((wave * NT + n) * 4 + r) * 64 + lane] = oacc[n][r];
        vs[wave * 64 + lane] = m;
        vs[(kWaves + wave) * 64 + lane] = l;
        __syncthreads();
        float mw[kWaves], sw[kWaves];
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mw[w] = vs[w * 64 + lane];
            mx = fmaxf(mx, mw[w]);
        }
        const float m_use = mx == -INFINITY ? 0.f : mx;
        float lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            sw[w] = fast_exp2((mw[w] - m_use) * c_exp);
            lsum += sw[w] * vs[(kWaves + w) * 64 + lane];
        }
        if (qi < (packed ? valid : a.seq)) {
            const bool zero_row = qi >= valid || lsum == 0.f;
            const float inv = zero_row ? 0.f : 1.f / lsum;
            float *orow = ob + (int64_t)qi * a.o_rs + g * DQ;
            for (int c = wave; c < DQ / 4; c += kWaves) {
                if (g * DQ + 4 * c < D) {
                    float e4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int n = (4 * c + e) % NT, r = (4 * c + e) / NT;
                        float acc = 0.f;
#pragma unroll
                        for (int w = 0; w < kWaves; ++w) acc += sw[w] * ks[((w * NT + n) * 4 + r) * 64 + lane];
                        e4[e] = zero_row ? 0.f : acc * inv;
                    }
                    float4 y = make_float4(e4[0], e4[1], e4[2], e4[3]);
                    if (ragged && !zero_row && !finite4(y))
                        y = exact_chunk(a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)qi * a.q_rs, kb, a.k_rs, vb,
                                        a.v_rs, rr.lo, rr.hi, D, a.scale, g * DQ + 4 * c);
                    *(float4 *)(orow + 4 * c) = y;
                }
            }
        }
        return;
    }

    // Register r of oacc[n] holds dim g DQ + NT r + n of row qi.  Rows at or
    // beyond valid, and rows with no weight (an empty key range), are stored as
    // literal zeros: their accumulators are zero weights times V, which is NaN
    // wherever V is not finite.  A NaN weight sum (a NaN or +Inf score) makes the
    // whole row NaN, as the reference's division by that sum does (naive.rs:53-61).
    if constexpr (FUSED) {
        // The wave's 16 x 64 output block goes through its quarter of the K tile
        // (no wave reads K after the last tile's V barrier) and leaves as whole
        // rows: each store instruction writes four 256-byte rows, streamed past
        // the caches.  In the accumulator layout a store covers 16-byte pieces
        // 64 bytes apart, which only the L2 can merge into lines.  The row's
        // 16-byte chunk c sits at chunk c ^ row, so both the writes (16 rows,
        // one chunk each) and the reads (one row, 16 chunks) touch 16
        // distinct chunk columns.
        float *st = ks + wave * 16 * 64;
        const bool zero_row = qi >= valid || l == 0.f;
        const float inv = zero_row ? 0.f : 1.f / l;
        bool bad = false;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
            if (!zero_row) {
                y.x = oacc[0][c] * inv;
                y.y = oacc[1][c] * inv;
                y.z = oacc[2][c] * inv;
                y.w = oacc[3][c] * inv;
            }
            bad |= !zero_row && !finite4(y);
            *(float4 *)(st + li * 64 + 4 * ((4 * g + c) ^ li)) = y;
        }
        // Non-finite chunks under ragged masks are recomputed (exact_chunk) in place.
        if (ragged && __any(bad)) {
#pragma unroll 1
            for (int c = 0; c < 4; ++c) {
                float4 *slot = (float4 *)(st + li * 64 + 4 * ((4 * g + c) ^ li));
                if (!zero_row && !finite4(*slot))
                    *slot = exact_chunk(a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)qi * a.q_rs, kb, a.k_rs, vb,
                                        a.v_rs, rr.lo, rr.hi, D, a.scale, 16 * g + 4 * c);
            }
        }
        // One wave's LDS accesses complete in order: the reads see the writes.
        const int rows = packed ? valid : a.seq;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = 4 * t + (lane >> 4), c = lane & 15;
            const float4 y = *(const float4 *)(st + r * 64 + 4 * (c ^ r));
            if (qw + r < rows) store_stream(ob + (int64_t)(qw + r) * a.o_rs + 4 * c, y);
        }
        return;
    }
    if (qi < (packed ? valid : a.seq)) {
        const bool zero_row = qi >= valid || l == 0.f;
        const float inv = zero_row ? 0.f : 1.f / l;
        float *orow = ob + (int64_t)qi * a.o_rs + g * DQ;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
            if (g * DQ + 4 * c < D) {
                float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
                if (!zero_row) {
                    y.x = oacc[(4 * c + 0) % NT][(4 * c + 0) / NT] * inv;
                    y.y = oacc[(4 * c + 1) % NT][(4 * c + 1) / NT] * inv;
                    y.z = oacc[(4 * c + 2) % NT][(4 * c + 2) / NT] * inv;
                    y.w = oacc[(4 * c + 3) % NT][(4 * c + 3) / NT] * inv;
                }
                if (ragged && !zero_row && !finite4(y))
                    y = exact_chunk(a.q + base(a.q_bs, a.q_hs, a.q_rs) + (int64_t)qi * a.q_rs, kb, a.k_rs, vb,
                                    a.v_rs, rr.lo, rr.hi, D, a.scale, g * DQ + 4 * c);
                *(float4 *)(orow + 4 * c) = y;
            }
        }
    }
}

template <int DP, bool FUSED, bool EXACTV>
__global__ void __launch_bounds__(kThreads, kMinWaves<DP>) attend_kernel(const AttnLaunch a, const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * DP];
    attend_body<DP, FUSED, false, false, false, -1, false, 0, EXACTV>(a, p, ks, vs, nullptr);
}

// Head_dim 64 under Window64 and Sliding(w): the fused kernel with subtile
// skipping (+7% on Window64 at L = 8192; no use for the block masks, whose
// items' key ranges cover whole subtiles).
// BlockDiag(b) with b dividing 64 at head_dim 64: every item is one 64-key tile,
// and the mask is known, so the item decode and key ranges compile to a few
// scalar instructions (the general kernel's first K/V load sits behind the
// decode of every mask kind and the tile walk's set-up): 64 VGPRs instead of
// 126, and the first load about 420 instructions earlier.  Blocks narrower than 64
// (SKIP) leave each wave's rows whole 16-key subtiles of other blocks' keys, which it
// skips: a quarter (b <= 16) or half (b = 32) of the matrix work, and no other block's
// V enters its rows even at weight 0 (0 * Inf would be NaN) when b is 16 or 32.
template <int DP, bool SKIP>
__global__ void __launch_bounds__(kThreads, kMinWaves<DP>) attend_blockdiag_kernel(const AttnLaunch a, const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * DP];
    // BlockDiag(64) rows of a wave share one range; narrower blocks may not.
    attend_body<DP, true, false, SKIP, false, RAYA_MASK_BLOCKDIAG, true, 0, SKIP>(a, p, ks, vs, nullptr);
}

template <int DP, int MK>
__global__ void __launch_bounds__(kThreads, kMinWaves<DP>) attend_sliding_kernel(const AttnLaunch a, const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * DP];
    attend_body<DP, true, false, true, false, MK>(a, p, ks, vs, nullptr);
}

// 16-row items with the key tiles split over the four waves, for grids that
// leave most compute units idle with 64-row items.
template <int DP, bool FUSED, int MK = -1, bool SINGLE = false, bool EXACTV = true>
__global__ void __launch_bounds__(kThreads, (kMinWavesOf<DP, true, FUSED>)) attend_split_kernel(const AttnLaunch a,
                                                                                               const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * DP];
    attend_body<DP, FUSED, false, false, true, MK, SINGLE, 0, EXACTV>(a, p, ks, vs, nullptr);
}

// The split kernel at head_dim 64 for items of at most MAXT tiles, every tile's K/V
// loads issued before the first tile is computed.  2 waves per SIMD hold the MAXT
// register sets (239 VGPRs at MAXT = 6); the small grids this kernel serves place at
// most two workgroups per compute unit.
template <int MAXT, bool EXACTV>
__global__ void __launch_bounds__(kThreads, 2) attend_split_all_kernel(const AttnLaunch a, const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * 64];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * 64];
    attend_body<64, true, false, false, true, -1, false, MAXT, EXACTV>(a, p, ks, vs, nullptr);
}

// The same kernel with the stage clock.  Per-wave totals are summed in LDS,
// then one thread per stage adds the workgroup's sum to the caller's totals.
// An item whose rows are all padding returns from the body in every wave with
// zero totals.
template <int DP, bool FUSED, bool SKIP, bool SPLIT = false>
__global__ void __launch_bounds__(kThreads, (kMinWavesOf<DP, SPLIT, FUSED>)) attend_timed_kernel(const AttnLaunch a,
                                                                                                const Plan p) {
    __shared__ __attribute__((aligned(16))) float ks[kKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kKeys * DP];
    __shared__ uint64_t part[kWaves][5];
    StageClock c{};
    attend_body<DP, FUSED, true, SKIP, SPLIT>(a, p, ks, vs, &c);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        part[wave][0] = c.qk;
        part[wave][1] = c.softmax;
        part[wave][2] = c.pv;
        part[wave][3] = c.load_wait;
        part[wave][4] = c.tiles;
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        uint64_t sum = 0;
        for (int w = 0; w < kWaves; ++w) sum += part[w][threadIdx.x];
        if (sum) atomicAdd((unsigned long long *)&a.stage_cycles->qk + threadIdx.x, (unsigned long long)sum);
    }
}

constexpr int64_t kMaxFusedRowStride = (int64_t(1) << 31) / (4 * kKeys) - kKeys;  // floats

// Half the bit width of the scatter domain: the smallest h with 4^h >= total.
int scatter_half_bits(int64_t total) {
    int h = 1;
    while ((int64_t(1) << (2 * h)) < total) ++h;
    return h;
}

// Grids of fewer 64-row items than this take the split kernel (16-row items,
// each tile's keys split over the waves).  At 192 items the two kernels take
// the same time; below, the split kernel is faster, above, the 64-row one (the
// split kernel runs 3 workgroups per compute unit).
constexpr int64_t kSplitBelow = 192;

// RAYA_ATTN_ITEMS=16 or 64 forces the item height (as the reference's
// RAYA_BACKEND forces a micro-kernel backend); anything else selects by grid.
bool use_split(const AttnLaunch &a) {
    if (const char *e = std::getenv("RAYA_ATTN_ITEMS")) {
        if (!std::strcmp(e, "16")) return true;
        if (!std::strcmp(e, "64")) return false;
    }
    const int64_t items = (a.seq + kQRows - 1) / kQRows * a.heads * a.batch;
    return items < kSplitBelow;
}

// The most 64-key tiles one 16-row item's key interval spans (every row valid; a
// shorter valid length only clips intervals).
int64_t max_item_tiles(const AttnLaunch &a) {
    const int64_t b = a.mask_arg;
    int64_t span;
    switch (a.mask_kind) {
    case RAYA_MASK_BLOCK3: span = 3 * RAYA_BLOCK; break;  // the rows share one 128-block
    case RAYA_MASK_WINDOW64: span = kSplitRows + 2 * RAYA_WINDOW; break;
    case RAYA_MASK_FULL: span = a.seq; break;
    case RAYA_MASK_SLIDING: span = kSplitRows + 2 * b; break;
    default:  // BlockDiag(b): one block when 16 divides b, else the blocks 16 rows touch
        span = b % kSplitRows == 0 ? b : b * ((kSplitRows - 1) / b + 2);
        break;
    }
    span = std::min<int64_t>(span, a.seq);
    return (span + kKeys - 1) / kKeys;
}

// RAYA_ATTN_PREFETCH=0 keeps the one-tile-ahead loads of the split kernel on items of
// up to six tiles.
bool prefetch_all() {
    const char *e = std::getenv("RAYA_ATTN_PREFETCH");
    return !(e && !std::strcmp(e, "0"));
}

// Item order of the 64-row kernels.  XCD x taking whole (sequence, head) pairs
// gives each XCD the padding of the sequences whose heads it holds: with 12
// heads on 8 XCDs, even sequences put two heads on XCDs 0-3 and odd ones on
// XCDs 4-7, so the XCDs' shares of the work differ by the two halves' valid
// lengths (7% on a batch of 32 sequences of U[512, 2048] valid rows).  Dealing
// each pair's units of 4 consecutive tiles round the XCDs, rotated by the
// pair's index, gives every XCD an equal share of every pair while a unit's
// items still share their key tiles in one L2: the MFMA-bound multi-tile lines
// gain about 1% (Block3 and BlockDiag(128) at 4 x 12 x 16384, Block3 at 32 x
// 12 x 2048).  A batch of one sequence gives every pair the same valid length
// and keeps whole pairs (16 heads x 2048 rows under Block3 ran 1% slower in
// units).  Single-tile BlockDiag(b <= 64) keeps whole pairs: HBM-bound, it runs
// the same either way (the XCD that finishes early leaves its bandwidth to the
// others), and units of 1 or 2 tiles, which scatter neighbouring rows over the
// XCDs, run it 16-20% slower.  Window64 and Sliding keep whole pairs too (units
// of 4 tiles: 0.4-1.5% slower on 16 heads x 4096 and 8192 rows).
// RAYA_ATTN_ORDER=pairs keeps whole pairs, rot1/rot2/rot4/rot8 deal units of
// that many tiles for any mask; the units must divide a pair's tiles 8 times
// over, else whole pairs.  Returns the shift, or -1 for whole pairs.
int rotate_shift(const AttnLaunch &a) {
    if (const char *e = std::getenv("RAYA_ATTN_ORDER")) {
        if (!std::strcmp(e, "pairs")) return -1;
        if (!std::strcmp(e, "rot1")) return 0;
        if (!std::strcmp(e, "rot2")) return 1;
        if (!std::strcmp(e, "rot4")) return 2;
        if (!std::strcmp(e, "rot8")) return 3;
    }
    const bool wide_block = a.mask_kind == RAYA_MASK_BLOCKDIAG && kKeys % a.mask_arg != 0;
    // One sequence gives every pair the same valid length: whole pairs are balanced.
    return (a.mask_kind == RAYA_MASK_BLOCK3 || wide_block) && a.batch > 1 ? 2 : -1;
}

template <bool EXACTV>
void launch_split_all(int64_t t, dim3 grid, dim3 block, hipStream_t stream, const AttnLaunch &a, const Plan &p) {
    if (t <= 2)
        hipLaunchKernelGGL((attend_split_all_kernel<2, EXACTV>), grid, block, 0, stream, a, p);
    else if (t <= 3)
        hipLaunchKernelGGL((attend_split_all_kernel<3, EXACTV>), grid, block, 0, stream, a, p);
    else if (t <= 4)
        hipLaunchKernelGGL((attend_split_all_kernel<4, EXACTV>), grid, block, 0, stream, a, p);
    else
        hipLaunchKernelGGL((attend_split_all_kernel<6, EXACTV>), grid, block, 0, stream, a, p);
}

template <int DP, bool FUSED = false>
hipError_t launch_dp(const AttnLaunch &a, hipStream_t stream) {
    const bool split = use_split(a);
    const int64_t rows = split ? kSplitRows : kQRows;
    const int64_t n_qt = (a.seq + rows - 1) / rows;
    const int64_t total = n_qt * a.heads * a.batch;
    if (total > 0x7fffffff) return hipErrorInvalidValue;
    Plan p;
    p.total = (int)total;
    p.half_bits = scatter_half_bits(total);
    p.n_qt = (int)n_qt;
    p.by_qt = make_fastdiv((uint32_t)n_qt);
    p.by_heads = make_fastdiv((uint32_t)a.heads);
    p.by_arg = make_fastdiv(a.mask_kind == RAYA_MASK_BLOCKDIAG ? (uint32_t)a.mask_arg : 1u);
    const int64_t pairs = (int64_t)a.heads * a.batch;
    p.pairs_per_xcd = pairs % kXcds == 0 ? (int)(pairs / kXcds) : 0;
    p.quads = split && p.pairs_per_xcd == 0 && total % (4 * kXcds) == 0;
    if (p.quads) {
        const char *e = std::getenv("RAYA_ATTN_QUADS");
        if (!(e && !std::strcmp(e, "plain"))) p.quads = 2;
    }
    p.rot_units = p.rot_shift = 0;
    p.by_rot = make_fastdiv(1u);
    const int shift = split ? -1 : rotate_shift(a);
    if (shift >= 0 && n_qt % (kXcds << shift) == 0) {
        p.rot_shift = shift;
        p.rot_units = (int)(n_qt / (kXcds << shift));
        p.by_rot = make_fastdiv((uint32_t)(p.rot_units << shift));
    }
    const dim3 grid((unsigned)total), block(kThreads);
    const bool sliding = a.mask_kind == RAYA_MASK_SLIDING || a.mask_kind == RAYA_MASK_WINDOW64;
    // Masks whose key ranges differ between the 16 rows of a wave take the kernels
    // that recompute non-finite output chunks (exact_chunk).
    const bool ragged = sliding || (a.mask_kind == RAYA_MASK_BLOCKDIAG && a.mask_arg % 16 != 0);
    if (split) {
        if (a.stage_cycles)
            hipLaunchKernelGGL((attend_timed_kernel<DP, FUSED, false, true>), grid, block, 0, stream, a, p);
        else if (FUSED && a.mask_kind == RAYA_MASK_BLOCKDIAG && kKeys % a.mask_arg == 0)
            if (a.mask_arg < 16)
                hipLaunchKernelGGL((attend_split_kernel<DP, FUSED, RAYA_MASK_BLOCKDIAG, true, true>), grid, block, 0, stream, a, p);
            else
                hipLaunchKernelGGL((attend_split_kernel<DP, FUSED, RAYA_MASK_BLOCKDIAG, true, false>), grid, block, 0, stream, a, p);
        else if (FUSED && prefetch_all() && max_item_tiles(a) >= 2 && max_item_tiles(a) <= 6) {
            // (Single-tile items have no later load to overlap.)
            const int64_t t = max_item_tiles(a);
            if (ragged)
                launch_split_all<true>(t, grid, block, stream, a, p);
            else
                launch_split_all<false>(t, grid, block, stream, a, p);
        }
        else if (ragged)
            hipLaunchKernelGGL((attend_split_kernel<DP, FUSED, -1, false, true>), grid, block, 0, stream, a, p);
        else
            hipLaunchKernelGGL((attend_split_kernel<DP, FUSED, -1, false, false>), grid, block, 0, stream, a, p);
        return hipGetLastError();
    }
    if constexpr (FUSED) {
        if (a.stage_cycles && sliding)
            hipLaunchKernelGGL((attend_timed_kernel<DP, true, true>), grid, block, 0, stream, a, p);
        else if (a.stage_cycles)
            hipLaunchKernelGGL((attend_timed_kernel<DP, true, false>), grid, block, 0, stream, a, p);
        else if (a.mask_kind == RAYA_MASK_WINDOW64)
            hipLaunchKernelGGL((attend_sliding_kernel<DP, RAYA_MASK_WINDOW64>), grid, block, 0, stream, a, p);
        else if (sliding)
            hipLaunchKernelGGL((attend_sliding_kernel<DP, RAYA_MASK_SLIDING>), grid, block, 0, stream, a, p);
        else if (a.mask_kind == RAYA_MASK_BLOCKDIAG && a.mask_arg == kKeys)
            hipLaunchKernelGGL((attend_blockdiag_kernel<DP, false>), grid, block, 0, stream, a, p);
        else if (a.mask_kind == RAYA_MASK_BLOCKDIAG && kKeys % a.mask_arg == 0)
            hipLaunchKernelGGL((attend_blockdiag_kernel<DP, true>), grid, block, 0, stream, a, p);
        else if (ragged)
            hipLaunchKernelGGL((attend_kernel<DP, true, true>), grid, block, 0, stream, a, p);
        else
            hipLaunchKernelGGL((attend_kernel<DP, true, false>), grid, block, 0, stream, a, p);
    } else {
        if (a.stage_cycles)
            hipLaunchKernelGGL((attend_timed_kernel<DP, false, false>), grid, block, 0, stream, a, p);
        else if (ragged)
            hipLaunchKernelGGL((attend_kernel<DP, false, true>), grid, block, 0, stream, a, p);
        else
            hipLaunchKernelGGL((attend_kernel<DP, false, false>), grid, block, 0, stream, a, p);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const AttnLaunch &a, hipStream_t stream) {
    const int dp = (a.head_dim + 15) / 16 * 16;
    switch (dp) {
    case 16: return launch_dp<16>(a, stream);
    case 32: return launch_dp<32>(a, stream);
    case 48: return launch_dp<48>(a, stream);
    case 64:
        // The fused issue forms K/V offsets within a tile in 32 bits: 63 rows of the
        // row stride plus the last chunk must stay below 2^31 bytes.
        return a.head_dim == 64 && a.k_rs < kMaxFusedRowStride && a.v_rs < kMaxFusedRowStride
                   ? launch_dp<64, true>(a, stream)
                   : launch_dp<64>(a, stream);
    case 80: return launch_dp<80>(a, stream);
    case 96: return launch_dp<96>(a, stream);
    case 112: return launch_dp<112>(a, stream);
    case 128: return launch_dp<128>(a, stream);
    // Above 128 the contraction is padded to the next of four widths (at most 1/8 of it
    // zeros from 144 up): K/V tiles of 64 keys take 2 x 64 x DP floats of LDS (128 KB at
    // 256, one workgroup per compute unit).
    case 144:
    case 160: return launch_dp<160>(a, stream);
    case 176:
    case 192: return launch_dp<192>(a, stream);
    case 208:
    case 224: return launch_dp<224>(a, stream);
    case 240:
    case 256: return launch_dp<256>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace raya
