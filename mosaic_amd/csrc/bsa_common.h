// bsa_common.h -- shared types, bf16 helpers and kernel parameter blocks for the gfx950
// block-sparse attention kernels.
//
// MFMA conventions used throughout (v_mfma_f32_32x32x16_bf16, one wave of 64 lanes):
//   lane l = 32*hh + r  (hh = l / 32, r = l % 32)
//   A operand (32 x 16): lane holds A[r][kidx(hh, i)], i = 0..7
//   B operand (16 x 32): lane holds B[kidx(hh, i)][r], i = 0..7
//   D (32 x 32, 16 fp32): register jj holds D[8*(jj/4) + 4*hh + jj%4][r]
// The contraction index kidx(hh, i) is the same function for A and B, so any consistent
// assignment of contraction elements to (hh, i) is correct.  Attention tiles are computed
// transposed (S^T = K Q^T, O^T = V^T P^T): a lane then owns one query column, so row
// statistics of the softmax are per-lane values plus one exchange between the two halves.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mosaic {

typedef uint16_t bf16_t;  // storage type of bfloat16 values
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.44269504089f;  // constant of the selected-branch kernel (ops.py:41)
constexpr int kHeadDim = 64;
constexpr int kTile = 64;                  // query rows / keys per attention tile

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 of two values, packed (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
// a rounded to bf16 (round to nearest even), as an fp32 value: the conversion puts bf16(a) in
// the high half of a word whose low half is bf16(0) = 0, which is that fp32 value (one
// instruction, no shift)
__device__ __forceinline__ float round_bf16(float a) { return __uint_as_float(pack_bf16x2(0.f, a)); }

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: A (16 x 32) lane holds A[l % 16][8*(l/16) + i]; B (32 x 16) lane
// holds B[8*(l/16) + i][l % 16]; D (16 x 16, 4 fp32) register e holds D[4*(l/16) + e][l % 16].
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Pooled K and V in MFMA-operand order for the compressed-attention kernel: per 32-block
// tile ut, every operand fragment is a contiguous 1 KB run (lane l's 16 bytes at 16*l), so a
// wave reads it with one coalesced 16-byte load per lane.  H heads, UT = nb_pad / 32 tiles.
//   K (A of S^T = K Q^T):  [B][H][UT][ds 4][lane 64][8]; lane 32*hh + r holds
//                          k[32*ut + r][16*ds + 8*hh .. +7]
//   V (A of O^T = V^T P^T): [B][H][UT][dt 2][s2 2][lane 64][8]; lane 32*hh + r holds
//                          v[32*ut + 16*s2 + 4*hh + i][32*dt + r] (i = 0..3), then the same
//                          for blocks + 8
__host__ __device__ __forceinline__ int64_t kfrag_index(int b, int h, int H, int UT, int ut, int ds, int lane) {
    return ((((int64_t)b * H + h) * UT + ut) * 4 + ds) * 512 + lane * 8;
}
__host__ __device__ __forceinline__ int64_t vfrag_index(int b, int h, int H, int UT, int ut, int dt, int s2, int lane) {
    return (((((int64_t)b * H + h) * UT + ut) * 2 + dt) * 2 + s2) * 512 + lane * 8;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const void* p) { return *reinterpret_cast<const uint2*>(p); }

// x[l] + x[l ^ 32] and max(x[l], x[l ^ 32]) in every lane l: one v_permlane32_swap (lanes
// l < 32 get x[l] and x[l + 32], lanes l >= 32 get x[l - 32] and x[l]) instead of an LDS
// permute round trip.  The operations are commutative, so both halves get the same value.
__device__ __forceinline__ float xor32_add(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Wave-uniform maximum of a non-negative float (or NaN, which wins) held per lane: DPP
// steps within each 16-lane row, then the four row maxima through scalar registers.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t x) {
    return max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max_nonneg(float v) {
    uint32_t x = __float_as_uint(v);
    x = dpp_max_u32<0xb1>(x);   // quad_perm [1,0,3,2]
    x = dpp_max_u32<0x4e>(x);   // quad_perm [2,3,0,1]
    x = dpp_max_u32<0x141>(x);  // row_half_mirror
    x = dpp_max_u32<0x140>(x);  // row_mirror
    const uint32_t a = __builtin_amdgcn_readlane(x, 0), b = __builtin_amdgcn_readlane(x, 16);
    const uint32_t c = __builtin_amdgcn_readlane(x, 32), d = __builtin_amdgcn_readlane(x, 48);
    return __uint_as_float(max(max(a, b), max(c, d)));
}

// Unsigned maximum over each group of LW consecutive lanes (16, 32 or 64), in every lane of
// the group and without scalar round trips: DPP steps within each 16-lane row, then
// v_permlane16_swap (rows 0 <-> 1 and 2 <-> 3) for groups of 32 and v_permlane32_swap
// (halves) for the whole wave, each followed by a max of the two swapped copies.
template <int LW>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t x) {
    static_assert(LW == 16 || LW == 32 || LW == 64, "groups of 16, 32 or 64 lanes");
    x = dpp_max_u32<0xb1>(x);   // quad_perm [1,0,3,2]
    x = dpp_max_u32<0x4e>(x);   // quad_perm [2,3,0,1]
    x = dpp_max_u32<0x141>(x);  // row_half_mirror
    x = dpp_max_u32<0x140>(x);  // row_mirror: every lane of a row holds the row max
    if constexpr (LW >= 32) {
        const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        x = max((uint32_t)a[0], (uint32_t)a[1]);
    }
    if constexpr (LW == 64) {
        const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        x = max((uint32_t)b[0], (uint32_t)b[1]);
    }
    return x;
}
__device__ __forceinline__ uint32_t wave_max_all_u32(uint32_t x) { return group_max_u32<64>(x); }

// ---------------------------------------------------------------------------------------
// Top-k of one row of bf16 selection scores held by a wave: torch.topk(k, largest=True,
// sorted=True) of attn_topk (primitives.py:50).  Lane l holds raw[i] = the bf16 bits of the
// score of block u = l + 64 i (blocks u >= nb are ignored).  Each score becomes a 32-bit key
// (order-preserving image of the bf16 bits << 16 | (0xffff - u)), so one unsigned max picks the
// largest score and, among equal scores, the lowest block index.  K rounds of a wave
// max-reduction emit the indices in descending score order (the order of exactly tied scores is
// unspecified in torch).  The wave max runs on DPP within each 16-lane row, then across rows
// with the two lane-swap permutes, leaving the maximum in every lane: no LDS or scalar round
// trips inside a selection round.  Indices go to idx32 / idx64 (either may be null) at
// out0 .. out0 + K - 1.

__device__ __forceinline__ uint32_t order16(uint32_t bits) {
    return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
}

// Insert x into the descending list (b0 >= b1 >= b2 >= b3); the smallest falls off.
__device__ __forceinline__ void insert4(uint32_t& b0, uint32_t& b1, uint32_t& b2, uint32_t& b3, uint32_t x) {
    uint32_t t = max(b0, x); x = min(b0, x); b0 = t;
    t = max(b1, x); x = min(b1, x); b1 = t;
    t = max(b2, x); x = min(b2, x); b2 = t;
    b3 = max(b3, x);
}

template <int PL>
__device__ __forceinline__ void select_topk(const uint32_t (&raw)[PL], int nb, int K, int lane, int64_t out0,
                                            int32_t* idx32, int64_t* idx64) {
    uint32_t key[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int u = lane + 64 * i;
        key[i] = (u < nb) ? ((order16(raw[i]) << 16) | (0xffffu - (uint32_t)u)) : 0u;
    }
    // Each lane keeps its four largest remaining keys.  Keys leave the wave in descending
    // order, so a lane's emitted keys are always its largest ones: after emitting key x the
    // lane's remaining keys are exactly those below x, and the buffer is refilled from them
    // only when all four buffered keys have been emitted.
    uint32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) insert4(b0, b1, b2, b3, key[i]);

    int mine = 0;  // lane (kk mod 64) keeps the kk-th index for one coalesced store
    for (int kk = 0; kk < K; ++kk) {
        const uint32_t mx = wave_max_all_u32(b0);
        const int u = (int)(0xffffu - (mx & 0xffffu));
        const bool win = b0 == mx;
        if (win) {
            b0 = b1;
            b1 = b2;
            b2 = b3;
            b3 = 0;
        }
        if (PL > 4 && __builtin_amdgcn_ballot_w64(win && b0 == 0)) {
            if (win && b0 == 0) {
#pragma unroll
                for (int i = 0; i < PL; ++i) insert4(b0, b1, b2, b3, key[i] < mx ? key[i] : 0u);
            }
        }
        if ((kk & 63) == lane) mine = u;
        if ((kk & 63) == 63 || kk == K - 1) {
            const int base = kk & ~63;
            if (lane <= kk - base) {
                if (idx32) idx32[out0 + base + lane] = mine;
                if (idx64) idx64[out0 + base + lane] = mine;
            }
        }
    }
}

// Batcher's odd-even merge sort network over N keys (N a power of two), descending.  All
// indices are compile-time constants, so the keys stay in registers; keys fixed at zero
// (padding) fold away.
template <int N>
__device__ __forceinline__ void sort_desc(uint32_t (&a)[N]) {
#pragma unroll
    for (int p = 1; p < N; p += p)
#pragma unroll
        for (int k = p; k > 0; k >>= 1)
#pragma unroll
            for (int j = k % p; j < N - k; j += k + k)
#pragma unroll
                for (int i = 0; i < k; ++i)
                    if (i + j + k < N && (i + j) / (p + p) == (i + j + k) / (p + p)) {
                        const uint32_t x = a[i + j], y = a[i + j + k];
                        a[i + j] = max(x, y);
                        a[i + j + k] = min(x, y);
                    }
}

// Row stride (words) of the per-lane sorted key lists of select_topk_sorted: at least PL + 1
// (the list and a zero sentinel), odd so the 64 lanes' reads of one round hit distinct banks.
template <int PL>
constexpr int kSortedStride = (PL + 1) | 1;

// The same selection as select_topk (same keys, same order of the emitted indices) for
// PL <= 16 and K <= LW, with no branch in a round.  The row is held by a group of LW
// consecutive lanes (the whole wave, or 2 or 4 rows per wave in groups of 32 or 16); lane lr of
// the group holds raw[i] = the score of block u = lr + LW i.  Each lane first sorts its keys
// (a sorting network in registers) and writes them, descending and followed by a zero, to its
// row of `list` (this wave's 64 x kSortedStride<PL> words of LDS, row = the lane).  A round is
// then the group maximum of the lanes' current keys (head), a compare, and the winner's step
// to its next key, read from LDS one round ahead (nxt), so the read's latency overlaps the
// next round's reduction.  Lane kk of the group keeps the kk-th emitted key; the indices are
// stored once at the end (not when `live` is false: a group past the last row).
typedef __attribute__((address_space(3))) uint32_t lds_u32;

template <int PL, int LW = 64>
__device__ __forceinline__ void select_topk_sorted(const uint32_t (&raw)[PL], int nb, int K, int lane,
                                                   int64_t out0, int32_t* idx32, int64_t* idx64,
                                                   lds_u32* list, int lr = -1, bool live = true) {
    constexpr int N = PL <= 1 ? 1 : PL <= 2 ? 2 : PL <= 4 ? 4 : PL <= 8 ? 8 : 16;
    static_assert(PL <= 16, "at most 16 keys per lane");
    if (LW == 64) lr = lane;
    uint32_t key[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int u = lr + LW * i;
        key[i] = (i < PL && u < nb) ? ((order16(raw[i < PL ? i : 0]) << 16) | (0xffffu - (uint32_t)u)) : 0u;
    }
    sort_desc<N>(key);
    lds_u32* row = list + lane * kSortedStride<PL>;
#pragma unroll
    for (int i = 0; i < PL; ++i) row[i] = key[i];
    row[PL] = 0u;
    uint32_t head = key[0], nxt = row[1];  // row[w], row[w + 1]
    int w = 0;  // keys of this lane emitted so far
    uint32_t mine = 0;
    for (int kk = 0; kk < K; ++kk) {
        const uint32_t mx = group_max_u32<LW>(head);
        const bool win = head == mx;
        w += win ? 1 : 0;
        head = win ? nxt : head;
        nxt = row[min(w + 1, PL)];
        mine = kk == lr ? mx : mine;
    }
    if (live && lr < K) {
        const int u = (int)(0xffffu - (mine & 0xffffu));
        if (idx32) idx32[out0 + lr] = u;
        if (idx64) idx64[out0 + lr] = u;
    }
}

// 2-D RoPE of one bf16 pair (x0, x1) packed in a word, by angle (c = cos, s = sin):
// (x0 c - x1 s, x1 c + x0 s) in fp32 with both products and the sum rounded separately (no
// fused multiply-add), as the reference's elementwise tensor ops round them
// (primitives.py:125-135), then rounded to bf16.
__device__ __forceinline__ float rope_mul_sub(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b - c * d;
}
__device__ __forceinline__ float rope_mul_add(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b + c * d;
}
__device__ __forceinline__ uint32_t rope_pair(uint32_t w, float c, float s) {
    const float x0 = bf_lo(w), x1 = bf_hi(w);
    return pack_bf16x2(rope_mul_sub(x0, c, x1, s), rope_mul_add(x1, c, x0, s));
}

// Map a linear workgroup id to a logical tile so that each of the 8 XCDs (which receive
// workgroups round-robin) works on one contiguous range of logical tiles and keeps that
// range's K/V blocks in its own L2.
__device__ __forceinline__ int xcd_remap(int id, int total) {
    const int xcd = id & 7, pos = id >> 3;
    const int per = total >> 3, rem = total & 7;
    return xcd * per + min(xcd, rem) + pos;
}

// ---------------------------------------------------------------------------------------
// Kernel parameter blocks (passed by value).

struct PoolParams {
    const bf16_t* x[3];        // q, k, v (x[i] may be null when that tensor is not pooled)
    int64_t sb[3], sn[3], sh[3];
    int heads[3];
    bf16_t* out_bnhd[3];       // [B, nb, H, 64] outputs (null: not written)
    // Optional MFMA-operand-ordered outputs for the compressed-attention kernel, zero past nb
    // (layouts at kfrag_index / vfrag_index):
    bf16_t* kfrag;             // tensor 1 as the A operand of S^T = K Q^T
    bf16_t* vfrag;             // tensor 2 as the A operand of O^T = V^T P^T
    float* kbnd;               // optional [B, nb, H1, 8]: per 8-dim chunk of tensor 1, the block's
                               // largest squared chunk norm (their sum bounds |k|^2 in the block)
    // Optional 2-D RoPE of tensors 0 and 1 before pooling: fp32 cos / sin tables [N, 32]
    // (one per token and rotated pair), rotated bf16 copies written to rot[0..1]
    // ([B, N, H, 64] contiguous); the pooled outputs and bounds are then those of the
    // rotated tensors.
    const float* rope_cos;
    const float* rope_sin;
    bf16_t* rot[2];
    int rope_lds;              // the block's table rows are staged in dynamic LDS (bs * 256 bytes)
    int B, nb, nb_pad, bs;
};

struct CmpParams {
    const bf16_t* qc; int64_t q_sb, q_sn, q_sh;   // pooled queries [B, nb, Hq, 64]
    const bf16_t* kfr;                             // pooled keys, operand order (kfrag_index)
    const bf16_t* vfr;                             // pooled values, operand order (vfrag_index)
    bf16_t* sbar;                                  // selection scores [B, Hk, nb, nb_pad]
    float* opart;                                  // [B, U, nb, Hq, 64] unnormalised O
    float2* ml;                                    // [B, U, nb, Hq] (running max, sum), log2 units
    bf16_t* ocmp;                                  // one split (nsplit == 1): the compressed-branch
                                                   // output [B, nb, Hq, 64] = bf16(O / l), written
                                                   // here instead of opart / ml; else null
    int B, nb, nb_pad, Hq, Hk, G, nsplit, ut_total;
    float scale_log2;                              // softmax_scale * log2(e)
};

// Combination of the compressed-attention split partials into the final compressed-branch
// output of one (batch, block) for all query heads (done by the top-k kernel, or by a
// combine-only kernel when there is no selection).
struct CombineParams {
    const float* opart;  // [B, U, nb, Hq, 64] unnormalised O per split
    const float2* ml;    // [B, U, nb, Hq] (max, sum) per split, log2 units
    bf16_t* ocmp;        // [B, nb, Hq, 64] compressed-branch output
    int nsplit, Hq;
};

struct TopkParams {
    const bf16_t* sbar;  // [B, Hk, nb, nb_pad]
    int32_t* idx32;      // optional [B, nb, Hk, K]
    int64_t* idx64;      // optional [B, nb, Hk, K]
    int B, nb, nb_pad, Hk, K, rows;
    int G;               // query heads per kv head (heads g*Hk + h of row h are combined)
    CombineParams cmb;   // cmb.ocmp == nullptr: no compressed-branch combine
    int* zero_ctr;       // optional: set to 0 (the attention kernel's dynamic-tail counter)
};

enum AttnMode : int {
    kModeFull = 0,
    kModeLocalOnly = 1,
    kModeNoCompression = 2,
    kModeNoSelection = 3,
    kModeSelectedOnly = 4,
};

struct AttnParams {
    const bf16_t* q; int64_t q_sb, q_sn, q_sh;
    const bf16_t* k; int64_t k_sb, k_sn, k_sh;
    const bf16_t* v; int64_t v_sb, v_sn, v_sh;
    const bf16_t* w; int64_t w_ss, w_sb, w_sn, w_sh;
    bf16_t* out;             // [B, N, Hq, 64], heads contiguous
    int64_t out_sb, out_sn;  // element strides of out's batch and token dimensions
    float* lse;              // [B, N, Hq] (selected-only mode, optional)
    const void* idx;         // [B, nb, Hk, K] int32 or int64
    const bf16_t* ocmp;      // compressed-branch output [B, nb, Hq, 64]
    const float* kbnd;       // key-norm bounds per selected block [B, nb, Hk, 8] (optional)
    // Optional 2-D RoPE of q inside the kernel (modes with a partial buffer): fp32 cos / sin
    // tables [N, 32]; q is read unrotated and rotated in registers.
    const float* rope_cos;
    const float* rope_sin;
    int B, N, Hq, Hk, G;
    int bs_l, bs, K, nb;
    int head_groups;         // G / waves-per-workgroup
    int qtiles;              // N / 64
    int total_wgs;           // work items (b, kv head, head group, query tile)
    // Dynamic tail: items [n_static, total_wgs) go to the tail_wgs workgroups launched after
    // the n_static statically mapped ones, each taking the next item from *tail_ctr (0 at
    // launch; the last taker resets it), so the compute units that finish their static items
    // first take more of the last items.  tail_ctr null: n_static = total_wgs, no tail.
    int n_static, tail_wgs;
    int* tail_ctr;
    float scale;             // softmax scale
    float scale_log2;        // softmax scale * log2(e)
};

// The attention block's input side (proj.hip): y = x W^T over the stacked q | k | v | gate
// weights, RoPE of q and k, the gate softmax and the block pooling in one kernel.
struct ProjParams {
    const bf16_t* x; int64_t x_sn, x_sb;   // token n of member b at x + n x_sn + b x_sb (D contiguous)
    const bf16_t* w;                       // [n_tiles * 256, D]: 64-row groups q heads | k | v | gates | zero
    int S, B, D, Hq, Hk;
    int gates;                             // a gate group follows the v heads (3 Hq <= 64 logits)
    int n_tiles;                           // 256-column tiles of w
    const float* rope_cos;                 // [S, 32] RoPE tables, or null (no rotation)
    const float* rope_sin;
    bf16_t* q; bf16_t* k; bf16_t* v;       // [B, S, H, 64] contiguous (q and k rotated)
    bf16_t* wts;                           // [B, S, Hq, 3] branch weights (gates)
    int bs;                                // pooled block size (64 or 128), 0: no pooling
    int nb, nb_pad;
    bf16_t* qc;                            // [B, nb, Hq, 64] pooled q
    bf16_t* kfrag;                         // pooled k, operand order (kfrag_index), zero past nb
    bf16_t* vfrag;                         // pooled v, operand order (vfrag_index), or null
    float* kbnd;                           // [B, nb, Hk, 8] largest squared chunk norms, or null
};

// Host-side launchers (defined next to each kernel).
hipError_t launch_proj(const ProjParams& p, hipStream_t s);
hipError_t launch_pool(const PoolParams& p, hipStream_t s);
hipError_t launch_cmp(const CmpParams& p, bool scores, bool attn, hipStream_t s);
hipError_t launch_topk(const TopkParams& p, hipStream_t s);
hipError_t launch_combine(const CombineParams& c, int B, int nb, hipStream_t s);
hipError_t launch_attn(const AttnParams& p, int mode, bool idx64, int waves, hipStream_t s);

// k-nearest-neighbour cross-attention between grids (interp.hip).
struct InterpParams {
    const bf16_t* k; int64_t k_sn, k_sb, k_sh;   // [S_from, B, H, 64]: point, member, head strides
    const bf16_t* v; int64_t v_sn, v_sb, v_sh;
    const int32_t* neighbors;                    // [S_to, K] source points of each target
    const int32_t* target_order;                 // [S_to] order the targets are taken in, or null
    const float* rel_pos;                        // [S_to, K, 3] normalised relative positions
    const bf16_t* w_q;                           // [H * 64, 3] query projection (to_q.weight)
    bf16_t* out;                                 // [S_to, B, H, 64] contiguous
    int S_from, S_to, B, H, K;
    float scale;
    float scale_log2e;                           // scale * log2 e
    int scale_pow2;                              // scale is a power of two
    int round_products;                          // products rounded to bf16 (eager) or fp32
};
hipError_t launch_knn_attn(const InterpParams& p, hipStream_t s);

// Tiles of consecutive targets (in the target order) for the LDS-staged k-NN kernel: each tile
// stages the distinct source rows its targets use once per (member, head).  Built on the host
// from the neighbour lists and the order (static per grid pair).
constexpr int kKnnTileTargets = 16;  // targets per tile at most (4 per wave)
constexpr int kKnnTileRows = 128;    // distinct source points per tile at most
struct KnnTiles {
    const int32_t* start;  // [n + 1]: tile i holds the targets at order positions [start[i], start[i + 1])
    const int32_t* src;    // [n, rows]: the tile's distinct source points (the first nsrc[i] used)
    const int32_t* nsrc;   // [n]
    const int32_t* slot;   // [S_to, K]: neighbour j of the target at order position pos is row
                           // slot[pos, j] of its tile's src
    int n, rows;           // rows: a multiple of 8, at most kKnnTileRows (the LDS staging capacity)
};
hipError_t launch_knn_attn_tiled(const InterpParams& p, const KnnTiles& t, hipStream_t s);
// whether launch_knn_attn_tiled takes p (fp32 products, 32-bit chunk offsets)
bool knn_tiled_supported(const InterpParams& p);

// Maximum number of selected blocks per query block (block indices are staged in LDS).
constexpr int kMaxSelected = 1024;

// Most compressed-attention splits (partials per row).
constexpr int kMaxSplits = 4;

// The compressed-branch output at block t of NH heads j0, j0 + jstep, ..., combined over the
// splits: lane owns dimension d = lane.  exp2 weights are relative to the largest split max.
// All loads of all heads and splits are issued before any arithmetic (one memory round trip).
// They are unconditional (past nsplit: the last split again, not used): loads under a branch
// leave the compiler's count of loads in flight unknown at the join, and the first wait after
// it then waits for all of them.  combine_load issues the loads and combine_store combines
// and stores; other work can sit between the two, so the loads' latency overlaps it.
template <int NH, int E = 1>  // E: elements (dimensions) of each head per lane
struct CombineRows {
    float2 mlv[NH][kMaxSplits];
    float ov[NH][kMaxSplits][E];
};

template <int NH>
__device__ __forceinline__ void combine_load(CombineRows<NH>& r, const CombineParams& c, int b, int nb, int t, int j0,
                                             int jstep, int lane) {
    const int64_t stride = (int64_t)nb * c.Hq;
    // written by an earlier launch and only read here: the constant address space lets the
    // compiler take the scalar path for the uniform (max, sum) rows
    typedef const __attribute__((address_space(4))) float cfloat;
    cfloat* ml = (cfloat*)c.ml;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int64_t row0 = ((int64_t)b * c.nsplit * nb + t) * c.Hq + j0 + h * jstep;
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; ++sp) {
            const int64_t row = row0 + min(sp, c.nsplit - 1) * stride;
            r.mlv[h][sp] = make_float2(ml[2 * row], ml[2 * row + 1]);
            r.ov[h][sp][0] = c.opart[row * kHeadDim + lane];
        }
    }
}

// Combined value of head h, element e of one lane's loaded partials: exp2 weights relative to
// the largest split max.  One split: its weight exp2(m - m) is exactly 1, so the value is
// o / l, taken directly (the same result without the exponentials).
template <int NH, int E = 1>
__device__ __forceinline__ float combine_value(const CombineRows<NH, E>& r, int h, int e, int nsplit) {
    if (nsplit == 1) return r.ov[h][0][e] / r.mlv[h][0].y;
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
        if (sp < nsplit) M = fmaxf(M, r.mlv[h][sp].x);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp) {
        if (sp < nsplit) {
            const float a = __builtin_amdgcn_exp2f(r.mlv[h][sp].x - M);
            L += a * r.mlv[h][sp].y;
            acc += a * r.ov[h][sp][e];
        }
    }
    return acc / L;
}

template <int NH>
__device__ __forceinline__ void combine_store(const CombineRows<NH>& r, const CombineParams& c, int b, int nb, int t,
                                              int j0, int jstep, int lane) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int j = j0 + h * jstep;
        c.ocmp[(((int64_t)b * nb + t) * c.Hq + j) * kHeadDim + lane] =
            (bf16_t)(pack_bf16x2(combine_value<NH>(r, h, 0, c.nsplit), 0.f) & 0xffffu);
    }
}

// The same for E = 64 / LW dimensions per lane, when a row's 64 dimensions are spread over a
// group of LW lanes (lane lr of the group: dimensions E lr .. E lr + E - 1).  The (max, sum)
// pairs differ between the groups of a wave, so they are vector loads here.
template <int NH, int E>
__device__ __forceinline__ void combine_load_group(CombineRows<NH, E>& r, const CombineParams& c, int b, int nb,
                                                   int t, int j0, int jstep, int lr) {
    const int64_t stride = (int64_t)nb * c.Hq;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int64_t row0 = ((int64_t)b * c.nsplit * nb + t) * c.Hq + j0 + h * jstep;
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; ++sp) {
            const int64_t row = row0 + min(sp, c.nsplit - 1) * stride;
            r.mlv[h][sp] = c.ml[row];
            const float* src = c.opart + row * kHeadDim + E * lr;
            if constexpr (E == 4) {
                const float4 v = *reinterpret_cast<const float4*>(src);
                r.ov[h][sp][0] = v.x; r.ov[h][sp][1] = v.y; r.ov[h][sp][2] = v.z; r.ov[h][sp][3] = v.w;
            } else if constexpr (E == 2) {
                const float2 v = *reinterpret_cast<const float2*>(src);
                r.ov[h][sp][0] = v.x; r.ov[h][sp][1] = v.y;
            } else {
                r.ov[h][sp][0] = src[0];
            }
        }
    }
}

template <int NH, int E>
__device__ __forceinline__ void combine_store_group(const CombineRows<NH, E>& r, const CombineParams& c, int b, int nb,
                                                    int t, int j0, int jstep, int lr) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int j = j0 + h * jstep;
        bf16_t* dst = c.ocmp + (((int64_t)b * nb + t) * c.Hq + j) * kHeadDim + E * lr;
        uint32_t w[(E + 1) / 2];
#pragma unroll
        for (int e = 0; e < E; e += 2) {
            const float v0 = combine_value<NH, E>(r, h, e, c.nsplit);
            const float v1 = e + 1 < E ? combine_value<NH, E>(r, h, e + 1 < E ? e + 1 : e, c.nsplit) : 0.f;
            w[e / 2] = pack_bf16x2(v0, v1);
        }
        if constexpr (E == 4) *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
        else if constexpr (E == 2) *reinterpret_cast<uint32_t*>(dst) = w[0];
        else *dst = (bf16_t)(w[0] & 0xffffu);
    }
}

template <int NH>
__device__ __forceinline__ void combine_ocmp(const CombineParams& c, int b, int nb, int t, int j0, int jstep, int lane) {
    CombineRows<NH> r;
    combine_load<NH>(r, c, b, nb, t, j0, jstep, lane);
    combine_store<NH>(r, c, b, nb, t, j0, jstep, lane);
}

}  // namespace mosaic
