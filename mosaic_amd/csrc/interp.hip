// interp.hip -- k-nearest-neighbour cross-attention between two grids (gfx950).
//
// Replaces the gather-attention of CrossAttentionInterpolate.forward (primitives.py:265-283):
//   q[s, j]    = to_q(rel_pos[s, j])            (Linear 3 -> H*64, bf16 out)
//   score      = sum_d bf16(q[s, j, h, d] * k[n(s, j), b, h, d])  -> bf16, * scale -> bf16
//   w          = softmax_j(score) in fp32, then bf16        (softmax over the K neighbours)
//   out[s,b,h] = sum_j bf16(w[j] * v[n(s, j), b, h, :])      -> bf16
// with the reference's rounding points (bf16 elementwise products, fp32 sums rounded once).
// The reference materialises q [S_to, K, H*64] and the gathered k, v [S_to, K, B, H*64];
// here q is formed in registers from the three rel_pos numbers and the head's 64x3 slice of
// to_q, and the k / v rows are read straight from [S_from, B, H, 64] (neighbouring targets
// share most of their neighbours, so rows are reused from L2).
//
// The work is VALU-bound: every (target, member, head) takes 2 K 64 bf16-rounded products.
// Each product is one v_dot2_f32_bf16 of the packed k / v pair against (x, 0) or (0, x)
// (exact: a bf16 x bf16 product fits fp32), then half a v_cvt_pk_bf16_f32 and half a
// v_dot2_f32_bf16 that adds the rounded pair; no k / v element is unpacked to fp32.
// Staging each tile of targets' neighbour union in LDS (cutting the L2 requests 4-7x)
// measured slower than this direct form: it halves the occupancy, and occupancy is what
// hides the latency of the reduction chains.
//
// One wave per (target s, head h) pair, looping over the batch members b with the next
// member's k / v loaded as soon as the current member is done with them.  Lane l = 8 jg + dc holds the 8-dim chunk dc of neighbours
// jg + 8 i (its "slots"): every k / v read is a 16-byte load and each 128-byte row is read
// by 8 adjacent lanes.  Scores are summed over the 8 chunk lanes with DPP (lanes l ^ 1,
// l ^ 2, l ^ 4), the softmax max / sum over the 8 neighbour groups with DPP row_ror:8,
// v_permlane16_swap and v_permlane32_swap; the output's 8 partial sums per lane are
// reduce-scattered over the groups by the same three exchanges, leaving one dimension per
// lane.  Workgroups are remapped so that each XCD takes one contiguous range of targets, in
// the caller's target order when one is given: with targets sorted along a space-filling
// curve, the waves in flight on an XCD share most of their neighbours' rows in its L2.
#include "bsa_common.h"

#include <type_traits>

namespace mosaic {
namespace {

constexpr int kInterpWaves = 4;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    // every lane's source lane exists for the patterns used here, so the old value and the
    // bound control never matter; with an undefined old value the compiler folds the move
    // into the add (with old = 0 it kept a separate move and a zeroing move for
    // row_half_mirror)
    return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
    return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false)));
}

// x summed over the 8 chunk lanes of its neighbour group (lanes l ^ 1, l ^ 2, l ^ 4)
__device__ __forceinline__ float chunk_sum(float x) {
    x = dpp_add<0xb1>(x);      // quad_perm [1,0,3,2]
    x = dpp_add<0x4e>(x);      // quad_perm [2,3,0,1]
    return dpp_add<0x141>(x);  // row_half_mirror
}

// v_permlane16_swap(a, b): rows 1 and 3 of a trade places with rows 0 and 2 of b.  The
// returned pair, summed, is a[l] + a[l ^ 16] in even rows and b[l] + b[l ^ 16] in odd rows.
__device__ __forceinline__ float swap16_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v_permlane32_swap(a, b): lanes 32-63 of a trade places with lanes 0-31 of b.  The pair,
// summed, is a[l] + a[l ^ 32] in lanes 0-31 and b[l] + b[l ^ 32] in lanes 32-63.
__device__ __forceinline__ float swap32_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x summed / maximised over the 8 neighbour groups (lanes l ^ 8, l ^ 16, l ^ 32)
__device__ __forceinline__ float group_sum(float x) {
    x = dpp_add<0x128>(x);  // row_ror:8 within a 16-lane row: lane l ^ 8
    return xor32_add(swap16_add(x, x));
}
__device__ __forceinline__ float group_max(float x) {
    x = dpp_max<0x128>(x);
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Exact bf16 products without unpacking: with a = (x, 0) or (0, x) (x bf16 in the low or
// high half), v_dot2_f32_bf16 of a and a packed bf16 pair b is x times the matching half of b,
// plus 0 (a bf16 x bf16 product is exact in fp32).  A dot product's result needs three wait
// states before another VALU instruction reads it, and the compiler does not track that
// through inline assembly, so the blocks below put their eight products first, every
// rounding (v_cvt_pk_bf16_f32 of a pair) reads products at least three instructions old, and
// each block ends with s_nop 2 before its sums are read.  The additions are dot products
// too, chained through the accumulator operand of the same instruction, which needs no wait.
//
// A neighbour's score partial over this lane's 8 dimensions: the eight products q[i] . k
// (q[i] = (x, 0) or (0, x) against the packed pairs of k), rounded to bf16 in pairs and added
// in fp32 by dot products with ones = (1, 1), in dimension order from 0.
__device__ __forceinline__ float score_partial(const uint32_t (&q)[8], const uint4& k, uint32_t ones) {
    float part, t0, t1, t2, t3, t4, t5, t6, t7;
    uint32_t c0, c1, c2, c3;
    asm("v_dot2_f32_bf16 %5, %13, %21, 0\n\t"
        "v_dot2_f32_bf16 %6, %14, %21, 0\n\t"
        "v_dot2_f32_bf16 %7, %15, %22, 0\n\t"
        "v_dot2_f32_bf16 %8, %16, %22, 0\n\t"
        "v_dot2_f32_bf16 %9, %17, %23, 0\n\t"
        "v_dot2_f32_bf16 %10, %18, %23, 0\n\t"
        "v_dot2_f32_bf16 %11, %19, %24, 0\n\t"
        "v_dot2_f32_bf16 %12, %20, %24, 0\n\t"
        "v_cvt_pk_bf16_f32 %1, %5, %6\n\t"
        "v_cvt_pk_bf16_f32 %2, %7, %8\n\t"
        "v_cvt_pk_bf16_f32 %3, %9, %10\n\t"
        "v_cvt_pk_bf16_f32 %4, %11, %12\n\t"
        "v_dot2_f32_bf16 %0, %1, %25, 0\n\t"
        "v_dot2_f32_bf16 %0, %2, %25, %0\n\t"
        "v_dot2_f32_bf16 %0, %3, %25, %0\n\t"
        "v_dot2_f32_bf16 %0, %4, %25, %0\n\t"
        "s_nop 2"
        : "=v"(part), "=v"(c0), "=v"(c1), "=v"(c2), "=v"(c3),
          "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)
        : "v"(q[0]), "v"(q[1]), "v"(q[2]), "v"(q[3]), "v"(q[4]), "v"(q[5]), "v"(q[6]), "v"(q[7]),
          "v"(k.x), "v"(k.y), "v"(k.z), "v"(k.w), "s"(ones));
    return part;
}

// Two neighbours' (weights a and b) contributions to four output dimensions 2m .. 2m + 3:
// acc[e] (+)= bf16(wa v_a[d]) + bf16(wb v_b[d]) for d = 2m + e, the products formed as above
// from (w, 0) / (0, w) and the packed pairs va0 = v_a[2m, 2m+1], va1 = v_a[2m+2, 2m+3] (vb0,
// vb1 of b), each pair rounded by one v_cvt_pk_bf16_f32 and added by a dot product with
// (1, 1) -- starting from 0 when FIRST.  Ends with the three wait states the sums need.
template <bool FIRST>
__device__ __forceinline__ void out_pair(uint32_t wa_lo, uint32_t wb_lo, uint32_t wa_hi, uint32_t wb_hi,
                                         uint32_t va0, uint32_t vb0, uint32_t va1, uint32_t vb1, uint32_t ones,
                                         float* acc) {
    float t0, t1, t2, t3, t4, t5, t6, t7;
    uint32_t c0, c1, c2, c3;
#define MOSAIC_OUT_PAIR_PRODUCTS                          \
    "v_dot2_f32_bf16 %8, %16, %20, 0\n\t"                \
    "v_dot2_f32_bf16 %9, %17, %21, 0\n\t"                \
    "v_dot2_f32_bf16 %10, %18, %20, 0\n\t"               \
    "v_dot2_f32_bf16 %11, %19, %21, 0\n\t"               \
    "v_dot2_f32_bf16 %12, %16, %22, 0\n\t"               \
    "v_dot2_f32_bf16 %13, %17, %23, 0\n\t"               \
    "v_dot2_f32_bf16 %14, %18, %22, 0\n\t"               \
    "v_dot2_f32_bf16 %15, %19, %23, 0\n\t"               \
    "v_cvt_pk_bf16_f32 %4, %8, %9\n\t"                   \
    "v_cvt_pk_bf16_f32 %5, %10, %11\n\t"                 \
    "v_cvt_pk_bf16_f32 %6, %12, %13\n\t"                 \
    "v_cvt_pk_bf16_f32 %7, %14, %15\n\t"
#define MOSAIC_OUT_PAIR_OPERANDS                                                                      \
    "=v"(c0), "=v"(c1), "=v"(c2), "=v"(c3),                                                           \
        "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)      \
        : "v"(wa_lo), "v"(wb_lo), "v"(wa_hi), "v"(wb_hi), "v"(va0), "v"(vb0), "v"(va1), "v"(vb1), "s"(ones)
    if constexpr (FIRST) {
        asm(MOSAIC_OUT_PAIR_PRODUCTS
            "v_dot2_f32_bf16 %0, %4, %24, 0\n\t"
            "v_dot2_f32_bf16 %1, %5, %24, 0\n\t"
            "v_dot2_f32_bf16 %2, %6, %24, 0\n\t"
            "v_dot2_f32_bf16 %3, %7, %24, 0\n\t"
            "s_nop 2"
            : "=v"(acc[0]), "=v"(acc[1]), "=v"(acc[2]), "=v"(acc[3]), MOSAIC_OUT_PAIR_OPERANDS);
    } else {
        asm(MOSAIC_OUT_PAIR_PRODUCTS
            "v_dot2_f32_bf16 %0, %4, %24, %0\n\t"
            "v_dot2_f32_bf16 %1, %5, %24, %1\n\t"
            "v_dot2_f32_bf16 %2, %6, %24, %2\n\t"
            "v_dot2_f32_bf16 %3, %7, %24, %3\n\t"
            "s_nop 2"
            : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), MOSAIC_OUT_PAIR_OPERANDS);
    }
#undef MOSAIC_OUT_PAIR_PRODUCTS
#undef MOSAIC_OUT_PAIR_OPERANDS
}

// One neighbour (weight w, as (w, 0) and (0, w)) against all eight output dimensions of the
// lane: acc[d] (+)= bf16(w v[d]), the pair (2m, 2m + 1) rounded by one v_cvt_pk_bf16_f32 and
// its halves added by dot products with pick_lo = (1, 0) and pick_hi = (0, 1) (scalar
// registers: as a constant operand the compiler would encode (1, 0) as the inline constant
// 1.0, which the dot product reads as (0, 1)) -- starting from 0 when FIRST.
template <bool FIRST>
__device__ __forceinline__ void out_single(uint32_t w_lo, uint32_t w_hi, const uint4& v, uint32_t pick_lo,
                                           uint32_t pick_hi, float* acc) {
    float t0, t1, t2, t3, t4, t5, t6, t7;
    uint32_t c0, c1, c2, c3;
#define MOSAIC_OUT_SINGLE_PRODUCTS                        \
    "v_dot2_f32_bf16 %12, %20, %22, 0\n\t"               \
    "v_dot2_f32_bf16 %13, %21, %22, 0\n\t"               \
    "v_dot2_f32_bf16 %14, %20, %23, 0\n\t"               \
    "v_dot2_f32_bf16 %15, %21, %23, 0\n\t"               \
    "v_dot2_f32_bf16 %16, %20, %24, 0\n\t"               \
    "v_dot2_f32_bf16 %17, %21, %24, 0\n\t"               \
    "v_dot2_f32_bf16 %18, %20, %25, 0\n\t"               \
    "v_dot2_f32_bf16 %19, %21, %25, 0\n\t"               \
    "v_cvt_pk_bf16_f32 %8, %12, %13\n\t"                 \
    "v_cvt_pk_bf16_f32 %9, %14, %15\n\t"                 \
    "v_cvt_pk_bf16_f32 %10, %16, %17\n\t"                \
    "v_cvt_pk_bf16_f32 %11, %18, %19\n\t"
#define MOSAIC_OUT_SINGLE_OPERANDS                                                                    \
    "=v"(c0), "=v"(c1), "=v"(c2), "=v"(c3),                                                           \
        "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)      \
        : "v"(w_lo), "v"(w_hi), "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w), "s"(pick_lo), "s"(pick_hi)
    if constexpr (FIRST) {
        asm(MOSAIC_OUT_SINGLE_PRODUCTS
            "v_dot2_f32_bf16 %0, %8, %26, 0\n\t"
            "v_dot2_f32_bf16 %1, %8, %27, 0\n\t"
            "v_dot2_f32_bf16 %2, %9, %26, 0\n\t"
            "v_dot2_f32_bf16 %3, %9, %27, 0\n\t"
            "v_dot2_f32_bf16 %4, %10, %26, 0\n\t"
            "v_dot2_f32_bf16 %5, %10, %27, 0\n\t"
            "v_dot2_f32_bf16 %6, %11, %26, 0\n\t"
            "v_dot2_f32_bf16 %7, %11, %27, 0\n\t"
            "s_nop 2"
            : "=v"(acc[0]), "=v"(acc[1]), "=v"(acc[2]), "=v"(acc[3]), "=v"(acc[4]), "=v"(acc[5]), "=v"(acc[6]),
              "=v"(acc[7]), MOSAIC_OUT_SINGLE_OPERANDS);
    } else {
        asm(MOSAIC_OUT_SINGLE_PRODUCTS
            "v_dot2_f32_bf16 %0, %8, %26, %0\n\t"
            "v_dot2_f32_bf16 %1, %8, %27, %1\n\t"
            "v_dot2_f32_bf16 %2, %9, %26, %2\n\t"
            "v_dot2_f32_bf16 %3, %9, %27, %3\n\t"
            "v_dot2_f32_bf16 %4, %10, %26, %4\n\t"
            "v_dot2_f32_bf16 %5, %10, %27, %5\n\t"
            "v_dot2_f32_bf16 %6, %11, %26, %6\n\t"
            "v_dot2_f32_bf16 %7, %11, %27, %7\n\t"
            "s_nop 2"
            : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]), "+v"(acc[6]),
              "+v"(acc[7]), MOSAIC_OUT_SINGLE_OPERANDS);
    }
#undef MOSAIC_OUT_SINGLE_PRODUCTS
#undef MOSAIC_OUT_SINGLE_OPERANDS
}

// fp32 products (the reference under torch.compile: its fused reductions of (q * k).sum and
// (w * v).sum multiply and add in fp32 and round only the sums).  A neighbour's score partial
// over this lane's 8 dimensions: four dot products of packed (q, q) pairs against k's pairs,
// chained through the accumulator, in dimension order from 0.
__device__ __forceinline__ bf16x2_t as_bf2(uint32_t w) { return __builtin_bit_cast(bf16x2_t, w); }
__device__ __forceinline__ float score_dot(const uint32_t (&q)[4], const uint4& k) {
    float a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q[0]), as_bf2(k.x), 0.f, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q[1]), as_bf2(k.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q[2]), as_bf2(k.z), a, false);
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q[3]), as_bf2(k.w), a, false);
}
// One neighbour (weight w as (w, 0) and (0, w)) against the lane's eight output dimensions in
// fp32: acc[d] (+)= w v[d], one dot product per product.
template <bool FIRST>
__device__ __forceinline__ void out_fp32(uint32_t w_lo, uint32_t w_hi, const uint4& v, float* acc) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        acc[2 * e] = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w_lo), as_bf2(vv[e]), FIRST ? 0.f : acc[2 * e], false);
        acc[2 * e + 1] = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w_hi), as_bf2(vv[e]), FIRST ? 0.f : acc[2 * e + 1], false);
    }
}

// The score of a slot in base-2 units, sc = bf16(bf16(part) * scale) * log2 e.  A power-of-two
// scale leaves bf16(part) * scale a bf16 value (a product too small to be normal is below
// 2^-126 in magnitude, and so is the difference its rounding would make), so that case takes
// one multiply by scale * log2 e.
template <bool POW2>
__device__ __forceinline__ float scaled_score(float part, const InterpParams& p) {
    return POW2 ? round_bf16(part) * p.scale_log2e : round_bf16(round_bf16(part) * p.scale) * kLog2e;
}

// Softmax weights of the lane's slots over the K neighbours, from the slots' base-2 scores and
// the lane's own maximum m: exp2(sc - max) / sum (0 for an absent neighbour: score -inf, the
// maximum finite).
template <int NSLOT>
__device__ __forceinline__ void softmax_weights(const float (&sc)[NSLOT], float m, float (&w)[NSLOT]) {
    m = group_max(m);
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
        w[i] = __builtin_amdgcn_exp2f(sc[i] - m);
        l += w[i];
    }
    const float inv = __builtin_amdgcn_rcpf(group_sum(l));
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) w[i] *= inv;
}

// acc[d] = sum over the lane's slots of w * v[d] with exact products, slot by slot
template <int NSLOT>
__device__ __forceinline__ void weighted_sum_fp32(const float (&w)[NSLOT], const uint4 (&vw)[NSLOT], float (&acc)[8]) {
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
        const uint32_t w_lo = pack_bf16x2(w[i], 0.f), w_hi = pack_bf16x2(0.f, w[i]);
        if (i == 0) out_fp32<true>(w_lo, w_hi, vw[i], acc);
        else out_fp32<false>(w_lo, w_hi, vw[i], acc);
    }
}

// The lane's 8 partial output dimensions reduce-scattered over the 8 neighbour groups: halves
// (dims e / e + 4), row pairs (e / e + 2), then lanes l ^ 8 (e / e + 1); the lane ends up with
// dimension 8 dc + 4 (l / 32) + 2 ((l / 16) % 2) + (l / 8) % 2 summed over all neighbours.
__device__ __forceinline__ float reduce_scatter(const float (&acc)[8], int lane) {
    float r4[4], r2[2];
#pragma unroll
    for (int e = 0; e < 4; ++e) r4[e] = swap32_add(acc[e], acc[e + 4]);
#pragma unroll
    for (int e = 0; e < 2; ++e) r2[e] = swap16_add(r4[e], r4[e + 2]);
    const bool odd8 = lane & 8;
    const float keep = odd8 ? r2[1] : r2[0], give = odd8 ? r2[0] : r2[1];
    return keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(give), 0x128, 0xf, 0xf, false));
}

__device__ __forceinline__ void unpack8(const uint4& w, float (&f)[8]) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) { f[2 * e] = bf_lo(a[e]); f[2 * e + 1] = bf_hi(a[e]); }
}

// The 16-byte chunk at byte offset off from a member's base (wave-uniform).  With 32-bit
// offsets the load is a raw buffer load: base in the resource (scalar registers), the offset
// as its per-lane offset, so the member loop spends no vector instruction on addresses.
template <bool OFF32, typename Off>
__device__ __forceinline__ uint4 ld_member(const bf16_t* base, Off off) {
    if constexpr (OFF32) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, -1, 0x00020000);
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        return make_uint4(v[0], v[1], v[2], v[3]);
    } else {
        return ld16(reinterpret_cast<const char*>(base) + off);
    }
}

// Waves per SIMD each instantiation is compiled for (the register budget): 6 at three slots
// with 32-bit offsets (the model's K = 24), what fits without spilling elsewhere.
constexpr int knn_waves(int nslot, bool off32) { return nslot <= 1 ? 8 : nslot == 2 ? 7 : nslot == 3 ? (off32 ? 6 : 5) : 4; }

// RP: products rounded to bf16 (the reference's eager elementwise ops); else fp32 products
template <int NSLOT, bool OFF32, bool POW2, bool RP>
__global__ __launch_bounds__(kInterpWaves * 64) __attribute__((amdgpu_waves_per_eu(knn_waves(NSLOT, OFF32)))) void knn_attn_kernel(InterpParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t pair = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * kInterpWaves + wave;
    if (pair >= (int64_t)p.S_to * p.H) return;  // wave-uniform; the kernel has no barrier
    const int pos = (int)(pair / p.H), h = (int)(pair - (int64_t)pos * p.H);
    // targets outside [0, S_to) in the order are clamped (memory safety)
    const int s = p.target_order ? min(max(p.target_order[pos], 0), p.S_to - 1) : pos;
    const int K = p.K, dc = lane & 7, jg = lane >> 3;

    // to_q rows h*64 + 8 dc .. + 7 (three bf16 weights each: 48 bytes, 16-byte aligned)
    float wq[24];
    {
        const bf16_t* wr = p.w_q + ((int64_t)h * 64 + 8 * dc) * 3;
        float t[8];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            unpack8(ld16(wr + 8 * c), t);
#pragma unroll
            for (int e = 0; e < 8; ++e) wq[8 * c + e] = t[e];
        }
    }
    // per slot: the neighbour's row offsets and this lane's 8 query values,
    // q[j][d] = bf16(rel[j] . W[h*64 + d]) (fp32 sum of the three bf16 products: the
    // Linear's bf16 inputs)
    // byte offsets of this lane's k / v chunks within a member (32 bits when they fit)
    using Off = typename std::conditional<OFF32, uint32_t, int64_t>::type;
    Off koff[NSLOT], voff[NSLOT];
    // RP: q[j][d] as a bf16 in the half of a word that k's dim d occupies; else the packed
    // pairs (q[j][2m], q[j][2m + 1])
    uint32_t qp[NSLOT][RP ? 8 : 4];
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
        const int64_t sj = (int64_t)s * K + min(jg + 8 * i, K - 1);
        // indices outside [0, S_from) are clamped (memory safety; the reference would raise)
        const int64_t n = min(max(p.neighbors[sj], 0), p.S_from - 1);
        koff[i] = (Off)(2 * (n * p.k_sn + (int64_t)h * p.k_sh + 8 * dc));
        voff[i] = (Off)(2 * (n * p.v_sn + (int64_t)h * p.v_sh + 8 * dc));
        const float r0 = round_bf16(p.rel_pos[3 * sj]), r1 = round_bf16(p.rel_pos[3 * sj + 1]),
                    r2 = round_bf16(p.rel_pos[3 * sj + 2]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t bits = __float_as_uint(round_bf16(fmaf(r2, wq[3 * e + 2], fmaf(r1, wq[3 * e + 1], r0 * wq[3 * e]))));
            if constexpr (RP) qp[i][e] = (e & 1) ? bits : bits >> 16;
            else if (e & 1) qp[i][e >> 1] |= bits;
            else qp[i][e >> 1] = bits >> 16;
        }
    }
    // the output dimension this lane ends up holding after the reduce-scatter
    const int dout = 8 * dc + 4 * (lane >> 5) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1);
    bf16_t* out = p.out + ((int64_t)s * p.B * p.H + h) * 64 + dout;

    // k / v chunks of the current member; the next member's k is loaded as soon as the scores
    // are done with k, its v once the output is done with v
    uint4 kw[NSLOT], vw[NSLOT];
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) { kw[i] = ld_member<OFF32>(p.k, koff[i]); vw[i] = ld_member<OFF32>(p.v, voff[i]); }
    const uint32_t ones = 0x3f803f80u, pick_lo = 0x3f80u, pick_hi = 0x3f800000u;  // bf16 pairs (1, 1), (1, 0), (0, 1)
    for (int b = 0; b < p.B; ++b) {
        const bool more = b + 1 < p.B;
        // the fp32-product form loads the next member unconditionally (the last member again
        // after the last): a conditional load made the compiler copy every k / v register at
        // the loop's end
        const int64_t bn = more ? b + 1 : b;
        // scores of this lane's slots (every lane of a neighbour group holds its score)
        float sc[NSLOT], m;
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
            float part;
            if constexpr (RP) part = chunk_sum(score_partial(qp[i], kw[i], ones));
            else part = chunk_sum(score_dot(qp[i], kw[i]));
            // the score in base-2 units, sc = bf16(bf16(part) * scale) * log2 e.  A power-of-two
            // scale leaves bf16(part) * scale a bf16 value (a product too small to be normal is
            // below 2^-126 in magnitude, and so is the difference its rounding would make), so
            // that case takes one multiply by scale * log2 e.
            const float t = POW2 ? round_bf16(part) * p.scale_log2e : round_bf16(round_bf16(part) * p.scale) * kLog2e;
            // only the last slot can hold absent neighbours (j >= K): NSLOT = ceil(K / 8)
            sc[i] = i < NSLOT - 1 || jg + 8 * i < K ? t : -INFINITY;
            m = i == 0 ? sc[0] : fmaxf(m, sc[i]);
        }
        if (!RP || more) {
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) kw[i] = ld_member<OFF32>(p.k + bn * p.k_sb, koff[i]);
        }
        m = group_max(m);
        float ex[NSLOT], l = 0.f;
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
            ex[i] = __builtin_amdgcn_exp2f(sc[i] - m);  // 0 for an absent neighbour (score -inf; m is finite)
            l += ex[i];
        }
        const float inv = __builtin_amdgcn_rcpf(group_sum(l));
        // out[d] = sum over slots of bf16(w * v[d]); two slots at a time share one rounding
        // instruction and one dot-product add.  An absent neighbour (j >= K) has weight 0; its
        // row (a duplicate of a present one) then adds bf16(0 * v) = 0.  The weights are bf16, so
        // each product is one dot product of (w, 0) or (0, w) with a packed pair of v.
        float acc[8];
        if constexpr (!RP) {
            // fp32 products: one dot product each, accumulated slot by slot
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) {
                const float x = ex[i] * inv;
                const uint32_t w_lo = pack_bf16x2(x, 0.f), w_hi = pack_bf16x2(0.f, x);
                if (i == 0) out_fp32<true>(w_lo, w_hi, vw[i], acc);
                else out_fp32<false>(w_lo, w_hi, vw[i], acc);
            }
        } else {
#pragma unroll
        for (int i = 0; i < NSLOT; i += 2) {
            // the weight as (w, 0) and (0, w): one conversion each
            const float xa = ex[i] * inv;
            const uint32_t wa_lo = pack_bf16x2(xa, 0.f), wa_hi = pack_bf16x2(0.f, xa);
            if (i + 1 < NSLOT) {
                const float xb = ex[i + 1] * inv;
                const uint32_t wb_lo = pack_bf16x2(xb, 0.f), wb_hi = pack_bf16x2(0.f, xb);
                const uint4 &va = vw[i], &vb = vw[i + 1];
                if (i == 0) {
                    out_pair<true>(wa_lo, wb_lo, wa_hi, wb_hi, va.x, vb.x, va.y, vb.y, ones, acc);
                    out_pair<true>(wa_lo, wb_lo, wa_hi, wb_hi, va.z, vb.z, va.w, vb.w, ones, acc + 4);
                } else {
                    out_pair<false>(wa_lo, wb_lo, wa_hi, wb_hi, va.x, vb.x, va.y, vb.y, ones, acc);
                    out_pair<false>(wa_lo, wb_lo, wa_hi, wb_hi, va.z, vb.z, va.w, vb.w, ones, acc + 4);
                }
            } else if (i == 0) {
                out_single<true>(wa_lo, wa_hi, vw[i], pick_lo, pick_hi, acc);
            } else {
                out_single<false>(wa_lo, wa_hi, vw[i], pick_lo, pick_hi, acc);
            }
        }
        }
        if (!RP || more) {
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) vw[i] = ld_member<OFF32>(p.v + bn * p.v_sb, voff[i]);
        }
        // reduce-scatter over the 8 neighbour groups: halves (dims e / e + 4), row pairs
        // (e / e + 2), then lanes l ^ 8 (e / e + 1)
        float r4[4], r2[2];
#pragma unroll
        for (int e = 0; e < 4; ++e) r4[e] = swap32_add(acc[e], acc[e + 4]);
#pragma unroll
        for (int e = 0; e < 2; ++e) r2[e] = swap16_add(r4[e], r4[e + 2]);
        const bool odd8 = lane & 8;
        const float keep = odd8 ? r2[1] : r2[0], give = odd8 ? r2[0] : r2[1];
        const float o = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(give), 0x128, 0xf, 0xf, false));
        out[(int64_t)b * p.H * 64] = (bf16_t)(pack_bf16x2(o, 0.f) & 0xffffu);
    }
}

// LDS-staged form (fp32 products): one workgroup per (tile of up to 16 targets, head).  The
// per-target kernel above issues 6 wave-wide 16-byte loads per (target, member, head), and at
// one wave-instruction per ~32 cycles the texture addresser is then busy all the time; here
// the tile's distinct source rows of k and v (the host-built tables) go into LDS once per
// member with direct-to-LDS loads (lane l of an instruction lands at byte 16 l of a 1 KB run
// of 8 rows), double-buffered, and the targets read them with ds_read_b128.  The arithmetic
// per (target, member, head) is the fp32-product form of the kernel above in the same lane
// layout and order, so both give the same bits.
//
// LDS: per group of 8 rows, four 1 KB runs [k buffer 0][k buffer 1][v buffer 0][v buffer 1],
// so a row's k and v in either buffer sit at fixed distances from its k in buffer 0 (the
// reads take them as immediate offsets; the member loop is unrolled by two for the buffer).
// Wave w takes targets t0 + w + 4 r of the tile and staging instructions w + 4 r over the k
// groups, then the v groups.  One barrier per member: after it the next member's rows have
// landed (every wave waited for its own loads) and no wave still reads the buffer that the
// next member's loads overwrite.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}
// address = base (uniform) + voff (per lane); LDS destination M0 + 16 l.  Inline assembly: the
// compiler's own direct-to-LDS builtin makes it wait for these loads before every LDS read of
// the other buffer.  M0 is declared clobbered; the compiler sets it again before its own uses.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Three slots' scores (K 17..24, the model's 24) as one block: the three dot-product chains
// interleaved, each from a literal 0 addend, accumulating through their own addend (no wait
// between them); the three wait states a dot product's result needs before another VALU
// instruction reads it; then the sums over the 8 chunk lanes of each neighbour group as DPP
// adds (lanes l ^ 1, l ^ 2, then the half-row mirror), the three slots interleaved so each
// DPP read of a register comes at least two instructions after its write.  Same products,
// order and sums as chunk_sum(score_dot(...)) (the builtin form moves 0 into each
// accumulator first, and two of its three half-mirror adds compiled to a move and an add).
__device__ __forceinline__ void score_dot3(const uint32_t (&q)[3][4], const uint4 (&k)[3], float (&a)[3]) {
    asm("v_dot2_f32_bf16 %0, %3, %15, 0\n\t"
        "v_dot2_f32_bf16 %1, %7, %19, 0\n\t"
        "v_dot2_f32_bf16 %2, %11, %23, 0\n\t"
        "v_dot2_f32_bf16 %0, %4, %16, %0\n\t"
        "v_dot2_f32_bf16 %1, %8, %20, %1\n\t"
        "v_dot2_f32_bf16 %2, %12, %24, %2\n\t"
        "v_dot2_f32_bf16 %0, %5, %17, %0\n\t"
        "v_dot2_f32_bf16 %1, %9, %21, %1\n\t"
        "v_dot2_f32_bf16 %2, %13, %25, %2\n\t"
        "v_dot2_f32_bf16 %0, %6, %18, %0\n\t"
        "v_dot2_f32_bf16 %1, %10, %22, %1\n\t"
        "v_dot2_f32_bf16 %2, %14, %26, %2\n\t"
        "s_nop 2\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %2, %2, %2 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %2, %2, %2 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %2, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2])
        : "v"(q[0][0]), "v"(q[0][1]), "v"(q[0][2]), "v"(q[0][3]), "v"(q[1][0]), "v"(q[1][1]), "v"(q[1][2]),
          "v"(q[1][3]), "v"(q[2][0]), "v"(q[2][1]), "v"(q[2][2]), "v"(q[2][3]), "v"(k[0].x), "v"(k[0].y),
          "v"(k[0].z), "v"(k[0].w), "v"(k[1].x), "v"(k[1].y), "v"(k[1].z), "v"(k[1].w), "v"(k[2].x), "v"(k[2].y),
          "v"(k[2].z), "v"(k[2].w));
}
// Three slots' weighted sum as one block: acc[2e] = sum_i (w_i, 0) . v_i[e], acc[2e + 1] =
// sum_i (0, w_i) . v_i[e], slot by slot from a literal 0 addend (the order of
// weighted_sum_fp32), then the three wait states.
__device__ __forceinline__ void weighted_sum3(const uint32_t (&wl)[3], const uint32_t (&wh)[3], const uint4 (&v)[3],
                                              float (&acc)[8]) {
#define MOSAIC_PV_FIRST(W0, W1, X, Y, Z, T)        \
    "v_dot2_f32_bf16 %0, " W0 ", " X ", 0\n\t"   \
    "v_dot2_f32_bf16 %1, " W1 ", " X ", 0\n\t"   \
    "v_dot2_f32_bf16 %2, " W0 ", " Y ", 0\n\t"   \
    "v_dot2_f32_bf16 %3, " W1 ", " Y ", 0\n\t"   \
    "v_dot2_f32_bf16 %4, " W0 ", " Z ", 0\n\t"   \
    "v_dot2_f32_bf16 %5, " W1 ", " Z ", 0\n\t"   \
    "v_dot2_f32_bf16 %6, " W0 ", " T ", 0\n\t"   \
    "v_dot2_f32_bf16 %7, " W1 ", " T ", 0\n\t"
#define MOSAIC_PV_NEXT(W0, W1, X, Y, Z, T)         \
    "v_dot2_f32_bf16 %0, " W0 ", " X ", %0\n\t"  \
    "v_dot2_f32_bf16 %1, " W1 ", " X ", %1\n\t"  \
    "v_dot2_f32_bf16 %2, " W0 ", " Y ", %2\n\t"  \
    "v_dot2_f32_bf16 %3, " W1 ", " Y ", %3\n\t"  \
    "v_dot2_f32_bf16 %4, " W0 ", " Z ", %4\n\t"  \
    "v_dot2_f32_bf16 %5, " W1 ", " Z ", %5\n\t"  \
    "v_dot2_f32_bf16 %6, " W0 ", " T ", %6\n\t"  \
    "v_dot2_f32_bf16 %7, " W1 ", " T ", %7\n\t"
    asm(MOSAIC_PV_FIRST("%8", "%9", "%14", "%15", "%16", "%17")
        MOSAIC_PV_NEXT("%10", "%11", "%18", "%19", "%20", "%21")
        MOSAIC_PV_NEXT("%12", "%13", "%22", "%23", "%24", "%25")
        "s_nop 2"
        : "=&v"(acc[0]), "=&v"(acc[1]), "=&v"(acc[2]), "=&v"(acc[3]), "=&v"(acc[4]), "=&v"(acc[5]), "=&v"(acc[6]),
          "=&v"(acc[7])
        : "v"(wl[0]), "v"(wh[0]), "v"(wl[1]), "v"(wh[1]), "v"(wl[2]), "v"(wh[2]), "v"(v[0].x), "v"(v[0].y),
          "v"(v[0].z), "v"(v[0].w), "v"(v[1].x), "v"(v[1].y), "v"(v[1].z), "v"(v[1].w), "v"(v[2].x), "v"(v[2].y),
          "v"(v[2].z), "v"(v[2].w));
#undef MOSAIC_PV_FIRST
#undef MOSAIC_PV_NEXT
}

constexpr int kTileWaveTargets = kKnnTileTargets / kInterpWaves;     // 4
constexpr int kTileWaveLoads = 2 * kKnnTileRows / 8 / kInterpWaves;  // 8 staging instructions per wave at most

template <int NSLOT, bool POW2>
__global__ __launch_bounds__(kInterpWaves * 64) void knn_tile_kernel(InterpParams p, KnnTiles tl) {
    extern __shared__ __attribute__((aligned(16))) uint4 kv_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pair = xcd_remap(blockIdx.x, gridDim.x);
    const int tile = pair / p.H, h = pair - tile * p.H;
    const int K = p.K, dc = lane & 7, jg = lane >> 3;
    const int rows = tl.rows;
    // the tables are clamped into range (memory safety; a malformed table gives wrong rows)
    const int t0 = __builtin_amdgcn_readfirstlane(min(max(tl.start[tile], 0), p.S_to));
    const int t1 = __builtin_amdgcn_readfirstlane(min(max(tl.start[tile + 1], t0), min(t0 + kKnnTileTargets, p.S_to)));
    const int nsrc = __builtin_amdgcn_readfirstlane(min(max(tl.nsrc[tile], 1), rows));
    const int ng = (nsrc + 7) >> 3;  // 8-row groups per tensor

    // staging offsets: instruction r of this wave loads group gi = wave + 4 r (k groups, then v)
    uint32_t soff[kTileWaveLoads];
#pragma unroll
    for (int r = 0; r < kTileWaveLoads; ++r) {
        const int gi = wave + kInterpWaves * r;
        const bool isv = gi >= ng;
        const int row = 8 * (isv ? gi - ng : gi) + (lane >> 3);
        const int n = min(max(tl.src[(int64_t)tile * rows + min(row, nsrc - 1)], 0), p.S_from - 1);
        soff[r] = isv ? (uint32_t)(2 * (n * p.v_sn + (int64_t)h * p.v_sh + 8 * dc))
                      : (uint32_t)(2 * (n * p.k_sn + (int64_t)h * p.k_sh + 8 * dc));
    }
    const uint32_t lds0 = lds_addr(kv_lds);
    auto stage = [&](int b, int buf) __attribute__((always_inline)) {
        const char* kb = reinterpret_cast<const char*>(p.k + (int64_t)b * p.k_sb);
        const char* vb = reinterpret_cast<const char*>(p.v + (int64_t)b * p.v_sb);
#pragma unroll
        for (int r = 0; r < kTileWaveLoads; ++r) {
            const int gi = wave + kInterpWaves * r;
            if (gi >= 2 * ng) break;  // uniform
            const bool isv = gi >= ng;
            const uint32_t dst = lds0 + (uint32_t)(4 * (isv ? gi - ng : gi) + 2 * isv + buf) * 1024u;
            if (isv) dma16(vb, soff[r], __builtin_amdgcn_readfirstlane(dst));
            else dma16(kb, soff[r], __builtin_amdgcn_readfirstlane(dst));
        }
    };

    // to_q rows h*64 + 8 dc .. + 7
    float wq[24];
    {
        const bf16_t* wr = p.w_q + ((int64_t)h * 64 + 8 * dc) * 3;
        float t[8];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            unpack8(ld16(wr + 8 * c), t);
#pragma unroll
            for (int e = 0; e < 8; ++e) wq[8 * c + e] = t[e];
        }
    }
    // per target of this wave: its index, its slots' k rows in buffer 0 (LDS byte offsets) and
    // its query pairs
    int tgt[kTileWaveTargets];
    uint32_t koff[kTileWaveTargets][NSLOT];
    uint32_t qp[kTileWaveTargets][NSLOT][4];
#pragma unroll
    for (int r = 0; r < kTileWaveTargets; ++r) {
        const int pos = min(t0 + wave + kInterpWaves * r, p.S_to - 1);
        const int s = __builtin_amdgcn_readfirstlane(p.target_order ? min(max(p.target_order[pos], 0), p.S_to - 1) : pos);
        tgt[r] = s;
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
            const int j = min(jg + 8 * i, K - 1);
            const int sl = min(max(tl.slot[(int64_t)pos * K + j], 0), rows - 1);
            koff[r][i] = lds0 + (uint32_t)(4096 * (sl >> 3) + 128 * (sl & 7) + 16 * dc);
            const int64_t sj = (int64_t)s * K + j;
            const float r0 = round_bf16(p.rel_pos[3 * sj]), r1 = round_bf16(p.rel_pos[3 * sj + 1]),
                        r2 = round_bf16(p.rel_pos[3 * sj + 2]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t bits = __float_as_uint(round_bf16(fmaf(r2, wq[3 * e + 2], fmaf(r1, wq[3 * e + 1], r0 * wq[3 * e]))));
                if (e & 1) qp[r][i][e >> 1] |= bits;
                else qp[r][i][e >> 1] = bits >> 16;
            }
        }
    }
    const int dout = 8 * dc + 4 * (lane >> 5) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1);

    // member b from buffer BUF (member b + 1 staged into the other one meanwhile)
    auto member = [&](int b, auto BUF) __attribute__((always_inline)) {
        constexpr int buf = decltype(BUF)::value;
        if (b + 1 < p.B) stage(b + 1, buf ^ 1);
        const char* lds = reinterpret_cast<const char*>(kv_lds) - lds0;  // koff holds absolute LDS addresses
#pragma unroll
        for (int r = 0; r < kTileWaveTargets; ++r) {
            if (t0 + wave + kInterpWaves * r >= t1) break;  // uniform
            uint4 kw[NSLOT], vw[NSLOT];
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) {
                kw[i] = *reinterpret_cast<const uint4*>(lds + koff[r][i] + 1024 * buf);
                vw[i] = *reinterpret_cast<const uint4*>(lds + koff[r][i] + 2048 + 1024 * buf);
            }
            float part[NSLOT], sc[NSLOT], m;
            if constexpr (NSLOT == 3) {
                score_dot3(qp[r], kw, part);
            } else {
#pragma unroll
                for (int i = 0; i < NSLOT; ++i) part[i] = score_dot(qp[r][i], kw[i]);
            }
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) {
                const float sum = NSLOT == 3 ? part[i] : chunk_sum(part[i]);  // score_dot3 sums the chunk lanes itself
                sc[i] = i < NSLOT - 1 || jg + 8 * i < K ? scaled_score<POW2>(sum, p) : -INFINITY;
                m = i == 0 ? sc[0] : fmaxf(m, sc[i]);
            }
            float wt[NSLOT], acc[8];
            softmax_weights(sc, m, wt);
            if constexpr (NSLOT == 3) {
                uint32_t wl[3], wh[3];
#pragma unroll
                for (int i = 0; i < 3; ++i) { wl[i] = pack_bf16x2(wt[i], 0.f); wh[i] = pack_bf16x2(0.f, wt[i]); }
                weighted_sum3(wl, wh, vw, acc);
            } else {
                weighted_sum_fp32(wt, vw, acc);
            }
            const float o = reduce_scatter(acc, lane);
            bf16_t* orow = p.out + (((int64_t)tgt[r] * p.B + b) * p.H + h) * 64;  // uniform
            orow[dout] = (bf16_t)(pack_bf16x2(o, 0.f) & 0xffffu);
        }
        wait_vmem();
        __syncthreads();
    };

    stage(0, 0);
    wait_vmem();
    __syncthreads();
    for (int b = 0; b < p.B; b += 2) {
        member(b, std::integral_constant<int, 0>{});
        if (b + 1 < p.B) member(b + 1, std::integral_constant<int, 1>{});
    }
}

template <int NSLOT, bool RP>
const void* pick(bool off32, bool pow2) {
    return off32 ? (pow2 ? (const void*)&knn_attn_kernel<NSLOT, true, true, RP> : (const void*)&knn_attn_kernel<NSLOT, true, false, RP>)
                 : (pow2 ? (const void*)&knn_attn_kernel<NSLOT, false, true, RP> : (const void*)&knn_attn_kernel<NSLOT, false, false, RP>);
}

bool knn_off32(const InterpParams& p) {
    // 32-bit chunk offsets when every chunk of a member lies within 4 GiB of its start
    const int64_t kmax = (int64_t)(p.S_from - 1) * p.k_sn + (int64_t)(p.H - 1) * p.k_sh + 64;
    const int64_t vmax = (int64_t)(p.S_from - 1) * p.v_sn + (int64_t)(p.H - 1) * p.v_sh + 64;
    return p.k_sn >= 0 && p.k_sh >= 0 && p.v_sn >= 0 && p.v_sh >= 0 && 2 * kmax <= 0xffffffffLL &&
           2 * vmax <= 0xffffffffLL;
}

template <int NSLOT>
hipError_t launch_slots(const InterpParams& p, unsigned wgs, hipStream_t s) {
    void* args[] = {const_cast<InterpParams*>(&p)};
    const bool off32 = knn_off32(p);
    const void* fn = p.round_products ? pick<NSLOT, true>(off32, p.scale_pow2) : pick<NSLOT, false>(off32, p.scale_pow2);
    return hipLaunchKernel(fn, dim3(wgs), dim3(kInterpWaves * 64), args, 0, s);
}

}  // namespace

hipError_t launch_knn_attn(const InterpParams& p, hipStream_t s) {
    const int64_t pairs = (int64_t)p.S_to * p.H;
    const int64_t wgs = (pairs + kInterpWaves - 1) / kInterpWaves;
    if (wgs <= 0) return hipSuccess;
    if (wgs > 0x7fffffff) return hipErrorInvalidValue;
    switch ((p.K + 7) / 8) {
        case 1: return launch_slots<1>(p, (unsigned)wgs, s);
        case 2: return launch_slots<2>(p, (unsigned)wgs, s);
        case 3: return launch_slots<3>(p, (unsigned)wgs, s);
        case 4: return launch_slots<4>(p, (unsigned)wgs, s);
        default: return hipErrorInvalidValue;
    }
}

// The LDS-staged form: fp32 products with 32-bit chunk offsets only (the caller falls back to
// launch_knn_attn otherwise).
bool knn_tiled_supported(const InterpParams& p) { return !p.round_products && knn_off32(p); }

hipError_t launch_knn_attn_tiled(const InterpParams& p, const KnnTiles& t, hipStream_t s) {
    if (!knn_tiled_supported(p) || t.rows <= 0 || t.rows % 8 || t.rows > kKnnTileRows) return hipErrorInvalidValue;
    const int64_t wgs = (int64_t)t.n * p.H;
    if (wgs <= 0) return hipSuccess;
    if (wgs > 0x7fffffff) return hipErrorInvalidValue;
    void* args[] = {const_cast<InterpParams*>(&p), const_cast<KnnTiles*>(&t)};
    const void* fn = nullptr;
    switch ((p.K + 7) / 8) {
        case 1: fn = p.scale_pow2 ? (const void*)&knn_tile_kernel<1, true> : (const void*)&knn_tile_kernel<1, false>; break;
        case 2: fn = p.scale_pow2 ? (const void*)&knn_tile_kernel<2, true> : (const void*)&knn_tile_kernel<2, false>; break;
        case 3: fn = p.scale_pow2 ? (const void*)&knn_tile_kernel<3, true> : (const void*)&knn_tile_kernel<3, false>; break;
        case 4: fn = p.scale_pow2 ? (const void*)&knn_tile_kernel<4, true> : (const void*)&knn_tile_kernel<4, false>; break;
        default: return hipErrorInvalidValue;
    }
    const size_t lds = 4u * (size_t)t.rows * 128u;  // per 8-row group: k and v, two buffers each
    return hipLaunchKernel(fn, dim3((unsigned)wgs), dim3(kInterpWaves * 64), args, lds, s);
}

}  // namespace mosaic
