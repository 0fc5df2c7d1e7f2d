// attn.hip -- fused local + selected-block attention with the gated merge (gfx950).
//
// One workgroup = (batch b, kv head c, 64-token query tile, group of NW query heads).
// Each wave owns one query head j of the GQA group and all 64 query rows of the tile; the
// K/V tiles of 64 keys are staged once in LDS and read by all NW waves.
//
//   local branch     block_attention / flash_attn_func (primitives.py:28-32): the keys of
//                    the query's block_attn_size block, logits q.k * scale, fp32 online
//                    softmax in base 2, P rounded to bf16 for the PV product.
//   selected branch  mosaic_attn_fwd_kernel (ops.py:41-134): q pre-scaled by scale*log2(e)
//                    and rounded to bf16 (:92), the sparse_block_size blocks named by the
//                    top-k indices in order (:94-95), base-2 online softmax (:120-128),
//                    P -> bf16 before PV (:128), O / l and LSE = m + log2(l) (:130-131).
//   merge            primitives.py:62-89 in fp32 in the epilogue; the compressed branch is
//                    read from the combined compressed-attention output (one row per block).
//
// Staging.  Tiles of both branches form one sequence [local tiles..., selected tiles...]
// streamed through two LDS buffers with one barrier per tile.  K and V rows go from global
// memory straight into LDS (global_load_lds_dwordx4: lane L of an instruction lands at
// byte 16*L of a 1 KB run), issued for tile t+1 right after the barrier of tile t, so no
// registers hold staged data.  Both keep 128-byte rows with the 16-byte chunks of a row
// permuted (XOR swizzle, chosen per tensor for its read pattern):
//   K  chunk c of key k at position c ^ ((k >> 1) & 7): a b128 read is served 16 lanes
//      (256 bytes, all 64 banks) at a time, and the 16 lanes that fetch chunk c of 16
//      consecutive keys then cover both 128-byte halves of the banks at 8 positions each;
//   V  chunk c of key k at position c ^ 2(k & 3): the 16 lanes of a transposing read that
//      fetch 2 chunks of 4 consecutive keys hit 8 different positions.
// The PV operand needs V^T (8 consecutive keys of one dimension per lane); it is read from
// the row-major tile with ds_read_b64_tr_b16, which hands lane 4a+b of each 16-lane group
// element b of the 8-byte rows addressed by lanes a, a+4, a+8, a+12.
//
// Softmax.  Local tiles: exact row max per tile with a lazy reference (a row's reference
// only moves when a tile's max exceeds it by more than kTau), fp32 row sums.  Selected
// tiles take one of two paths, chosen per wave at the first selected tile:
//   bounded     the pooling kernel's per-block key-norm bounds and |q'| bound every logit
//               of the wave by kLogitBound, so P = exp2(s) needs no reference, no max and
//               no rescale; row sums of the bf16 P run on the matrix pipe (row_sums).
//   running     the first tile's exact row max is the reference m; later tiles take
//               exp2(s - m) without a max pass, and a tile whose row sums exceed kSumLimit
//               (or are not finite) is recomputed from LDS with the reference moved up to
//               its row max.  Row sums add the fp32 P, as the selected-branch kernel does
//               (ops.py:125).
// Numerator and denominator share the reference, so both give the same softmax.
//
// Two workgroups share a CU (2 waves per SIMD): one wave's softmax VALU work overlaps the
// other's MFMA work.  The local branch's partial merge (w0 * o_ba) waits in LDS as bf16.
// In the modes with that partial buffer, the same per-wave region first receives the wave's
// Q rows (row-contiguous DMA) and finally stages the merged output, so Q loads and O stores
// move whole 128-byte rows instead of 16-byte pieces of 32 rows.
//
// S^T = K Q^T and O^T = V^T P^T are computed so a lane owns one query column (see
// bsa_common.h).
#include <type_traits>

#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int kTileElems = 64 * 64;  // one K or V tile: 64 keys x 64 dims, 128-byte rows
constexpr int PS = 68;               // merge-partial row stride in bf16
constexpr float kTau = 8.0f;
// Largest accepted partial row sum of a selected tile under the reference max: every P is
// then <= 2^16, far from fp32 / bf16 overflow.
constexpr float kSumLimit = 65536.0f;
// Bounded-logit path of the selected branch: largest |s| (base-2 logit) it accepts, and the
// most selected blocks whose key-norm bounds are staged.
constexpr float kLogitBound = 64.0f;
constexpr int kMaxBounded = 64;

typedef __attribute__((address_space(3))) void lds_void;
typedef short v4i16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Direct-to-LDS loads of one 64-key tile (K and V rows key0 .. key0+63): NW waves, 8/NW
// 1 KB runs per wave and tensor.  The per-lane byte offsets (key row * stride + swizzled
// chunk) do not change between tiles and are computed once as unsigned 32-bit values, so
// each load is a wave-uniform base (key0 * stride, scalar) plus a lane offset.
template <int NW>
__device__ __forceinline__ void dma_init(uint32_t* dk, uint32_t* dv, int wave_u, int lane, int64_t ksn, int64_t vsn) {
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
        const int row = 8 * (wave_u * (8 / NW) + i) + (lane >> 3), pos = lane & 7;
        dk[i] = 2u * (uint32_t)(row * ksn + 8 * (pos ^ ((row >> 1) & 7)));  // global chunk at position pos
        dv[i] = 2u * (uint32_t)(row * vsn + 8 * (pos ^ ((row & 3) << 1)));
    }
}
template <int NW>
__device__ __forceinline__ void dma_issue(const uint32_t* dk, const uint32_t* dv, const bf16_t* kb, const bf16_t* vb,
                                          int64_t ksn, int64_t vsn, int key0, bf16_t* Kd, bf16_t* Vd, int wave_u) {
    const int k0 = __builtin_amdgcn_readfirstlane(key0);
    const char* kt = reinterpret_cast<const char*>(kb + (int64_t)k0 * ksn);
    const char* vt = reinterpret_cast<const char*>(vb + (int64_t)k0 * vsn);
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
        const int row0 = 8 * (wave_u * (8 / NW) + i);
        __builtin_amdgcn_global_load_lds(kt + dk[i], (lds_void*)(Kd + row0 * 64), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vt + dv[i], (lds_void*)(Vd + row0 * 64), 16, 0, 0);
    }
}

__device__ __forceinline__ void zero(f32x16 (&x)[2][2]) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) x[a][b][e] = 0.f;
}

// Per-lane element offsets of the operand reads (constant over tiles).
struct ReadOffsets {
    int k[4];  // K row r, chunk 2*ds + hh (swizzled), for ds = 0..3; + 32*kt*64 per key tile
    int v[2];  // V transposing read for dim tile dt; + (32*kt + 16*s2 + 8*sec)*64
    __device__ __forceinline__ void init(int lane) {
        const int r = lane & 31, hh = lane >> 5;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) k[ds] = r * 64 + 8 * ((2 * ds + hh) ^ ((r >> 1) & 7));
        const int s = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
            v[dt] = (4 * hh + (s >> 2)) * 64 + 8 * ((4 * dt + 2 * half + ((s & 3) >> 1)) ^ (2 * (s >> 2))) + 4 * (s & 1);
    }
};

// S^T = K Q^T for one 64-key tile: s[key tile][query tile].
__device__ __forceinline__ void s_tile(const bf16_t* Ks, const ReadOffsets& ro, const bf16x8 (&qf)[2][4],
                                       f32x16 (&s)[2][2]) {
    zero(s);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + 32 * kt * 64 + ro.k[ds]));
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[kt][qt] = mfma32(a, qf[qt][ds], s[kt][qt]);
        }
    }
}

// S^T = K Q^T (as s_tile) with the key tiles in sequence: the scores of keys 0..31
// are complete after half of the MFMAs, so their exponentials can overlap the other half.
__device__ __forceinline__ void s_tile_seq(const bf16_t* Ks, const ReadOffsets& ro, const bf16x8 (&qf)[2][4],
                                           f32x16 (&s)[2][2]) {
    zero(s);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + 32 * kt * 64 + ro.k[ds]));
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[kt][qt] = mfma32(a, qf[qt][ds], s[kt][qt]);
        }
}

// One query tile of s_tile (rare recompute path), as s[key tile].
__device__ __forceinline__ void s_half(const bf16_t* Ks, const ReadOffsets& ro, const bf16x8 (&qf)[4], f32x16 (&s)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[kt][e] = 0.f;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
            s[kt] = mfma32(as_bf16x8(*reinterpret_cast<const uint4*>(Ks + 32 * kt * 64 + ro.k[ds])), qf[ds], s[kt]);
}

// O^T += V^T P^T for one 64-key tile; V^T operands come from transposing reads of the
// row-major tile (keys 4hh + 0..3 and 8 + 4hh + 0..3 of each 16-key step, matching the
// packing of P in exp_pack).
__device__ __forceinline__ void pv_tile(const bf16_t* Vs, const ReadOffsets& ro, const bf16x8 (&pb)[2][2][2],
                                        f32x16 (&o)[2][2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const bf16_t* vp = Vs + (32 * kt + 16 * s2) * 64 + ro.v[dt];
                const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                               (__attribute__((address_space(3))) v4i16*)(vp)));
                const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                               (__attribute__((address_space(3))) v4i16*)(vp + 8 * 64)));
                const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) o[dt][qt] = mfma32(a, pb[qt][kt][s2], o[dt][qt]);
            }
}

// P = exp2(s * c - m[qt]) (SCALED), exp2(s - m[qt]) (SHIFT) or exp2(s), packed to bf16 for
// the PV product; lt = this lane's partial row sums of P (fp32, before rounding).
template <bool SCALED, bool SHIFT>
__device__ __forceinline__ void exp_pack(const f32x16 (&s)[2][2], const float (&m)[2], float c, bf16x8 (&pb)[2][2][2],
                                         float (&lt)[2]) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float lsum[4] = {0.f, 0.f, 0.f, 0.f};
        const float mm = m[qt];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x0 = s[kt][qt][8 * s2 + 2 * i], x1 = s[kt][qt][8 * s2 + 2 * i + 1];
                    const float a0 = SCALED ? fmaf(x0, c, -mm) : (SHIFT ? x0 - mm : x0);
                    const float a1 = SCALED ? fmaf(x1, c, -mm) : (SHIFT ? x1 - mm : x1);
                    const float p0 = __builtin_amdgcn_exp2f(a0), p1 = __builtin_amdgcn_exp2f(a1);
                    w[i] = pack_bf16x2(p0, p1);
                    lsum[2 * kt + s2] += p0 + p1;
                }
                pb[qt][kt][s2] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
            }
        lt[qt] = (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
    }
}

// exp_pack<false, true> of one query tile
__device__ __forceinline__ void exp_pack_half(const f32x16 (&s)[2], float m, bf16x8 (&pb)[2][2], float& lt) {
    float lsum[2] = {0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p0 = __builtin_amdgcn_exp2f(s[kt][8 * s2 + 2 * i] - m);
                const float p1 = __builtin_amdgcn_exp2f(s[kt][8 * s2 + 2 * i + 1] - m);
                w[i] = pack_bf16x2(p0, p1);
                lsum[kt] += p0 + p1;
            }
            pb[kt][s2] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
        }
    lt = lsum[0] + lsum[1];
}

// P = exp2(s) packed to bf16 for the PV product; the row sums are taken on the matrix pipe
// (row_sums).
__device__ __forceinline__ void exp_pack_raw(const f32x16 (&s)[2][2], bf16x8 (&pb)[2][2][2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    w[i] = pack_bf16x2(__builtin_amdgcn_exp2f(s[kt][qt][8 * s2 + 2 * i]),
                                       __builtin_amdgcn_exp2f(s[kt][qt][8 * s2 + 2 * i + 1]));
                pb[qt][kt][s2] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
            }
}

// Selector A of the row-sum product D = A B on v_mfma_f32_16x16x32_bf16, where B is a PV
// operand pb[qt][kt][s2] (lane l: 8 keys of query l % 32 from key half l / 32).  Lane l of B
// lands in column l % 16, contraction chunk c = l / 16, so chunks 0 and 2 carry queries
// 0..15 and chunks 1 and 3 queries 16..31.  A[i][chunk c] = 1 when (c & 1) == ((i >> 2) & 1):
// output lane l (rows 4*(l/16)..+3, column l % 16) then receives the 16-key sum of P for
// query l % 32, both key halves included.
__device__ __forceinline__ bf16x8 row_sum_selector(int lane) {
    const uint32_t h = ((((lane & 15) >> 2) ^ (lane >> 4)) & 1) ? 0u : 0x3f80u;
    const uint32_t w = h | (h << 16);
    return as_bf16x8(make_uint4(w, w, w, w));
}

// acc[qt] += row sums of the bf16 P of one tile (every lane of a query column holds its total)
__device__ __forceinline__ void row_sums(const bf16x8& sel, const bf16x8 (&pb)[2][2][2], f32x4 (&acc)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) acc[qt] = mfma16(sel, pb[qt][kt][s2], acc[qt]);
}

// Row max of a tile (both lane halves) for query tile qt.
__device__ __forceinline__ float tile_max(const f32x16 (&s)[2][2], int qt) {
    float mx = s[0][qt][0];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][qt][e]);
    return xor32_max(mx);
}

__device__ __forceinline__ float half_max(const f32x16 (&s)[2]) {
    float mx = s[0][0];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
    return xor32_max(mx);
}

using Buf0 = std::integral_constant<int, 0>;
using Buf1 = std::integral_constant<int, 1>;

// Waves per SIMD the kernel is compiled for: 2 where the registers allow it.  The one- and
// two-wave workgroups of the modes with a selected branch (GQA groups of 1, 2 or an odd
// size) need more than 256 registers per lane and run one wave per SIMD.
template <int NW, int MODE>
constexpr int kWavesPerSimd = (NW == 1 && MODE != kModeLocalOnly) ||
                                      (NW == 2 && (MODE == kModeFull || MODE == kModeNoCompression))
                                  ? 1
                                  : 2;

template <int NW, int MODE, typename IdxT>
__global__ __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64),
                          amdgpu_waves_per_eu(kWavesPerSimd<NW, MODE>, kWavesPerSimd<NW, MODE>)))
void bsa_attn_kernel(AttnParams p) {
    constexpr bool kLocal = MODE != kModeSelectedOnly;
    constexpr bool kSel = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeSelectedOnly;
    constexpr bool kCmp = MODE == kModeFull || MODE == kModeNoSelection;
    constexpr bool kWeights = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeNoSelection;
    constexpr bool kPartial = MODE == kModeFull || MODE == kModeNoCompression;
    // selected tiles may take the bounded-logit path (key-norm bounds come with the pooling)
    constexpr bool kFastSel = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeSelectedOnly;

    // two staging buffers as separate objects, so the compiler can tell the loads in flight
    // into one buffer from the reads of the other
    __shared__ __attribute__((aligned(1024))) bf16_t Ks0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Ks1[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Vs0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Vs1[kTileElems];
    __shared__ __attribute__((aligned(16))) bf16_t Part[kPartial ? NW * 64 * PS : 8];
    __shared__ __attribute__((aligned(16))) bf16_t Ocmp[kCmp ? NW * 64 : 8];  // compressed-branch rows
    __shared__ int sel_key0[kSel ? kMaxSelected : 1];  // first key of each in-range selected block
    __shared__ int sel_count;
    __shared__ uint32_t Gw[kWeights ? NW * 3 * 64 : 1];  // gate words [wave][branch][row]
    __shared__ __attribute__((aligned(16))) float sel_kbnd[kFastSel ? kMaxBounded * 8 : 4];  // key-norm bounds

    const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int L;
    if ((int)blockIdx.x < p.n_static) {
        L = xcd_remap(blockIdx.x, p.n_static);
    } else {
        // dynamic tail: the next unclaimed item, or none (the whole workgroup leaves before
        // any other barrier); the last of the tail_wgs takers resets the counter for the next
        // launch
        __shared__ int claimed;
        if (tid == 0) {
            const int t = __hip_atomic_fetch_add(p.tail_ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (t == p.tail_wgs - 1) __hip_atomic_store(p.tail_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            claimed = t;
        }
        __syncthreads();
        const int t = claimed;
        if (t >= p.total_wgs - p.n_static) return;
        L = p.n_static + t;
    }
    const int qtile = L % p.qtiles;
    const int rest = L / p.qtiles;
    const int hgs = p.Hk * p.head_groups;
    const int hg = rest % hgs;
    const int b = rest / hgs;
    const int c = hg / p.head_groups;
    const int j = c * p.G + (hg % p.head_groups) * NW + wave;
    const int n0 = qtile * kTile;

    const bf16_t* qb = p.q + b * p.q_sb + (int64_t)j * p.q_sh;
    const bf16_t* kb = p.k + b * p.k_sb + (int64_t)c * p.k_sh;
    const bf16_t* vb = p.v + b * p.v_sb + (int64_t)c * p.v_sh;

    // tile sequence: [local tiles][tiles of the in-range selected blocks, in top-k order]
    const int tl_count = kLocal ? p.bs_l / kTile : 0;
    const int lstart = (n0 / p.bs_l) * p.bs_l;
    const int sub = p.bs / kTile;
    // Prologue.  The Q rows, the gate weights, the compressed-branch row and (with a local
    // branch) the first tile do not depend on the top-k indices: their loads are issued
    // first, so they are in flight while wave 0 stages the indices.
    bf16x8 qf[2][4];
    if constexpr (kPartial) {
        // The wave's 64 Q rows go to its (still unused) partial buffer in LDS as full 128-byte
        // rows, chunks swizzled as the K tiles, and are read into registers after the first
        // barrier: 8 row-contiguous 1 KB requests instead of 16-byte pieces of 32 rows.
        bf16_t* qs = Part + wave * 64 * PS;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = 8 * i + (lane >> 3), pos = lane & 7;
            __builtin_amdgcn_global_load_lds(qb + (int64_t)(n0 + row) * p.q_sn + 8 * (pos ^ ((row >> 1) & 7)),
                                             (lds_void*)(qs + 8 * i * 64), 16, 0, 0);
        }
        // With RoPE, the 64 query rows' cos / sin table rows (128 bytes each) go to the K and V
        // buffers of tile 1, unused until the first barrier; q is rotated from them there.
        if (p.rope_cos != nullptr) {
#pragma unroll
            for (int i = 0; i < 8 / NW; ++i) {
                const int row0 = 8 * ((8 / NW) * wave + i);
                __builtin_amdgcn_global_load_lds(p.rope_cos + (int64_t)(n0 + row0) * 32 + 4 * lane,
                                                 (lds_void*)(Ks1 + row0 * 64), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(p.rope_sin + (int64_t)(n0 + row0) * 32 + 4 * lane,
                                                 (lds_void*)(Vs1 + row0 * 64), 16, 0, 0);
            }
        }
    } else {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
                qf[qt][ds] = as_bf16x8(ld16(qb + (int64_t)(n0 + 32 * qt + r) * p.q_sn + 16 * ds + 8 * hh));
    }
    // Gate weights of the 64 rows: the aligned 4-byte word holding each bf16 gate goes straight
    // to LDS (lane L: row n0 + L), so no register waits on them; gate(s, qt) picks the half.
    auto gate_ptr = [&](int sidx, int row) -> const bf16_t* {
        return p.w + sidx * p.w_ss + b * p.w_sb + (int64_t)(n0 + row) * p.w_sn + (int64_t)j * p.w_sh;
    };
    if constexpr (kWeights) {
#pragma unroll
        for (int sidx = 0; sidx < 3; ++sidx) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(gate_ptr(sidx, lane)) & ~uintptr_t(3);
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a), (lds_void*)(Gw + (wave * 3 + sidx) * 64),
                                             4, 0, 0);
        }
    }
    auto gate = [&](int sidx, int qt) -> float {
        const uint32_t wd = Gw[(wave * 3 + sidx) * 64 + 32 * qt + r];
        return (reinterpret_cast<uintptr_t>(gate_ptr(sidx, 32 * qt + r)) & 2) ? bf_hi(wd) : bf_lo(wd);
    };
    if constexpr (kCmp) {  // compressed-branch output row of (block, head j): 128 bytes into LDS
        const bf16_t* ocp = p.ocmp + (((int64_t)b * p.nb + n0 / p.bs) * p.Hq + j) * kHeadDim;
        if (lane < 32) __builtin_amdgcn_global_load_lds(ocp + 2 * lane, (lds_void*)(Ocmp + wave * 64), 4, 0, 0);
    }
    uint32_t dk[8 / NW], dv[8 / NW];
    dma_init<NW>(dk, dv, wave, lane, p.k_sn, p.v_sn);
    if constexpr (kLocal) dma_issue<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, lstart, Ks0, Vs0, wave);

    // Selected blocks: wave 0 compacts the in-range indices (top-k order kept) into LDS once,
    // so tile addresses never wait on a global load inside the loop.
    if constexpr (kSel) {
        if (wave == 0) {
            const IdxT* ip = reinterpret_cast<const IdxT*>(p.idx) + ((int64_t)(b * p.nb + n0 / p.bs) * p.Hk + c) * p.K;
            int count = 0;
            for (int base = 0; base < p.K; base += 64) {
                const int i = base + lane;
                const int64_t blk = i < p.K ? (int64_t)ip[i] : -1;
                const bool ok = blk >= 0 && blk < p.nb;
                const uint64_t mask = __builtin_amdgcn_ballot_w64(ok);
                const int pos = count + (int)__builtin_popcountll(mask & ((1ull << lane) - 1ull));
                if (ok) sel_key0[pos] = (int)(blk * p.bs);
                count += (int)__builtin_popcountll(mask);
            }
            if (lane == 0) sel_count = count;
        }
        __syncthreads();
    }
    const int nvalid = kSel ? sel_count : 0;
    const int total_tiles = tl_count + nvalid * sub;
    // first key of tile t >= 1 (tile 0 of a local branch is issued above); tiles are
    // requested in order
    int cur_k = 0, cur_s = 0;
    // up to 64 selected blocks: every wave keeps their first keys in a register (lane i,
    // block i), so a tile address is a readlane instead of an LDS round trip
    const int selv = (kSel && lane < nvalid) ? sel_key0[lane] : 0;
    auto next_key0 = [&](int t) -> int {
        if (kLocal && t < tl_count) return lstart + kTile * t;
        const int base = nvalid <= 64 ? __builtin_amdgcn_readlane(selv, cur_k) : sel_key0[cur_k];
        const int key0 = base + cur_s * kTile;
        if (++cur_s == sub) {
            cur_s = 0;
            ++cur_k;
        }
        return key0;
    };
    // With the first selected tile, the key-norm bounds of the selected blocks (32 bytes each)
    // go to LDS; they arrive with that tile (when the caller supplied them).
    auto load_kbnd = [&]() {
        if (wave == 0 && p.kbnd != nullptr && nvalid <= kMaxBounded) {
            for (int i0 = 0; i0 < nvalid; i0 += 32) {
                const int i = i0 + (lane >> 1);
                if (i < nvalid) {
                    const int64_t blk = sel_key0[i] / p.bs;
                    const float* src = p.kbnd + ((b * p.nb + blk) * p.Hk + c) * 8 + 4 * (lane & 1);
                    __builtin_amdgcn_global_load_lds(src, (lds_void*)(sel_kbnd + 8 * i0), 16, 0, 0);
                }
            }
        }
    };
    if (!kLocal && total_tiles > 0) {
        dma_issue<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, next_key0(0), Ks0, Vs0, wave);
        if constexpr (kFastSel) load_kbnd();
    }

    ReadOffsets ro;
    ro.init(lane);

    f32x16 o[2][2], s[2][2];
    bf16x8 pb[2][2][2];
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
    zero(o);

    // Start of tile t in buffer BUF: wait for this wave's loads of tile t, then the barrier
    // makes every wave's loads visible and guarantees the other buffer (tile t-1) is no
    // longer read; the loads of tile t+1 go there.
    auto issue_next = [&](auto bufc, int t) {
        const int BUF = bufc;  // compile-time (Buf0 / Buf1) or runtime (t & 1)
        if (t + 1 < total_tiles)
            dma_issue<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, next_key0(t + 1), BUF ? Ks0 : Ks1, BUF ? Vs0 : Vs1, wave);
        if constexpr (kFastSel && kLocal) {
            if (t + 1 == tl_count) load_kbnd();
        }
    };
    auto begin_tile = [&](auto bufc, int t) {
        wait_vmem();
        __syncthreads();
        issue_next(bufc, t);
    };

    bf16_t* outp = p.out + (int64_t)b * p.out_sb + (int64_t)n0 * p.out_sn + (int64_t)j * kHeadDim;

    // ------------------------------------------------------------------ local branch
    if constexpr (kLocal) {
        // Start of local tile t: tile 0 of the modes with a partial buffer first takes the Q rows
        // staged in the prologue (and rotates them).
        auto local_begin = [&](auto bufc, int t) {
            if (kPartial && t == 0) {
                wait_vmem();
                __syncthreads();
                // the Q rows staged in the prologue (same layout as a K tile)
                const bf16_t* qs = Part + wave * 64 * PS;
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                    for (int ds = 0; ds < 4; ++ds)
                        qf[qt][ds] = as_bf16x8(*reinterpret_cast<const uint4*>(qs + 32 * qt * 64 + ro.k[ds]));
                if (p.rope_cos != nullptr) {
                    // RoPE of q: this lane's dims 16 ds + 8 hh .. + 7 of query row 32 qt + r are
                    // the pairs 8 ds + 4 hh .. + 3 of that row's table entries
                    const float* cs = reinterpret_cast<const float*>(Ks1);
                    const float* sn = reinterpret_cast<const float*>(Vs1);
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                        for (int ds = 0; ds < 4; ++ds) {
                            const int e = (32 * qt + r) * 32 + 8 * ds + 4 * hh;
                            const float4 c4 = *reinterpret_cast<const float4*>(cs + e);
                            const float4 s4 = *reinterpret_cast<const float4*>(sn + e);
                            const uint4 u = __builtin_bit_cast(uint4, qf[qt][ds]);
                            qf[qt][ds] = as_bf16x8(make_uint4(rope_pair(u.x, c4.x, s4.x), rope_pair(u.y, c4.y, s4.y),
                                                              rope_pair(u.z, c4.z, s4.z), rope_pair(u.w, c4.w, s4.w)));
                        }
                    __syncthreads();  // every wave is done with the tables before tile 1 lands there
                }
                issue_next(bufc, t);
            } else {
                begin_tile(bufc, t);
            }
        };
        // The tile's compute.  The buffer is a compile-time choice (Buf0 / Buf1): with a runtime
        // choice the compiler cannot tell the buffer read here from the one the next tile's
        // loads are landing in, and it waits for those loads before the first V read.
        auto local_run = [&](auto bufc, int t) {
            const bf16_t* Kc = decltype(bufc)::value ? Ks1 : Ks0;
            const bf16_t* Vc = decltype(bufc)::value ? Vs1 : Vs0;
            s_tile(Kc, ro, qf, s);
            float mt[2];
            bool need = false;
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                mt[qt] = tile_max(s, qt) * p.scale_log2;
                need |= mt[qt] > m[qt] + kTau;
            }
            if (t == 0) {  // first tile: O and l are still zero, the reference is the tile max
                m[0] = mt[0];
                m[1] = mt[1];
            } else if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform; rare after the first tile
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) {
                    const float mnew = mt[qt] > m[qt] + kTau ? mt[qt] : m[qt];
                    const float alpha = __builtin_amdgcn_exp2f(m[qt] - mnew);
                    l[qt] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) o[dt][qt] *= alpha;
                    m[qt] = mnew;
                }
            }
            float lt[2];
            exp_pack<true, true>(s, m, p.scale_log2, pb, lt);
            l[0] += lt[0];
            l[1] += lt[1];
            pv_tile(Vc, ro, pb, o);
        };
        // tile 0 (with the Q rows), then the rest in pairs over the two buffers
        local_begin(Buf0{}, 0);
        local_run(Buf0{}, 0);
        for (int t = 1; t < tl_count; t += 2) {
            begin_tile(Buf1{}, t);
            local_run(Buf1{}, t);
            if (t + 1 >= tl_count) break;
            begin_tile(Buf0{}, t + 1);
            local_run(Buf0{}, t + 1);
        }
        float inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) inv[qt] = 1.f / xor32_add(l[qt]);

        if constexpr (MODE == kModeLocalOnly || MODE == kModeNoSelection || kPartial) {
            float f[2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f[qt] = inv[qt];
                if constexpr (kWeights) f[qt] *= gate(0, qt);
            }
            if constexpr (MODE == kModeLocalOnly) {
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                        for (int g4 = 0; g4 < 4; ++g4) {
                            uint2 w2;
                            w2.x = pack_bf16x2(o[dt][qt][4 * g4 + 0] * f[qt], o[dt][qt][4 * g4 + 1] * f[qt]);
                            w2.y = pack_bf16x2(o[dt][qt][4 * g4 + 2] * f[qt], o[dt][qt][4 * g4 + 3] * f[qt]);
                            *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.out_sn + 32 * dt + 8 * g4 + 4 * hh) = w2;
                        }
                return;
            } else if constexpr (kPartial) {
                // w0 * o_ba waits in LDS (bf16) while the selected branch runs
                bf16_t* pp = Part + wave * 64 * PS;
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                        for (int g4 = 0; g4 < 4; ++g4) {
                            uint2 w2;
                            w2.x = pack_bf16x2(o[dt][qt][4 * g4 + 0] * f[qt], o[dt][qt][4 * g4 + 1] * f[qt]);
                            w2.y = pack_bf16x2(o[dt][qt][4 * g4 + 2] * f[qt], o[dt][qt][4 * g4 + 3] * f[qt]);
                            *reinterpret_cast<uint2*>(pp + (32 * qt + r) * PS + 32 * dt + 8 * g4 + 4 * hh) = w2;
                        }
            } else {  // no selection: keep w0 * o_ba in registers for the epilogue
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) o[dt][qt] *= f[qt];
            }
        }
    }

    // ------------------------------------------------------------------ selected branch
    if constexpr (kSel) {
        // ops.py:92: q * softmax_scale * LOG2_E in fp32, rounded to bf16
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
                const uint4 u = __builtin_bit_cast(uint4, qf[qt][ds]);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
                uint32_t o4[4];
#pragma unroll
                for (int mm = 0; mm < 4; ++mm)
                    o4[mm] = pack_bf16x2((bf_lo(w[mm]) * p.scale) * kLog2e, (bf_hi(w[mm]) * p.scale) * kLog2e);
                qf[qt][ds] = as_bf16x8(make_uint4(o4[0], o4[1], o4[2], o4[3]));
            }
        zero(o);
        l[0] = l[1] = 0.f;

        // Bounded-logit path.  |s| <= |q'| * |k|; with the pooled key-norm bounds of the
        // selected blocks, a wave whose rows all have |s| <= kLogitBound takes P = exp2(s)
        // directly (reference 0: P stays within [2^-64, 2^64], far from fp32 / bf16 limits)
        // and sums the bf16 P on the matrix pipe.  Otherwise the running-reference path below.
        float qn2[2] = {0.f, 0.f};  // |q'|^2 of this lane's rows
        if constexpr (kFastSel) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
                for (int ds = 0; ds < 4; ++ds) {
                    const uint4 u = __builtin_bit_cast(uint4, qf[qt][ds]);
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int mm = 0; mm < 4; ++mm) {
                        const bf16x2 h = __builtin_bit_cast(bf16x2, w[mm]);
                        qn2[qt] = __builtin_amdgcn_fdot2_f32_bf16(h, h, qn2[qt], false);
                    }
                }
                qn2[qt] = xor32_add(qn2[qt]);
            }
        }
        // after the barrier of the first selected tile: every row of this wave bounded?
        auto bounded = [&]() -> bool {
            if (p.kbnd == nullptr || nvalid > kMaxBounded) return false;
            float kb2 = 0.f;
            for (int i = lane; i < nvalid; i += 64) {
                const float4 a = *reinterpret_cast<const float4*>(sel_kbnd + 8 * i);
                const float4 c4 = *reinterpret_cast<const float4*>(sel_kbnd + 8 * i + 4);
                kb2 = fmaxf(kb2, ((a.x + a.y) + (a.z + a.w)) + ((c4.x + c4.y) + (c4.z + c4.w)));
            }
            kb2 = wave_max_nonneg(kb2);
            const float lim = kLogitBound * kLogitBound;
            return !__builtin_amdgcn_ballot_w64(!(qn2[0] * kb2 <= lim && qn2[1] * kb2 <= lim));
        };

        // running-reference path: the first tile's exact row max is the reference
        auto first_body = [&](auto bufc) __attribute__((always_inline)) {
            const int BUF = bufc;  // compile-time (Buf0 / Buf1) or runtime (t & 1)
            s_tile(BUF ? Ks1 : Ks0, ro, qf, s);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) m[qt] = tile_max(s, qt);
            float lt[2];
            exp_pack<false, true>(s, m, 1.f, pb, lt);
            l[0] += lt[0];
            l[1] += lt[1];
            pv_tile(BUF ? Vs1 : Vs0, ro, pb, o);
        };
        auto sel_body = [&](auto bufc) __attribute__((always_inline)) {
            const int BUF = bufc;  // compile-time (Buf0 / Buf1) or runtime (t & 1)
            const bf16_t* Kc = BUF ? Ks1 : Ks0;
            s_tile(Kc, ro, qf, s);
            float lt[2];
            exp_pack<false, true>(s, m, 1.f, pb, lt);
            if (__builtin_amdgcn_ballot_w64(!(lt[0] <= kSumLimit && lt[1] <= kSumLimit))) {
                // rare: recompute one query tile at a time with the reference moved up to
                // the tile's row max (K of this tile stays in LDS until the next barrier)
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) {
                    f32x16 sh[2];
                    s_half(Kc, ro, qf[qt], sh);
                    const float mx = half_max(sh);
                    const float mnew = mx > m[qt] ? mx : m[qt];
                    const float alpha = __builtin_amdgcn_exp2f(m[qt] - mnew);
                    l[qt] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) o[dt][qt] *= alpha;
                    m[qt] = mnew;
                    exp_pack_half(sh, mnew, pb[qt], lt[qt]);
                }
            }
            l[0] += lt[0];
            l[1] += lt[1];
            pv_tile(BUF ? Vs1 : Vs0, ro, pb, o);
        };

        int t = tl_count;
        bool fast = false;
        if (t < total_tiles) {  // barrier of the first selected tile, then the path choice
            begin_tile(t & 1, t);
            if constexpr (kFastSel) fast = bounded();
        }
        if (fast) {
            const bf16x8 rsel = row_sum_selector(lane);
            f32x4 lacc[2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) lacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
            auto fast_body = [&](auto bufc) __attribute__((always_inline)) {
                const int BUF = bufc;  // compile-time (Buf0 / Buf1) or runtime (t & 1)
                s_tile_seq(BUF ? Ks1 : Ks0, ro, qf, s);
                if constexpr (MODE == kModeSelectedOnly) {
                    // the LSE is an output: row sums of the fp32 P, as the reference forms l
                    // (ops.py:125), per lane on the VALU
                    float lt[2];
                    exp_pack<false, false>(s, m, 1.f, pb, lt);
                    l[0] += lt[0];
                    l[1] += lt[1];
                } else {
                    exp_pack_raw(s, pb);
                    row_sums(rsel, pb, lacc);
                }
                pv_tile(BUF ? Vs1 : Vs0, ro, pb, o);
            };
            // the first selected tile has begun; enter the two-buffer loop at its parity
            if (t & 1) {
                fast_body(Buf1{});
                if (++t < total_tiles) begin_tile(Buf0{}, t);
            }
            while (t < total_tiles) {
                fast_body(Buf0{});
                if (++t >= total_tiles) break;
                begin_tile(Buf1{}, t);
                fast_body(Buf1{});
                if (++t >= total_tiles) break;
                begin_tile(Buf0{}, t);
            }
            // every lane holds its row's whole sum (matrix-pipe sums) or its partial sum (VALU
            // sums of the selected-only mode); the epilogue adds the two key halves
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                if constexpr (MODE != kModeSelectedOnly) l[qt] = hh == 0 ? lacc[qt][0] : 0.f;
                m[qt] = 0.f;
            }
        } else if (t < total_tiles) {
            first_body(t & 1);
            ++t;
            if constexpr (MODE == kModeSelectedOnly) {  // the only path of this mode: unrolled
                if ((t & 1) && t < total_tiles) {
                    begin_tile(Buf1{}, t);
                    sel_body(Buf1{});
                    ++t;
                }
                for (; t + 1 < total_tiles; t += 2) {
                    begin_tile(Buf0{}, t);
                    sel_body(Buf0{});
                    begin_tile(Buf1{}, t + 1);
                    sel_body(Buf1{});
                }
                if (t < total_tiles) {
                    begin_tile(Buf0{}, t);
                    sel_body(Buf0{});
                }
            } else {  // fallback of the bounded path: one copy, runtime buffers
#pragma clang loop unroll(disable)
                for (; t < total_tiles; ++t) {
                    begin_tile(t & 1, t);
                    sel_body(t & 1);
                }
            }
        }
    }

    // ------------------------------------------------------------------ epilogue
    if constexpr (MODE == kModeSelectedOnly) {
        float ltot[2], inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            ltot[qt] = xor32_add(l[qt]);
            inv[qt] = 1.f / ltot[qt];
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    uint2 w2;
                    w2.x = pack_bf16x2(o[dt][qt][4 * g4 + 0] * inv[qt], o[dt][qt][4 * g4 + 1] * inv[qt]);
                    w2.y = pack_bf16x2(o[dt][qt][4 * g4 + 2] * inv[qt], o[dt][qt][4 * g4 + 3] * inv[qt]);
                    *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.out_sn + 32 * dt + 8 * g4 + 4 * hh) = w2;
                }
        if (p.lse != nullptr && hh == 0) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
                p.lse[((int64_t)b * p.N + n0 + 32 * qt + r) * p.Hq + j] = m[qt] + __log2f(ltot[qt]);
        }
        return;
    } else if constexpr (kWeights) {
        // per-row weights of the selected and compressed branches and the renormalisation
        float fs[2], fc[2], nrm[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const float w0 = gate(0, qt), w1 = gate(1, qt), w2 = gate(2, qt);
            if constexpr (kSel) fs[qt] = w2 / xor32_add(l[qt]);
            fc[qt] = w1;
            nrm[qt] = MODE == kModeNoCompression ? 1.f / (w0 + w2 + 1e-8f)
                    : MODE == kModeNoSelection ? 1.f / (w0 + w1 + 1e-8f) : 1.f;
        }
        f32x16 oc[2];  // compressed-branch output of block n0 / bs for head j (same for all rows)
        if constexpr (kCmp) {
            uint2 ocw[2][4];
            wait_vmem();  // the row was requested in the prologue; the wave reads its own bytes
            const bf16_t* ocp = Ocmp + wave * 64 + 4 * hh;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) ocw[dt][g4] = *reinterpret_cast<const uint2*>(ocp + 32 * dt + 8 * g4);
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    oc[dt][4 * g4 + 0] = bf_lo(ocw[dt][g4].x);
                    oc[dt][4 * g4 + 1] = bf_hi(ocw[dt][g4].x);
                    oc[dt][4 * g4 + 2] = bf_lo(ocw[dt][g4].y);
                    oc[dt][4 * g4 + 3] = bf_hi(ocw[dt][g4].y);
                }
        }
        bf16_t* pp = Part + wave * 64 * PS;
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    float v[4];
                    if constexpr (kPartial) {
                        const uint2 pw = *reinterpret_cast<const uint2*>(pp + (32 * qt + r) * PS + 32 * dt + 8 * g4 + 4 * hh);
                        v[0] = bf_lo(pw.x); v[1] = bf_hi(pw.x); v[2] = bf_lo(pw.y); v[3] = bf_hi(pw.y);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int jj = 4 * g4 + e;
                        float x;
                        if constexpr (kPartial) x = v[e] + o[dt][qt][jj] * fs[qt];
                        else x = o[dt][qt][jj];  // no selection: o holds w0 * o_ba
                        if constexpr (kCmp) x += oc[dt][jj] * fc[qt];
                        v[e] = x * nrm[qt];
                    }
                    uint2 w2;
                    w2.x = pack_bf16x2(v[0], v[1]);
                    w2.y = pack_bf16x2(v[2], v[3]);
                    if constexpr (kPartial)  // back into this lane's own Part slot, stored below
                        *reinterpret_cast<uint2*>(pp + (32 * qt + r) * PS + 32 * dt + 8 * g4 + 4 * hh) = w2;
                    else
                        *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.out_sn + 32 * dt + 8 * g4 + 4 * hh) = w2;
                }
        if constexpr (kPartial) {
            // Row-major read-back: lane l stores 16 bytes at chunk l % 8 of row l / 8 (+ 8 i),
            // 8 full 128-byte rows per store instead of 16-byte pieces of 32 rows.  Only this
            // wave's lanes touch its Part rows; LDS operations of a wave complete in order.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int rr = lane >> 3, cc = (lane & 7) * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = 8 * i + rr;
                const uint2 lo = *reinterpret_cast<const uint2*>(pp + row * PS + cc);
                const uint2 hi = *reinterpret_cast<const uint2*>(pp + row * PS + cc + 4);
                *reinterpret_cast<uint4*>(outp + (int64_t)row * p.out_sn + cc) = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
        }
    }
}

template <int NW>
hipError_t launch_nw(const AttnParams& p, int mode, bool idx64, hipStream_t s) {
    const dim3 grid(p.n_static + p.tail_wgs), block(NW * 64);
    void* args[] = {const_cast<AttnParams*>(&p)};
    const void* fn = nullptr;
    switch (mode) {
        case kModeFull: fn = (const void*)bsa_attn_kernel<NW, kModeFull, int32_t>; break;
        case kModeLocalOnly: fn = (const void*)bsa_attn_kernel<NW, kModeLocalOnly, int32_t>; break;
        case kModeNoCompression: fn = (const void*)bsa_attn_kernel<NW, kModeNoCompression, int32_t>; break;
        case kModeNoSelection: fn = (const void*)bsa_attn_kernel<NW, kModeNoSelection, int32_t>; break;
        case kModeSelectedOnly:
            fn = idx64 ? (const void*)bsa_attn_kernel<NW, kModeSelectedOnly, int64_t>
                       : (const void*)bsa_attn_kernel<NW, kModeSelectedOnly, int32_t>;
            break;
        default: return hipErrorInvalidValue;
    }
    return hipLaunchKernel(fn, grid, block, args, 0, s);
}

}  // namespace

hipError_t launch_attn(const AttnParams& p, int mode, bool idx64, int waves, hipStream_t s) {
    switch (waves) {
        case 1: return launch_nw<1>(p, mode, idx64, s);
        case 2: return launch_nw<2>(p, mode, idx64, s);
        case 4: return launch_nw<4>(p, mode, idx64, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mosaic
