// attn.hip -- fused local + selected-block attention with the gated merge (gfx950).
//
// One workgroup = (batch b, kv head c, 64-token query tile, group of NW query heads).
// Each wave owns one query head j of the GQA group and all 64 query rows of the tile; the
// K/V tiles of 64 keys are loaded once into LDS and read by all NW waves.
//
//   local branch     block_attention / flash_attn_func (primitives.py:28-32): the keys of
//                    the query's block_attn_size block, logits q.k * scale, fp32 online
//                    softmax in base 2, P rounded to bf16 for the PV product.
//   selected branch  mosaic_attn_fwd_kernel (ops.py:41-134): q pre-scaled by scale*log2(e)
//                    and rounded to bf16 (:92), the sparse_block_size blocks named by the
//                    top-k indices in order (:94-95), base-2 online softmax (:120-128),
//                    P -> bf16 before PV (:128), O / l and LSE = m + log2(l) (:130-131).
//   merge            primitives.py:62-89 in fp32 in the epilogue; the compressed branch is
//                    read from the split partial results of the compressed-attention kernel.
//
// Tiles of both branches form one sequence [local tiles..., selected tiles...] streamed
// through a double-buffered LDS ring with one barrier per tile: tile t+1 is written to the
// other buffer after tile t's compute, from registers loaded one tile earlier.
//
// The softmax rescale is lazy: a row's reference max only moves when a tile's max exceeds
// it by more than kTau (log2 units), so P = exp2(s - m) <= 2^kTau and, after the first tile,
// the O accumulators are touched by MFMA only.  The result is the same softmax: numerator
// and denominator share the reference max.  Row sums are taken from the bf16-rounded P with
// v_dot2c_f32_bf16, i.e. from the same values that enter the PV product.
//
// Two workgroups share a CU (2 waves per SIMD): one wave's softmax VALU work overlaps the
// other's MFMA work.  The local branch's partial merge (w0 * o_ba) waits in LDS as bf16.
//
// S^T = K Q^T and O^T = V^T P^T are computed so a lane owns one query column (see
// bsa_common.h).  K is kept row-major in LDS (A operand rows = keys); V is transposed while
// being written to LDS so the PV A operand reads 8-byte runs of consecutive keys.
#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int KS = 72;  // K tile row stride in bf16 (144 B): 16-lane b128 reads hit distinct banks
constexpr int VS = 68;  // V^T tile row stride in bf16 (136 B): 32-lane b64 reads hit distinct banks
constexpr int PS = 68;  // merge-partial row stride in bf16
constexpr int kKTile = 64 * KS;
constexpr int kVTile = 64 * VS;
constexpr float kTau = 8.0f;

template <int NW>
struct TileLoader {
    static constexpr int NT = NW * 64;
    static constexpr int KCH = 512 / NT;               // 16-byte K chunks per thread
    static constexpr int VCH = (256 + NT - 1) / NT;    // (key pair, 8 dims) V chunks per thread
    uint4 kr[KCH];
    uint4 v0[VCH], v1[VCH];

    __device__ __forceinline__ void load(const bf16_t* kb, const bf16_t* vb, int64_t ksn, int64_t vsn, int key0,
                                         int tid) {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int c = tid + i * NT, row = c >> 3, ch = c & 7;
            kr[i] = ld16(kb + (int64_t)(key0 + row) * ksn + ch * 8);
        }
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int c = tid + i * NT;
            if (VCH * NT == 256 || c < 256) {
                const int pr = c & 31, ch = c >> 5;
                const bf16_t* src = vb + (int64_t)(key0 + 2 * pr) * vsn + ch * 8;
                v0[i] = ld16(src);
                v1[i] = ld16(src + vsn);
            }
        }
    }

    __device__ __forceinline__ void store(bf16_t* Ks, bf16_t* Vt, int tid) const {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int c = tid + i * NT, row = c >> 3, ch = c & 7;
            *reinterpret_cast<uint4*>(Ks + row * KS + ch * 8) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int c = tid + i * NT;
            if (VCH * NT == 256 || c < 256) {
                const int pr = c & 31, ch = c >> 5;
                const uint32_t a[4] = {v0[i].x, v0[i].y, v0[i].z, v0[i].w};
                const uint32_t b[4] = {v1[i].x, v1[i].y, v1[i].z, v1[i].w};
                bf16_t* dst = Vt + (ch * 8) * VS + 2 * pr;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    *reinterpret_cast<uint32_t*>(dst + (2 * m) * VS) = (a[m] & 0xffffu) | (b[m] << 16);
                    *reinterpret_cast<uint32_t*>(dst + (2 * m + 1) * VS) = (a[m] >> 16) | (b[m] & 0xffff0000u);
                }
            }
        }
    }
};

__device__ __forceinline__ void zero(f32x16 (&x)[2][2]) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) x[a][b][e] = 0.f;
}

// S^T = K Q^T for one 64-key tile: s[key tile][query tile]
__device__ __forceinline__ void s_tile(const bf16_t* Ks, const bf16x8 (&qf)[2][4], f32x16 (&s)[2][2], int r, int hh) {
    zero(s);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + (32 * kt + r) * KS + 16 * ds + 8 * hh));
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[kt][qt] = mfma32(a, qf[qt][ds], s[kt][qt]);
        }
    }
}

// O^T += V^T P^T for one 64-key tile
__device__ __forceinline__ void pv_tile(const bf16_t* Vt, const bf16x8 (&pb)[2][2][2], f32x16 (&o)[2][2], int r,
                                        int hh) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const bf16_t* vp = Vt + (32 * dt + r) * VS + 32 * kt + 16 * s2 + 4 * hh;
                const uint2 lo = ld8(vp), hi = ld8(vp + 8);
                const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) o[dt][qt] = mfma32(a, pb[qt][kt][s2], o[dt][qt]);
            }
}

// Online softmax of one tile with lazy rescaling.  Logits are s * c when SCALED, else s.
// m: reference max per query tile (log2 units); l: this lane's partial denominators.
template <bool SCALED>
__device__ __forceinline__ void softmax_tile(f32x16 (&s)[2][2], float (&m)[2], float (&l)[2], f32x16 (&o)[2][2],
                                             bf16x8 (&pb)[2][2][2], float c) {
    float mt[2];
    bool need = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float mx = s[0][qt][0];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][qt][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        mt[qt] = SCALED ? mx * c : mx;
        need |= mt[qt] > m[qt] + kTau;
    }
    if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform; rare after a row's first tile
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const float mnew = mt[qt] > m[qt] + kTau ? mt[qt] : m[qt];
            const float alpha = __builtin_amdgcn_exp2f(m[qt] - mnew);  // 0 on a row's first tile
            l[qt] *= alpha;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) o[dt][qt] *= alpha;
            m[qt] = mnew;
        }
    }
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3f803f80u);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const float mm = m[qt];
        float lsum[2] = {0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x0 = s[kt][qt][8 * s2 + 2 * i], x1 = s[kt][qt][8 * s2 + 2 * i + 1];
                    const float p0 = __builtin_amdgcn_exp2f(SCALED ? fmaf(x0, c, -mm) : x0 - mm);
                    const float p1 = __builtin_amdgcn_exp2f(SCALED ? fmaf(x1, c, -mm) : x1 - mm);
                    w[i] = pack_bf16x2(p0, p1);
                    lsum[kt] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[i]), ones, lsum[kt], false);
                }
                pb[qt][kt][s2] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
            }
        l[qt] += lsum[0] + lsum[1];
    }
}

__device__ __forceinline__ float load_bf16(const bf16_t* p) { return bf2f(*p); }

template <int MODE>
struct AttnLds {
    static constexpr bool kPartial = MODE == kModeFull || MODE == kModeNoCompression;
};

template <int NW, int MODE, typename IdxT>
__global__ __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(2, 2)))
void bsa_attn_kernel(AttnParams p) {
    constexpr bool kLocal = MODE != kModeSelectedOnly;
    constexpr bool kSel = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeSelectedOnly;
    constexpr bool kCmp = MODE == kModeFull || MODE == kModeNoSelection;
    constexpr bool kWeights = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeNoSelection;
    constexpr bool kPartial = AttnLds<MODE>::kPartial;

    __shared__ __attribute__((aligned(16))) bf16_t Ks[2 * kKTile];
    __shared__ __attribute__((aligned(16))) bf16_t Vt[2 * kVTile];
    __shared__ __attribute__((aligned(16))) bf16_t Part[kPartial ? NW * 64 * PS : 8];
    __shared__ int sel_key0[kSel ? kMaxSelected : 1];  // first key of each in-range selected block
    __shared__ int sel_count;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 31, hh = lane >> 5;
    const int L = xcd_remap(blockIdx.x, p.total_wgs);
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
    const IdxT* ip = reinterpret_cast<const IdxT*>(p.idx) + ((int64_t)(b * p.nb + n0 / p.bs) * p.Hk + c) * p.K;
    // Selected blocks: wave 0 compacts the in-range indices (top-k order kept) into LDS once,
    // so the tile loop reads block offsets from LDS instead of waiting on a global load.
    if constexpr (kSel) {
        if (wave == 0) {
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
    // The loader asks for tiles in order 0, 1, 2, ...
    int cur_k = 0, cur_s = 0;
    auto next_key0 = [&](int t) -> int {
        if (kLocal && t < tl_count) return lstart + kTile * t;
        const int key0 = sel_key0[cur_k] + cur_s * kTile;
        if (++cur_s == sub) {
            cur_s = 0;
            ++cur_k;
        }
        return key0;
    };

    bf16x8 qf[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
            qf[qt][ds] = as_bf16x8(ld16(qb + (int64_t)(n0 + 32 * qt + r) * p.q_sn + 16 * ds + 8 * hh));

    // compressed-branch output of this block and head (bf16), consumed in the epilogue
    uint2 ocw[2][4];
    if constexpr (kCmp) {
        const bf16_t* ocp = p.ocmp + (((int64_t)b * p.nb + n0 / p.bs) * p.Hq + j) * kHeadDim + 4 * hh;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) ocw[dt][g4] = ld8(ocp + 32 * dt + 8 * g4);
    }

    TileLoader<NW> tl;
    if (total_tiles > 0) {
        tl.load(kb, vb, p.k_sn, p.v_sn, next_key0(0), tid);
        tl.store(Ks, Vt, tid);
        if (total_tiles > 1) tl.load(kb, vb, p.k_sn, p.v_sn, next_key0(1), tid);
    }

    f32x16 o[2][2], s[2][2];
    bf16x8 pb[2][2][2];
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
    zero(o);

    auto advance = [&](int t) {
        // after tile t's compute: publish tile t+1 into the other buffer, prefetch tile t+2
        if (t + 1 < total_tiles) {
            tl.store(Ks + ((t + 1) & 1) * kKTile, Vt + ((t + 1) & 1) * kVTile, tid);
            if (t + 2 < total_tiles) tl.load(kb, vb, p.k_sn, p.v_sn, next_key0(t + 2), tid);
        }
    };

    bf16_t* outp = p.out + ((int64_t)b * p.N + n0) * p.Hq * kHeadDim + (int64_t)j * kHeadDim;

    // ------------------------------------------------------------------ local branch
    if constexpr (kLocal) {
        for (int t = 0; t < tl_count; ++t) {
            __syncthreads();
            const int buf = t & 1;
            s_tile(Ks + buf * kKTile, qf, s, r, hh);
            softmax_tile<true>(s, m, l, o, pb, p.scale_log2);
            pv_tile(Vt + buf * kVTile, pb, o, r, hh);
            advance(t);
        }
        float inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) inv[qt] = 1.f / (l[qt] + __shfl_xor(l[qt], 32));

        if constexpr (MODE == kModeLocalOnly || MODE == kModeNoSelection || kPartial) {
            float f[2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f[qt] = inv[qt];
                if constexpr (kWeights) {
                    const float w0 = load_bf16(p.w + b * p.w_sb + (int64_t)(n0 + 32 * qt + r) * p.w_sn + (int64_t)j * p.w_sh);
                    f[qt] *= w0;
                }
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
                            *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.Hq * kHeadDim + 32 * dt + 8 * g4 + 4 * hh) = w2;
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
        m[0] = m[1] = -INFINITY;
        l[0] = l[1] = 0.f;
        for (int t = tl_count; t < total_tiles; ++t) {
            __syncthreads();
            const int buf = t & 1;
            s_tile(Ks + buf * kKTile, qf, s, r, hh);
            softmax_tile<false>(s, m, l, o, pb, 1.f);
            pv_tile(Vt + buf * kVTile, pb, o, r, hh);
            advance(t);
        }
    }

    // ------------------------------------------------------------------ epilogue
    if constexpr (MODE == kModeSelectedOnly) {
        float ltot[2], inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            ltot[qt] = l[qt] + __shfl_xor(l[qt], 32);
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
                    *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.Hq * kHeadDim + 32 * dt + 8 * g4 + 4 * hh) = w2;
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
            const int64_t woff = b * p.w_sb + (int64_t)(n0 + 32 * qt + r) * p.w_sn + (int64_t)j * p.w_sh;
            const float w0 = load_bf16(p.w + woff);
            const float w1 = load_bf16(p.w + p.w_ss + woff);
            const float w2 = load_bf16(p.w + 2 * p.w_ss + woff);
            if constexpr (kSel) fs[qt] = w2 / (l[qt] + __shfl_xor(l[qt], 32));
            fc[qt] = w1;
            nrm[qt] = MODE == kModeNoCompression ? 1.f / (w0 + w2 + 1e-8f)
                    : MODE == kModeNoSelection ? 1.f / (w0 + w1 + 1e-8f) : 1.f;
        }
        f32x16 oc[2];  // compressed-branch output of block n0 / bs for head j (same for all rows)
        if constexpr (kCmp) {
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
        const bf16_t* pp = Part + wave * 64 * PS;
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
                    *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.Hq * kHeadDim + 32 * dt + 8 * g4 + 4 * hh) = w2;
                }
    }
}

template <int NW>
hipError_t launch_nw(const AttnParams& p, int mode, bool idx64, hipStream_t s) {
    const dim3 grid(p.total_wgs), block(NW * 64);
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
