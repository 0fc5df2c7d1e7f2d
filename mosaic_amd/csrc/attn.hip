// attn.hip -- fused local + selected-block attention with the gated merge (gfx950).
//
// One workgroup = (batch b, kv head c, 64-token query tile, group of NW query heads).
// Each wave owns one query head j = c*G + ... of the GQA group and all 64 query rows of the
// tile; the K/V tiles of 64 keys are loaded once into LDS and read by all NW waves.
//
//   local branch     block_attention / flash_attn_func (primitives.py:28-32): the keys of
//                    the query's block_attn_size block, logits q.k * scale, fp32 online
//                    softmax in base 2, P rounded to bf16 for the PV product.
//   selected branch  mosaic_attn_fwd_kernel (ops.py:41-134): q pre-scaled by scale*log2(e)
//                    and rounded to bf16 (:92), the sparse_block_size blocks named by the
//                    top-k indices in order (:94-95), base-2 online softmax (:120-128),
//                    P -> bf16 before PV (:128), O / l and LSE = m + log2(l) (:130-131).
//   merge            primitives.py:62-89 in fp32 in the epilogue, with the compressed branch
//                    read from the partial results of the compressed-attention kernel.
//
// S^T = K Q^T and O^T = V^T P^T are computed so a lane owns one query column (see
// bsa_common.h).  K is kept row-major in LDS (A operand rows = keys); V is transposed while
// being written to LDS so the PV A operand reads 8-byte runs of consecutive keys.
#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int KS = 72;  // K tile row stride in bf16 (144 B): 16-lane b128 reads hit distinct banks
constexpr int VS = 68;  // V^T tile row stride in bf16 (136 B): 32-lane b64 reads hit distinct banks

template <int NW>
struct TileLoader {
    static constexpr int NT = NW * 64;
    static constexpr int KCH = 512 / NT;               // 16-byte K chunks per thread
    static constexpr int VCH = (256 + NT - 1) / NT;    // (key pair, 8 dims) V chunks per thread
    uint4 kr[KCH];
    uint4 v0[VCH], v1[VCH];

    __device__ __forceinline__ void load(const bf16_t* kb, const bf16_t* vb, int64_t ksn,
                                         int64_t vsn, int key0, int tid) {
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

struct WaveState {
    f32x16 o[2][2];  // O^T accumulators [d tile][query tile]
    float m[2];      // running max of the logits (log2 units) per query tile
    float l[2];      // this lane's partial softmax denominator per query tile

    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[dt][qt][e] = 0.f;
        m[0] = m[1] = -INFINITY;
        l[0] = l[1] = 0.f;
    }
};

__device__ __forceinline__ bf16x8 pack8(const f32x16& s, int base) {
    uint4 u;
    u.x = pack_bf16x2(s[base + 0], s[base + 1]);
    u.y = pack_bf16x2(s[base + 2], s[base + 3]);
    u.z = pack_bf16x2(s[base + 4], s[base + 5]);
    u.w = pack_bf16x2(s[base + 6], s[base + 7]);
    return as_bf16x8(u);
}

// One 64-key tile: S^T = K Q^T, online softmax update, O^T += V^T P^T.
// SCALED: logits = S * c (local branch, unscaled q); otherwise logits = S (q pre-scaled).
template <bool SCALED>
__device__ __forceinline__ void attend_tile(const bf16_t* Ks, const bf16_t* Vt, const bf16x8 (&qf)[2][4],
                                            WaveState& st, float c, int r, int hh) {
    f32x16 s[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[kt][qt][e] = 0.f;

#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + (32 * kt + r) * KS + 16 * ds + 8 * hh));
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[kt][qt] = mfma32(a, qf[qt][ds], s[kt][qt]);
        }
    }

    bf16x8 pb[2][2][2];  // [query tile][key tile][16-key step]
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][qt][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(st.m[qt], SCALED ? mx * c : mx);
        const float alpha = __builtin_amdgcn_exp2f(st.m[qt] - mnew);
        float sum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float x = SCALED ? fmaf(s[kt][qt][e], c, -mnew) : s[kt][qt][e] - mnew;
                const float pe = __builtin_amdgcn_exp2f(x);
                s[kt][qt][e] = pe;
                sum += pe;
            }
        st.l[qt] = st.l[qt] * alpha + sum;
        st.m[qt] = mnew;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) st.o[dt][qt] *= alpha;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            pb[qt][kt][0] = pack8(s[kt][qt], 0);
            pb[qt][kt][1] = pack8(s[kt][qt], 8);
        }
    }

#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const bf16_t* vp = Vt + (32 * dt + r) * VS + 32 * kt + 16 * s2 + 4 * hh;
                const uint2 lo = ld8(vp), hi = ld8(vp + 8);
                const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) st.o[dt][qt] = mfma32(a, pb[qt][kt][s2], st.o[dt][qt]);
            }
}

__device__ __forceinline__ float load_bf16(const bf16_t* p) { return bf2f(*p); }

template <int NW, int MODE, typename IdxT>
__global__ __launch_bounds__(NW * 64) void bsa_attn_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) bf16_t Ks[64 * KS];
    __shared__ __attribute__((aligned(16))) bf16_t Vt[64 * VS];

    constexpr bool kLocal = MODE != kModeSelectedOnly;
    constexpr bool kSel = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeSelectedOnly;
    constexpr bool kCmp = MODE == kModeFull || MODE == kModeNoSelection;
    constexpr bool kWeights = MODE == kModeFull || MODE == kModeNoCompression || MODE == kModeNoSelection;

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

    bf16x8 qf[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
            qf[qt][ds] = as_bf16x8(ld16(qb + (int64_t)(n0 + 32 * qt + r) * p.q_sn + 16 * ds + 8 * hh));

    // gate weights of this lane's two query rows
    float wgt[2][3];
    if constexpr (kWeights) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int sidx = 0; sidx < 3; ++sidx)
                wgt[qt][sidx] = load_bf16(p.w + sidx * p.w_ss + b * p.w_sb + (int64_t)(n0 + 32 * qt + r) * p.w_sn +
                                          (int64_t)j * p.w_sh);
    }

    TileLoader<NW> tl;
    WaveState st;
    f32x16 acc[2][2];  // merge accumulator (fp32), same layout as st.o

    bf16_t* outp = p.out + ((int64_t)b * p.N + n0) * p.Hq * kHeadDim + (int64_t)j * kHeadDim;
    auto store_out = [&](const f32x16 (&val)[2][2]) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    uint2 w2;
                    w2.x = pack_bf16x2(val[dt][qt][4 * g4 + 0], val[dt][qt][4 * g4 + 1]);
                    w2.y = pack_bf16x2(val[dt][qt][4 * g4 + 2], val[dt][qt][4 * g4 + 3]);
                    *reinterpret_cast<uint2*>(outp + (int64_t)(32 * qt + r) * p.Hq * kHeadDim + 32 * dt + 8 * g4 + 4 * hh) = w2;
                }
    };

    // ------------------------------------------------------------------ local branch
    if constexpr (kLocal) {
        st.reset();
        const int lstart = (n0 / p.bs_l) * p.bs_l;
        const int ntiles = p.bs_l / kTile;
        tl.load(kb, vb, p.k_sn, p.v_sn, lstart, tid);
        for (int t = 0; t < ntiles; ++t) {
            __syncthreads();
            tl.store(Ks, Vt, tid);
            __syncthreads();
            if (t + 1 < ntiles) tl.load(kb, vb, p.k_sn, p.v_sn, lstart + kTile * (t + 1), tid);
            attend_tile<true>(Ks, Vt, qf, st, p.scale_log2, r, hh);
        }
        float inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) inv[qt] = 1.f / (st.l[qt] + __shfl_xor(st.l[qt], 32));

        if constexpr (MODE == kModeLocalOnly) {
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) acc[dt][qt] = st.o[dt][qt] * inv[qt];
            store_out(acc);
            return;
        } else {
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) acc[dt][qt] = st.o[dt][qt] * (inv[qt] * wgt[qt][0]);
        }
    }

    // ------------------------------------------------------------------ compressed branch
    if constexpr (kCmp) {
        // Combine the split partial results of block tq for head j: each split holds an
        // unnormalised O and its (max, sum) in log2 units.
        const int tq = n0 / p.bs;
        const int64_t row0 = ((int64_t)b * p.nsplit * p.nb + tq) * p.Hq + j;  // split 0
        const int64_t split_stride = (int64_t)p.nb * p.Hq;
        float M = -INFINITY;
        for (int sp = 0; sp < p.nsplit; ++sp) M = fmaxf(M, p.ml[row0 + sp * split_stride].x);
        f32x16 oc[2];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) oc[dt][e] = 0.f;
        float Lsum = 0.f;
        for (int sp = 0; sp < p.nsplit; ++sp) {
            const float2 mlv = p.ml[row0 + sp * split_stride];
            const float a = __builtin_amdgcn_exp2f(mlv.x - M);
            Lsum += a * mlv.y;
            const float* op = p.opart + (row0 + sp * split_stride) * kHeadDim;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(op + 32 * dt + 8 * g4 + 4 * hh);
                    oc[dt][4 * g4 + 0] += a * v4.x;
                    oc[dt][4 * g4 + 1] += a * v4.y;
                    oc[dt][4 * g4 + 2] += a * v4.z;
                    oc[dt][4 * g4 + 3] += a * v4.w;
                }
        }
        const float linv = 1.f / Lsum;
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const float w1 = wgt[qt][1] * linv;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) acc[dt][qt] += oc[dt] * w1;
        }
        if constexpr (MODE == kModeNoSelection) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                const float nrm = 1.f / (wgt[qt][0] + wgt[qt][1] + 1e-8f);
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) acc[dt][qt] *= nrm;
            }
            store_out(acc);
            return;
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
                for (int m = 0; m < 4; ++m)
                    o4[m] = pack_bf16x2((bf_lo(w[m]) * p.scale) * kLog2e, (bf_hi(w[m]) * p.scale) * kLog2e);
                qf[qt][ds] = as_bf16x8(make_uint4(o4[0], o4[1], o4[2], o4[3]));
            }
        st.reset();
        const int qblk = n0 / p.bs;
        const IdxT* ip = reinterpret_cast<const IdxT*>(p.idx) + ((int64_t)(b * p.nb + qblk) * p.Hk + c) * p.K;
        const int sub = p.bs / kTile;
        const int ntiles = p.K * sub;
        auto tile_key0 = [&](int t, bool& valid) {
            const int64_t blk = (int64_t)ip[t / sub];
            valid = blk >= 0 && blk < p.nb;
            return (int)((valid ? blk : 0) * p.bs) + (t % sub) * kTile;
        };
        bool valid_next;
        int key0 = tile_key0(0, valid_next);
        tl.load(kb, vb, p.k_sn, p.v_sn, key0, tid);
        for (int t = 0; t < ntiles; ++t) {
            const bool valid = valid_next;
            __syncthreads();
            tl.store(Ks, Vt, tid);
            __syncthreads();
            if (t + 1 < ntiles) {
                key0 = tile_key0(t + 1, valid_next);
                tl.load(kb, vb, p.k_sn, p.v_sn, key0, tid);
            }
            if (valid) attend_tile<false>(Ks, Vt, qf, st, 1.f, r, hh);
        }
        float ltot[2], inv[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            ltot[qt] = st.l[qt] + __shfl_xor(st.l[qt], 32);
            inv[qt] = 1.f / ltot[qt];
        }
        if constexpr (MODE == kModeSelectedOnly) {
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) acc[dt][qt] = st.o[dt][qt] * inv[qt];
            store_out(acc);
            if (p.lse != nullptr && hh == 0) {
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
                    p.lse[((int64_t)b * p.N + n0 + 32 * qt + r) * p.Hq + j] = st.m[qt] + __log2f(ltot[qt]);
            }
            return;
        } else if constexpr (MODE == kModeFull) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                const float w2 = wgt[qt][2] * inv[qt];
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) acc[dt][qt] += st.o[dt][qt] * w2;
            }
            store_out(acc);
        } else {  // no compression: (o_ba*w0 + o_slc*w2) / (w0 + w2 + 1e-8)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                const float nrm = 1.f / (wgt[qt][0] + wgt[qt][2] + 1e-8f);
                const float w2 = wgt[qt][2] * inv[qt];
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) acc[dt][qt] = (acc[dt][qt] + st.o[dt][qt] * w2) * nrm;
            }
            store_out(acc);
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
