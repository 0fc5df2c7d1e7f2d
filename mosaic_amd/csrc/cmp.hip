// cmp.hip -- compressed (block-to-block) attention and top-k selection scores (gfx950).
//
// Both consume S = q_cmp . k_cmp^T over the mean-pooled blocks, so one kernel computes the
// 32x32 score tile once with bf16 MFMA and uses it twice:
//
//   scores      attn_topk (primitives.py:35-49): bf16(S) per query head (the matmul output
//               dtype), then the mean over the G query heads g*Hk + h of selection row h
//               (einops '(g h)' grouping, :47), rounded to bf16, written row-major in u.
//   attention   flash_attn_func(q_cmp, k_cmp, v_cmp) (primitives.py:77): logits S*scale,
//               online softmax in base 2 over this split's range of key blocks, P -> bf16,
//               O^T += v_cmp^T P^T.  Each split writes its unnormalised O and (max, sum);
//               the top-k kernel combines the splits.  With one split the kernel writes
//               the output bf16(O / l) itself.
//
// Grid: (query-block tiles of 32, selection row h, batch * splits).  Workgroup: G waves;
// wave g handles query head j = g*Hk + h against kv head j / G, so the G heads averaged by
// selection row h sit in one workgroup and are reduced through LDS (bf16 tiles, 8-byte
// reads and stores).
//
// The loop over key-block tiles is latency-bound (little arithmetic per tile, one wave per
// SIMD at the usual sizes): it is software-pipelined by one tile (the S product of the next
// tile runs on the matrix cores during the mean and softmax of the current one), and the K
// and V^T fragments are requested one to two tiles ahead into separate double-buffered
// register sets (unrolled by two).  The pooling kernel writes K and V in MFMA
// operand order (kfrag_index / vfrag_index), so each fragment is one coalesced 16-byte load
// per lane; gathering them from row-major K and transposed V (32 rows per instruction) made
// this kernel memory-pipeline bound (27.5 us against 15.7 us at Nside 64).  All loads are
// unconditional, so the compiler's wait counts stay exact and a wait for the prefetched
// fragments never waits for the score stores issued after them.
#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int XSB = 40;  // row stride (bf16) of the per-head score exchange tile [32 t][32 u]
constexpr float kTau = 8.0f;

struct KFrags {
    uint4 k[4];  // A operand of S^T = K Q^T: k_cmp[u0 + r][16*ds + 8*hh ..]
};
struct VFrags {
    uint2 v[2][2][2];  // A operand of O^T += V^T P^T: [dt][s2][lo/hi]
};

// One 32-block tile's fragments: contiguous 1 KB runs of the operand-ordered pooled K / V
// (blocks past nb are zero there; their scores are masked or never stored).
__device__ __forceinline__ void load_k(KFrags& f, const CmpParams& p, int b, int c, int ut, int lane) {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) f.k[ds] = ld16(p.kfr + kfrag_index(b, c, p.Hk, p.ut_total, ut, ds, lane));
}
__device__ __forceinline__ void load_v(VFrags& f, const CmpParams& p, int b, int c, int ut, int lane) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const uint4 w = ld16(p.vfr + vfrag_index(b, c, p.Hk, p.ut_total, ut, dt, s2, lane));
            f.v[dt][s2][0] = make_uint2(w.x, w.y);
            f.v[dt][s2][1] = make_uint2(w.z, w.w);
        }
}

// Mean over the G heads of one 32x32 tile of bf16 scores in LDS, rounded to bf16 and stored
// (rows past the last block are skipped; columns up to nb_pad are written, the padding is
// never read).  Thread tid handles 16/G consecutive columns of row (tid * 16/G) / 32.
template <int G>
__device__ __forceinline__ void store_mean(const bf16_t* xb, bf16_t* dst_row0, int64_t row_stride, int rows_left,
                                           int tid, int gcount) {
    if constexpr (G == 0) {  // head count not a power of two: one element at a time
        for (int e = tid; e < 32 * 32; e += gcount * 64) {
            const int t = e >> 5, u = e & 31;
            if (t >= rows_left) break;
            float sum = 0.f;
            for (int gg = 0; gg < gcount; ++gg) sum += bf2f(xb[(gg * 32 + t) * XSB + u]);
            dst_row0[t * row_stride + u] = (bf16_t)(pack_bf16x2(sum / (float)gcount, 0.f) & 0xffffu);
        }
        return;
    }
    constexpr int GG = G > 0 ? G : 1;
    constexpr int EPT = 16 / GG;            // elements per thread
    constexpr int CH = EPT >= 4 ? 4 : EPT;  // elements per LDS read / global store
    const int e0 = tid * EPT, t = e0 >> 5, u = e0 & 31;
    if (t >= rows_left) return;
#pragma unroll
    for (int c0 = 0; c0 < EPT; c0 += CH) {
        float acc[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) acc[i] = 0.f;
#pragma unroll
        for (int g = 0; g < GG; ++g) {
            const bf16_t* src = xb + (g * 32 + t) * XSB + u + c0;
            if constexpr (CH == 4) {
                const uint2 w = *reinterpret_cast<const uint2*>(src);
                acc[0] += bf_lo(w.x); acc[1] += bf_hi(w.x); acc[2] += bf_lo(w.y); acc[3] += bf_hi(w.y);
            } else if constexpr (CH == 2) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
                acc[0] += bf_lo(w); acc[1] += bf_hi(w);
            } else {
                acc[0] += bf2f(*src);
            }
        }
        bf16_t* dst = dst_row0 + t * row_stride + u + c0;
        constexpr float kInvG = 1.f / GG;  // exact: GG is a power of two
        if constexpr (CH == 4) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(pack_bf16x2(acc[0] * kInvG, acc[1] * kInvG), pack_bf16x2(acc[2] * kInvG, acc[3] * kInvG));
        } else if constexpr (CH == 2) {
            *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(acc[0] * kInvG, acc[1] * kInvG);
        } else {
            *dst = (bf16_t)(pack_bf16x2(acc[0] * kInvG, 0.f) & 0xffffu);
        }
    }
}

// G > 0: query heads per kv head as a compile-time constant (a power of two); G == 0: any
// head count (p.G waves, at most 16).
template <bool SCORES, bool ATTN, int G>
__global__ __attribute__((amdgpu_flat_work_group_size(1, G > 0 ? G * 64 : 1024), amdgpu_waves_per_eu(1, 3)))
void cmp_kernel(CmpParams p) {
    constexpr int kMaxG = G > 0 ? G : 16;
    __shared__ __attribute__((aligned(16))) bf16_t xs[SCORES ? 2 * kMaxG * 32 * XSB : 8];  // [2][G][32 t][XSB]
    const int ng = G > 0 ? G : p.G;

    const int tid = threadIdx.x, g = tid >> 6, lane = tid & 63, r = lane & 31, hh = lane >> 5;
    const int t0 = blockIdx.x * 32, h = blockIdx.y;
    const int b = blockIdx.z / p.nsplit, split = blockIdx.z % p.nsplit;
    const int j = g * p.Hk + h;
    const int c = j / ng;
    const int ut0 = split * p.ut_total / p.nsplit, ut1 = (split + 1) * p.ut_total / p.nsplit;

    const bool tvalid = t0 + r < p.nb;
    bf16x8 qf[4];
    {
        const int trow = min(t0 + r, p.nb - 1);  // rows past the last block: clamped, never stored
        const bf16_t* qp = p.qc + b * p.q_sb + (int64_t)trow * p.q_sn + (int64_t)j * p.q_sh + 8 * hh;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) qf[ds] = as_bf16x8(ld16(qp + 16 * ds));
    }
    bf16_t* srow0 = SCORES ? p.sbar + ((int64_t)(b * p.Hk + h) * p.nb + t0) * p.nb_pad : nullptr;

    f32x16 o[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    float m = -INFINITY, l = 0.f;

    // S^T of one key tile for this head (fp32)
    auto scores_of = [&](const KFrags& kf) __attribute__((always_inline)) {
        f32x16 s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) s = mfma32(as_bf16x8(kf.k[ds]), qf[ds], s);
        return s;
    };
    // lane holds S^T[u0 + 8*(e/4) + 4*hh + e%4][t0 + r]: bf16(S) of this head to exchange buffer buf
    auto publish = [&](const f32x16& s, int buf) __attribute__((always_inline)) {
        bf16_t* xb = xs + buf * (kMaxG * 32 * XSB);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
            *reinterpret_cast<uint2*>(xb + (g * 32 + r) * XSB + 8 * g4 + 4 * hh) =
                make_uint2(pack_bf16x2(s[4 * g4 + 0], s[4 * g4 + 1]), pack_bf16x2(s[4 * g4 + 2], s[4 * g4 + 3]));
    };
    // the online softmax of one tile's logits and O^T += V^T P^T
    auto attend = [&](f32x16 s, const VFrags& vf, int ut) __attribute__((always_inline)) {
        const int u0 = ut * 32;
        if (u0 + 32 > p.nb) {  // last, partial tile: blocks past the end get no weight
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (u0 + 8 * (e >> 2) + 4 * hh + (e & 3) >= p.nb) s[e] = -INFINITY;
        }
        float mx = s[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s[e]);
        mx = xor32_max(mx) * p.scale_log2;
        // lazy reference: moves only when a tile's max exceeds it by more than kTau (the
        // first tile always moves it), so P <= 2^kTau and O is rarely rescaled
        if (__builtin_amdgcn_ballot_w64(mx > m + kTau)) {
            const float mnew = mx > m + kTau ? mx : m;
            const float alpha = __builtin_amdgcn_exp2f(m - mnew);
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) o[dt] *= alpha;
            m = mnew;
        }
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float pe = __builtin_amdgcn_exp2f(fmaf(s[e], p.scale_log2, -m));
            s[e] = pe;
            sum += pe;
        }
        l += sum;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            uint4 pu;
            pu.x = pack_bf16x2(s[8 * s2 + 0], s[8 * s2 + 1]);
            pu.y = pack_bf16x2(s[8 * s2 + 2], s[8 * s2 + 3]);
            pu.z = pack_bf16x2(s[8 * s2 + 4], s[8 * s2 + 5]);
            pu.w = pack_bf16x2(s[8 * s2 + 6], s[8 * s2 + 7]);
            const bf16x8 pb = as_bf16x8(pu);
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const uint2 lo = vf.v[dt][s2][0], hi = vf.v[dt][s2][1];
                o[dt] = mfma32(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb, o[dt]);
            }
        }
    };
    // Software-pipelined by one tile: the S product of tile ut + 1 is issued before the score
    // mean and the softmax of tile ut, so the matrix cores run it while those execute, and
    // bf16(S) of tile ut + 1 is published (one barrier per tile) after them.  K and V
    // fragments are double-buffered separately: K of tile ut + 2 and V of tile ut + 1 are
    // requested while tile ut is processed.  Past the last tile the requests repeat the last
    // tile (never used), so every load is unconditional and every wait targets exactly the
    // fragments about to be used.  Exchange buffer (ut - ut0) & 1 holds tile ut; it is
    // rewritten two tiles later, after the barrier that follows every wave's mean of it.
    if (ut0 < ut1) {
        KFrags ka, kb;
        VFrags va, vb;
        load_k(ka, p, b, c, ut0, lane);
        load_v(va, p, b, c, ut0, lane);
        load_k(kb, p, b, c, min(ut0 + 1, ut1 - 1), lane);
        f32x16 sa = scores_of(ka), sb;
        if constexpr (SCORES) {
            publish(sa, 0);
            __syncthreads();
        }
        for (int ut = ut0;; ut += 2) {
            // tile ut: S in sa (published in buffer 0), V in va; K of tile ut + 1 in kb
            sb = scores_of(kb);
            load_k(ka, p, b, c, min(ut + 2, ut1 - 1), lane);
            if constexpr (ATTN) load_v(vb, p, b, c, min(ut + 1, ut1 - 1), lane);
            if constexpr (SCORES) store_mean<G>(xs, srow0 + ut * 32, p.nb_pad, p.nb - t0, tid, ng);
            if constexpr (ATTN) attend(sa, va, ut);
            if (ut + 1 >= ut1) break;
            if constexpr (SCORES) {
                publish(sb, 1);
                __syncthreads();
            }
            // tile ut + 1: S in sb (buffer 1), V in vb; K of tile ut + 2 in ka
            sa = scores_of(ka);
            load_k(kb, p, b, c, min(ut + 3, ut1 - 1), lane);
            if constexpr (ATTN) load_v(va, p, b, c, min(ut + 2, ut1 - 1), lane);
            if constexpr (SCORES)
                store_mean<G>(xs + kMaxG * 32 * XSB, srow0 + (ut + 1) * 32, p.nb_pad, p.nb - t0, tid, ng);
            if constexpr (ATTN) attend(sb, vb, ut + 1);
            if (ut + 2 >= ut1) break;
            if constexpr (SCORES) {
                publish(sa, 0);
                __syncthreads();
            }
        }
    }

    if constexpr (ATTN) {
        const float ltot = xor32_add(l);
        if (tvalid && p.ocmp != nullptr) {
            // one split: the output itself, O / l rounded to bf16 (the combine's value for one
            // split, the same division)
            bf16_t* op = p.ocmp + (((int64_t)b * p.nb + t0 + r) * p.Hq + j) * kHeadDim;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4)
                    *reinterpret_cast<uint2*>(op + 32 * dt + 8 * g4 + 4 * hh) =
                        make_uint2(pack_bf16x2(o[dt][4 * g4 + 0] / ltot, o[dt][4 * g4 + 1] / ltot),
                                   pack_bf16x2(o[dt][4 * g4 + 2] / ltot, o[dt][4 * g4 + 3] / ltot));
        } else if (tvalid) {
            const int64_t row = (((int64_t)b * p.nsplit + split) * p.nb + t0 + r) * p.Hq + j;
            if (hh == 0) p.ml[row] = make_float2(m, ltot);
            float* op = p.opart + row * kHeadDim;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4)
                    *reinterpret_cast<float4*>(op + 32 * dt + 8 * g4 + 4 * hh) =
                        make_float4(o[dt][4 * g4 + 0], o[dt][4 * g4 + 1], o[dt][4 * g4 + 2], o[dt][4 * g4 + 3]);
        }
    }
}

template <int G>
const void* pick(bool scores, bool attn) {
    if (scores && attn) return (const void*)cmp_kernel<true, true, G>;
    if (scores) return (const void*)cmp_kernel<true, false, G>;
    if (attn) return (const void*)cmp_kernel<false, true, G>;
    return nullptr;
}

}  // namespace

hipError_t launch_cmp(const CmpParams& p, bool scores, bool attn, hipStream_t s) {
    const dim3 grid((p.nb + 31) / 32, p.Hk, p.B * p.nsplit), block(p.G * 64);
    void* args[] = {const_cast<CmpParams*>(&p)};
    const void* fn = nullptr;
    switch (p.G) {
        case 1: fn = pick<1>(scores, attn); break;
        case 2: fn = pick<2>(scores, attn); break;
        case 4: fn = pick<4>(scores, attn); break;
        case 8: fn = pick<8>(scores, attn); break;
        case 16: fn = pick<16>(scores, attn); break;
        default: fn = pick<0>(scores, attn); break;
    }
    if (fn == nullptr) return hipSuccess;
    return hipLaunchKernel(fn, grid, block, args, 0, s);
}

}  // namespace mosaic
