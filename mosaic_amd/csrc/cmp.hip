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
//               the attention kernel combines the splits in its epilogue.
//
// Grid: (query-block tiles of 32, selection row h, batch * splits).  Workgroup: G waves;
// wave g handles query head j = g*Hk + h against kv head j / G, so the G heads averaged by
// selection row h sit in one workgroup and are reduced through LDS.
//
// The loop over key-block tiles is latency-bound (little arithmetic per tile), so the next
// tile's K and V^T fragments are loaded into registers while the current one is computed,
// and the per-head score exchange is double-buffered (one barrier per tile).
#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int XS = 36;  // row stride (floats) of the per-head score exchange buffer

struct CmpFrags {
    uint4 k[4];      // A operand of S^T = K Q^T: k_cmp[u0 + r][16*ds + 8*hh ..]
    uint2 v[2][2][2];  // A operand of O^T += V^T P^T: [dt][s2][lo/hi]
};

template <bool ATTN>
__device__ __forceinline__ void load_frags(CmpFrags& f, const CmpParams& p, const bf16_t* kp0, const bf16_t* vtp,
                                           int u0, int r, int hh) {
    const bool uvalid = u0 + r < p.nb;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
        f.k[ds] = uvalid ? ld16(kp0 + (int64_t)(u0 + r) * p.k_sn + 16 * ds) : make_uint4(0, 0, 0, 0);
    if constexpr (ATTN) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const bf16_t* vp = vtp + (int64_t)(32 * dt + r) * p.nb_pad + u0 + 16 * s2 + 4 * hh;
                f.v[dt][s2][0] = ld8(vp);
                f.v[dt][s2][1] = ld8(vp + 8);
            }
    }
}

template <bool SCORES, bool ATTN, int MAXT>
__global__ __launch_bounds__(MAXT) void cmp_kernel(CmpParams p) {
    extern __shared__ float xs[];  // [2][G][32 t][XS] bf16-rounded scores per head (SCORES)

    const int tid = threadIdx.x, g = tid >> 6, lane = tid & 63, r = lane & 31, hh = lane >> 5;
    const int t0 = blockIdx.x * 32, h = blockIdx.y;
    const int b = blockIdx.z / p.nsplit, split = blockIdx.z % p.nsplit;
    const int j = g * p.Hk + h;
    const int c = j / p.G;
    const int ut0 = split * p.ut_total / p.nsplit, ut1 = (split + 1) * p.ut_total / p.nsplit;
    const int nthreads = blockDim.x;
    const int xs_half = p.G * 32 * XS;

    const bool tvalid = t0 + r < p.nb;
    bf16x8 qf[4];
    {
        const bf16_t* qp = p.qc + b * p.q_sb + (int64_t)(t0 + r) * p.q_sn + (int64_t)j * p.q_sh + 8 * hh;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) qf[ds] = as_bf16x8(tvalid ? ld16(qp + 16 * ds) : make_uint4(0, 0, 0, 0));
    }
    const bf16_t* kp0 = p.kc + b * p.k_sb + (int64_t)c * p.k_sh + 8 * hh;
    const bf16_t* vtp = ATTN ? p.vct + ((int64_t)(b * p.Hk + c) * kHeadDim) * p.nb_pad : nullptr;

    f32x16 o[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    float m = -INFINITY, l = 0.f;

    CmpFrags cur, nxt;
    if (ut0 < ut1) load_frags<ATTN>(nxt, p, kp0, vtp, ut0 * 32, r, hh);

    for (int ut = ut0; ut < ut1; ++ut) {
        const int u0 = ut * 32;
        cur = nxt;
        if (ut + 1 < ut1) load_frags<ATTN>(nxt, p, kp0, vtp, u0 + 32, r, hh);

        f32x16 s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) s = mfma32(as_bf16x8(cur.k[ds]), qf[ds], s);

        if constexpr (SCORES) {
            // lane holds S^T[u0 + 8*(e/4) + 4*hh + e%4][t0 + r]
            float* xb = xs + ((ut - ut0) & 1) * xs_half;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                float4 v4;
                v4.x = round_bf16(s[4 * g4 + 0]);
                v4.y = round_bf16(s[4 * g4 + 1]);
                v4.z = round_bf16(s[4 * g4 + 2]);
                v4.w = round_bf16(s[4 * g4 + 3]);
                *reinterpret_cast<float4*>(xb + (g * 32 + r) * XS + 8 * g4 + 4 * hh) = v4;
            }
            __syncthreads();  // buffer (ut & 1) is next written two tiles later, after another barrier
            for (int e = tid; e < 32 * 32; e += nthreads) {
                const int tl = e >> 5, ul = e & 31;
                float sum = 0.f;
                for (int gg = 0; gg < p.G; ++gg) sum += xb[(gg * 32 + tl) * XS + ul];
                const float mean = sum / (float)p.G;
                if (t0 + tl < p.nb && u0 + ul < p.nb)
                    p.sbar[((int64_t)(b * p.Hk + h) * p.nb + t0 + tl) * p.nb_pad + u0 + ul] =
                        (bf16_t)(pack_bf16x2(mean, 0.f) & 0xffffu);
            }
        }

        if constexpr (ATTN) {
            float mx = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int u = u0 + 8 * (e >> 2) + 4 * hh + (e & 3);
                if (u >= p.nb) s[e] = -INFINITY;
                mx = fmaxf(mx, s[e]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(m, mx * p.scale_log2);
            const float alpha = __builtin_amdgcn_exp2f(m - mnew);
            float sum = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float pe = __builtin_amdgcn_exp2f(fmaf(s[e], p.scale_log2, -mnew));
                s[e] = pe;
                sum += pe;
            }
            l = l * alpha + sum;
            m = mnew;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) o[dt] *= alpha;
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
                    const uint2 lo = cur.v[dt][s2][0], hi = cur.v[dt][s2][1];
                    o[dt] = mfma32(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb, o[dt]);
                }
            }
        }
    }

    if constexpr (ATTN) {
        const float ltot = l + __shfl_xor(l, 32);
        if (tvalid) {
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

}  // namespace

hipError_t launch_cmp(const CmpParams& p, bool scores, bool attn, hipStream_t s) {
    const dim3 grid((p.nb + 31) / 32, p.Hk, p.B * p.nsplit), block(p.G * 64);
    const size_t shmem = scores ? (size_t)2 * p.G * 32 * XS * sizeof(float) : 0;
    void* args[] = {const_cast<CmpParams*>(&p)};
    const void* fn = nullptr;
    const int nt = p.G * 64;
#define MOSAIC_CMP_PICK(MAXT)                                                    \
    if (scores && attn) fn = (const void*)cmp_kernel<true, true, MAXT>;          \
    else if (scores) fn = (const void*)cmp_kernel<true, false, MAXT>;            \
    else if (attn) fn = (const void*)cmp_kernel<false, true, MAXT>;              \
    else return hipSuccess;
    if (nt <= 256) {
        MOSAIC_CMP_PICK(256)
    } else if (nt <= 512) {
        MOSAIC_CMP_PICK(512)
    } else {
        MOSAIC_CMP_PICK(1024)
    }
#undef MOSAIC_CMP_PICK
    if (shmem > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
        if (e != hipSuccess) return e;
    }
    return hipLaunchKernel(fn, grid, block, args, shmem, s);
}

}  // namespace mosaic
