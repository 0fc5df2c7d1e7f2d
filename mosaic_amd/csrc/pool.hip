// pool.hip -- mean pooling of q, k, v over runs of sparse_block_size tokens (gfx950).
//
// Replaces reduce(x, 'b (nb bs) h d -> b nb h d', 'mean') (primitives.py:65-66,76): fp32
// sum over the block's tokens in token order, divided by the block size, rounded to bf16.
// One workgroup per (pooled block t, batch b) reads the block's q, k and v rows once
// (HBM-bound: each thread streams one 16-byte column chunk down the block's tokens).
// Outputs: [B, nb, H, 64] for the pooled tensors and, for k and v, the MFMA-operand-ordered
// layouts read by the compressed-attention kernel (kfrag_index / vfrag_index; zero for the
// padding blocks nb .. nb_pad-1).
// Optionally, for the keys (tensor 1), the largest squared norm of each 8-dim chunk over the
// block's tokens: the sum of a head's 8 values bounds |k|^2 for every key of the block, which
// the attention kernel uses to bound its logits.
// Optionally, q and k (tensors 0 and 1) are first rotated by the 2-D RoPE of the tokens'
// positions (primitives.py:125-135: x * cos + rotate_half(x) * sin in fp32, back to bf16):
// pair m = (2m, 2m+1) of a head becomes (x0 c_m - x1 s_m, x1 c_m + x0 s_m), each product and
// the sum rounded as the reference rounds them.  The rotated rows are written out (the
// attention reads them) and pooled, so the rotation costs no extra read of q and k.
#include "bsa_common.h"

namespace mosaic {
namespace {

// ROPE: 0 no rotation; 1 rotation with the block's table rows staged in LDS; 2 rotation with
// the table rows read from global memory (blocks too large for the LDS staging).  Separate
// instantiations keep the LDS reads ds_read instructions (a runtime choice between the two
// address spaces compiled to generic loads).
template <int ROPE>
__global__ __launch_bounds__(256) void pool_kernel(PoolParams p) {
    const int t = blockIdx.x, b = blockIdx.y;
    // RoPE tables of the block's tokens, read once per workgroup: [token][8 float4] of cos,
    // then of sin (every head of a token uses the same row)
    extern __shared__ float4 rope_rows[];
    if (ROPE == 1 && t < p.nb) {
        const float4* c4 = reinterpret_cast<const float4*>(p.rope_cos) + (int64_t)t * p.bs * 8;
        const float4* s4 = reinterpret_cast<const float4*>(p.rope_sin) + (int64_t)t * p.bs * 8;
        for (int i = threadIdx.x; i < 16 * p.bs; i += blockDim.x)
            rope_rows[i] = i < 8 * p.bs ? c4[i] : s4[i - 8 * p.bs];
        __syncthreads();
    }
    const int c0 = p.heads[0] * 8, c1 = p.heads[1] * 8, c2 = p.heads[2] * 8;
    const int ctot = c0 + c1 + c2;
    for (int col = threadIdx.x; col < ctot; col += blockDim.x) {
        const int which = col < c0 ? 0 : (col < c0 + c1 ? 1 : 2);
        const int cc = col - (which == 0 ? 0 : (which == 1 ? c0 : c0 + c1));
        const int hd = cc >> 3, ch = cc & 7;
        bf16_t* frag = which == 1 ? p.kfrag : (which == 2 ? p.vfrag : nullptr);
        // operand-ordered output of this thread's 8 dims of block t (zero past nb)
        auto store_frag = [&](const float (&x)[8]) {
            const int UT = p.nb_pad >> 5, ut = t >> 5, w = t & 31;
            if (which == 1) {
                uint4 u;
                u.x = pack_bf16x2(x[0], x[1]); u.y = pack_bf16x2(x[2], x[3]);
                u.z = pack_bf16x2(x[4], x[5]); u.w = pack_bf16x2(x[6], x[7]);
                *reinterpret_cast<uint4*>(frag + kfrag_index(b, hd, p.heads[1], UT, ut, ch >> 1, 32 * (ch & 1) + w)) = u;
            } else {
                const int s2 = w >> 4, rem = w & 15, slot = 4 * (rem >> 3) + (rem & 3), hh = (rem & 7) >> 2;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = 8 * ch + e;
                    frag[vfrag_index(b, hd, p.heads[2], UT, ut, d >> 5, s2, 32 * hh + (d & 31)) + slot] =
                        (bf16_t)(pack_bf16x2(x[e], 0.f) & 0xffffu);
                }
            }
        };
        if (t >= p.nb) {  // padding blocks of the operand-ordered outputs
            if (frag) {
                const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                store_frag(zero);
            }
            continue;
        }
        const int64_t sn = p.sn[which];
        const bf16_t* src = p.x[which] + b * p.sb[which] + (int64_t)t * p.bs * sn + (int64_t)hd * p.sh[which] + ch * 8;
        // RoPE of this thread's 4 pairs (frequencies 4 ch .. 4 ch + 3) of token n of the block
        const bool rope = ROPE != 0 && which < 2;
        const int64_t tok0 = (int64_t)t * p.bs;
        bf16_t* rdst = rope && p.rot[which] != nullptr
                           ? p.rot[which] + (((int64_t)b * p.nb * p.bs + tok0) * p.heads[which] + hd) * kHeadDim + ch * 8
                           : nullptr;
        auto rotate = [&](uint4 v, int n) __attribute__((always_inline)) -> uint4 {
            float4 c, s;
            if constexpr (ROPE == 1) {
                c = rope_rows[n * 8 + ch];
                s = rope_rows[8 * p.bs + n * 8 + ch];
            } else {
                c = *reinterpret_cast<const float4*>(p.rope_cos + (tok0 + n) * 32 + 4 * ch);
                s = *reinterpret_cast<const float4*>(p.rope_sin + (tok0 + n) * 32 + 4 * ch);
            }
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            const float cf[4] = {c.x, c.y, c.z, c.w}, sf[4] = {s.x, s.y, s.z, s.w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = rope_pair(w[i], cf[i], sf[i]);
            const uint4 r = make_uint4(o[0], o[1], o[2], o[3]);
            if (rdst) *reinterpret_cast<uint4*>(rdst + (int64_t)n * p.heads[which] * kHeadDim) = r;
            return r;
        };
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        float sqmax = 0.f;  // largest squared norm of this 8-dim chunk over the block's tokens
        auto add_token = [&](uint4 v, int n) __attribute__((always_inline)) {
            if (rope) v = rotate(v, n);
            const float x[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y),
                                bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
            float sq = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                acc[e] += x[e];
                sq = fmaf(x[e], x[e], sq);
            }
            sqmax = fmaxf(sqmax, sq);
        };
        int n = 0;
        for (; n + 8 <= p.bs; n += 8) {  // eight tokens' loads in flight, summed in token order
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld16(src + (int64_t)(n + u) * sn);
#pragma unroll
            for (int u = 0; u < 8; ++u) add_token(v[u], n + u);
        }
        for (; n < p.bs; ++n) add_token(ld16(src + (int64_t)n * sn), n);
        if (which == 1 && p.kbnd != nullptr)
            p.kbnd[(((int64_t)b * p.nb + t) * p.heads[1] + hd) * 8 + ch] = sqmax;
        const float denom = (float)p.bs;
        float mean[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) mean[e] = acc[e] / denom;
        bf16_t* out = p.out_bnhd[which];
        if (out) {
            uint4 w;
            w.x = pack_bf16x2(mean[0], mean[1]);
            w.y = pack_bf16x2(mean[2], mean[3]);
            w.z = pack_bf16x2(mean[4], mean[5]);
            w.w = pack_bf16x2(mean[6], mean[7]);
            *reinterpret_cast<uint4*>(out + (((int64_t)b * p.nb + t) * p.heads[which] + hd) * kHeadDim + ch * 8) = w;
        }
        if (frag) store_frag(mean);
    }
}

}  // namespace

hipError_t launch_pool(const PoolParams& p, hipStream_t s) {
    PoolParams q = p;
    // stage the RoPE rows in LDS when the block's rows fit the default dynamic limit (256 tokens, 64 KB)
    q.rope_lds = p.rope_cos != nullptr && p.bs <= 256;
    void* args[] = {&q};
    const int tgrid = (p.kfrag || p.vfrag) ? p.nb_pad : p.nb;
    const size_t lds = q.rope_lds ? (size_t)p.bs * 256 : 0;
    const void* fn = p.rope_cos == nullptr ? (const void*)pool_kernel<0>
                   : q.rope_lds ? (const void*)pool_kernel<1> : (const void*)pool_kernel<2>;
    return hipLaunchKernel(fn, dim3(tgrid, p.B), dim3(256), args, lds, s);
}

}  // namespace mosaic
