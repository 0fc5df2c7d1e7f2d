// pool.hip -- mean pooling of q, k, v over runs of sparse_block_size tokens (gfx950).
//
// Replaces reduce(x, 'b (nb bs) h d -> b nb h d', 'mean') (primitives.py:65-66,76): fp32
// sum over the block's tokens in token order, divided by the block size, rounded to bf16.
// One workgroup per (pooled block t, batch b) reads the block's q, k and v rows once
// (HBM-bound: each thread streams one 16-byte column chunk down the block's tokens).
// Outputs: [B, nb, H, 64] for the pooled tensors and, for v, the transposed layout
// [B, Hk, 64, nb_pad] (zero beyond nb) read by the compressed-attention PV product.
// Optionally, for the keys (tensor 1), the largest squared norm of each 8-dim chunk over the
// block's tokens: the sum of a head's 8 values bounds |k|^2 for every key of the block, which
// the attention kernel uses to bound its logits.
#include "bsa_common.h"

namespace mosaic {
namespace {

__global__ __launch_bounds__(256) void pool_kernel(PoolParams p) {
    const int t = blockIdx.x, b = blockIdx.y;
    const int c0 = p.heads[0] * 8, c1 = p.heads[1] * 8, c2 = p.heads[2] * 8;
    const int ctot = c0 + c1 + c2;
    for (int col = threadIdx.x; col < ctot; col += blockDim.x) {
        const int which = col < c0 ? 0 : (col < c0 + c1 ? 1 : 2);
        const int cc = col - (which == 0 ? 0 : (which == 1 ? c0 : c0 + c1));
        const int hd = cc >> 3, ch = cc & 7;
        bf16_t* out_t = (which == 2) ? p.out_t : nullptr;
        if (t >= p.nb) {  // padding columns of the transposed output
            if (out_t) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    out_t[((int64_t)(b * p.heads[2] + hd) * kHeadDim + ch * 8 + e) * p.nb_pad + t] = 0;
            }
            continue;
        }
        const int64_t sn = p.sn[which];
        const bf16_t* src = p.x[which] + b * p.sb[which] + (int64_t)t * p.bs * sn + (int64_t)hd * p.sh[which] + ch * 8;
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        float sqmax = 0.f;  // largest squared norm of this 8-dim chunk over the block's tokens
        for (int n = 0; n < p.bs; n += 8) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld16(src + (int64_t)(n + u) * sn);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float x[8] = {bf_lo(v[u].x), bf_hi(v[u].x), bf_lo(v[u].y), bf_hi(v[u].y),
                                    bf_lo(v[u].z), bf_hi(v[u].z), bf_lo(v[u].w), bf_hi(v[u].w)};
                float sq = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    acc[e] += x[e];
                    sq = fmaf(x[e], x[e], sq);
                }
                sqmax = fmaxf(sqmax, sq);
            }
        }
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
        if (out_t) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                out_t[((int64_t)(b * p.heads[2] + hd) * kHeadDim + ch * 8 + e) * p.nb_pad + t] =
                    (bf16_t)(pack_bf16x2(mean[e], 0.f) & 0xffffu);
        }
    }
}

}  // namespace

hipError_t launch_pool(const PoolParams& p, hipStream_t s) {
    void* args[] = {const_cast<PoolParams*>(&p)};
    const int tgrid = p.out_t ? p.nb_pad : p.nb;
    return hipLaunchKernel((const void*)pool_kernel, dim3(tgrid, p.B), dim3(256), args, 0, s);
}

}  // namespace mosaic
