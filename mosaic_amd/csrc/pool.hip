// pool.hip -- mean pooling of q, k, v over runs of sparse_block_size tokens (gfx950).
//
// Replaces reduce(x, 'b (nb bs) h d -> b nb h d', 'mean') (primitives.py:65-66,76): fp32
// sum over the block's tokens in token order, divided by the block size, rounded to bf16.
// One workgroup per (pooled block t, batch b) reads the block's q, k and v rows once
// (HBM-bound).  Each thread streams one 16-byte column chunk down the block's tokens, summing in
// token order; with RoPE two adjacent threads share a chunk, each taking one half of the
// tokens, and their partial sums are added through a lane swap, which spreads the rotation
// arithmetic over twice as many waves.
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

// a[which] for which in 0..2 through selects, so a per-thread choice of tensor does not index
// the kernel's parameter block at run time (which would read it from memory)
template <typename T>
__device__ __forceinline__ T sel3(const T (&a)[3], int which) {
    return which == 0 ? a[0] : (which == 1 ? a[1] : a[2]);
}

// x of the other lane of the pair (l, l ^ 1): DPP quad_perm [1, 0, 3, 2]
__device__ __forceinline__ float swap_pair(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xb1, 0xf, 0xf, false));
}
// (first half) + (second half) in both lanes of a pair, in that order (half = this lane's half)
__device__ __forceinline__ float acc_pair(float x, int half) {
    const float y = swap_pair(x);
    return half ? y + x : x + y;
}

// ROPE: 0 no rotation; 1 rotation with the block's table rows staged in LDS; 2 rotation with
// the table rows read from global memory (blocks too large for the LDS staging).  Separate
// instantiations keep the LDS reads ds_read instructions (a runtime choice between the two
// address spaces compiled to generic loads).
template <int ROPE>
constexpr int kPoolMaxThreads = ROPE == 2 ? 512 : 1024;  // the global-table variant needs more registers
template <int ROPE>
constexpr int kThreadsPerChunk = ROPE != 0 ? 2 : 1;

template <int ROPE>
__global__ __launch_bounds__(kPoolMaxThreads<ROPE>) void pool_kernel(PoolParams p) {
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
    constexpr int TPC = kThreadsPerChunk<ROPE>;
    const int hb = TPC == 2 ? (p.bs + 1) >> 1 : p.bs;  // tokens of the first (or only) half
    // blockDim.x is even, so the two threads of a column are adjacent lanes of one iteration
    for (int col2 = threadIdx.x; col2 < TPC * ctot; col2 += blockDim.x) {
        const int col = TPC == 2 ? col2 >> 1 : col2, half = TPC == 2 ? col2 & 1 : 0;
        const int which = col < c0 ? 0 : (col < c0 + c1 ? 1 : 2);
        const int cc = col - (which == 0 ? 0 : (which == 1 ? c0 : c0 + c1));
        const int hd = cc >> 3, ch = cc & 7;
        // this thread's tensor, selected once (no runtime indexing of the parameter block)
        const int heads = sel3(p.heads, which);
        bf16_t* frag = which == 1 ? p.kfrag : (which == 2 ? p.vfrag : nullptr);
        // operand-ordered output of this thread's 8 dims of block t (zero past nb)
        auto store_frag = [&](const float (&x)[8]) {
            const int UT = p.nb_pad >> 5, ut = t >> 5, w = t & 31;
            if (which == 1) {
                uint4 u;
                u.x = pack_bf16x2(x[0], x[1]); u.y = pack_bf16x2(x[2], x[3]);
                u.z = pack_bf16x2(x[4], x[5]); u.w = pack_bf16x2(x[6], x[7]);
                *reinterpret_cast<uint4*>(frag + kfrag_index(b, hd, heads, UT, ut, ch >> 1, 32 * (ch & 1) + w)) = u;
            } else {
                const int s2 = w >> 4, rem = w & 15, slot = 4 * (rem >> 3) + (rem & 3), hh = (rem & 7) >> 2;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = 8 * ch + e;
                    frag[vfrag_index(b, hd, heads, UT, ut, d >> 5, s2, 32 * hh + (d & 31)) + slot] =
                        (bf16_t)(pack_bf16x2(x[e], 0.f) & 0xffffu);
                }
            }
        };
        if (t >= p.nb) {  // padding blocks of the operand-ordered outputs
            if (frag && half == 0) {
                const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                store_frag(zero);
            }
            continue;
        }
        // tokens n0 .. n1-1 of the block: this thread's half
        const int n0 = half ? hb : 0, n1 = half ? p.bs : hb;
        const int64_t sn = sel3(p.sn, which);
        const int64_t tok0 = (int64_t)t * p.bs + n0;
        const bf16_t* src = sel3(p.x, which) + b * sel3(p.sb, which) + tok0 * sn + (int64_t)hd * sel3(p.sh, which) + ch * 8;
        // RoPE of this thread's 4 pairs (frequencies 4 ch .. 4 ch + 3): table rows of token n0 + i
        const bool rope = ROPE != 0 && which < 2;
        bf16_t* rot = which == 0 ? p.rot[0] : (which == 1 ? p.rot[1] : nullptr);
        bf16_t* rdst = rope && rot != nullptr
                           ? rot + (((int64_t)b * p.nb * p.bs + tok0) * heads + hd) * kHeadDim + ch * 8
                           : nullptr;
        const int64_t rstride = (int64_t)heads * kHeadDim;
        const float4* ctab = ROPE == 1 ? rope_rows + n0 * 8 + ch
                                       : reinterpret_cast<const float4*>(p.rope_cos + tok0 * 32 + 4 * ch);
        const float4* stab = ROPE == 1 ? rope_rows + 8 * p.bs + n0 * 8 + ch
                                       : reinterpret_cast<const float4*>(p.rope_sin + tok0 * 32 + 4 * ch);
        auto rotate = [&](uint4 v, int i) __attribute__((always_inline)) -> uint4 {
            const float4 c = ctab[8 * i], s = stab[8 * i];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            const float cf[4] = {c.x, c.y, c.z, c.w}, sf[4] = {s.x, s.y, s.z, s.w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = rope_pair(w[k], cf[k], sf[k]);
            return make_uint4(o[0], o[1], o[2], o[3]);
        };
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        float sqmax = 0.f;  // largest squared norm of this 8-dim chunk over the block's tokens
        auto add_token = [&](uint4 v) __attribute__((always_inline)) {
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
        const int count = n1 - n0;
        int i = 0;
        for (; i + 8 <= count; i += 8) {  // eight tokens' loads in flight, summed in token order
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld16(src + (int64_t)u * sn);
            src += 8 * sn;
            if (rope) {
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = rotate(v[u], i + u);
                if (rdst) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) *reinterpret_cast<uint4*>(rdst + (int64_t)u * rstride) = v[u];
                    rdst += 8 * rstride;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) add_token(v[u]);
        }
        for (; i < count; ++i) {
            uint4 v = ld16(src);
            src += sn;
            if (rope) {
                v = rotate(v, i);
                if (rdst) {
                    *reinterpret_cast<uint4*>(rdst) = v;
                    rdst += rstride;
                }
            }
            add_token(v);
        }
        // first half + second half, the same sum in both lanes of the pair (a one-token block
        // has no second half: its sum is kept as is)
        if (p.bs > hb) {
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = acc_pair(acc[e], half);
            sqmax = fmaxf(sqmax, swap_pair(sqmax));
        }
        if (which == 1 && p.kbnd != nullptr && half == 0)
            p.kbnd[(((int64_t)b * p.nb + t) * heads + hd) * 8 + ch] = sqmax;
        const float denom = (float)p.bs;
        float mean[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) mean[e] = acc[e] / denom;
        bf16_t* out = sel3(p.out_bnhd, which);
        if (out && half == 0) {
            uint4 w;
            w.x = pack_bf16x2(mean[0], mean[1]);
            w.y = pack_bf16x2(mean[2], mean[3]);
            w.z = pack_bf16x2(mean[4], mean[5]);
            w.w = pack_bf16x2(mean[6], mean[7]);
            *reinterpret_cast<uint4*>(out + (((int64_t)b * p.nb + t) * heads + hd) * kHeadDim + ch * 8) = w;
        }
        if (frag && half == (p.bs > hb ? 1 : 0)) store_frag(mean);  // both halves hold the mean
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
    // one thread (two with RoPE) per 16-byte column chunk of the q, k, v rows, in whole waves
    const int items = (p.rope_cos != nullptr ? 2 : 1) * 8 * (p.heads[0] + p.heads[1] + p.heads[2]);
    const int cap = p.rope_cos == nullptr ? kPoolMaxThreads<0> : q.rope_lds ? kPoolMaxThreads<1> : kPoolMaxThreads<2>;
    const int threads = items >= cap ? cap : (items + 63) / 64 * 64;
    return hipLaunchKernel(fn, dim3(tgrid, p.B), dim3(threads), args, lds, s);
}

}  // namespace mosaic
