// topk.hip -- per-row top-k block selection over the bf16 selection scores (gfx950).
//
// Replaces scores.topk(k=block_count, dim=-1, largest=True) of attn_topk
// (primitives.py:50).  One wave per row (b, h, t).  Each score is turned into a 32-bit key
// (order-preserving image of the bf16 bits << 16 | (0xffff - u)), so one unsigned max picks
// the largest score and, among equal scores, the lowest block index.  K rounds of a wave
// max-reduction emit the indices in descending score order (torch's sorted=True order; the
// order of exactly tied scores is unspecified there).
#include "bsa_common.h"

namespace mosaic {
namespace {

__device__ __forceinline__ uint32_t order16(uint32_t bits) {
    return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
}

template <int PL>  // keys per lane: nb <= 64 * PL
__global__ __launch_bounds__(256) void topk_kernel(TopkParams p) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // uniform per wave; no barriers in this kernel
    const int lane = threadIdx.x & 63;
    const bf16_t* src = p.sbar + (int64_t)row * p.nb_pad;

    uint32_t key[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int u = lane + 64 * i;
        key[i] = (u < p.nb) ? ((order16(src[u]) << 16) | (0xffffu - (uint32_t)u)) : 0u;
    }
    const int t = row % p.nb;
    const int bh = row / p.nb;
    const int h = bh % p.Hk, b = bh / p.Hk;
    const int64_t out0 = (((int64_t)b * p.nb + t) * p.Hk + h) * p.K;

    for (int kk = 0; kk < p.K; ++kk) {
        uint32_t mx = 0;
#pragma unroll
        for (int i = 0; i < PL; ++i) mx = max(mx, key[i]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
#pragma unroll
        for (int i = 0; i < PL; ++i) key[i] = (key[i] == mx) ? 0u : key[i];
        const int u = (int)(0xffffu - (mx & 0xffffu));
        if (lane == 0) {
            if (p.idx32) p.idx32[out0 + kk] = u;
            if (p.idx64) p.idx64[out0 + kk] = u;
        }
    }
}

template <int PL>
hipError_t launch_pl(const TopkParams& p, hipStream_t s) {
    void* args[] = {const_cast<TopkParams*>(&p)};
    return hipLaunchKernel((const void*)topk_kernel<PL>, dim3((p.rows + 3) / 4), dim3(256), args, 0, s);
}

}  // namespace

hipError_t launch_topk(const TopkParams& p, hipStream_t s) {
    const int per_lane = (p.nb + 63) / 64;
    if (per_lane <= 1) return launch_pl<1>(p, s);
    if (per_lane <= 2) return launch_pl<2>(p, s);
    if (per_lane <= 4) return launch_pl<4>(p, s);
    if (per_lane <= 8) return launch_pl<8>(p, s);
    if (per_lane <= 16) return launch_pl<16>(p, s);
    if (per_lane <= 32) return launch_pl<32>(p, s);
    if (per_lane <= 64) return launch_pl<64>(p, s);
    if (per_lane <= 128) return launch_pl<128>(p, s);
    return hipErrorInvalidValue;
}

}  // namespace mosaic
