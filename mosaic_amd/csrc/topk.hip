// topk.hip -- per-row top-k block selection over the bf16 selection scores (gfx950).
//
// Replaces scores.topk(k=block_count, dim=-1, largest=True) of attn_topk
// (primitives.py:50).  One wave per row (b, h, t).  Each score becomes a 32-bit key
// (order-preserving image of the bf16 bits << 16 | (0xffff - u)), so one unsigned max picks
// the largest score and, among equal scores, the lowest block index.  K rounds of a wave
// max-reduction emit the indices in descending score order (torch's sorted=True order; the
// order of exactly tied scores is unspecified there).
//
// The wave max runs on DPP within each 16-lane row (quad swaps, half-row and row mirrors),
// then across rows with the two lane-swap permutes, leaving the maximum in every lane: no
// LDS or scalar round trips inside a selection round.
#include "bsa_common.h"

namespace mosaic {
namespace {

__device__ __forceinline__ uint32_t order16(uint32_t bits) {
    return (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
}

// Insert x into the descending list (b0 >= b1 >= b2 >= b3); the smallest falls off.
__device__ __forceinline__ void insert4(uint32_t& b0, uint32_t& b1, uint32_t& b2, uint32_t& b3, uint32_t x) {
    uint32_t t = max(b0, x); x = min(b0, x); b0 = t;
    t = max(b1, x); x = min(b1, x); b1 = t;
    t = max(b2, x); x = min(b2, x); b2 = t;
    b3 = max(b3, x);
}

template <int PL>  // keys per lane: nb <= 64 * PL
__global__ __launch_bounds__(256) void topk_kernel(TopkParams p) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // uniform per wave; no barriers in this kernel
    const int lane = threadIdx.x & 63;
    const bf16_t* src = p.sbar + (int64_t)row * p.nb_pad;
    const int t = row % p.nb;
    const int bh = row / p.nb;
    const int h = bh % p.Hk, b = bh / p.Hk;

    // The row's scores are loaded unconditionally (index clamped into the padded row) and
    // before the combine's loads, so all of them share one memory round trip.
    uint32_t raw[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) raw[i] = src[min(lane + 64 * i, p.nb_pad - 1)];

    // compressed-branch output of block t for the G query heads g*Hk + h of this row
    if (p.cmb.ocmp != nullptr) {
        int g = 0;
        for (; g + 4 <= p.G; g += 4) combine_ocmp<4>(p.cmb, b, p.nb, t, g * p.Hk + h, p.Hk, lane);
        for (; g < p.G; ++g) combine_ocmp<1>(p.cmb, b, p.nb, t, g * p.Hk + h, p.Hk, lane);
    }

    uint32_t key[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int u = lane + 64 * i;
        key[i] = (u < p.nb) ? ((order16(raw[i]) << 16) | (0xffffu - (uint32_t)u)) : 0u;
    }
    // Each lane keeps its four largest remaining keys.  Keys leave the wave in descending
    // order, so a lane's emitted keys are always its largest ones: after emitting key x the
    // lane's remaining keys are exactly those below x, and the buffer is refilled from them
    // only when all four buffered keys have been emitted.
    uint32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) insert4(b0, b1, b2, b3, key[i]);

    const int64_t out0 = (((int64_t)b * p.nb + t) * p.Hk + h) * p.K;

    int mine = 0;  // lane (kk mod 64) keeps the kk-th index for one coalesced store
    for (int kk = 0; kk < p.K; ++kk) {
        const uint32_t mx = wave_max_all_u32(b0);
        const int u = (int)(0xffffu - (mx & 0xffffu));
        const bool win = b0 == mx;
        if (win) {
            b0 = b1;
            b1 = b2;
            b2 = b3;
            b3 = 0;
        }
        if (PL > 4 && __builtin_amdgcn_ballot_w64(win && b0 == 0)) {
            if (win && b0 == 0) {
#pragma unroll
                for (int i = 0; i < PL; ++i) insert4(b0, b1, b2, b3, key[i] < mx ? key[i] : 0u);
            }
        }
        if ((kk & 63) == lane) mine = u;
        if ((kk & 63) == 63 || kk == p.K - 1) {
            const int base = kk & ~63;
            if (lane <= kk - base) {
                if (p.idx32) p.idx32[out0 + base + lane] = mine;
                if (p.idx64) p.idx64[out0 + base + lane] = mine;
            }
        }
    }
}

template <int PL>
hipError_t launch_pl(const TopkParams& p, hipStream_t s) {
    void* args[] = {const_cast<TopkParams*>(&p)};
    return hipLaunchKernel((const void*)topk_kernel<PL>, dim3((p.rows + 3) / 4), dim3(256), args, 0, s);
}

// Compressed-branch split combine alone (no selection): one wave per (batch, block).
__global__ __launch_bounds__(256) void combine_kernel(CombineParams c, int rows, int nb) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    const int t = row % nb, b = row / nb;
    int j = 0;
    for (; j + 4 <= c.Hq; j += 4) combine_ocmp<4>(c, b, nb, t, j, 1, lane);
    for (; j < c.Hq; ++j) combine_ocmp<1>(c, b, nb, t, j, 1, lane);
}

}  // namespace

hipError_t launch_combine(const CombineParams& c, int B, int nb, hipStream_t s) {
    const int rows = B * nb;
    void* args[] = {const_cast<CombineParams*>(&c), const_cast<int*>(&rows), &nb};
    return hipLaunchKernel((const void*)combine_kernel, dim3((rows + 3) / 4), dim3(256), args, 0, s);
}

hipError_t launch_topk(const TopkParams& p, hipStream_t s) {
    const int per_lane = (p.nb + 63) / 64;
    if (per_lane <= 1) return launch_pl<1>(p, s);
    if (per_lane <= 2) return launch_pl<2>(p, s);
    if (per_lane <= 3) return launch_pl<3>(p, s);
    if (per_lane <= 4) return launch_pl<4>(p, s);
    if (per_lane <= 6) return launch_pl<6>(p, s);
    if (per_lane <= 8) return launch_pl<8>(p, s);
    if (per_lane <= 12) return launch_pl<12>(p, s);
    if (per_lane <= 16) return launch_pl<16>(p, s);
    if (per_lane <= 24) return launch_pl<24>(p, s);
    if (per_lane <= 32) return launch_pl<32>(p, s);
    if (per_lane <= 48) return launch_pl<48>(p, s);
    if (per_lane <= 64) return launch_pl<64>(p, s);
    if (per_lane <= 96) return launch_pl<96>(p, s);
    if (per_lane <= 128) return launch_pl<128>(p, s);
    return hipErrorInvalidValue;
}

}  // namespace mosaic
