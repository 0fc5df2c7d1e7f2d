// topk.hip -- per-row top-k block selection over the bf16 selection scores (gfx950).
//
// Replaces scores.topk(k=block_count, dim=-1, largest=True) of attn_topk
// (primitives.py:50).  One wave per row (b, h, t), or 2 or 4 rows per wave when the rows are
// many and short (topk_rows_kernel); the selection itself is select_topk_sorted (up to 16 keys
// per lane of the row's lanes and 64 selected) or select_topk (bsa_common.h).  When the row's
// compressed-branch output is combined here too, for 1, 2 or 4 query heads per kv head (NH)
// the split partials are requested before the selection and combined after it, so their
// memory latency overlaps the selection rounds.
#include "bsa_common.h"

namespace mosaic {
namespace {

template <int PL, int NH>  // keys per lane: nb <= 64 * PL; NH > 0: G == NH, partials prefetched
__global__ __launch_bounds__(256) void topk_kernel(TopkParams p) {
    constexpr bool kSorted = PL <= 16;
    __shared__ uint32_t lists[kSorted ? 4 * 64 * kSortedStride<PL> : 1];
    const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));  // one per wave
    if (p.zero_ctr != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(p.zero_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

    const int64_t out0 = (((int64_t)b * p.nb + t) * p.Hk + h) * p.K;
    auto select = [&]() __attribute__((always_inline)) {
        if constexpr (kSorted) {
            if (p.K <= 64) {
                select_topk_sorted<PL>(raw, p.nb, p.K, lane, out0, p.idx32, p.idx64,
                                       (lds_u32*)lists + (threadIdx.x >> 6) * 64 * kSortedStride<PL>);
                return;
            }
        }
        select_topk<PL>(raw, p.nb, p.K, lane, out0, p.idx32, p.idx64);
    };
    // compressed-branch output of block t for the G query heads g*Hk + h of this row
    if constexpr (NH > 0) {
        const bool cmb = p.cmb.ocmp != nullptr;
        CombineRows<NH> rows;
        if (cmb) combine_load<NH>(rows, p.cmb, b, p.nb, t, h, p.Hk, lane);
        select();
        if (cmb) combine_store<NH>(rows, p.cmb, b, p.nb, t, h, p.Hk, lane);
    } else {
        if (p.cmb.ocmp != nullptr) {
            int g = 0;
            for (; g + 4 <= p.G; g += 4) combine_ocmp<4>(p.cmb, b, p.nb, t, g * p.Hk + h, p.Hk, lane);
            for (; g < p.G; ++g) combine_ocmp<1>(p.cmb, b, p.nb, t, g * p.Hk + h, p.Hk, lane);
        }
        select();
    }
}

// R rows per wave (groups of 64 / R lanes) when the rows are many and short: the selection
// rounds' instructions then serve R rows at once.  Group lane lr holds the scores of blocks
// lr + (64 / R) i (PL of them) and combines dimensions R lr .. R lr + R - 1 of the row's NH
// query heads (NH == 0: no combine).  Groups past the last row load row rows - 1 and store
// nothing.
template <int PL, int R, int NH>
__global__ __launch_bounds__(256) void topk_rows_kernel(TopkParams p) {
    constexpr int LW = 64 / R;
    __shared__ uint32_t lists[4 * 64 * kSortedStride<PL>];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (p.zero_ctr != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(p.zero_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int row0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + wave) * R);
    if (row0 >= p.rows) return;  // uniform per wave; no barriers in this kernel
    const int lr = lane % LW;
    const int row_any = row0 + lane / LW;
    const bool live = row_any < p.rows;
    const int row = live ? row_any : p.rows - 1;
    const bf16_t* src = p.sbar + (int64_t)row * p.nb_pad;
    const int t = row % p.nb;
    const int bh = row / p.nb;
    const int h = bh % p.Hk, b = bh / p.Hk;

    uint32_t raw[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) raw[i] = src[min(lr + LW * i, p.nb_pad - 1)];
    const int64_t out0 = (((int64_t)b * p.nb + t) * p.Hk + h) * p.K;
    CombineRows<(NH > 0 ? NH : 1), R> rows;
    const bool cmb = NH > 0 && p.cmb.ocmp != nullptr;
    if constexpr (NH > 0) {
        if (cmb) combine_load_group<NH, R>(rows, p.cmb, b, p.nb, t, h, p.Hk, lr);
    }
    select_topk_sorted<PL, LW>(raw, p.nb, p.K, lane, out0, p.idx32, p.idx64,
                               (lds_u32*)lists + wave * 64 * kSortedStride<PL>, lr, live);
    if constexpr (NH > 0) {
        if (cmb && live) combine_store_group<NH, R>(rows, p.cmb, b, p.nb, t, h, p.Hk, lr);
    }
}

template <int PL, int R>
const void* rows_kernel(const TopkParams& p) {
    if (p.cmb.ocmp == nullptr) return (const void*)topk_rows_kernel<PL, R, 0>;
    if (p.G == 1) return (const void*)topk_rows_kernel<PL, R, 1>;
    if (p.G == 2) return (const void*)topk_rows_kernel<PL, R, 2>;
    if (p.G == 4) return (const void*)topk_rows_kernel<PL, R, 4>;
    return nullptr;
}

// Rows per wave: 4 (groups of 16 lanes) or 2 (of 32) when a group holds at most 16 keys per
// lane and K indices, and the grouped grid still has at least two waves per SIMD (2048).
template <int R>
const void* pick_rows(const TopkParams& p) {
    constexpr int LW = 64 / R;
    if (p.K > LW || p.nb > 16 * LW || p.rows < 2048 * R) return nullptr;
    const int pl = (p.nb + LW - 1) / LW;
    if (pl <= 1) return rows_kernel<1, R>(p);
    if (pl <= 2) return rows_kernel<2, R>(p);
    if (pl <= 3) return rows_kernel<3, R>(p);
    if (pl <= 4) return rows_kernel<4, R>(p);
    if (pl <= 6) return rows_kernel<6, R>(p);
    if (pl <= 8) return rows_kernel<8, R>(p);
    if (pl <= 12) return rows_kernel<12, R>(p);
    return rows_kernel<16, R>(p);
}

template <int PL>
hipError_t launch_pl(const TopkParams& p, hipStream_t s) {
    void* args[] = {const_cast<TopkParams*>(&p)};
    const void* fn = (const void*)topk_kernel<PL, 0>;
    if constexpr (PL <= 16) {
        if (p.G == 1) fn = (const void*)topk_kernel<PL, 1>;
        if (p.G == 2) fn = (const void*)topk_kernel<PL, 2>;
        if (p.G == 4) fn = (const void*)topk_kernel<PL, 4>;
    }
    return hipLaunchKernel(fn, dim3((p.rows + 3) / 4), dim3(256), args, 0, s);
}

// Compressed-branch split combine alone (no selection): one wave per (batch, block).
__global__ __launch_bounds__(256) void combine_kernel(CombineParams c, int rows, int nb) {
    const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));  // one per wave
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
    for (int R : {4, 2}) {
        const void* fn = R == 4 ? pick_rows<4>(p) : pick_rows<2>(p);
        if (fn != nullptr) {
            void* args[] = {const_cast<TopkParams*>(&p)};
            const int waves = (p.rows + R - 1) / R;
            return hipLaunchKernel(fn, dim3((waves + 3) / 4), dim3(256), args, 0, s);
        }
    }
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
