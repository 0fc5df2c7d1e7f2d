// bwd.hip -- backward of the selected-block attention (gfx950).
//
// Replaces MosaicAttnFunction.backward / mosaic_attn_bwd (ops.py:437-507, 541-554) and its
// kernels (ops.py:179-273 grad q, 276-297 block mask, 300-434 grad k / v) with the same
// arithmetic and rounding points:
//   q'    = bf16((q * scale) * log2 e)                      (ops.py:236-237, 412-414)
//   delta = bf16(sum_d bf16(o * do))                        (ops.py:458, eager bf16 ops)
//   dq    = bf16(((sum over selected keys of bf16(P ln2 (dP - delta)) k) * scale) * log2 e)
//           with P = exp2(q'.k - lse), dP = do.v            (ops.py:265-273)
//   dv    = sum over the queries that selected the key of bf16(P) do
//   dk    = sum of bf16(P (dP - delta) ln2) q'              (ops.py:425-431)
// Products run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  One difference in order:
// grad k/v accumulates S and dP onto -lse and -delta, so those subtractions happen inside the
// fp32 accumulation rather than after it.
//
// The reference's grad-k/v program scans a dense [B, Hk, nb, nb] boolean block mask for every
// key block.  Here each key-tile workgroup marks, in LDS, the query blocks whose selection row
// holds its block (one pass over the [nb, K] index rows of its kv head) and then walks the
// marked blocks in ascending order -- the reference's loop order, without the mask tensor.
//
// Tiles reach LDS by direct-to-LDS loads (no register staging, issued as inline assembly) in a
// layout that both 16-byte row reads and ds_read_b64_tr_b16 transposing reads take without
// bank conflicts, so no transposed copy of any operand is stored.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsa_common.h"
#include "mosaic_bsa.h"

namespace mosaic {

namespace {

constexpr float kLn2 = 0.69314718056f;   // ops.py:197
constexpr int kMaxBwdBlocks = 4096;      // query blocks a key tile can mark (LDS flags)

struct BwdParams {
    const bf16_t* q; int64_t q_sb, q_sn, q_sh;
    const bf16_t* k; int64_t k_sb, k_sn, k_sh;
    const bf16_t* v; int64_t v_sb, v_sn, v_sh;
    const bf16_t* go; int64_t go_sb, go_sn, go_sh;
    const bf16_t* o;        // forward output [B, N, Hq, 64] contiguous
    const float* lse;       // [B, N, Hq] base-2 log-sum-exp of the scaled logits
    float* nlse;            // [B, N, Hq] -lse (workspace), written by the grad-q kernel
    float* ndelta;          // [B, N, Hq] -delta (workspace), written by the grad-q kernel
    bf16_t* qs;             // q' = bf16((q scale) log2 e), [B, N, Hq, 64] contiguous (workspace):
                            // written by the grad-q kernel, read by the grad-k/v kernel
    const int64_t* idx;     // [B, nb, Hk, K]
    bf16_t* dq; bf16_t* dk; bf16_t* dv;   // contiguous [B, N, H, 64]
    int B, N, Hq, Hk, G, bs, K, nb;
    float scale;
};

typedef short v4i16 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ grad q
// One workgroup = (batch b, kv head c, 64-query tile, NW query heads of the GQA group); wave w
// owns query head j = c G + NW h + w and all 64 rows of the tile, as the forward kernel does:
// the selected blocks' 64-key K and V tiles go from global memory straight into LDS (two
// buffers, one barrier per tile) and are read by every wave of the group.  Per tile and 32-key
// half kt, computed transposed so a lane owns one query column (lse and delta are per-lane
// registers):
//   S^T  = K Q'^T          A = K rows (b128 reads),  B = q' fragments (registers)
//   dP^T = V dO^T          A = V rows,               B = do fragments (registers)
//   dS   = bf16(exp2(S - lse) ln2 (dP - delta)), packed in accumulator order as B operands
//   dQ^T += K^T dS^T       A = K^T (transposing ds_read_b64_tr_b16 reads of the K tile)
// Both tiles use the bwd_swz layout.
constexpr int kTileElems = 64 * 64;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Workgroup barrier for LDS data whose direct-to-LDS loads each wave has already waited for
// itself: __syncthreads() would also wait for every load still in flight (its release fence
// covers the loads' LDS writes), which takes the prefetch of the next step out of the overlap.
// The memory clobber keeps the compiler from moving LDS accesses across it; lgkmcnt(0) retires
// this wave's LDS reads of the slot that is refilled after the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS layout of the backward's 64-row tiles: 128-byte rows, chunk c of row r at position
// c ^ bwd_swz(r).  The tiles are read both along rows (ds_read_b128 of one chunk of 16
// consecutive rows) and transposed (ds_read_b64_tr_b16 of two chunks of 4 consecutive rows,
// two such groups per cycle); bwd_swz makes both conflict-free: over rows of one parity in 16
// consecutive rows it is a permutation of 0..7, and rows r and r + 2 of an aligned group of
// four differ in bit 2, so their four-chunk runs land on disjoint banks.
__device__ __forceinline__ int bwd_swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }

// Per-lane byte offsets of one 64-row tile's direct-to-LDS loads: NW waves, 8/NW runs of
// 8 rows each; chunk pos of row r holds global chunk pos ^ bwd_swz(r).
template <int NW>
__device__ __forceinline__ void tile_dma_init(uint32_t* dk, uint32_t* dv, int wave, int lane, int64_t ksn, int64_t vsn) {
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
        const int row = 8 * (wave * (8 / NW) + i) + (lane >> 3), pos = lane & 7;
        const int src = 8 * (pos ^ bwd_swz(row));
        dk[i] = 2u * (uint32_t)(row * ksn + src);
        dv[i] = 2u * (uint32_t)(row * vsn + src);
    }
}

// Direct-to-LDS loads issued as inline assembly, address = base (uniform) + voff (per lane),
// LDS destination M0 + 16 l (dwordx4) or M0 + 4 l (dword) for lane l.  The compiler's wait
// insertion does not see them: across the joins of a ring loop its tracking of which LDS
// object a direct-to-LDS load writes becomes conservative, and it waited for the loads just
// requested for a later step before the current step's LDS reads.  The caller waits for these
// loads (s_waitcnt vmcnt) and synchronises the workgroup itself.  M0 is declared clobbered;
// the compiler sets M0 again before each of its own uses, so nothing it holds is lost.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// One 64-row tile's direct-to-LDS loads (offsets from tile_dma_init), issued as dma16
template <int NW>
__device__ __forceinline__ void tile_dma(const uint32_t* dk, const uint32_t* dv, const bf16_t* kb, const bf16_t* vb,
                                             int64_t ksn, int64_t vsn, int key0, bf16_t* Kd, bf16_t* Vd, int wave) {
    const int k0 = __builtin_amdgcn_readfirstlane(key0);
    const bf16_t* kt = kb + (int64_t)k0 * ksn;
    const bf16_t* vt = vb + (int64_t)k0 * vsn;
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
        const int row0 = 8 * (wave * (8 / NW) + i);
        dma16(kt, dk[i], lds_addr(Kd + row0 * 64));
        dma16(vt, dv[i], lds_addr(Vd + row0 * 64));
    }
}

template <int NW>
__global__ __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(2, 2)))
void bwd_dq_kernel(BwdParams p, int head_groups, int total_wgs) {
    __shared__ __attribute__((aligned(1024))) bf16_t Ks0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Ks1[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Vs0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t Vs1[kTileElems];
    __shared__ int sel_key0[kMaxSelected];  // first key of each in-range selected block, top-k order
    __shared__ int sel_count;

    const int lane = threadIdx.x & 63, r = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qtiles = p.N / 64;
    const int L = xcd_remap(blockIdx.x, total_wgs);
    const int qtile = L % qtiles, rest = L / qtiles;
    const int hg = rest % (p.Hk * head_groups), b = rest / (p.Hk * head_groups);
    const int c = hg / head_groups;
    const int j = c * p.G + (hg % head_groups) * NW + wave;
    const int n0 = qtile * 64;
    const bf16_t* kb = p.k + (int64_t)b * p.k_sb + (int64_t)c * p.k_sh;
    const bf16_t* vb = p.v + (int64_t)b * p.v_sb + (int64_t)c * p.v_sh;

    // wave 0 compacts the in-range selected blocks (duplicates kept: each entry counts, as the
    // reference's loop over the entries does)
    if (wave == 0) {
        const int64_t* ip = p.idx + (((int64_t)b * p.nb + n0 / p.bs) * p.Hk + c) * p.K;
        int count = 0;
        for (int base = 0; base < p.K; base += 64) {
            const int i = base + lane;
            const int64_t blk = i < p.K ? ip[i] : -1;
            const bool ok = blk >= 0 && blk < p.nb;
            const uint64_t mask = __builtin_amdgcn_ballot_w64(ok);
            const int pos = count + (int)__builtin_popcountll(mask & ((1ull << lane) - 1ull));
            if (ok) sel_key0[pos] = (int)(blk * p.bs);
            count += (int)__builtin_popcountll(mask);
        }
        if (lane == 0) sel_count = count;
    }
    // this wave's rows: q' = bf16((q scale) log2 e) and do as MFMA B fragments, lse, and
    // delta = bf16(sum_d bf16(o do)) formed here from o rows loaded in the fragments' layout
    // (each lane sums its 32 dims in fp32, the two lane halves add once) and written for the
    // grad-k/v kernel
    bf16x8 qf[2][4], gf[2][4];
    float lse[2], dlt[2];
    {
        const bf16_t* qb = p.q + (int64_t)b * p.q_sb + (int64_t)j * p.q_sh;
        const bf16_t* gb = p.go + (int64_t)b * p.go_sb + (int64_t)j * p.go_sh;
        const bf16_t* ob = p.o + ((int64_t)b * p.N * p.Hq + j) * 64;
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const int n = n0 + 32 * qt + r;
            uint4 ov[4];
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
                qf[qt][ds] = as_bf16x8(ld16(qb + (int64_t)n * p.q_sn + 16 * ds + 8 * hh));
                gf[qt][ds] = as_bf16x8(ld16(gb + (int64_t)n * p.go_sn + 16 * ds + 8 * hh));
                ov[ds] = ld16(ob + (int64_t)n * p.Hq * 64 + 16 * ds + 8 * hh);
            }
            const int64_t row = ((int64_t)b * p.N + n) * p.Hq + j;
            lse[qt] = p.lse[row];
            float sum = 0.f;
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
                const uint4 gv = __builtin_bit_cast(uint4, gf[qt][ds]);
                const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, ow[4] = {ov[ds].x, ov[ds].y, ov[ds].z, ov[ds].w};
#pragma unroll
                for (int mm = 0; mm < 4; ++mm) {
                    sum += round_bf16(bf_lo(ow[mm]) * bf_lo(gw[mm]));
                    sum += round_bf16(bf_hi(ow[mm]) * bf_hi(gw[mm]));
                }
            }
            dlt[qt] = round_bf16(xor32_add(sum));
            if (hh == 0) {   // negated for the grad-k/v kernel's accumulator start values
                p.nlse[row] = -lse[qt];
                p.ndelta[row] = -dlt[qt];
            }
        }
        // q' for the grad-k/v kernel (the rows this lane holds: query 32 qt + r, dims 16 ds + 8 hh)
        bf16_t* qsb = p.qs + (((int64_t)b * p.N + n0) * p.Hq + j) * 64;
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
                const uint4 sc = make_uint4(o4[0], o4[1], o4[2], o4[3]);
                qf[qt][ds] = as_bf16x8(sc);
                *reinterpret_cast<uint4*>(qsb + (int64_t)(32 * qt + r) * p.Hq * 64 + 16 * ds + 8 * hh) = sc;
            }
    }
    __syncthreads();
    const int sub = p.bs / 64;
    const int total = sel_count * sub;
    int cur_k = 0, cur_s = 0;
    const int selv = lane < sel_count ? sel_key0[lane] : 0;
    auto next_key0 = [&]() -> int {   // tiles are requested in order
        const int base = sel_count <= 64 ? __builtin_amdgcn_readlane(selv, cur_k) : sel_key0[cur_k];
        const int key0 = base + cur_s * 64;
        if (++cur_s == sub) {
            cur_s = 0;
            ++cur_k;
        }
        return key0;
    };
    uint32_t dk[8 / NW], dv[8 / NW];
    tile_dma_init<NW>(dk, dv, wave, lane, p.k_sn, p.v_sn);
    if (total > 0) tile_dma<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, next_key0(), Ks0, Vs0, wave);

    // per-lane LDS element offsets: row reads of key row 32 kt + r, chunk 2 ds + hh; transposing
    // reads of dims 32 dt + (lane % 32) for keys 16 s2 + 4 hh + 0..3 (+ 8 for sec = 1)
    int rk[4], tk[2][2];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) rk[ds] = r * 64 + 8 * ((2 * ds + hh) ^ bwd_swz(r));
    {
        const int s = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int sec = 0; sec < 2; ++sec) {
                const int row = 4 * hh + (s >> 2) + 8 * sec;
                const int chunk = 4 * dt + 2 * half + ((s & 3) >> 1);
                tk[dt][sec] = row * 64 + 8 * (chunk ^ bwd_swz(row)) + 4 * (s & 1);
            }
    }
    f32x16 acc[2][2];  // dQ^T [dim block dt][query block qt]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[dt][qt][e] = 0.f;

    auto tile = [&](const bf16_t* Kc, const bf16_t* Vc) __attribute__((always_inline)) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x16 s[2], dp[2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int e = 0; e < 16; ++e) { s[qt][e] = 0.f; dp[qt][e] = 0.f; }
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
                const bf16x8 ka = as_bf16x8(*reinterpret_cast<const uint4*>(Kc + 32 * kt * 64 + rk[ds]));
                const bf16x8 va = as_bf16x8(*reinterpret_cast<const uint4*>(Vc + 32 * kt * 64 + rk[ds]));
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) {
                    s[qt] = mfma32(ka, qf[qt][ds], s[qt]);
                    dp[qt] = mfma32(va, gf[qt][ds], dp[qt]);
                }
            }
            // dS in accumulator order, packed as the B operand: keys 16 s2 + 4 hh + 0..3, + 8
            bf16x8 db[2][2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    uint32_t w4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int e0 = 8 * s2 + 2 * i;
                        const float p0 = __builtin_amdgcn_exp2f(s[qt][e0] - lse[qt]) * kLn2;
                        const float p1 = __builtin_amdgcn_exp2f(s[qt][e0 + 1] - lse[qt]) * kLn2;
                        w4[i] = pack_bf16x2(p0 * (dp[qt][e0] - dlt[qt]), p1 * (dp[qt][e0 + 1] - dlt[qt]));
                    }
                    db[qt][s2] = as_bf16x8(make_uint4(w4[0], w4[1], w4[2], w4[3]));
                }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const bf16_t* kp = Kc + (32 * kt + 16 * s2) * 64;
                    const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                                   (__attribute__((address_space(3))) v4i16*)(kp + tk[dt][0])));
                    const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                                   (__attribute__((address_space(3))) v4i16*)(kp + tk[dt][1])));
                    const bf16x8 kT = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt) acc[dt][qt] = mfma32(kT, db[qt][s2], acc[dt][qt]);
                }
        }
    };
    // tile t in buffer t & 1: wait for this wave's loads, the barrier publishes every wave's loads
    // and frees the other buffer, whose next tile is requested right away.  Two tiles per
    // round and one exit (an odd count skips the last tile's products): with an exit after
    // each tile the accumulators lived in rotating register sets (316 registers, one wave per
    // SIMD); now 240, two waves per SIMD.
    for (int t = 0; t < total; t += 2) {
        wait_vmem();
        __syncthreads();
        if (t + 1 < total) tile_dma<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, next_key0(), Ks1, Vs1, wave);
        tile(Ks0, Vs0);
        wait_vmem();
        __syncthreads();
        if (t + 2 < total) tile_dma<NW>(dk, dv, kb, vb, p.k_sn, p.v_sn, next_key0(), Ks0, Vs0, wave);
        if (t + 1 < total) tile(Ks1, Vs1);
    }
    // dq = bf16((dQ scale) log2 e), rows n0 + 32 qt + r, dims 32 dt + 8 g4 + 4 hh + 0..3
    bf16_t* out = p.dq + (((int64_t)b * p.N + n0) * p.Hq + j) * 64;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const f32x16& a = acc[dt][qt];
                uint2 w2;
                w2.x = pack_bf16x2((a[4 * g4 + 0] * p.scale) * kLog2e, (a[4 * g4 + 1] * p.scale) * kLog2e);
                w2.y = pack_bf16x2((a[4 * g4 + 2] * p.scale) * kLog2e, (a[4 * g4 + 3] * p.scale) * kLog2e);
                *reinterpret_cast<uint2*>(out + (int64_t)(32 * qt + r) * p.Hq * 64 + 32 * dt + 8 * g4 + 4 * hh) = w2;
            }
}

// ------------------------------------------------------------------ grad k, grad v
// grid (N / 64 key tiles, Hk, B).  Wave w = (key half kh = w / 2, query half qh = w % 2).  Per
// step -- one (marked query block tile, query head of the group) -- a wave forms S = q' k^T and
// dP = do v^T for its 32 queries x 32 keys; P and dS stay in registers, where the accumulator
// layout (lane: one key column, 16 query rows) is exactly the MFMA B operand of
// dV^T += do^T P and dK^T += q'^T dS with k running over those query rows; the A operands
// (do^T, q'^T) come from transposing LDS reads of the row-major tiles in the same row order.
// The wave's K and V rows stay in registers for all steps.  S and dP accumulate onto -lse and
// -delta of their rows (written by the grad-q kernel), so P = exp2(S) and dS = P dP ln2 take
// no subtraction (the subtraction happens inside the fp32 accumulation instead of after it).
// The step's q' rows (pre-scaled by the grad-q kernel), do rows, -lse and -delta go from global
// memory straight into LDS: a ring of three slots, loads requested two steps ahead, one barrier
// per step.  All tiles use the bwd_swz layout.  The two waves of a key half sum their partial
// dV^T / dK^T once, at the end.
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_dkv_kernel(BwdParams p) {
    __shared__ __attribute__((aligned(1024))) bf16_t kvs[2 * kTileElems];   // K tile, V tile
    bf16_t* Ks = kvs;
    bf16_t* Vs = kvs + kTileElems;
    // Three steps in a ring; a slot holds the step's q' tile, do tile, then -lse and -delta of
    // its 64 rows (fp32).  The loop below is unrolled over the slots (each an array of its own)
    // and its loads are issued as inline assembly, so no compiler-inserted wait holds a step's
    // LDS reads until the loads in flight into the other slots land.  The final reduction
    // reuses slots 0 and 1.
    constexpr int kSlotElems = 2 * kTileElems + 256;
    __shared__ __attribute__((aligned(1024))) bf16_t ring0[kSlotElems], ring1[kSlotElems], ring2[kSlotElems];
    __shared__ uint64_t mark[kMaxBwdBlocks / 64];   // bit t: query block t selected this block
    // key tiles in XCD-contiguous ranges: with selections that follow spatial proximity,
    // neighbouring key tiles are selected by the same query blocks and share their (q', do)
    // tiles in one L2
    const int ntiles = gridDim.x;
    const int L = xcd_remap(blockIdx.x + ntiles * (blockIdx.y + gridDim.y * blockIdx.z), ntiles * gridDim.y * gridDim.z);
    const int kt = L % ntiles, c = (L / ntiles) % (int)gridDim.y, b = L / (ntiles * (int)gridDim.y);
    const int key0 = kt * 64;
    const int64_t u = key0 / p.bs;
    const int lane = threadIdx.x & 63, r = lane & 31, hh = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // K and V of the key tile
    uint32_t dk[2], dv[2];
    tile_dma_init<4>(dk, dv, w, lane, p.k_sn, p.v_sn);
    {
        const bf16_t* kt = p.k + (int64_t)b * p.k_sb + (int64_t)c * p.k_sh + (int64_t)key0 * p.k_sn;
        const bf16_t* vt = p.v + (int64_t)b * p.v_sb + (int64_t)c * p.v_sh + (int64_t)key0 * p.v_sn;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row0 = 8 * (2 * w + i);
            dma16(kt, dk[i], lds_addr(Ks + row0 * 64));
            dma16(vt, dv[i], lds_addr(Vs + row0 * 64));
        }
    }
    // query blocks whose selection row (kv head c) holds block u, as a bitmap: lane l of a wave
    // scans row 64 i + l (eight entries per step, all loads of a step issued before any
    // compare) and the wave's ballot is word i
    for (int i = w; i < (p.nb + 63) / 64; i += 4) {
        const int t = 64 * i + lane;
        bool hit = false;
        if (t < p.nb) {
            const int64_t* row = p.idx + (((int64_t)b * p.nb + t) * p.Hk + c) * p.K;
            for (int i0 = 0; i0 < p.K; i0 += 8) {
                int64_t e[8];
#pragma unroll
                for (int k8 = 0; k8 < 8; ++k8) e[k8] = i0 + k8 < p.K ? row[i0 + k8] : -1;
#pragma unroll
                for (int k8 = 0; k8 < 8; ++k8) hit |= e[k8] == u;
            }
        }
        const uint64_t bits = __builtin_amdgcn_ballot_w64(hit);
        if (lane == 0) mark[i] = bits;
    }
    __syncthreads();
    const int kh = w >> 1, qh = w & 1;
    f32x16 dkT[2], dvT[2];  // [d block]: rows d = 32 db + row(e), column key 32 kh + lane % 32
#pragma unroll
    for (int e = 0; e < 16; ++e) { dkT[0][e] = 0.f; dkT[1][e] = 0.f; dvT[0][e] = 0.f; dvT[1][e] = 0.f; }
    // steps: (marked query block t, its 64-row tile tt, query head g of the group), ascending
    const int tiles = p.bs / 64;
    auto next_marked = [&](int t) {   // first marked block >= t, or nb (uniform LDS reads)
        const int words = (p.nb + 63) / 64;
        int i = t >> 6;
        if (i >= words) return p.nb;
        uint64_t m = mark[i] & (~0ull << (t & 63));
        while (m == 0) {
            if (++i >= words) return p.nb;
            m = mark[i];
        }
        return 64 * i + (int)__builtin_ctzll(m);
    };
    int t = next_marked(0), tt = 0, g = 0;
    auto advance = [&]() {
        if (++g == p.G) {
            g = 0;
            if (++tt == tiles) { tt = 0; t = next_marked(t + 1); }
        }
    };
    // per-lane byte offsets of the step's q' and do rows (8 rows per 1 KB run, two runs per wave)
    uint32_t dq_[2], dg_[2];
    tile_dma_init<4>(dq_, dg_, w, lane, (int64_t)p.Hq * 64, p.go_sn);
    // one step's loads: every wave issues exactly six direct-to-LDS instructions (two 1 KB runs
    // each of q' and do, and -lse / -delta of 16 rows), so a wait for all but the newest step's
    // loads is one fixed s_waitcnt.  Past the last step, and for the virtual steps before the
    // first, it loads query rows 0..63 into the free slot (never read), so that no branch
    // depends on the step count.
    auto issue_step = [&](bf16_t* slot, bool real) __attribute__((always_inline)) {
        bf16_t* Qd = slot;
        bf16_t* Gd = slot + kTileElems;
        float* ld = reinterpret_cast<float*>(slot + 2 * kTileElems);
        const int n0 = __builtin_amdgcn_readfirstlane(real && t < p.nb ? t * p.bs + 64 * tt : 0);
        const int j = c * p.G + g;
        const bf16_t* qt = p.qs + ((int64_t)b * p.N * p.Hq + j) * 64 + (int64_t)n0 * p.Hq * 64;
        const bf16_t* gt = p.go + (int64_t)b * p.go_sb + (int64_t)j * p.go_sh + (int64_t)n0 * p.go_sn;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row0 = 8 * (2 * w + i);
            dma16(qt, dq_[i], lds_addr(Qd + row0 * 64));
            dma16(gt, dg_[i], lds_addr(Gd + row0 * 64));
        }
        const int64_t row0 = ((int64_t)b * p.N + n0 + 16 * w) * p.Hq + j;
        if (lane < 16) {   // lane l -> 4 bytes at 4 l of this wave's 16 rows
            const uint32_t off = 4u * (uint32_t)(lane * p.Hq);
            dma4(p.nlse + row0, off, lds_addr(ld + 16 * w));
            dma4(p.ndelta + row0, off, lds_addr(ld + 64 + 16 * w));
        }
    };
    // per-lane LDS element offsets: row reads (row 32 h + r, chunk 2 kk + hh) and transposing
    // reads (dims 32 dt + lane % 32, rows 4 hh + 0..3 (+ 8) of a 16-row group)
    int rd[4], tr[2][2];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) rd[kk] = r * 64 + 8 * ((2 * kk + hh) ^ bwd_swz(r));
    {
        const int s4 = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int sec = 0; sec < 2; ++sec) {
                const int row = 4 * hh + (s4 >> 2) + 8 * sec;
                const int chunk = 4 * dt + 2 * half + ((s4 & 3) >> 1);
                tr[dt][sec] = row * 64 + 8 * (chunk ^ bwd_swz(row)) + 4 * (s4 & 1);
            }
    }
    auto tr_read = [&](const bf16_t* T, int q0, int dt) __attribute__((always_inline)) -> bf16x8 {
        const bf16_t* tp = T + q0 * 64;
        const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                       (__attribute__((address_space(3))) v4i16*)(tp + tr[dt][0])));
        const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                       (__attribute__((address_space(3))) v4i16*)(tp + tr[dt][1])));
        return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
    };
    bf16x8 kf[4], vf[4];   // this wave's K and V rows (key half kh), constant over the steps
    auto step = [&](const bf16_t* slot) __attribute__((always_inline)) {
        const bf16_t* Qc = slot;
        const bf16_t* Gc = slot + kTileElems;
        const float* lc = reinterpret_cast<const float*>(slot + 2 * kTileElems);
        const float* dc = lc + 64;
        // S and dP start from -lse and -delta of their rows (accumulator element 4 g4 + i is
        // row 32 qh + 8 g4 + 4 hh + i): one 16-byte read each, and the products add to them
        f32x16 s, dp;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const float4 l4 = *reinterpret_cast<const float4*>(lc + 32 * qh + 8 * g4 + 4 * hh);
            const float4 d4 = *reinterpret_cast<const float4*>(dc + 32 * qh + 8 * g4 + 4 * hh);
            s[4 * g4 + 0] = l4.x; s[4 * g4 + 1] = l4.y; s[4 * g4 + 2] = l4.z; s[4 * g4 + 3] = l4.w;
            dp[4 * g4 + 0] = d4.x; dp[4 * g4 + 1] = d4.y; dp[4 * g4 + 2] = d4.z; dp[4 * g4 + 3] = d4.w;
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const bf16x8 qa = as_bf16x8(*reinterpret_cast<const uint4*>(Qc + 32 * qh * 64 + rd[kk]));
            const bf16x8 ga = as_bf16x8(*reinterpret_cast<const uint4*>(Gc + 32 * qh * 64 + rd[kk]));
            s = mfma32(qa, kf[kk], s);     // S: queries x keys
            dp = mfma32(ga, vf[kk], dp);   // dP
        }
        bf16x8 pb[2], db[2];
#pragma unroll
        for (int e = 0; e < 16; ++e) {   // s = q'.k - lse, dp = do.v - delta
            const float pr = __builtin_amdgcn_exp2f(s[e]);
            const float ds = pr * dp[e] * kLn2;
            pb[e >> 3][e & 7] = (__bf16)pr;
            db[e >> 3][e & 7] = (__bf16)ds;
        }
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                const int q0 = 32 * qh + 16 * ch;
                dvT[dblk] = mfma32(tr_read(Gc, q0, dblk), pb[ch], dvT[dblk]);
                dkT[dblk] = mfma32(tr_read(Qc, q0, dblk), db[ch], dkT[dblk]);
            }
        }
    };
    // a key tile that no query block selected has no steps (its gradients are zero)
    int marked = 0;
    for (int i = 0; i < (p.nb + 63) / 64; ++i) marked += __builtin_popcountll(mark[i]);
    const int steps = marked * tiles * p.G;
    // The loop below runs whole rounds of three steps with one exit.  pad = 0..2 virtual steps
    // come first (their slots get the rows past the end like the steps after the last one, and
    // their products are skipped), so real step k uses slot (k + pad) % 3.
    const int pad = (3 - steps % 3) % 3;
    issue_step(ring0, pad == 0);
    if (pad == 0) advance();
    issue_step(ring1, pad <= 1);
    if (pad <= 1) advance();
    // K and V were requested before the two steps' twelve loads; every wave's K / V rows are in
    // LDS after the barrier, and this wave's half goes to registers
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    lds_barrier();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        kf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + 32 * kh * 64 + rd[kk]));
        vf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(Vs + 32 * kh * 64 + rd[kk]));
    }
    // Padded step i uses ring slot i % 3.  Its loads were requested two steps earlier; wait for
    // them, leaving the next step's six in flight, and the barrier publishes every wave's loads
    // and frees slot (i + 2) % 3, whose step is requested right away.
    auto ring_step = [&](const bf16_t* cur, bf16_t* next, bool real) __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        lds_barrier();
        issue_step(next, true);
        advance();
        if (real) step(cur);
    };
    for (int i = 0; i < steps + pad; i += 3) {
        ring_step(ring0, ring2, i >= pad);
        ring_step(ring1, ring0, i + 1 >= pad);
        ring_step(ring2, ring1, true);
    }
    // sum the two query halves' partials: qh = 1 parks its accumulators in LDS (the staging
    // buffers; with no steps the K / V loads may still be in flight, so wait for them first)
    wait_vmem();
    __syncthreads();
    // value v of lane r at v * 32 + r: consecutive lanes on consecutive banks
    float* red = reinterpret_cast<float*>((kh == 0 ? ring0 : ring1) + hh * kTileElems) + r;
    if (qh == 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            red[32 * e] = dkT[0][e];
            red[32 * (16 + e)] = dkT[1][e];
            red[32 * (32 + e)] = dvT[0][e];
            red[32 * (48 + e)] = dvT[1][e];
        }
    }
    __syncthreads();
    if (qh == 0) {
        const int64_t base = (((int64_t)b * p.N + key0 + 32 * kh + r) * p.Hk + c) * 64;
        // registers 4 g .. 4 g + 3 hold dims 32 dblk + 8 g + 4 hh + 0..3: one 8-byte store each
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float kx[4], vx[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int e = 4 * g + i;
                    kx[i] = dkT[dblk][e] + red[32 * (16 * dblk + e)];
                    vx[i] = dvT[dblk][e] + red[32 * (32 + 16 * dblk + e)];
                }
                const int d = 32 * dblk + 8 * g + 4 * hh;
                *reinterpret_cast<uint2*>(p.dk + base + d) = make_uint2(pack_bf16x2(kx[0], kx[1]), pack_bf16x2(kx[2], kx[3]));
                *reinterpret_cast<uint2*>(p.dv + base + d) = make_uint2(pack_bf16x2(vx[0], vx[1]), pack_bf16x2(vx[2], vx[3]));
            }
        }
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }
int check_rows(const mosaic_bnhd& t) {
    if (t.ptr == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(t.ptr) || t.stride_b % 8 || t.stride_n % 8 || t.stride_h % 8) return MOSAIC_ERR_ALIGNMENT;
    return MOSAIC_OK;
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" {

// -lse and -delta (fp32 per row), then q' (bf16 rows of 64), each 256-byte aligned
static size_t bwd_row_bytes(int32_t batch, int32_t seq_len, int32_t num_q_heads) {
    return ((size_t)batch * seq_len * num_q_heads * sizeof(float) + 255) / 256 * 256;
}

size_t mosaic_sparse_attn_bwd_workspace_size(int32_t batch, int32_t seq_len, int32_t num_q_heads) {
    if (batch <= 0 || seq_len <= 0 || num_q_heads <= 0) return 0;
    const size_t qs = ((size_t)batch * seq_len * num_q_heads * kHeadDim * sizeof(bf16_t) + 255) / 256 * 256;
    return 2 * bwd_row_bytes(batch, seq_len, num_q_heads) + qs;
}

int mosaic_sparse_attn_bwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, const void* out, const float* lse,
                           mosaic_bnhd grad_out, const int64_t* block_indices, int32_t batch, int32_t seq_len,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                           int32_t block_count, float softmax_scale, void* grad_q, void* grad_k, void* grad_v,
                           void* workspace, size_t workspace_bytes, void* stream) {
    if (batch <= 0 || seq_len <= 0) return MOSAIC_ERR_SHAPE;
    if (head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return MOSAIC_ERR_HEADS;
    if (block_size <= 0 || block_size % 64 || seq_len % block_size) return MOSAIC_ERR_BLOCK_SIZE;
    if (block_count <= 0 || block_count > kMaxSelected) return MOSAIC_ERR_BLOCK_COUNT;
    if (seq_len / block_size > kMaxBwdBlocks) return MOSAIC_ERR_UNSUPPORTED;
    for (const mosaic_bnhd* t : {&q, &k, &v, &grad_out})
        if (int e = check_rows(*t)) return e;
    if (!out || !lse || !block_indices || !grad_q || !grad_k || !grad_v) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(out) || !aligned16(grad_q) || !aligned16(grad_k) || !aligned16(grad_v)) return MOSAIC_ERR_ALIGNMENT;
    const size_t need = mosaic_sparse_attn_bwd_workspace_size(batch, seq_len, num_q_heads);
    if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)) return MOSAIC_ERR_WORKSPACE;
    if ((int64_t)seq_len / 64 > 0x7fffffff || batch > 65535 || num_q_heads > 65535) return MOSAIC_ERR_SHAPE;

    BwdParams p{};
    p.q = static_cast<const bf16_t*>(q.ptr); p.q_sb = q.stride_b; p.q_sn = q.stride_n; p.q_sh = q.stride_h;
    p.k = static_cast<const bf16_t*>(k.ptr); p.k_sb = k.stride_b; p.k_sn = k.stride_n; p.k_sh = k.stride_h;
    p.v = static_cast<const bf16_t*>(v.ptr); p.v_sb = v.stride_b; p.v_sn = v.stride_n; p.v_sh = v.stride_h;
    p.go = static_cast<const bf16_t*>(grad_out.ptr);
    p.go_sb = grad_out.stride_b; p.go_sn = grad_out.stride_n; p.go_sh = grad_out.stride_h;
    p.o = static_cast<const bf16_t*>(out);
    p.lse = lse;
    const size_t row_bytes = bwd_row_bytes(batch, seq_len, num_q_heads);
    p.nlse = static_cast<float*>(workspace);
    p.ndelta = reinterpret_cast<float*>(static_cast<char*>(workspace) + row_bytes);
    p.qs = reinterpret_cast<bf16_t*>(static_cast<char*>(workspace) + 2 * row_bytes);
    p.idx = block_indices;
    p.dq = static_cast<bf16_t*>(grad_q); p.dk = static_cast<bf16_t*>(grad_k); p.dv = static_cast<bf16_t*>(grad_v);
    p.B = batch; p.N = seq_len; p.Hq = num_q_heads; p.Hk = num_kv_heads; p.G = num_q_heads / num_kv_heads;
    p.bs = block_size; p.K = block_count; p.nb = seq_len / block_size;
    p.scale = softmax_scale > 0.f ? softmax_scale : 0.125f;   // head_dim^-0.5 for head_dim 64
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* args[] = {&p};
    // grad q: one workgroup per (batch, kv head, query tile, group of NW query heads); it also
    // writes delta and q' for grad k/v
    if ((int64_t)batch * seq_len * num_q_heads >= ((int64_t)1 << 40)) return MOSAIC_ERR_SHAPE;
    const int G = num_q_heads / num_kv_heads;
    const int nw = (G == 1 || G == 2 || G == 4) ? G : (G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1));
    int head_groups = G / nw;
    const int64_t dq_wgs = (int64_t)batch * num_kv_heads * head_groups * (seq_len / 64);
    if (dq_wgs > 0x7fffffff) return MOSAIC_ERR_SHAPE;
    int total_wgs = (int)dq_wgs;
    void* dq_args[] = {&p, &head_groups, &total_wgs};
    const void* dq_fn = nw == 4 ? (const void*)&bwd_dq_kernel<4>
                      : nw == 2 ? (const void*)&bwd_dq_kernel<2> : (const void*)&bwd_dq_kernel<1>;
    if (hipLaunchKernel(dq_fn, dim3(total_wgs), dim3(64 * nw), dq_args, 0, s) != hipSuccess) return MOSAIC_ERR_LAUNCH;
    if (hipLaunchKernel((const void*)&bwd_dkv_kernel, dim3(seq_len / 64, num_kv_heads, batch), dim3(256), args, 0,
                        s) != hipSuccess)
        return MOSAIC_ERR_LAUNCH;
    return MOSAIC_OK;
}

}  // extern "C"
