// proj.hip -- the attention block's input side in one kernel (gfx950): the q / k / v / gate
// projection GEMM with RoPE, block pooling and the gate softmax in its epilogue.
//
// Replaces, for MosaicAttention.forward (primitives.py:182-195, 171-180, 125-135, 65-66, 76):
//   y      = x W^T over the stacked rows of to_q | to_k | to_v | to_strategy_combine_mlp
//            (bf16 operands, fp32 accumulation, rounded to bf16 like the reference's bf16 Linear)
//   q, k   = RoPE(y) per head: pair (2m, 2m+1) -> (x0 c - x1 s, x1 c + x0 s) in fp32, products
//            and sum rounded separately, then bf16 (primitives.py:125-135)
//   w      = bf16(softmax over the three branch logits of each head, fp32) (primitives.py:173-180)
//   pooled = bf16(fp32 sum of the block's rounded (rotated) rows / block size), for q, k, v
//            (the compressed branch's inputs), plus for k the largest squared 8-dim chunk norm
//            over the block's rows (the attention kernel's logit bound)
// so q, k and v are written once and never read back by a pooling pass.
//
// Tiling: one workgroup = 256 tokens of one member x 128 output columns (two 64-column
// groups: a q, k or v head, the gate logits, or zero padding), K = model dim in steps of 32.
// Four waves, one per SIMD, and two workgroups per CU (72 KB of LDS each), so one
// workgroup's epilogue overlaps the other's products; wave (wm, wn) computes rows
// 128 wm .. + 127 of group wn with v_mfma_f32_32x32x16_bf16 (eight 32 x 32 accumulators), so
// each wave's epilogue handles one head (or the gates) and whole pooled blocks.  x rows and W
// rows go from global memory straight into LDS (direct-to-LDS loads, a three-slot ring),
// XOR-swizzled so the 16-byte operand reads are conflict-free.  The rounded results are
// staged in LDS (reusing the stages) and leave as 16-byte row chunks; RoPE and pooling run on
// those chunks (a RoPE pair in one lane, the pooled sums of a chunk added across the lanes
// that hold its rows).  Workgroups that share an x tile are dispatched to the same XCD.
#include "bsa_common.h"

namespace mosaic {
namespace {

constexpr int kProjM = 256;                 // tokens per workgroup
constexpr int kProjN = 128;                 // output columns per workgroup
constexpr int kProjK = 32;                  // reduction step
constexpr int kSlotA = kProjM * kProjK;     // bf16 elements of an x ring slot (16 KB)
constexpr int kSlotB = kProjN * kProjK;     // bf16 elements of a weight ring slot (8 KB)
constexpr int kRing = 3;                    // ring slots (k steps in flight)

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Workgroup barrier for LDS data whose direct-to-LDS loads each wave has already waited for
// itself: __syncthreads() would also wait for every load still in flight (its release fence
// covers the loads' LDS writes), which takes the prefetched steps out of the overlap.  The
// memory clobber keeps the compiler from moving LDS accesses across it; lgkmcnt(0) retires this
// wave's reads of the slot that is refilled after the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS byte address of a pointer into a __shared__ array
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}
// 16-byte LDS read issued as inline assembly: the compiler does not see an LDS access, so it
// inserts no wait for direct-to-LDS loads in flight (its alias tracking of those loads is
// conservative at the ring's loop head and would wait for the prefetched steps too).  The
// caller waits with lgkm_wait before using the result.
template <int OFF>
__device__ __forceinline__ bf16x8 lds_read16(uint32_t addr) {
    bf16x8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
// s_waitcnt lgkmcnt(N) that the six operand registers depend on, so no use of them is
// scheduled before the wait
template <int N>
__device__ __forceinline__ void lgkm_wait(bf16x8& a0, bf16x8& a1, bf16x8& a2, bf16x8& a3, bf16x8& b0, bf16x8& b1) {
    asm volatile("s_waitcnt lgkmcnt(%6)" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1) : "i"(N));
}

// DPP moves in which every lane reads a valid lane (no old value to keep)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}
// x of the other lane of the pair (l, l ^ 1): quad_perm [1, 0, 3, 2]
__device__ __forceinline__ float swap_pair(float x) { return dpp<0xb1>(x); }
// x[l] + x[l ^ 16] and max(x[l], x[l ^ 16]) in every lane: one v_permlane16_swap (rows 1 and
// 3 of one copy trade places with rows 0 and 2 of the other)
__device__ __forceinline__ float swap16_add(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

enum GroupRole { kRoleQ = 0, kRoleK = 1, kRoleV = 2, kRoleGate = 3, kRolePad = 4 };

__device__ __forceinline__ int group_role(const ProjParams& p, int g, int& head) {
    if (g < p.Hq) { head = g; return kRoleQ; }
    if (g < p.Hq + p.Hk) { head = g - p.Hq; return kRoleK; }
    if (g < p.Hq + 2 * p.Hk) { head = g - p.Hq - p.Hk; return kRoleV; }
    head = 0;
    return (p.gates && g == p.Hq + 2 * p.Hk) ? kRoleGate : kRolePad;
}

// staging layout of a wave's 128 x 64 result (128 rows x 128 bytes): 16-byte chunk c of row r
// at position c ^ (4 ((r / 4) % 2)).  A pair-write instruction covers 64 bytes of each of the
// rows r, r + 1, r + 4, r + 5; rows of one parity share a 128-byte half of the 64 banks, and
// r and r + 4 take opposite 64-byte quarters of it
__device__ __forceinline__ int stage_off(int row, int col) {
    return row * 64 + 8 * ((col >> 3) ^ (4 * ((row >> 2) & 1))) + (col & 7);
}

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void proj_kernel(ProjParams p) {
    // a ring of three k-steps (x rows in As, weight rows in Bs); after the loop each wave
    // stages its 128 x 64 result (16 KB) in As[w] (waves 0-2) or Bs[0..1] (wave 3).  72 KB per
    // workgroup: two workgroups share a CU, so one's epilogue overlaps the other's products.
    __shared__ __attribute__((aligned(1024))) bf16_t As[kRing][kSlotA];
    __shared__ __attribute__((aligned(1024))) bf16_t Bs[kRing][kSlotB];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = w >> 1, wn = w & 1;
    // logical tile: n fastest, then member, then token range, so the n tiles of one x tile
    // are neighbours and xcd_remap keeps them on one XCD (its L2 serves the x tile's re-reads)
    const int id = xcd_remap(blockIdx.x, gridDim.x);
    const int n_tiles = p.n_tiles * (256 / kProjN);
    const int ntile = id % n_tiles;
    const int mtile = id / n_tiles;
    const int b = mtile % p.B, s0 = (mtile / p.B) * kProjM;
    const int n0 = ntile * kProjN;

    // direct-to-LDS loads of a slot (rows of 32 k = 64 bytes), sixteen rows (1 KB) per
    // instruction: wave w fills x rows 64 w .. + 63 and weight rows 32 w .. + 31; lane l lands
    // at row 16 i + l / 4, position l % 4, and fetches the row's chunk (l % 4) ^ ((row / 4) % 4).
    // A 16-byte LDS read serves 16 lanes per cycle from 64 banks (256 bytes): the 16
    // consecutive rows of one read then cover the four 64-byte quarters of the banks (row % 4)
    // with four distinct chunk positions each ((row / 4) % 4), so no two lanes share a bank.
    const int r16 = lane >> 2, gch = (lane & 3) ^ ((lane >> 4) & 3);
    // uniform bases (scalar registers) plus one 32-bit byte offset per lane and operand
    const char* xbase = reinterpret_cast<const char*>(p.x + (int64_t)(s0 + 64 * w) * p.x_sn + (int64_t)b * p.x_sb);
    const char* wbase = reinterpret_cast<const char*>(p.w + (int64_t)(n0 + 32 * w) * p.D);
    const uint32_t xoff = 2u * (uint32_t)(r16 * p.x_sn + 8 * gch);
    const uint32_t woff = 2u * (uint32_t)(r16 * p.D + 8 * gch);
    const int64_t xstep = 32 * p.x_sn, wstep = 32 * (int64_t)p.D;   // bytes per 16 rows
    auto issue = [&](int k0, int slot) __attribute__((always_inline)) {
        const char* xk = xbase + 2 * k0;
        const char* wk = wbase + 2 * k0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(xk + i * xstep + xoff, (lds_void*)(As[slot] + (64 * w + 16 * i) * kProjK), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(wk + i * wstep + woff, (lds_void*)(Bs[slot] + (32 * w + 16 * i) * kProjK), 16, 0, 0);
    };
    // operand reads: row 32 t + lane % 32 of a 32-row block, chunk 2 kk + lane / 32 (kk = 0, 1)
    int rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) rd[kk] = (lane & 31) * kProjK + 8 * ((2 * kk + (lane >> 5)) ^ ((lane >> 2) & 3));

    f32x16 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mt][nt][e] = 0.f;
    // both k sub-steps' operands are requested at once; the first six reads are waited for
    // (lgkmcnt 6: LDS reads complete in order) while the second six are in flight
    auto compute = [&](int slot) __attribute__((always_inline)) {
        bf16x8 a[2][4], bb[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint32_t aa = lds_addr(As[slot] + 128 * wm * kProjK + rd[kk]);
            const uint32_t ba = lds_addr(Bs[slot] + 64 * wn * kProjK + rd[kk]);
            constexpr int T = 32 * kProjK * 2;   // bytes between 32-row blocks
            a[kk][0] = lds_read16<0>(aa);
            a[kk][1] = lds_read16<T>(aa);
            a[kk][2] = lds_read16<2 * T>(aa);
            a[kk][3] = lds_read16<3 * T>(aa);
            bb[kk][0] = lds_read16<0>(ba);
            bb[kk][1] = lds_read16<T>(ba);
        }
        lgkm_wait<6>(a[0][0], a[0][1], a[0][2], a[0][3], bb[0][0], bb[0][1]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma32(a[0][mt], bb[0][nt], acc[mt][nt]);
        lgkm_wait<0>(a[1][0], a[1][1], a[1][2], a[1][3], bb[1][0], bb[1][1]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma32(a[1][mt], bb[1][nt], acc[mt][nt]);
    };
    // Step i uses slot i % 3; its loads (six per wave) were requested two steps earlier.  Wait
    // for them, leaving the next step's six in flight, then the barrier publishes every wave's
    // loads and frees slot (i + 2) % 3 (computed at step i - 1 by every wave), whose step is
    // requested before step i is computed.
    const int steps = p.D / kProjK;
    issue(0, 0);
    issue(kProjK, 1);
    auto ring_step = [&](int i, int slot, int next_slot) __attribute__((always_inline)) {
        if (i + 1 < steps) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else wait_vmem();
        lds_barrier();
        if (i + 2 < steps) issue(kProjK * (i + 2), next_slot);
        compute(slot);
    };
    for (int i = 0; i < steps; i += 3) {
        ring_step(i, 0, 2);
        if (i + 1 < steps) ring_step(i + 1, 1, 0);
        if (i + 2 < steps) ring_step(i + 2, 2, 1);
    }
    __syncthreads();  // every wave is done with the ring: its arrays become the output staging

    // ------------------------------------------------------------------ epilogue
    // Phase 1: each wave rounds its accumulators to bf16 and stages its 128 x 64 result.  The
    // accumulator layout gives lane l column 32 nt + l % 32 of the wave's group and rows
    // 8 (e / 4) + 4 (l / 32) + e % 4 of each 32-row tile mt of its 128 rows.
    const int hh = lane >> 5, odd = lane & 1;
    int head;
    const int role = group_role(p, n0 / 64 + wn, head);
    // this wave's staging array (128 rows x 64 columns, 16 KB)
    bf16_t* stg = w < 3 ? As[w] : Bs[0];
    if (role != kRolePad) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {                   // tile i: 32-column half j, 32-row tile mt
            const int j = i >> 2, mt = i & 3;
            const int col = 32 * j + (lane & 31);       // column within the group (head dim)
            float x[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) x[e] = round_bf16(acc[mt][j][e]);
            // stage rows r, r + 1 as bf16 pairs of columns (c, c + 1): even lanes write row r,
            // odd lanes row r + 1, each after one swap with the pair's other lane
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const float other = swap_pair(odd ? x[e] : x[e + 1]);
                const uint32_t word = odd ? pack_bf16x2(other, x[e + 1]) : pack_bf16x2(x[e], other);
                const int row = 32 * mt + 4 * hh + 8 * (e >> 2) + (e & 3) + odd;   // row of the wave's 128
                *reinterpret_cast<uint32_t*>(stg + stage_off(row, col & ~1)) = word;
            }
        }
    }

    // Phase 2, from each wave's own staging (no workgroup barrier: a wave's LDS writes and
    // reads are ordered).  q / k / v: lane l takes the 8 columns 8 (l % 8) .. + 7 of rows
    // 8 it + l / 8 (it = 0 .. 15), so a RoPE pair lies in one lane and the table values of its
    // four frequencies are one 16-byte load each of cos and sin; each rotated chunk leaves as
    // a 16-byte row chunk to [B, S, H, 64], and the lane sums its rows of each pooled block,
    // which three exchanges (lanes l ^ 8, l ^ 16, l ^ 32) then add up.  The gates: the softmax
    // of each head's three logits to [B, S, Hq, 3].
    if (role == kRoleQ || role == kRoleK || role == kRoleV) {
        bf16_t* dst = role == kRoleQ ? p.q : (role == kRoleK ? p.k : p.v);
        const int H = role == kRoleQ ? p.Hq : p.Hk;
        bf16_t* rowp = dst + (((int64_t)b * p.S + s0 + 128 * wm) * H + head) * 64;
        const bool rope = p.rope_cos != nullptr && role != kRoleV;
        const bool pool = p.bs > 0;
        const bool bound = role == kRoleK && p.kbnd != nullptr;
        const int ch = lane & 7, r8 = lane >> 3;
        const int bpw = p.bs == 64 ? 2 : 1;             // pooled blocks per 128 rows (bs 64 or 128)
        float ps[2][8], sqm[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            sqm[k2] = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ps[k2][e] = 0.f;
        }
        const float* ctab = rope ? p.rope_cos + (int64_t)(s0 + 128 * wm) * 32 + 4 * ch : nullptr;
        const float* stab = rope ? p.rope_sin + (int64_t)(s0 + 128 * wm) * 32 + 4 * ch : nullptr;
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int row = 8 * it + r8;
            uint4 u = *reinterpret_cast<const uint4*>(stg + stage_off(row, 8 * ch));
            if (rope) {
                // (x0, x1) -> (x0 c - x1 s, x1 c + x0 s), products and sum rounded separately
                const float4 c = *reinterpret_cast<const float4*>(ctab + row * 32);
                const float4 sn = *reinterpret_cast<const float4*>(stab + row * 32);
                u.x = rope_pair(u.x, c.x, sn.x);
                u.y = rope_pair(u.y, c.y, sn.y);
                u.z = rope_pair(u.z, c.z, sn.z);
                u.w = rope_pair(u.w, c.w, sn.w);
            }
            *reinterpret_cast<uint4*>(rowp + (int64_t)row * H * 64 + 8 * ch) = u;
            if (pool) {
                const int k2 = bpw == 2 ? it >> 3 : 0;   // rows 0-63 and 64-127 at bs 64
                const float xs[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y),
                                     bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
                float sq = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    ps[k2][e] += xs[e];
                    sq = fmaf(xs[e], xs[e], sq);
                }
                sqm[k2] = fmaxf(sqm[k2], sq);
            }
        }
        if (pool) {
            // pooled outputs: every lane holds its chunk's block sums after the exchanges; lanes
            // 0-7 (l / 8 = 0) write them
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                if (k2 >= bpw) break;
                const int t = (s0 + 128 * wm) / p.bs + k2;    // block index
                float mean[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float v = ps[k2][e];
                    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));  // l ^ 8
                    v = xor32_add(swap16_add(v));
                    mean[e] = v / (float)p.bs;
                }
                float mx = sqm[k2];
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x128, 0xf, 0xf, false)));
                mx = xor32_max(swap16_max(mx));
                if (r8 == 0) {
                    uint4 m4;
                    m4.x = pack_bf16x2(mean[0], mean[1]); m4.y = pack_bf16x2(mean[2], mean[3]);
                    m4.z = pack_bf16x2(mean[4], mean[5]); m4.w = pack_bf16x2(mean[6], mean[7]);
                    if (role == kRoleQ) {
                        *reinterpret_cast<uint4*>(p.qc + (((int64_t)b * p.nb + t) * p.Hq + head) * 64 + 8 * ch) = m4;
                    } else if (role == kRoleK) {
                        *reinterpret_cast<uint4*>(p.kfrag + kfrag_index(b, head, p.Hk, p.nb_pad >> 5, t >> 5, ch >> 1,
                                                                         32 * (ch & 1) + (t & 31))) = m4;
                        if (bound) p.kbnd[(((int64_t)b * p.nb + t) * p.Hk + head) * 8 + ch] = mx;
                    } else if (p.vfrag != nullptr) {
                        const int wt = t & 31, s2 = wt >> 4, rem = wt & 15;
                        const int slot = 4 * (rem >> 3) + (rem & 3), h2 = (rem & 7) >> 2;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int col = 8 * ch + e;
                            p.vfrag[vfrag_index(b, head, p.Hk, p.nb_pad >> 5, t >> 5, col >> 5, s2, 32 * h2 + (col & 31)) +
                                    slot] = (bf16_t)(pack_bf16x2(mean[e], 0.f) & 0xffffu);
                        }
                    }
                }
            }
            // operand-ordered k / v of the padding blocks nb .. nb_pad - 1 are zero: written by
            // the workgroups of each member's last token range (wave wm = 0 of the group)
            if ((role == kRoleK || (role == kRoleV && p.vfrag != nullptr)) && s0 + kProjM == p.S && wm == 0) {
                const int UT = p.nb_pad >> 5;
                for (int i = lane; i < (p.nb_pad - p.nb) * 64; i += 64) {
                    const int t = p.nb + (i >> 6), col = i & 63;
                    if (role == kRoleK) {
                        const int c8 = col >> 3;
                        p.kfrag[kfrag_index(b, head, p.Hk, UT, t >> 5, c8 >> 1, 32 * (c8 & 1) + (t & 31)) + (col & 7)] = 0;
                    } else {
                        const int wt = t & 31, s2 = wt >> 4, rem = wt & 15;
                        const int slot = 4 * (rem >> 3) + (rem & 3), h2 = (rem & 7) >> 2;
                        p.vfrag[vfrag_index(b, head, p.Hk, UT, t >> 5, col >> 5, s2, 32 * h2 + (col & 31)) + slot] = 0;
                    }
                }
            }
        }
    } else if (role == kRoleGate) {
        for (int idx = lane; idx < 128 * p.Hq; idx += 64) {
            const int row = idx / p.Hq, h = idx - row * p.Hq;
            float l3[3];
#pragma unroll
            for (int sb = 0; sb < 3; ++sb) l3[sb] = bf2f(reinterpret_cast<const uint16_t*>(stg)[stage_off(row, 3 * h + sb)]);
            const float mx = fmaxf(fmaxf(l3[0], l3[1]), l3[2]);
            float ex[3];
#pragma unroll
            for (int sb = 0; sb < 3; ++sb) ex[sb] = expf(l3[sb] - mx);
            const float den = (ex[0] + ex[1]) + ex[2];
            bf16_t* o = p.wts + (((int64_t)b * p.S + s0 + 128 * wm + row) * p.Hq + h) * 3;
#pragma unroll
            for (int sb = 0; sb < 3; ++sb) o[sb] = (bf16_t)(pack_bf16x2(ex[sb] / den, 0.f) & 0xffffu);
        }
    }
}

}  // namespace

hipError_t launch_proj(const ProjParams& p, hipStream_t s) {
    ProjParams q = p;
    void* args[] = {&q};
    const int grid = (p.S / kProjM) * p.B * p.n_tiles * (256 / kProjN);
    return hipLaunchKernel((const void*)proj_kernel, dim3(grid), dim3(256), args, 0, s);
}

}  // namespace mosaic
