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
// Products run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation.
//
// The reference's grad-k/v program scans a dense [B, Hk, nb, nb] boolean block mask for every
// key block.  Here each key-tile workgroup marks, in LDS, the query blocks whose selection row
// holds its block (one pass over the [nb, K] index rows of its kv head) and then walks the
// marked blocks in ascending order -- the reference's loop order, without the mask tensor.
//
// Workgroups are 4 waves.  Each phase of a 64 x 64 tile step gives every wave one 32 x 32
// quadrant; operands come from LDS rows (16-byte reads), with transposed copies of the
// operands whose MFMA B side runs along the token dimension.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsa_common.h"
#include "mosaic_bsa.h"

namespace mosaic {

namespace {

constexpr float kLn2 = 0.69314718056f;   // ops.py:197
constexpr int kLd = 72;                  // LDS row stride in bf16 (144 bytes: 16-byte aligned rows)
constexpr int kMaxBwdBlocks = 4096;      // query blocks a key tile can mark (LDS flags)

struct BwdParams {
    const bf16_t* q; int64_t q_sb, q_sn, q_sh;
    const bf16_t* k; int64_t k_sb, k_sn, k_sh;
    const bf16_t* v; int64_t v_sb, v_sn, v_sh;
    const bf16_t* go; int64_t go_sb, go_sn, go_sh;
    const bf16_t* o;        // forward output [B, N, Hq, 64] contiguous
    const float* lse;       // [B, N, Hq] base-2 log-sum-exp of the scaled logits
    float* delta;           // [B, N, Hq] (workspace)
    const int64_t* idx;     // [B, nb, Hk, K]
    bf16_t* dq; bf16_t* dk; bf16_t* dv;   // contiguous [B, N, H, 64]
    int B, N, Hq, Hk, G, bs, K, nb;
    float scale;
};

__device__ __forceinline__ void unpack8(const uint4& u, float f[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { f[2 * i] = bf_lo(w[i]); f[2 * i + 1] = bf_hi(w[i]); }
}
__device__ __forceinline__ uint4 pack8(const float f[8]) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ bf16x8 lds8(const bf16_t* p) { return as_bf16x8(*reinterpret_cast<const uint4*>(p)); }

// A 64-row x 64-dim tile of a [B, N, H, 64] tensor moves global -> registers -> LDS in two
// steps, so the loads of the next tile are in flight while the current one is computed.
// 256 threads, two 16-byte chunks each: chunk c = thread + 256 i is row c / 8, dims 8 (c % 8).
__device__ __forceinline__ void load_rows(const bf16_t* base, int64_t sn, uint4 reg[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i;
        reg[i] = ld16(base + (int64_t)(c >> 3) * sn + (c & 7) * 8);
    }
}

// Registers -> LDS rows (row-major, optionally also transposed), scaled to q' when QSCALE.
template <bool QSCALE, bool TRANSPOSE>
__device__ __forceinline__ void store_rows(const uint4 reg[2], bf16_t* rows, bf16_t* cols, float scale) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i;
        const int r = c >> 3, c8 = (c & 7) * 8;
        uint4 u = reg[i];
        if (QSCALE || TRANSPOSE) {
            float f[8];
            unpack8(u, f);
            if (QSCALE) {
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = (f[e] * scale) * kLog2e;
                u = pack8(f);
                unpack8(u, f);
            }
            if (TRANSPOSE) {
#pragma unroll
                for (int e = 0; e < 8; ++e) cols[(c8 + e) * kLd + r] = (bf16_t)(pack_bf16x2(f[e], 0.f) & 0xffffu);
            }
        }
        *reinterpret_cast<uint4*>(rows + r * kLd + c8) = u;
    }
}

template <bool QSCALE, bool TRANSPOSE>
__device__ __forceinline__ void stage_rows(const bf16_t* base, int64_t sn, bf16_t* rows, bf16_t* cols,
                                           float scale) {
    uint4 reg[2];
    load_rows(base, sn, reg);
    store_rows<QSCALE, TRANSPOSE>(reg, rows, cols, scale);
}

// D(32x32) += A(32 x 64) B(64 x 32) with A rows and B columns read as 16-byte LDS runs:
// a_rows[m][k], b_rows[n][k] (both "row = output index, 64 contiguous k").
__device__ __forceinline__ f32x16 mma_32x32x64(const bf16_t* a_rows, const bf16_t* b_rows, f32x16 acc, int lane) {
    const int r = lane & 31, kh = 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        acc = mfma32(lds8(a_rows + r * kLd + 16 * kk + kh), lds8(b_rows + r * kLd + 16 * kk + kh), acc);
    return acc;
}

// ------------------------------------------------------------------ delta
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdParams p) {
    // one wave per 8 (b, n, h) rows; lane l: row l / 8, dims 8 (l % 8) .. +7
    const int64_t rows = (int64_t)p.B * p.N * p.Hq;
    const int lane = threadIdx.x & 63;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    if (row >= rows) return;
    const int h = (int)(row % p.Hq);
    const int64_t bn = row / p.Hq;
    const int n = (int)(bn % p.N), b = (int)(bn / p.N);
    const int c8 = (lane & 7) * 8;
    float o[8], g[8];
    unpack8(ld16(p.o + row * 64 + c8), o);
    unpack8(ld16(p.go + (int64_t)b * p.go_sb + (int64_t)n * p.go_sn + (int64_t)h * p.go_sh + c8), g);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += round_bf16(o[e] * g[e]);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if ((lane & 7) == 0) p.delta[row] = round_bf16(s);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// MFMA A operand of the transpose of a row-major LDS tile T[token][dim] (row stride kLd): lane
// l receives dim d0 + l % 32 for tokens t0 + 4 (l / 32) + 0..3 and t0 + 8 + 4 (l / 32) + 0..3,
// the accumulator row order of P and dS.  ds_read_b64_tr_b16 hands lane 4a + b of each
// 16-lane group element b of the 8-byte rows addressed by lanes a, a + 4, a + 8, a + 12, so
// lane s of a group addresses token 4 (l / 32) + s / 4, dims 16 ((l / 16) % 2) + 4 (s % 4).
__device__ __forceinline__ bf16x8 lds_tr_operand(const bf16_t* T, int t0, int d0, int lane) {
    const int s = lane & 15;
    const bf16_t* p = T + (t0 + 4 * (lane >> 5) + (s >> 2)) * kLd + d0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
    const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                   (__attribute__((address_space(3))) v4i16*)(p)));
    const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                   (__attribute__((address_space(3))) v4i16*)(p + 8 * kLd)));
    return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// The same row order from a row-major tile read along its rows: elements k0 + 4 (l / 32) + 0..3
// and k0 + 8 + 4 (l / 32) + 0..3 of row r.
__device__ __forceinline__ bf16x8 lds_row_perm(const bf16_t* T, int r, int k0, int lane) {
    const bf16_t* p = T + r * kLd + k0 + 4 * (lane >> 5);
    const uint2 lo = *reinterpret_cast<const uint2*>(p);
    const uint2 hi = *reinterpret_cast<const uint2*>(p + 8);
    return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// ------------------------------------------------------------------ grad q
// grid (N / 64 query tiles, Hq, B)
__global__ __launch_bounds__(256) void bwd_dq_kernel(BwdParams p) {
    __shared__ __attribute__((aligned(16))) bf16_t Qs[64 * kLd], Gs[64 * kLd], Ks[64 * kLd], Vs[64 * kLd],
        Ds[64 * kLd];
    __shared__ float lse_s[64], dl_s[64];
    const int qt = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
    const int c = j / p.G;
    const int n0 = qt * 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    stage_rows<true, false>(p.q + (int64_t)b * p.q_sb + (int64_t)n0 * p.q_sn + (int64_t)j * p.q_sh, p.q_sn, Qs,
                            nullptr, p.scale);
    stage_rows<false, false>(p.go + (int64_t)b * p.go_sb + (int64_t)n0 * p.go_sn + (int64_t)j * p.go_sh, p.go_sn,
                             Gs, nullptr, 0.f);
    if (threadIdx.x < 64) {
        const int64_t r = ((int64_t)b * p.N + n0 + threadIdx.x) * p.Hq + j;
        lse_s[threadIdx.x] = p.lse[r];
        dl_s[threadIdx.x] = p.delta[r];
    }
    const int64_t* sel = p.idx + (((int64_t)b * p.nb + n0 / p.bs) * p.Hk + c) * p.K;
    const int rh = w & 1, kh = w >> 1;   // phase 2: query half, key half
    const int dh = w >> 1;               // phase 3: dim half (query half rh)
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    // steps: the 64-key tiles of the valid selected blocks, in top-k order
    const int tiles = p.bs / 64;
    auto next_valid = [&](int i) {   // first entry >= i holding a block in range (uniform)
        while (i < p.K && (sel[i] < 0 || sel[i] >= p.nb)) ++i;
        return i;
    };
    int i = next_valid(0), t = 0;
    uint4 kr[2], vr[2];
    auto load_kv = [&](int i_, int t_) {
        const int key0 = (int)sel[i_] * p.bs + 64 * t_;
        load_rows(p.k + (int64_t)b * p.k_sb + (int64_t)key0 * p.k_sn + (int64_t)c * p.k_sh, p.k_sn, kr);
        load_rows(p.v + (int64_t)b * p.v_sb + (int64_t)key0 * p.v_sn + (int64_t)c * p.v_sh, p.v_sn, vr);
    };
    if (i < p.K) load_kv(i, 0);
    while (i < p.K) {
        __syncthreads();   // previous step's readers of Ks / Vs / Ds are done
        store_rows<false, false>(kr, Ks, nullptr, 0.f);
        store_rows<false, false>(vr, Vs, nullptr, 0.f);
        if (++t == tiles) { t = 0; i = next_valid(i + 1); }
        if (i < p.K) load_kv(i, t);   // next step's tiles, in flight during this step
        __syncthreads();
        f32x16 s, dp;
#pragma unroll
        for (int e = 0; e < 16; ++e) { s[e] = 0.f; dp[e] = 0.f; }
        s = mma_32x32x64(Qs + 32 * rh * kLd, Ks + 32 * kh * kLd, s, lane);
        dp = mma_32x32x64(Gs + 32 * rh * kLd, Vs + 32 * kh * kLd, dp, lane);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 32 * rh + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            const float pr = exp2f(s[e] - lse_s[r]) * kLn2;
            const float ds = pr * (dp[e] - dl_s[r]);
            Ds[r * kLd + 32 * kh + (lane & 31)] = (bf16_t)(pack_bf16x2(ds, 0.f) & 0xffffu);
        }
        __syncthreads();
        // dQ += dS k: A = dS rows and B = k^T (transposing reads of the row-major k tile), both
        // with the keys of each 16-key step in the order 4 (l / 32) + 0..3, 8 + 4 (l / 32) + 0..3
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            acc = mfma32(lds_row_perm(Ds, 32 * rh + (lane & 31), 16 * kk, lane),
                         lds_tr_operand(Ks, 16 * kk, 32 * dh, lane), acc);
    }
    bf16_t* out = p.dq + (((int64_t)b * p.N + n0) * p.Hq + j) * 64;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int r = 32 * rh + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        out[(int64_t)r * p.Hq * 64 + 32 * dh + (lane & 31)] =
            (bf16_t)(pack_bf16x2((acc[e] * p.scale) * kLog2e, 0.f) & 0xffffu);
    }
}

// ------------------------------------------------------------------ grad k, grad v
// grid (N / 64 key tiles, Hk, B).  Wave w = (key half kh = w / 2, query half qh = w % 2).  Per
// step a wave forms S = q' k^T and dP = do v^T for its 32 queries x 32 keys; P and dS stay in
// registers, where the accumulator layout (lane: one key column, 16 query rows) is exactly the
// MFMA B operand of dV^T += do^T P and dK^T += q'^T dS with k running over those query rows;
// the A operands (do^T, q'^T) come from transposing LDS reads of the row-major tiles in the
// same row order, so no transposed copy is staged.
// The two waves of a key half sum their partial dV^T / dK^T once, at the end.
__global__ __launch_bounds__(256) void bwd_dkv_kernel(BwdParams p) {
    __shared__ __attribute__((aligned(16))) bf16_t smem[4 * 64 * kLd];   // also the final 32 KB reduction
    __shared__ float lse_s[64], dl_s[64];
    __shared__ uint8_t mark[kMaxBwdBlocks];
    bf16_t* Ks = smem;
    bf16_t* Vs = smem + 64 * kLd;
    bf16_t* Qs = smem + 2 * 64 * kLd;
    bf16_t* Gs = smem + 3 * 64 * kLd;
    const int kt = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const int key0 = kt * 64;
    const int64_t u = key0 / p.bs;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // query blocks whose selection row (kv head c) holds block u: eight entries per step, all
    // loads of a step issued before any compare
    for (int t = threadIdx.x; t < p.nb; t += 256) {
        const int64_t* row = p.idx + (((int64_t)b * p.nb + t) * p.Hk + c) * p.K;
        bool hit = false;
        for (int i0 = 0; i0 < p.K; i0 += 8) {
            int64_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = i0 + i < p.K ? row[i0 + i] : -1;
#pragma unroll
            for (int i = 0; i < 8; ++i) hit |= e[i] == u;
        }
        mark[t] = hit;
    }
    stage_rows<false, false>(p.k + (int64_t)b * p.k_sb + (int64_t)key0 * p.k_sn + (int64_t)c * p.k_sh, p.k_sn, Ks,
                             nullptr, 0.f);
    stage_rows<false, false>(p.v + (int64_t)b * p.v_sb + (int64_t)key0 * p.v_sn + (int64_t)c * p.v_sh, p.v_sn, Vs,
                             nullptr, 0.f);
    __syncthreads();
    const int kh = w >> 1, qh = w & 1;
    const int hq = 4 * (lane >> 5);         // this lane's row offset inside each group of 8 rows
    f32x16 dkT[2], dvT[2];                  // [d block]: rows d = 32 db + row(e), column key 32 kh + lane % 32
#pragma unroll
    for (int e = 0; e < 16; ++e) { dkT[0][e] = 0.f; dkT[1][e] = 0.f; dvT[0][e] = 0.f; dvT[1][e] = 0.f; }
    // steps: (marked query block t, its 64-row tile tt, query head g of the group), ascending
    const int tiles = p.bs / 64;
    auto next_marked = [&](int t) {   // first marked block >= t (uniform LDS reads)
        while (t < p.nb && !mark[t]) ++t;
        return t;
    };
    int t = next_marked(0), tt = 0, g = 0;
    uint4 qr[2], gr[2];
    float lr = 0.f, dr = 0.f;
    auto load_q = [&](int t_, int tt_, int g_) {
        const int n0 = t_ * p.bs + 64 * tt_;
        const int j = c * p.G + g_;
        load_rows(p.q + (int64_t)b * p.q_sb + (int64_t)n0 * p.q_sn + (int64_t)j * p.q_sh, p.q_sn, qr);
        load_rows(p.go + (int64_t)b * p.go_sb + (int64_t)n0 * p.go_sn + (int64_t)j * p.go_sh, p.go_sn, gr);
        if (threadIdx.x < 64) {
            const int64_t r = ((int64_t)b * p.N + n0 + threadIdx.x) * p.Hq + j;
            lr = p.lse[r];
            dr = p.delta[r];
        }
    };
    if (t < p.nb) load_q(t, 0, 0);
    while (t < p.nb) {
        __syncthreads();   // previous step's readers are done with Qs / Gs
        store_rows<true, false>(qr, Qs, nullptr, p.scale);
        store_rows<false, false>(gr, Gs, nullptr, 0.f);
        if (threadIdx.x < 64) {
            lse_s[threadIdx.x] = lr;
            dl_s[threadIdx.x] = dr;
        }
        if (++g == p.G) {
            g = 0;
            if (++tt == tiles) { tt = 0; t = next_marked(t + 1); }
        }
        if (t < p.nb) load_q(t, tt, g);   // next step's rows, in flight during this step
        __syncthreads();
        f32x16 s, dp;
#pragma unroll
        for (int e = 0; e < 16; ++e) { s[e] = 0.f; dp[e] = 0.f; }
        s = mma_32x32x64(Qs + 32 * qh * kLd, Ks + 32 * kh * kLd, s, lane);    // S: queries x keys
        dp = mma_32x32x64(Gs + 32 * qh * kLd, Vs + 32 * kh * kLd, dp, lane);  // dP
        bf16x8 pb[2], db[2];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int q = 32 * qh + 8 * (e >> 2) + hq + (e & 3);
            const float pr = exp2f(s[e] - lse_s[q]);
            const float ds = pr * (dp[e] - dl_s[q]) * kLn2;
            pb[e >> 3][e & 7] = (__bf16)pr;
            db[e >> 3][e & 7] = (__bf16)ds;
        }
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                const int q0 = 32 * qh + 16 * ch;
                dvT[dblk] = mfma32(lds_tr_operand(Gs, q0, 32 * dblk, lane), pb[ch], dvT[dblk]);
                dkT[dblk] = mfma32(lds_tr_operand(Qs, q0, 32 * dblk, lane), db[ch], dkT[dblk]);
            }
        }
    }
    // sum the two query halves' partials: qh = 1 parks its accumulators in LDS
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem) + (kh * 64 + lane) * 64;
    if (qh == 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            red[e] = dkT[0][e]; red[16 + e] = dkT[1][e]; red[32 + e] = dvT[0][e]; red[48 + e] = dvT[1][e];
        }
    }
    __syncthreads();
    if (qh == 0) {
        const int64_t base = (((int64_t)b * p.N + key0 + 32 * kh + (lane & 31)) * p.Hk + c) * 64;
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int d = 32 * dblk + 8 * (e >> 2) + hq + (e & 3);
                p.dk[base + d] = (bf16_t)(pack_bf16x2(dkT[dblk][e] + red[16 * dblk + e], 0.f) & 0xffffu);
                p.dv[base + d] = (bf16_t)(pack_bf16x2(dvT[dblk][e] + red[32 + 16 * dblk + e], 0.f) & 0xffffu);
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

size_t mosaic_sparse_attn_bwd_workspace_size(int32_t batch, int32_t seq_len, int32_t num_q_heads) {
    if (batch <= 0 || seq_len <= 0 || num_q_heads <= 0) return 0;
    return ((size_t)batch * seq_len * num_q_heads * sizeof(float) + 255) / 256 * 256;
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
    p.delta = static_cast<float*>(workspace);
    p.idx = block_indices;
    p.dq = static_cast<bf16_t*>(grad_q); p.dk = static_cast<bf16_t*>(grad_k); p.dv = static_cast<bf16_t*>(grad_v);
    p.B = batch; p.N = seq_len; p.Hq = num_q_heads; p.Hk = num_kv_heads; p.G = num_q_heads / num_kv_heads;
    p.bs = block_size; p.K = block_count; p.nb = seq_len / block_size;
    p.scale = softmax_scale > 0.f ? softmax_scale : 0.125f;   // head_dim^-0.5 for head_dim 64
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* args[] = {&p};
    const int64_t rows = (int64_t)batch * seq_len * num_q_heads;
    const int64_t dgrid = (rows + 31) / 32;
    if (dgrid > 0x7fffffff) return MOSAIC_ERR_SHAPE;
    if (hipLaunchKernel((const void*)&bwd_delta_kernel, dim3((unsigned)dgrid), dim3(256), args, 0, s) != hipSuccess)
        return MOSAIC_ERR_LAUNCH;
    if (hipLaunchKernel((const void*)&bwd_dq_kernel, dim3(seq_len / 64, num_q_heads, batch), dim3(256), args, 0, s) !=
        hipSuccess)
        return MOSAIC_ERR_LAUNCH;
    if (hipLaunchKernel((const void*)&bwd_dkv_kernel, dim3(seq_len / 64, num_kv_heads, batch), dim3(256), args, 0,
                        s) != hipSuccess)
        return MOSAIC_ERR_LAUNCH;
    return MOSAIC_OK;
}

}  // extern "C"
