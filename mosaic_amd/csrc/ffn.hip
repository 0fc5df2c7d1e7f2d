// ffn.hip -- cSwiGLU's first projection with the gate in its epilogue (gfx950).
//
// Replaces, for cSwiGLU.forward (primitives.py:92-105), h = w13(x) (a bf16 Linear: fp32
// accumulation, rounded to bf16) followed by the gate with the rounding points of the
// reference's eager bf16 ops (the same ones swiglu_kernel in fused.hip applies):
//   a = bf16(x1 + noise[member]),  s = bf16(a / (1 + exp(-a))),  g = bf16(s * x3)
// for x1, x3 = h.chunk(2): h (two hidden-wide halves per row) is never written or read back.
//
// The weight is w13 with its rows permuted in 64-row groups: group t holds rows 32 t .. + 31
// of the x1 half, then the same rows of the x3 half.  A wave's 64 output columns are then one
// x1 block and the matching x3 block, and the MFMA accumulator layout (lane: one column, 16
// rows) gives a lane both values of each of its (row, hidden index) pairs.
//
// Tiling, operand staging and the k ring follow proj.hip: 256 rows x 256 permuted columns per
// workgroup, eight waves (two per SIMD), wave (wm, wn) computes rows 128 wm .. + 127 of the
// 64-column group wn with v_mfma_f32_32x32x16_bf16, K in steps of 32 through a ring of four
// LDS slots filled by direct-to-LDS loads.  Workgroups go in groups of kGroupRows row tiles
// with the column tile varying slowest inside a group, so the workgroups an XCD runs at one
// time share both their x tiles and their weight tiles in its L2.
#include "bsa_common.h"
#include "mosaic_bsa.h"

namespace mosaic {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kM = 256;              // rows per workgroup
constexpr int kN = 256;              // permuted columns per workgroup (128 hidden indices)
constexpr int kK = 32;               // reduction step
constexpr int kSlot = kM * kK;       // bf16 elements of one operand's ring slot (16 KB)
constexpr int kGroupRows = 4;        // row tiles per L2 group

struct SwigluLinearParams {
    const bf16_t* x;        // [rows, D], row stride x_sr (elements)
    const bf16_t* w;        // [2 hidden, D] permuted w13, contiguous
    const bf16_t* noise;    // [noise_rows, hidden] contiguous, or null
    bf16_t* out;            // [rows, hidden] contiguous
    int64_t x_sr;
    int D, hidden, noise_rows, n_tiles, row_tiles;
};

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// barrier for LDS data whose direct-to-LDS loads each wave has already waited for itself
// (__syncthreads() would also wait for every load still in flight)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}
// 16-byte LDS read issued as inline assembly (no compiler wait for the loads in flight into
// the other ring slots); the caller waits with lgkm_wait before using the result
template <int OFF>
__device__ __forceinline__ bf16x8 lds_read16(uint32_t addr) {
    bf16x8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
// s_waitcnt lgkmcnt(N) that the six operand registers depend on
template <int N>
__device__ __forceinline__ void lgkm_wait(bf16x8& a0, bf16x8& a1, bf16x8& a2, bf16x8& a3, bf16x8& b0, bf16x8& b1) {
    asm volatile("s_waitcnt lgkmcnt(%6)" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1) : "i"(N));
}

__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void swiglu_linear_kernel(SwigluLinearParams p) {
    __shared__ __attribute__((aligned(1024))) bf16_t A0[kSlot], A1[kSlot], A2[kSlot], A3[kSlot];
    __shared__ __attribute__((aligned(1024))) bf16_t B0[kSlot], B1[kSlot], B2[kSlot], B3[kSlot];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = w >> 2, wn = w & 3;
    // logical tile: groups of kGroupRows row tiles (the last group may hold fewer); inside a
    // group the row tile varies fastest, so xcd_remap's contiguous ranges per XCD cover a few
    // column tiles of a few row tiles
    const int id = xcd_remap(blockIdx.x, gridDim.x);
    const int per_group = kGroupRows * p.n_tiles;
    const int grp = id / per_group, within = id - grp * per_group;
    const int rows_here = min(kGroupRows, p.row_tiles - grp * kGroupRows);
    const int ntile = within / rows_here;
    const int rtile = grp * kGroupRows + (within - ntile * rows_here);
    const int64_t r0 = (int64_t)rtile * kM;
    const int n0 = ntile * kN;

    // direct-to-LDS loads of a slot (rows of 32 k = 64 bytes): wave w fills rows 32 w .. + 31 of
    // both operands, sixteen rows per instruction; lane l lands at row 16 i + l / 4, position
    // l % 4, and fetches the row's chunk (l % 4) ^ ((row / 4) % 4), so the 16-byte operand reads
    // (16 consecutive rows per cycle over 64 banks) are conflict-free
    const int r16 = lane >> 2, gch = (lane & 3) ^ ((lane >> 4) & 3);
    const char* xbase = reinterpret_cast<const char*>(p.x + (r0 + 32 * w) * p.x_sr);
    const char* wbase = reinterpret_cast<const char*>(p.w + (int64_t)(n0 + 32 * w) * p.D);
    const uint32_t xoff = 2u * (uint32_t)(r16 * p.x_sr + 8 * gch);
    const uint32_t woff = 2u * (uint32_t)(r16 * p.D + 8 * gch);
    const int64_t xstep = 32 * p.x_sr, wstep = 32 * (int64_t)p.D;   // bytes per 16 rows
    auto issue = [&](int k0, bf16_t* As, bf16_t* Bs) __attribute__((always_inline)) {
        const char* xk = xbase + 2 * k0;
        const char* wk = wbase + 2 * k0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            __builtin_amdgcn_global_load_lds(xk + i * xstep + xoff, (lds_void*)(As + (32 * w + 16 * i) * kK), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(wk + i * wstep + woff, (lds_void*)(Bs + (32 * w + 16 * i) * kK), 16, 0, 0);
        }
    };
    // operand reads: row 32 t + lane % 32 of a 32-row block, chunk 2 kk + lane / 32 (kk = 0, 1)
    int rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) rd[kk] = (lane & 31) * kK + 8 * ((2 * kk + (lane >> 5)) ^ ((lane >> 2) & 3));

    f32x16 acc[4][2];   // [32-row tile][x1 block, x3 block]
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mt][nt][e] = 0.f;
    auto compute = [&](const bf16_t* As, const bf16_t* Bs) __attribute__((always_inline)) {
        bf16x8 a[2][4], bb[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint32_t aa = lds_addr(As + 128 * wm * kK + rd[kk]);
            const uint32_t ba = lds_addr(Bs + 64 * wn * kK + rd[kk]);
            constexpr int T = 32 * kK * 2;   // bytes between 32-row blocks
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
    // Step i uses slot i % 4; its loads were requested three steps earlier.  Wait for them,
    // leaving the two newer steps' loads in flight (four per wave and step), then the barrier
    // publishes every wave's loads and frees slot (i + 3) % 4, whose step is requested before
    // step i is computed.  D is a multiple of 128, so the loop runs whole rings and has one exit.
    const int steps = p.D / kK;
    issue(0, A0, B0);
    issue(kK, A1, B1);
    issue(2 * kK, A2, B2);
    auto ring_step = [&](int i, const bf16_t* As, const bf16_t* Bs, bf16_t* An, bf16_t* Bn) __attribute__((always_inline)) {
        if (i + 2 < steps) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (i + 1 < steps) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else wait_vmem();
        lds_barrier();
        if (i + 3 < steps) issue(kK * (i + 3), An, Bn);
        compute(As, Bs);
    };
    for (int i = 0; i < steps; i += 4) {
        ring_step(i, A0, B0, A3, B3);
        ring_step(i + 1, A1, B1, A0, B0);
        ring_step(i + 2, A2, B2, A1, B1);
        ring_step(i + 3, A3, B3, A2, B2);
    }

    // ------------------------------------------------------------------ epilogue
    // lane: hidden index j (column lane % 32 of the wave's x1 and x3 blocks), rows
    // 8 (e / 4) + 4 (lane / 32) + e % 4 of each 32-row tile mt of its 128 rows
    const int hh = lane >> 5;
    const int j = 32 * (n0 / 64 + wn) + (lane & 31);
    bf16_t* outj = p.out + j;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int64_t rb = r0 + 128 * wm + 32 * mt + 4 * hh;
        float nv[16];
        if (p.noise != nullptr) {   // noise row = row % noise_rows (rows are [sequence, member])
            const int m0 = (int)(rb % p.noise_rows);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int nr = (m0 + 8 * (e >> 2) + (e & 3)) % p.noise_rows;
                nv[e] = bf2f(p.noise[(int64_t)nr * p.hidden + j]);
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float a = round_bf16(acc[mt][0][e]);
            if (p.noise != nullptr) a = round_bf16(a + nv[e]);
            const float sl = round_bf16(a / (1.0f + expf(-a)));
            const float g = sl * round_bf16(acc[mt][1][e]);
            const int64_t row = rb + 8 * (e >> 2) + (e & 3);
            outj[row * p.hidden] = (bf16_t)(pack_bf16x2(g, 0.f) & 0xffffu);
        }
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" {

int mosaic_swiglu_linear_fwd(const void* x, int64_t rows, int32_t dim, int64_t x_row_stride, const void* weight,
                             int32_t hidden, const void* noise, int32_t noise_rows, void* out, void* stream) {
    if (rows <= 0 || dim <= 0 || hidden <= 0) return MOSAIC_ERR_SHAPE;
    if (!x || !weight || !out) return MOSAIC_ERR_NULL_POINTER;
    if (noise && noise_rows <= 0) return MOSAIC_ERR_SHAPE;
    if (rows % kM || dim % (4 * kK) || (2 * (int64_t)hidden) % kN) return MOSAIC_ERR_UNSUPPORTED;
    if (x_row_stride < dim || x_row_stride % 8) return MOSAIC_ERR_ALIGNMENT;
    if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (noise && !aligned16(noise)))
        return MOSAIC_ERR_ALIGNMENT;
    // per-lane byte offsets within 16 rows are 32-bit
    if (x_row_stride >= ((int64_t)1 << 26) || dim >= (1 << 26)) return MOSAIC_ERR_UNSUPPORTED;
    const int64_t row_tiles = rows / kM, n_tiles = 2 * (int64_t)hidden / kN;
    if (row_tiles * n_tiles > 0x7fffffff || row_tiles > 0x7fffffff) return MOSAIC_ERR_SHAPE;
    SwigluLinearParams p{};
    p.x = static_cast<const bf16_t*>(x);
    p.w = static_cast<const bf16_t*>(weight);
    p.noise = static_cast<const bf16_t*>(noise);
    p.out = static_cast<bf16_t*>(out);
    p.x_sr = x_row_stride;
    p.D = dim;
    p.hidden = hidden;
    p.noise_rows = noise ? noise_rows : 1;
    p.n_tiles = (int)n_tiles;
    p.row_tiles = (int)row_tiles;
    void* args[] = {&p};
    const hipError_t e = hipLaunchKernel((const void*)&swiglu_linear_kernel, dim3((unsigned)(row_tiles * n_tiles)),
                                         dim3(512), args, 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MOSAIC_OK : MOSAIC_ERR_LAUNCH;
}

}  // extern "C"
