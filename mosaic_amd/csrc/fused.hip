// fused.hip -- the model's row-wise elementwise work as single HBM passes (gfx950).
//
// rms_norm_kernel replaces torch.nn.RMSNorm (used by MosaicBlock, primitives.py:220-227, and
// by the U-Net's pre/post-processing and resampling, mosaic.py:163-217, primitives.py:313-359),
// optionally fused with the residual add in front of it (primitives.py:225-226):
//   y   = x + r                       rounded to x's dtype, as torch's add rounds
//   out = y * rsqrt(mean(y^2) + eps) [* weight]   fp32 statistics, rounded once to out's dtype
// swiglu_kernel replaces the gate of cSwiGLU.forward (primitives.py:102-105):
//   a = x1 + noise[member]  (rounded),  s = silu(a) = a / (1 + exp(-a))  (rounded),  g = s * x3
// with the rounding points of the reference's eager bf16 ops.  In eager torch these are 3-6
// kernels, each reading and writing the full activation; here each is one read and one write.
//
// Both kernels are HBM-bound: rms_norm moves (1 + residual + sum_out + 1) rows of `cols`
// elements, swiglu reads 2 hidden and writes 1 hidden element per (row, column).  Each lane
// moves 8 contiguous elements per access (16-byte bf16 / 2x16-byte fp32 loads and stores).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsa_common.h"
#include "mosaic_bsa.h"

namespace mosaic {
namespace {

constexpr int kNormWaves = 4;      // rows per workgroup (one wave per row)
constexpr int kMaxNormChunks = 8;  // 8-element chunks per lane: cols <= 8 * 64 * 8 = 4096
constexpr int kGluThreads = 256;

__device__ __forceinline__ void load8(const float* p, float v[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load8(const bf16_t* p, float v[8]) {
    const uint4 u = ld16(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = bf_lo(w[i]); v[2 * i + 1] = bf_hi(w[i]); }
}
__device__ __forceinline__ void store8(float* p, const float v[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void store8(bf16_t* p, const float v[8]) {
    uint4 u;
    u.x = pack_bf16x2(v[0], v[1]); u.y = pack_bf16x2(v[2], v[3]);
    u.z = pack_bf16x2(v[4], v[5]); u.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = u;
}
// the value a tensor of element type T holds for the fp32 result x
__device__ __forceinline__ float as_stored(float x, const float*) { return x; }
__device__ __forceinline__ float as_stored(float x, const bf16_t*) { return round_bf16(x); }

__device__ __forceinline__ float wave_sum(float s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    return s;
}

struct NormParams {
    const void* x; const void* res; const float* weight;
    void* sum_out; void* out;
    int64_t rows, x_stride, r_stride;
    int cols; float eps;
};

template <typename T, typename TO, int NCH, bool RES>
__global__ __launch_bounds__(kNormWaves * 64) void rms_norm_kernel(NormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const T* x = static_cast<const T*>(p.x) + row * p.x_stride;
    const T* r = RES ? static_cast<const T*>(p.res) + row * p.r_stride : nullptr;
    const int nchunk = p.cols >> 3;
    float v[NCH][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunk) {
            load8(x + 8 * c, v[i]);
            if (RES) {
                float rv[8];
                load8(r + 8 * c, rv);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[i][e] = as_stored(v[i][e] + rv[e], x);
                if (p.sum_out) store8(static_cast<T*>(p.sum_out) + row * p.cols + 8 * c, v[i]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
        }
    }
    const float inv = rsqrtf(wave_sum(ss) / (float)p.cols + p.eps);
    TO* out = static_cast<TO*>(p.out) + row * p.cols;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunk) {
            float o[8];
            if (p.weight) {
                const float* w = p.weight + 8 * c;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = v[i][e] * inv * w[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = v[i][e] * inv;
            }
            store8(out + 8 * c, o);
        }
    }
}

template <typename T, typename TO, bool RES>
hipError_t launch_norm_t(const NormParams& p, hipStream_t s) {
    const unsigned grid = (unsigned)((p.rows + kNormWaves - 1) / kNormWaves);
    void* args[] = {const_cast<NormParams*>(&p)};
    const void* k = nullptr;
    switch ((p.cols / 8 + 63) / 64) {
        case 1: k = (const void*)&rms_norm_kernel<T, TO, 1, RES>; break;
        case 2: k = (const void*)&rms_norm_kernel<T, TO, 2, RES>; break;
        case 3: k = (const void*)&rms_norm_kernel<T, TO, 3, RES>; break;
        case 4: k = (const void*)&rms_norm_kernel<T, TO, 4, RES>; break;
        case 5: case 6: k = (const void*)&rms_norm_kernel<T, TO, 6, RES>; break;
        case 7: case 8: k = (const void*)&rms_norm_kernel<T, TO, 8, RES>; break;
        default: return hipErrorInvalidValue;
    }
    return hipLaunchKernel(k, dim3(grid), dim3(kNormWaves * 64), args, 0, s);
}

template <typename T, typename TO>
hipError_t launch_norm_res(const NormParams& p, hipStream_t s) {
    return p.res ? launch_norm_t<T, TO, true>(p, s) : launch_norm_t<T, TO, false>(p, s);
}

// HEALPix resampling epilogue (primitives.py:313-359): the resampled rows of the projection P
// plus the broadcast position term, plus the skip connection, normalised:
//   output row R = (n f + j) B + b  (sequence-first [(n f), B, d]) takes
//   y = bf16(P[n B + b, j d .. j d + d) + pos[n, j d .. j d + d))     (the '(f d)' split)
//   y = bf16(y + shortcut[R])                                        (upsampling only)
//   out = y * rsqrt(mean(y^2) + eps) * weight
// f = 1 with no shortcut is the downsampling epilogue.  One wave per output row; the eager
// form is an add, a transposed copy, an add and the norm, each a pass over the activations.
struct ResampleParams {
    const bf16_t* p; const bf16_t* pos; const bf16_t* shortcut; const float* weight;
    bf16_t* out;
    int64_t rows, p_stride;
    int members, factor, dim;
    float eps;
};

template <int NCH, bool SC>
__global__ __launch_bounds__(kNormWaves * 64) void resample_norm_kernel(ResampleParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int64_t fb = (int64_t)p.factor * p.members;
    const int64_t n = row / fb;
    const int rem = (int)(row - n * fb);
    const int j = rem / p.members, b = rem - j * p.members;
    const bf16_t* prow = p.p + (n * p.members + b) * p.p_stride + (int64_t)j * p.dim;
    const bf16_t* qrow = p.pos + n * ((int64_t)p.factor * p.dim) + (int64_t)j * p.dim;
    const int nchunk = p.dim >> 3;
    float v[NCH][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunk) {
            float a[8];
            load8(prow + 8 * c, v[i]);
            load8(qrow + 8 * c, a);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = round_bf16(v[i][e] + a[e]);
            if (SC) {
                load8(p.shortcut + row * p.dim + 8 * c, a);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[i][e] = round_bf16(v[i][e] + a[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
        }
    }
    const float inv = rsqrtf(wave_sum(ss) / (float)p.dim + p.eps);
    bf16_t* out = p.out + row * p.dim;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunk) {
            float o[8];
            if (p.weight) {
                const float* w = p.weight + 8 * c;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = v[i][e] * inv * w[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = v[i][e] * inv;
            }
            store8(out + 8 * c, o);
        }
    }
}

template <bool SC>
hipError_t launch_resample_t(const ResampleParams& p, hipStream_t s) {
    const unsigned grid = (unsigned)((p.rows + kNormWaves - 1) / kNormWaves);
    void* args[] = {const_cast<ResampleParams*>(&p)};
    const void* k = nullptr;
    switch ((p.dim / 8 + 63) / 64) {
        case 1: k = (const void*)&resample_norm_kernel<1, SC>; break;
        case 2: k = (const void*)&resample_norm_kernel<2, SC>; break;
        case 3: k = (const void*)&resample_norm_kernel<3, SC>; break;
        case 4: k = (const void*)&resample_norm_kernel<4, SC>; break;
        case 5: case 6: k = (const void*)&resample_norm_kernel<6, SC>; break;
        case 7: case 8: k = (const void*)&resample_norm_kernel<8, SC>; break;
        default: return hipErrorInvalidValue;
    }
    return hipLaunchKernel(k, dim3(grid), dim3(kNormWaves * 64), args, 0, s);
}

// The end of an encoder stage and the input of its downsampling (mosaic.py:318-321,
// primitives.py:322-326): s = bf16(x + pending) (the stage's last residual add, kept as the skip
// connection) and the same sums merged per coarse pixel, '(n f) b c -> n b (f c)', for the
// downsampling projection.  One thread per 8-element chunk of s; both stores are 16 bytes.
struct MergeParams {
    const bf16_t* x; const bf16_t* r; bf16_t* s; bf16_t* merged;
    int64_t rows;  // (n f) B rows of s
    int members, factor, dim;
};

__global__ __launch_bounds__(256) void add_merge_kernel(MergeParams p) {
    const int chunks = p.dim >> 3;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= p.rows * chunks) return;
    const int64_t row = i / chunks;
    const int c = (int)(i - row * chunks) * 8;
    float a[8], b[8];
    load8(p.x + row * p.dim + c, a);
    load8(p.r + row * p.dim + c, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = round_bf16(a[e] + b[e]);
    store8(p.s + row * p.dim + c, a);
    const int64_t fb = (int64_t)p.factor * p.members;
    const int64_t n = row / fb;
    const int rem = (int)(row - n * fb);
    const int j = rem / p.members, m = rem - j * p.members;
    store8(p.merged + ((n * p.members + m) * p.factor + j) * p.dim + c, a);
}

// generate_strategy_weights (primitives.py:173-180) on the gate slice of the stacked projection:
//   w[s, b, n, h] = bf16(softmax over s of fp32(logits[n, b, 3 h + s]))
// as torch.softmax(logits.float(), dim=0).type_as(x) computes it: m = max, e_s = exp(l_s - m),
// w_s = e_s / (e_0 + e_1 + e_2).  One thread per (b, n, h) in the order of w, so the stores of
// a wave are contiguous in each plane (in logits order they were 24-byte pieces B rows apart:
// 106 us at 1.18 M rows of 12 heads); the eager form is a strided fp32 copy, a softmax launch
// over a dimension of 3 and a cast, each a separate pass.
struct GateParams {
    const bf16_t* logits; bf16_t* w;
    int64_t rows, row_stride;  // rows = S * B, logits row (n, b) at (n B + b) row_stride
    int members, heads;
};

__global__ __launch_bounds__(256) void gate_softmax_kernel(GateParams p) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= p.rows * p.heads) return;
    const int64_t t = i / p.heads, seq = p.rows / p.members;  // t = b seq + n
    const int h = (int)(i - t * p.heads);
    const int64_t b = t / seq, n = t - b * seq;
    const bf16_t* l = p.logits + (n * p.members + b) * p.row_stride + 3 * h;
    const float l0 = bf2f(l[0]), l1 = bf2f(l[1]), l2 = bf2f(l[2]);
    const float m = fmaxf(fmaxf(l0, l1), l2);
    const float e0 = expf(l0 - m), e1 = expf(l1 - m), e2 = expf(l2 - m);
    const float sum = e0 + e1 + e2;
    const int64_t plane = p.rows * p.heads;  // one [B, S, H] plane per branch s
    bf16_t* w = p.w + i;
    w[0] = (bf16_t)(pack_bf16x2(e0 / sum, 0.f) & 0xffffu);
    w[plane] = (bf16_t)(pack_bf16x2(e1 / sum, 0.f) & 0xffffu);
    w[2 * plane] = (bf16_t)(pack_bf16x2(e2 / sum, 0.f) & 0xffffu);
}

struct GluParams {
    const void* h; const void* noise; void* out;
    int64_t rows, h_stride;
    int hidden, noise_rows;
};

template <typename T, bool NOISE>
__global__ __launch_bounds__(kGluThreads) void swiglu_kernel(GluParams p) {
    const int64_t chunks = p.hidden >> 3;
    const int64_t i = (int64_t)blockIdx.x * kGluThreads + threadIdx.x;
    if (i >= p.rows * chunks) return;
    const int64_t row = i / chunks;
    const int c = (int)(i - row * chunks) * 8;
    const T* h = static_cast<const T*>(p.h) + row * p.h_stride + c;
    float x1[8], x3[8], g[8];
    load8(h, x1);
    load8(h + p.hidden, x3);
    if (NOISE) {
        float n[8];
        load8(static_cast<const T*>(p.noise) + (row % p.noise_rows) * p.hidden + c, n);
#pragma unroll
        for (int e = 0; e < 8; ++e) x1[e] = as_stored(x1[e] + n[e], h);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float a = x1[e];
        const float sl = as_stored(a / (1.0f + expf(-a)), h);
        g[e] = sl * x3[e];
    }
    store8(static_cast<T*>(p.out) + row * p.hidden + c, g);
}

template <typename T>
hipError_t launch_glu(const GluParams& p, hipStream_t s) {
    const int64_t total = p.rows * (p.hidden / 8);
    const int64_t grid = (total + kGluThreads - 1) / kGluThreads;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    void* args[] = {const_cast<GluParams*>(&p)};
    const void* k = p.noise ? (const void*)&swiglu_kernel<T, true> : (const void*)&swiglu_kernel<T, false>;
    return hipLaunchKernel(k, dim3((unsigned)grid), dim3(kGluThreads), args, 0, s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool valid_dtype(int32_t d) { return d == MOSAIC_DTYPE_F32 || d == MOSAIC_DTYPE_BF16; }
// element strides that keep every 8-element chunk 16-byte aligned
bool chunk_stride(int64_t stride, int32_t dtype) { return stride % (dtype == MOSAIC_DTYPE_F32 ? 4 : 8) == 0; }
int status(hipError_t e) { return e == hipSuccess ? MOSAIC_OK : MOSAIC_ERR_LAUNCH; }

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" {

int mosaic_rms_norm_fwd(const void* x, const void* residual, int32_t dtype, int64_t rows, int32_t cols,
                        int64_t x_row_stride, int64_t residual_row_stride, const float* weight, float eps,
                        void* sum_out, void* out, int32_t out_dtype, void* stream) {
    if (rows <= 0 || cols <= 0) return MOSAIC_ERR_SHAPE;
    if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return MOSAIC_ERR_UNSUPPORTED;
    if (cols % 8 || cols > kMaxNormChunks * 64 * 8) return MOSAIC_ERR_UNSUPPORTED;
    if (rows > (int64_t)0x7fffffff * kNormWaves) return MOSAIC_ERR_SHAPE;
    if (!x || !out) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(x) || !aligned16(out) || !chunk_stride(x_row_stride, dtype)) return MOSAIC_ERR_ALIGNMENT;
    if (residual && (!aligned16(residual) || !aligned16(sum_out) || !chunk_stride(residual_row_stride, dtype)))
        return MOSAIC_ERR_ALIGNMENT;
    if (weight && !aligned16(weight)) return MOSAIC_ERR_ALIGNMENT;
    NormParams p{x, residual, weight, sum_out, out, rows, x_row_stride, residual_row_stride, cols, eps};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == MOSAIC_DTYPE_BF16)
        return status(out_dtype == MOSAIC_DTYPE_BF16 ? launch_norm_res<bf16_t, bf16_t>(p, s)
                                                     : launch_norm_res<bf16_t, float>(p, s));
    return status(out_dtype == MOSAIC_DTYPE_BF16 ? launch_norm_res<float, bf16_t>(p, s)
                                                 : launch_norm_res<float, float>(p, s));
}

int mosaic_resample_norm_fwd(const void* p, int64_t p_row_stride, const void* pos, const void* shortcut,
                             const float* weight, float eps, int64_t coarse_rows, int32_t members,
                             int32_t factor, int32_t dim, void* out, void* stream) {
    if (coarse_rows <= 0 || members <= 0 || factor <= 0 || dim <= 0) return MOSAIC_ERR_SHAPE;
    if (dim % 8 || dim > kMaxNormChunks * 64 * 8) return MOSAIC_ERR_UNSUPPORTED;
    if (p_row_stride < (int64_t)factor * dim) return MOSAIC_ERR_SHAPE;
    const int64_t rows = coarse_rows * factor * members;
    if (rows / factor / members != coarse_rows || rows > (int64_t)0x7fffffff * kNormWaves) return MOSAIC_ERR_SHAPE;
    if (!p || !pos || !out) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(p) || !aligned16(pos) || !aligned16(out) || p_row_stride % 8) return MOSAIC_ERR_ALIGNMENT;
    if ((shortcut && !aligned16(shortcut)) || (weight && !aligned16(weight))) return MOSAIC_ERR_ALIGNMENT;
    ResampleParams rp{static_cast<const bf16_t*>(p), static_cast<const bf16_t*>(pos),
                      static_cast<const bf16_t*>(shortcut), weight, static_cast<bf16_t*>(out),
                      rows, p_row_stride, members, factor, dim, eps};
    hipStream_t s = static_cast<hipStream_t>(stream);
    return status(shortcut ? launch_resample_t<true>(rp, s) : launch_resample_t<false>(rp, s));
}

int mosaic_add_merge_fwd(const void* x, const void* residual, int64_t coarse_rows, int32_t members,
                         int32_t factor, int32_t dim, void* sum_out, void* merged_out, void* stream) {
    if (coarse_rows <= 0 || members <= 0 || factor <= 0 || dim <= 0) return MOSAIC_ERR_SHAPE;
    if (dim % 8) return MOSAIC_ERR_UNSUPPORTED;
    const int64_t rows = coarse_rows * factor * members, total = rows * (dim / 8);
    if (rows / factor / members != coarse_rows || (total + 255) / 256 > 0x7fffffff) return MOSAIC_ERR_SHAPE;
    if (!x || !residual || !sum_out || !merged_out) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(x) || !aligned16(residual) || !aligned16(sum_out) || !aligned16(merged_out))
        return MOSAIC_ERR_ALIGNMENT;
    MergeParams mp{static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(residual), static_cast<bf16_t*>(sum_out),
                   static_cast<bf16_t*>(merged_out), rows, members, factor, dim};
    void* args[] = {&mp};
    return status(hipLaunchKernel((const void*)add_merge_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                                  args, 0, static_cast<hipStream_t>(stream)));
}

int mosaic_gate_softmax_fwd(const void* logits, int64_t logits_row_stride, int64_t seq, int32_t members,
                            int32_t heads, void* w, void* stream) {
    if (seq <= 0 || members <= 0 || heads <= 0) return MOSAIC_ERR_SHAPE;
    if (logits_row_stride < 3 * (int64_t)heads) return MOSAIC_ERR_SHAPE;
    const int64_t rows = seq * members, total = rows * heads;
    if (rows / members != seq || total / heads != rows || (total + 255) / 256 > 0x7fffffff) return MOSAIC_ERR_SHAPE;
    if (!logits || !w) return MOSAIC_ERR_NULL_POINTER;
    if ((reinterpret_cast<uintptr_t>(logits) & 1u) || (reinterpret_cast<uintptr_t>(w) & 1u)) return MOSAIC_ERR_ALIGNMENT;
    GateParams gp{static_cast<const bf16_t*>(logits), static_cast<bf16_t*>(w), rows, logits_row_stride, members, heads};
    void* args[] = {&gp};
    return status(hipLaunchKernel((const void*)gate_softmax_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                                  args, 0, static_cast<hipStream_t>(stream)));
}

int mosaic_swiglu_fwd(const void* h, int32_t dtype, int64_t rows, int32_t hidden, int64_t h_row_stride,
                      const void* noise, int32_t noise_rows, void* out, void* stream) {
    if (rows <= 0 || hidden <= 0) return MOSAIC_ERR_SHAPE;
    if (!valid_dtype(dtype)) return MOSAIC_ERR_UNSUPPORTED;
    if (hidden % 8) return MOSAIC_ERR_UNSUPPORTED;
    if (!h || !out) return MOSAIC_ERR_NULL_POINTER;
    if (noise && noise_rows <= 0) return MOSAIC_ERR_SHAPE;
    if (h_row_stride < 2 * (int64_t)hidden) return MOSAIC_ERR_SHAPE;
    if (!aligned16(h) || !aligned16(out) || !chunk_stride(h_row_stride, dtype)) return MOSAIC_ERR_ALIGNMENT;
    if (noise && !aligned16(noise)) return MOSAIC_ERR_ALIGNMENT;
    GluParams p{h, noise, out, rows, h_row_stride, hidden, noise_rows};
    hipStream_t s = static_cast<hipStream_t>(stream);
    return status(dtype == MOSAIC_DTYPE_BF16 ? launch_glu<bf16_t>(p, s) : launch_glu<float>(p, s));
}

}  // extern "C"
