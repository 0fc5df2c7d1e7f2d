// api.hip -- the extern "C" entry points of include/mosaic_bsa.h.
//
// Host side only: argument validation (before any launch), workspace layout, choice of the
// compressed-attention split count, and the launch sequence on the caller's stream:
//   pool (q, k, v -> pooled)  ->  cmp (compressed attention partials + selection scores)
//   ->  top-k (indices)  ->  attn (local + selected + merge)
// Nothing here allocates device memory or synchronises the host.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>

#include "bsa_common.h"
#include "mosaic_bsa.h"

using namespace mosaic;

// Workspace of mosaic_bsa_fwd_noalloc: a static device array, one copy per GPU, alive until the
// process ends.  Its host-side name is only a handle for hipGetSymbolAddress; kernels receive
// the device address that call returns (scratch_of_current_device).
static __device__ __align__(256) unsigned char scratch[MOSAIC_BSA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kAlign = 256;
constexpr int kMaxBlocksTopk = 8192;  // selection rows live in registers: 128 keys per lane
constexpr int kMaxGroup = 16;         // query heads per kv head (one wave each in cmp_kernel)

size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_bnhd(const mosaic_bnhd& t) {
    if (t.ptr == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(t.ptr) || (t.stride_b % 8) || (t.stride_n % 8) || (t.stride_h % 8)) return MOSAIC_ERR_ALIGNMENT;
    return MOSAIC_OK;
}

float resolve_scale(float s, int d) { return s > 0.f ? s : 1.f / std::sqrt((float)d); }

int check_heads(int Hq, int Hk) {
    if (Hq <= 0 || Hk <= 0 || Hq % Hk) return MOSAIC_ERR_HEADS;
    if (Hq / Hk > kMaxGroup) return MOSAIC_ERR_UNSUPPORTED;
    return MOSAIC_OK;
}

// Waves per attention workgroup: the whole GQA group when it is 1, 2 or 4 heads, otherwise
// groups of 4 (G a multiple of 4) or single heads.
int attn_waves(int G) {
    if (G == 1 || G == 2 || G == 4) return G;
    if (G % 4 == 0) return 4;
    if (G % 2 == 0) return 2;
    return 1;
}

// Key-range splits of the scores / compressed-attention pass.  Its tile loop is issue-bound
// at one wave per SIMD, so while the grid fits one workgroup per compute unit, more splits
// shorten every workgroup's walk; a second workgroup on a unit runs at about half speed and
// the grid then waits for that unit (Nside 64, 72 workgroups per split: 2 splits 14.0 us,
// 3 splits 11.7 us, 4 splits 13.9 us).  Larger grids keep two splits up to two workgroups per
// unit.  A pure function of the shape, so the workspace size does not depend on the device.
constexpr int kCmpSlots = 256;  // compute units of an MI355X
int choose_splits(int B, int nb, int Hk) {
    const int tt = (nb + 31) / 32;
    const int wgs = tt * Hk * B;
    if (wgs <= kCmpSlots) return std::max(1, std::min({kMaxSplits, kCmpSlots / wgs, tt}));
    return wgs < 2 * kCmpSlots && tt >= 2 ? 2 : 1;
}

struct Layout {
    int nb = 0, nb_pad = 0, nsplit = 1;
    size_t qc = 0, kfr = 0, vfr = 0, sbar = 0, idx = 0, kbnd = 0, opart = 0, ml = 0, ocmp = 0, tail = 0, total = 0;
};

bool uses_selection(int mode) { return mode == MOSAIC_BSA_FULL || mode == MOSAIC_BSA_NO_COMPRESSION; }
bool uses_compression(int mode) { return mode == MOSAIC_BSA_FULL || mode == MOSAIC_BSA_NO_SELECTION; }

int validate(const mosaic_bsa_args* a) {
    if (a == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (a->mode < MOSAIC_BSA_FULL || a->mode > MOSAIC_BSA_NO_SELECTION) return MOSAIC_ERR_MODE;
    if (a->batch <= 0 || a->seq_len <= 0) return MOSAIC_ERR_SHAPE;
    if (a->head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (int e = check_heads(a->num_q_heads, a->num_kv_heads)) return e;
    if (int e = check_bnhd(a->q)) return e;
    if (int e = check_bnhd(a->k)) return e;
    if (int e = check_bnhd(a->v)) return e;
    if (a->out == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(a->out)) return MOSAIC_ERR_ALIGNMENT;
    if (a->out_stride_b < 0 || a->out_stride_n < 0 || a->out_stride_b % 8 || a->out_stride_n % 8)
        return MOSAIC_ERR_ALIGNMENT;
    if ((int64_t)a->batch * a->seq_len * a->num_q_heads * kHeadDim >= ((int64_t)1 << 40)) return MOSAIC_ERR_SHAPE;
    if (a->block_attn_size <= 0 || a->block_attn_size % kTile || a->seq_len % a->block_attn_size)
        return MOSAIC_ERR_BLOCK_SIZE;
    if (a->mode == MOSAIC_BSA_LOCAL_ONLY) return MOSAIC_OK;
    if (a->weights == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (a->sparse_block_size <= 0 || a->sparse_block_size % kTile || a->seq_len % a->sparse_block_size)
        return MOSAIC_ERR_BLOCK_SIZE;
    const int nb = a->seq_len / a->sparse_block_size;
    if (a->sparse_block_count < 0 || a->sparse_block_count > nb) return MOSAIC_ERR_BLOCK_COUNT;
    if (uses_selection(a->mode)) {
        if (a->sparse_block_count == 0) return MOSAIC_ERR_BLOCK_COUNT;
        if (nb > kMaxBlocksTopk || nb > 65535) return MOSAIC_ERR_UNSUPPORTED;
        if (a->sparse_block_count > kMaxSelected) return MOSAIC_ERR_UNSUPPORTED;
    }
    return MOSAIC_OK;
}

Layout layout_of(const mosaic_bsa_args* a) {
    Layout L;
    if (a->mode == MOSAIC_BSA_LOCAL_ONLY) return L;
    const size_t B = a->batch, Hq = a->num_q_heads, Hk = a->num_kv_heads;
    L.nb = a->seq_len / a->sparse_block_size;
    L.nb_pad = (L.nb + 31) / 32 * 32;
    L.nsplit = choose_splits(a->batch, L.nb, a->num_kv_heads);
    const size_t nb = L.nb, nbp = L.nb_pad, K = a->sparse_block_count, U = L.nsplit;
    size_t off = 0;
    L.qc = off; off = align_up(off + B * nb * Hq * kHeadDim * 2);
    L.kfr = off; off = align_up(off + B * Hk * nbp * kHeadDim * 2);
    if (uses_compression(a->mode)) {
        L.vfr = off; off = align_up(off + B * Hk * nbp * kHeadDim * 2);
        L.opart = off; off = align_up(off + B * U * nb * Hq * kHeadDim * 4);
        L.ml = off; off = align_up(off + B * U * nb * Hq * 8);
        L.ocmp = off; off = align_up(off + B * nb * Hq * kHeadDim * 2);
    }
    if (uses_selection(a->mode)) {
        L.sbar = off; off = align_up(off + B * Hk * nb * nbp * 2);
        L.idx = off; off = align_up(off + B * nb * Hk * K * 4);
        L.kbnd = off; off = align_up(off + B * nb * Hk * 8 * 4);
        L.tail = off; off = align_up(off + 4);  // the attention kernel's dynamic-tail counter
    }
    L.total = off;
    return L;
}

AttnParams attn_params(const mosaic_bnhd& q, const mosaic_bnhd& k, const mosaic_bnhd& v, int B, int N,
                       int Hq, int Hk, float scale) {
    AttnParams p{};
    p.q = static_cast<const bf16_t*>(q.ptr); p.q_sb = q.stride_b; p.q_sn = q.stride_n; p.q_sh = q.stride_h;
    p.k = static_cast<const bf16_t*>(k.ptr); p.k_sb = k.stride_b; p.k_sn = k.stride_n; p.k_sh = k.stride_h;
    p.v = static_cast<const bf16_t*>(v.ptr); p.v_sb = v.stride_b; p.v_sn = v.stride_n; p.v_sh = v.stride_h;
    p.B = B; p.N = N; p.Hq = Hq; p.Hk = Hk; p.G = Hq / Hk;
    const int waves = attn_waves(p.G);
    p.head_groups = p.G / waves;
    p.qtiles = N / kTile;
    p.total_wgs = B * Hk * p.head_groups * p.qtiles;
    p.n_static = p.total_wgs;  // no dynamic tail unless set_dynamic_tail
    p.scale = scale;
    p.scale_log2 = scale * kLog2e;
    return p;
}

int launch_status(hipError_t e) { return e == hipSuccess ? MOSAIC_OK : MOSAIC_ERR_LAUNCH; }

// The attention kernel's dynamic tail (modes with a top-k pass, which zeroes the counter): the
// last kTailItems items are taken by kTailItems + kTailExtra workgroups launched after the
// static ones.  Launches of fewer than 4 * kTailItems items keep the static mapping.
#ifndef MOSAIC_TAIL_ITEMS
#define MOSAIC_TAIL_ITEMS 512
#endif
#ifndef MOSAIC_TAIL_EXTRA
#define MOSAIC_TAIL_EXTRA 512
#endif
constexpr int kTailItems = MOSAIC_TAIL_ITEMS, kTailExtra = MOSAIC_TAIL_EXTRA;
void set_dynamic_tail(AttnParams& p, int* ctr) {
    if (kTailItems <= 0 || p.total_wgs < 4 * kTailItems) return;
    p.tail_ctr = ctr;
    p.n_static = p.total_wgs - kTailItems;
    p.tail_wgs = kTailItems + kTailExtra;
}

// Device address of `scratch` on the current device, resolved once per device (each GPU holds
// its own copy of the array at its own address) and cached.
constexpr int kMaxDevices = 256;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

int scratch_of_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return MOSAIC_ERR_LAUNCH;
    if (dev >= kMaxDevices) return MOSAIC_ERR_UNSUPPORTED;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return MOSAIC_ERR_LAUNCH;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MOSAIC_OK;
}

int record(void* const* events, int i, hipStream_t s) {
    if (events == nullptr || events[i] == nullptr) return MOSAIC_OK;
    return launch_status(hipEventRecord(static_cast<hipEvent_t>(events[i]), s));
}

// Inputs of the fused RoPE path: fp32 cos / sin tables [N, 32] and the rotated q, k outputs
// (bf16 [B, N, H, 64] contiguous).
struct RopeIO {
    const float* cos;
    const float* sin;
    void* q_rot;
    void* k_rot;
};

// proj: the input side's projection kernel runs in place of the pooling pass (its q, k, v,
// weights and pooled outputs feed the later kernels; a's q / k / v / weights point at them)
// stages: bit k launches stage k (mosaic_bsa_stage); all four for a whole forward.
constexpr unsigned kAllStages = 0xfu;
int bsa_forward(const mosaic_bsa_args* a, void* ws, size_t ws_bytes, void* stream, void* const* events,
                const RopeIO* rope = nullptr, const ProjParams* proj = nullptr, unsigned stages = kAllStages) {
    if (int e = validate(a)) return e;
    auto run = [stages](int stage) { return (stages >> stage) & 1u; };
    // With RoPE, the modes with both local and selected branches rotate q inside the attention
    // kernel, so the rotated q is an optional output there; the other modes read it back.
    const bool q_in_kernel = a->mode == MOSAIC_BSA_FULL || a->mode == MOSAIC_BSA_NO_COMPRESSION;
    if (rope != nullptr) {
        if (!rope->cos || !rope->sin || !rope->k_rot || (!rope->q_rot && !q_in_kernel)) return MOSAIC_ERR_NULL_POINTER;
        if (!aligned16(rope->cos) || !aligned16(rope->sin) || !aligned16(rope->k_rot) ||
            (rope->q_rot && !aligned16(rope->q_rot)))
            return MOSAIC_ERR_ALIGNMENT;
    }
    const Layout L = layout_of(a);
    if (L.total > 0) {
        if (ws == nullptr || ws_bytes < L.total) return MOSAIC_ERR_WORKSPACE;
        if ((reinterpret_cast<uintptr_t>(ws) & (kAlign - 1)) != 0) return MOSAIC_ERR_WORKSPACE;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* w = static_cast<char*>(ws);
    const int B = a->batch, N = a->seq_len, Hq = a->num_q_heads, Hk = a->num_kv_heads;
    const float scale = resolve_scale(a->softmax_scale, a->head_dim);
    const bool sel = uses_selection(a->mode), cmp = uses_compression(a->mode);

    AttnParams ap = attn_params(a->q, a->k, a->v, B, N, Hq, Hk, scale);
    ap.out = static_cast<bf16_t*>(a->out);
    ap.out_sb = a->out_stride_b ? a->out_stride_b : (int64_t)N * Hq * kHeadDim;
    ap.out_sn = a->out_stride_n ? a->out_stride_n : (int64_t)Hq * kHeadDim;
    ap.bs_l = a->block_attn_size;
    ap.bs = a->mode == MOSAIC_BSA_LOCAL_ONLY ? kTile : a->sparse_block_size;
    ap.K = a->sparse_block_count;
    ap.nb = N / ap.bs;
    ap.w = static_cast<const bf16_t*>(a->weights);
    ap.w_ss = a->w_stride_s; ap.w_sb = a->w_stride_b; ap.w_sn = a->w_stride_n; ap.w_sh = a->w_stride_h;
    const int waves = attn_waves(ap.G);
    // With RoPE, the pooling pass rotates q and k (reading them once) and the later kernels
    // read the rotated copies.
    auto set_rope = [&](PoolParams& pp) {
        pp.rope_cos = rope->cos;
        pp.rope_sin = rope->sin;
        pp.rot[0] = static_cast<bf16_t*>(rope->q_rot);
        pp.rot[1] = static_cast<bf16_t*>(rope->k_rot);
    };
    auto use_rotated = [&]() {
        if (q_in_kernel) {
            ap.rope_cos = rope->cos;
            ap.rope_sin = rope->sin;
        } else {
            ap.q = static_cast<const bf16_t*>(rope->q_rot);
            ap.q_sb = (int64_t)N * Hq * kHeadDim; ap.q_sn = (int64_t)Hq * kHeadDim; ap.q_sh = kHeadDim;
        }
        ap.k = static_cast<const bf16_t*>(rope->k_rot);
        ap.k_sb = (int64_t)N * Hk * kHeadDim; ap.k_sn = (int64_t)Hk * kHeadDim; ap.k_sh = kHeadDim;
    };

    if (int e = record(events, 0, s)) return e;
    if (a->mode != MOSAIC_BSA_LOCAL_ONLY) {
        const bf16_t* qc = reinterpret_cast<const bf16_t*>(w + L.qc);

        PoolParams pp{};
        pp.x[0] = ap.q; pp.sb[0] = ap.q_sb; pp.sn[0] = ap.q_sn; pp.sh[0] = ap.q_sh; pp.heads[0] = Hq;
        pp.x[1] = ap.k; pp.sb[1] = ap.k_sb; pp.sn[1] = ap.k_sn; pp.sh[1] = ap.k_sh; pp.heads[1] = Hk;
        pp.out_bnhd[0] = reinterpret_cast<bf16_t*>(w + L.qc);
        pp.kfrag = reinterpret_cast<bf16_t*>(w + L.kfr);
        if (cmp) {
            pp.x[2] = ap.v; pp.sb[2] = ap.v_sb; pp.sn[2] = ap.v_sn; pp.sh[2] = ap.v_sh; pp.heads[2] = Hk;
            pp.vfrag = reinterpret_cast<bf16_t*>(w + L.vfr);
        }
        pp.B = B; pp.nb = L.nb; pp.nb_pad = L.nb_pad; pp.bs = a->sparse_block_size;
        if (sel) pp.kbnd = reinterpret_cast<float*>(w + L.kbnd);
        if (proj) {
            ProjParams jp = *proj;
            jp.bs = a->sparse_block_size; jp.nb = L.nb; jp.nb_pad = L.nb_pad;
            jp.qc = pp.out_bnhd[0]; jp.kfrag = pp.kfrag; jp.vfrag = pp.vfrag; jp.kbnd = pp.kbnd;
            if (run(MOSAIC_BSA_STAGE_POOL))
                if (int e = launch_status(launch_proj(jp, s))) return e;
        } else {
            if (rope) set_rope(pp);
            if (run(MOSAIC_BSA_STAGE_POOL))
                if (int e = launch_status(launch_pool(pp, s))) return e;
            if (rope) use_rotated();
        }
        if (int e = record(events, 1, s)) return e;

        CmpParams cp{};
        cp.qc = qc; cp.q_sb = (int64_t)L.nb * Hq * kHeadDim; cp.q_sn = (int64_t)Hq * kHeadDim; cp.q_sh = kHeadDim;
        cp.kfr = reinterpret_cast<const bf16_t*>(w + L.kfr);
        cp.vfr = cmp ? reinterpret_cast<const bf16_t*>(w + L.vfr) : nullptr;
        cp.sbar = sel ? reinterpret_cast<bf16_t*>(w + L.sbar) : nullptr;
        cp.opart = cmp ? reinterpret_cast<float*>(w + L.opart) : nullptr;
        cp.ml = cmp ? reinterpret_cast<float2*>(w + L.ml) : nullptr;
        cp.B = B; cp.nb = L.nb; cp.nb_pad = L.nb_pad; cp.Hq = Hq; cp.Hk = Hk; cp.G = Hq / Hk;
        cp.nsplit = L.nsplit; cp.ut_total = L.nb_pad / 32;
        cp.scale_log2 = scale * kLog2e;
        // one split: the scores pass writes the compressed-branch output, nothing to combine
        cp.ocmp = (cmp && L.nsplit == 1) ? reinterpret_cast<bf16_t*>(w + L.ocmp) : nullptr;
        if (run(MOSAIC_BSA_STAGE_CMP))
            if (int e = launch_status(launch_cmp(cp, sel, cmp, s))) return e;
        if (int e = record(events, 2, s)) return e;

        CombineParams cb{};
        cb.opart = cp.opart; cb.ml = cp.ml; cb.nsplit = L.nsplit; cb.Hq = Hq;
        cb.ocmp = cmp ? reinterpret_cast<bf16_t*>(w + L.ocmp) : nullptr;
        if (sel) {
            TopkParams tp{};
            tp.G = Hq / Hk;
            tp.cmb = cb;
            if (cp.ocmp != nullptr) tp.cmb.ocmp = nullptr;
            tp.sbar = cp.sbar;
            tp.idx32 = reinterpret_cast<int32_t*>(w + L.idx);
            tp.idx64 = a->block_indices_out;
            tp.B = B; tp.nb = L.nb; tp.nb_pad = L.nb_pad; tp.Hk = Hk; tp.K = a->sparse_block_count;
            tp.rows = B * Hk * L.nb;
            tp.zero_ctr = reinterpret_cast<int*>(w + L.tail);
            set_dynamic_tail(ap, tp.zero_ctr);
            if (run(MOSAIC_BSA_STAGE_TOPK))
                if (int e = launch_status(launch_topk(tp, s))) return e;
            ap.idx = tp.idx32;
            ap.kbnd = pp.kbnd;
        } else if (cmp && cp.ocmp == nullptr) {
            if (run(MOSAIC_BSA_STAGE_TOPK))
                if (int e = launch_status(launch_combine(cb, B, L.nb, s))) return e;
        }
        if (int e = record(events, 3, s)) return e;
        ap.ocmp = cb.ocmp;
    } else {
        if (proj) {  // local attention only: the projection without pooling
            if (run(MOSAIC_BSA_STAGE_POOL))
                if (int e = launch_status(launch_proj(*proj, s))) return e;
        } else if (rope) {  // local attention only: the pooling pass just rotates q and k
            PoolParams pp{};
            pp.x[0] = ap.q; pp.sb[0] = ap.q_sb; pp.sn[0] = ap.q_sn; pp.sh[0] = ap.q_sh; pp.heads[0] = Hq;
            pp.x[1] = ap.k; pp.sb[1] = ap.k_sb; pp.sn[1] = ap.k_sn; pp.sh[1] = ap.k_sh; pp.heads[1] = Hk;
            pp.B = B; pp.nb = N / kTile; pp.nb_pad = pp.nb; pp.bs = kTile;
            set_rope(pp);
            if (run(MOSAIC_BSA_STAGE_POOL))
                if (int e = launch_status(launch_pool(pp, s))) return e;
            use_rotated();
        }
        if (int e = record(events, 1, s)) return e;
        if (int e = record(events, 2, s)) return e;
        if (int e = record(events, 3, s)) return e;
    }
    static const int mode_map[4] = {kModeFull, kModeLocalOnly, kModeNoCompression, kModeNoSelection};
    if (run(MOSAIC_BSA_STAGE_ATTN))
        if (int e = launch_status(launch_attn(ap, mode_map[a->mode], false, waves, s))) return e;
    return record(events, 4, s);
}

}  // namespace

extern "C" {

size_t mosaic_bsa_workspace_size(const mosaic_bsa_args* args) {
    if (validate(args) != MOSAIC_OK) return 0;
    return layout_of(args).total;
}

int mosaic_bsa_fwd(const mosaic_bsa_args* args, void* workspace, size_t workspace_bytes, void* stream) {
    return bsa_forward(args, workspace, workspace_bytes, stream, nullptr);
}

int mosaic_bsa_fwd_noalloc(const mosaic_bsa_args* args, void* stream) {
    if (int e = validate(args)) return e;
    const size_t need = layout_of(args).total;
    if (need > MOSAIC_BSA_NOALLOC_SCRATCH_BYTES) return MOSAIC_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (need > 0)
        if (int e = scratch_of_current_device(&ws)) return e;
    return bsa_forward(args, ws, need, stream, nullptr);
}

int mosaic_bsa_fwd_profiled(const mosaic_bsa_args* args, void* workspace, size_t workspace_bytes, void* stream,
                            void* const* events) {
    return bsa_forward(args, workspace, workspace_bytes, stream, events);
}

int mosaic_bsa_fwd_stage(const mosaic_bsa_args* args, void* workspace, size_t workspace_bytes, void* stream,
                         int stage) {
    if (stage < MOSAIC_BSA_STAGE_POOL || stage > MOSAIC_BSA_STAGE_ATTN) return MOSAIC_ERR_UNSUPPORTED;
    return bsa_forward(args, workspace, workspace_bytes, stream, nullptr, nullptr, nullptr, 1u << stage);
}

int mosaic_bsa_fwd_rope(const mosaic_bsa_args* args, const float* rope_cos, const float* rope_sin, void* q_rot,
                        void* k_rot, void* workspace, size_t workspace_bytes, void* stream) {
    const RopeIO rope{rope_cos, rope_sin, q_rot, k_rot};
    return bsa_forward(args, workspace, workspace_bytes, stream, nullptr, &rope);
}

int mosaic_bsa_fwd_proj(const mosaic_bsa_args* args, const mosaic_proj_args* proj, void* workspace,
                        size_t workspace_bytes, void* stream) {
    if (args == nullptr || proj == nullptr) return MOSAIC_ERR_NULL_POINTER;
    const mosaic_proj_args& j = *proj;
    if (!j.x || !j.weight || !j.q || !j.k || !j.v) return MOSAIC_ERR_NULL_POINTER;
    const bool local = args->mode == MOSAIC_BSA_LOCAL_ONLY;
    if (!local && !j.weights) return MOSAIC_ERR_NULL_POINTER;
    if ((j.rope_cos == nullptr) != (j.rope_sin == nullptr)) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(j.x) || !aligned16(j.weight) || !aligned16(j.q) || !aligned16(j.k) || !aligned16(j.v) ||
        (j.rope_cos && (!aligned16(j.rope_cos) || !aligned16(j.rope_sin))) || j.x_stride_n % 8 || j.x_stride_b % 8)
        return MOSAIC_ERR_ALIGNMENT;
    const int32_t B = args->batch, N = args->seq_len, Hq = args->num_q_heads, Hk = args->num_kv_heads;
    if (B <= 0 || N <= 0 || j.dim <= 0 || j.x_stride_n < 0 || j.x_stride_b < 0) return MOSAIC_ERR_SHAPE;
    if (int e = check_heads(Hq, Hk)) return e;
    if (args->head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (j.dim % 128 || N % 256 || (!local && 3 * Hq > 64)) return MOSAIC_ERR_UNSUPPORTED;
    if (!local && args->sparse_block_size != 64 && args->sparse_block_size != 128) return MOSAIC_ERR_UNSUPPORTED;
    const int groups = Hq + 2 * Hk + (local ? 0 : 1);
    const int n_tiles = (groups + 3) / 4;
    if (j.weight_rows != 256 * n_tiles) return MOSAIC_ERR_SHAPE;
    // every row the kernel reads: x rows up to (N - 1, B - 1), weight rows up to weight_rows
    if ((int64_t)(N - 1) * j.x_stride_n + (int64_t)(B - 1) * j.x_stride_b + j.dim >= ((int64_t)1 << 40))
        return MOSAIC_ERR_SHAPE;
    if (j.x_stride_n >= ((int64_t)1 << 27) || j.dim >= (1 << 27))
        return MOSAIC_ERR_UNSUPPORTED;   // per-lane byte offsets within 8 rows are 32-bit
    mosaic_bsa_args a = *args;
    a.q = mosaic_bnhd{j.q, (int64_t)N * Hq * kHeadDim, (int64_t)Hq * kHeadDim, kHeadDim};
    a.k = mosaic_bnhd{j.k, (int64_t)N * Hk * kHeadDim, (int64_t)Hk * kHeadDim, kHeadDim};
    a.v = mosaic_bnhd{j.v, (int64_t)N * Hk * kHeadDim, (int64_t)Hk * kHeadDim, kHeadDim};
    a.weights = local ? nullptr : j.weights;
    a.w_stride_s = 1; a.w_stride_h = 3; a.w_stride_n = (int64_t)Hq * 3; a.w_stride_b = (int64_t)N * Hq * 3;
    ProjParams p{};
    p.x = static_cast<const bf16_t*>(j.x); p.x_sn = j.x_stride_n; p.x_sb = j.x_stride_b;
    p.w = static_cast<const bf16_t*>(j.weight);
    p.S = N; p.B = B; p.D = j.dim; p.Hq = Hq; p.Hk = Hk; p.gates = local ? 0 : 1; p.n_tiles = n_tiles;
    p.rope_cos = j.rope_cos; p.rope_sin = j.rope_sin;
    p.q = static_cast<bf16_t*>(j.q); p.k = static_cast<bf16_t*>(j.k); p.v = static_cast<bf16_t*>(j.v);
    p.wts = static_cast<bf16_t*>(j.weights);
    return bsa_forward(&a, workspace, workspace_bytes, stream, nullptr, nullptr, &p);
}

// The selected branch alone; with kbnd (the key-norm bounds of k's blocks, [B, nb, Hk, 8])
// a workgroup whose logits are all within the bound takes the bounded path.
static int sparse_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, const int64_t* block_indices, int32_t batch,
                      int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t block_size, int32_t block_count, float softmax_scale, void* out, float* lse,
                      float* kbnd, void* stream) {
    if (batch <= 0 || seq_len <= 0 || block_count <= 0) return block_count <= 0 ? MOSAIC_ERR_BLOCK_COUNT : MOSAIC_ERR_SHAPE;
    if (head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (int e = check_heads(num_q_heads, num_kv_heads)) return e;
    if (int e = check_bnhd(q)) return e;
    if (int e = check_bnhd(k)) return e;
    if (int e = check_bnhd(v)) return e;
    if (block_indices == nullptr || out == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(out)) return MOSAIC_ERR_ALIGNMENT;
    if (block_size <= 0 || block_size % kTile || seq_len % block_size) return MOSAIC_ERR_BLOCK_SIZE;
    if (block_count > kMaxSelected) return MOSAIC_ERR_UNSUPPORTED;
    AttnParams ap = attn_params(q, k, v, batch, seq_len, num_q_heads, num_kv_heads,
                                resolve_scale(softmax_scale, head_dim));
    ap.out = static_cast<bf16_t*>(out);
    ap.out_sb = (int64_t)seq_len * num_q_heads * kHeadDim;
    ap.out_sn = (int64_t)num_q_heads * kHeadDim;
    ap.lse = lse;
    ap.idx = block_indices;
    ap.bs = block_size;
    ap.bs_l = block_size;
    ap.K = block_count;
    ap.nb = seq_len / block_size;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kbnd != nullptr) {   // k's block bounds: the pooling pass over k alone, bounds only
        PoolParams pp{};
        pp.x[1] = ap.k; pp.sb[1] = ap.k_sb; pp.sn[1] = ap.k_sn; pp.sh[1] = ap.k_sh; pp.heads[1] = num_kv_heads;
        pp.kbnd = kbnd;
        pp.B = batch; pp.nb = ap.nb; pp.nb_pad = ap.nb; pp.bs = block_size;
        if (int e = launch_status(launch_pool(pp, s))) return e;
        ap.kbnd = kbnd;
    }
    return launch_status(launch_attn(ap, kModeSelectedOnly, true, attn_waves(ap.G), s));
}

int mosaic_sparse_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, const int64_t* block_indices,
                           int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t block_size, int32_t block_count, float softmax_scale,
                           void* out, float* lse, void* stream) {
    return sparse_fwd(q, k, v, block_indices, batch, seq_len, num_q_heads, num_kv_heads, head_dim, block_size,
                      block_count, softmax_scale, out, lse, nullptr, stream);
}

size_t mosaic_sparse_attn_fwd_workspace_size(int32_t batch, int32_t seq_len, int32_t num_kv_heads,
                                             int32_t block_size) {
    if (batch <= 0 || seq_len <= 0 || num_kv_heads <= 0 || block_size <= 0 || seq_len % block_size) return 0;
    return (size_t)batch * (seq_len / block_size) * num_kv_heads * 8 * sizeof(float);
}

int mosaic_sparse_attn_fwd_ws(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, const int64_t* block_indices,
                              int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t block_size, int32_t block_count, float softmax_scale,
                              void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
    const size_t need = mosaic_sparse_attn_fwd_workspace_size(batch, seq_len, num_kv_heads, block_size);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
        return MOSAIC_ERR_WORKSPACE;
    return sparse_fwd(q, k, v, block_indices, batch, seq_len, num_q_heads, num_kv_heads, head_dim, block_size,
                      block_count, softmax_scale, out, lse, need > 0 ? static_cast<float*>(workspace) : nullptr, stream);
}

int mosaic_block_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, int32_t batch, int32_t seq_len,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          float softmax_scale, void* out, void* stream) {
    mosaic_bsa_args a{};
    a.batch = batch; a.seq_len = seq_len; a.num_q_heads = num_q_heads; a.num_kv_heads = num_kv_heads;
    a.head_dim = head_dim; a.block_attn_size = block_size; a.mode = MOSAIC_BSA_LOCAL_ONLY;
    a.softmax_scale = softmax_scale; a.q = q; a.k = k; a.v = v; a.out = out;
    return bsa_forward(&a, nullptr, 0, stream, nullptr);
}

int mosaic_dense_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, int32_t batch, int32_t seq_len,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
                          void* out, void* stream) {
    return mosaic_block_attn_fwd(q, k, v, batch, seq_len, num_q_heads, num_kv_heads, head_dim, seq_len,
                                 softmax_scale, out, stream);
}

int mosaic_pool_mean_fwd(mosaic_bnhd x, int32_t batch, int32_t seq_len, int32_t num_heads, int32_t head_dim,
                         int32_t block_size, void* out, void* stream) {
    if (batch <= 0 || seq_len <= 0 || num_heads <= 0) return MOSAIC_ERR_SHAPE;
    if (head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (int e = check_bnhd(x)) return e;
    if (out == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(out)) return MOSAIC_ERR_ALIGNMENT;
    if (block_size <= 0 || block_size % 8 || seq_len % block_size) return MOSAIC_ERR_BLOCK_SIZE;
    PoolParams pp{};
    pp.x[0] = static_cast<const bf16_t*>(x.ptr);
    pp.sb[0] = x.stride_b; pp.sn[0] = x.stride_n; pp.sh[0] = x.stride_h; pp.heads[0] = num_heads;
    pp.out_bnhd[0] = static_cast<bf16_t*>(out);
    pp.B = batch; pp.nb = seq_len / block_size; pp.nb_pad = pp.nb; pp.bs = block_size;
    return launch_status(launch_pool(pp, static_cast<hipStream_t>(stream)));
}

int mosaic_knn_interp_fwd(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors, const float* rel_pos,
                          const void* w_q, int32_t num_from, int32_t num_to, int32_t batch, int32_t num_heads,
                          int32_t head_dim, int32_t num_neighbors, float scale, void* out, void* stream) {
    return mosaic_knn_interp_fwd_ordered(k, v, neighbors, rel_pos, w_q, nullptr, num_from, num_to, batch,
                                         num_heads, head_dim, num_neighbors, scale, out, stream);
}

int mosaic_knn_interp_fwd_ordered(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors, const float* rel_pos,
                                  const void* w_q, const int32_t* target_order, int32_t num_from, int32_t num_to,
                                  int32_t batch, int32_t num_heads, int32_t head_dim, int32_t num_neighbors,
                                  float scale, void* out, void* stream) {
    return mosaic_knn_interp_fwd_ex(k, v, neighbors, rel_pos, w_q, target_order, nullptr, num_from, num_to, batch,
                                    num_heads, head_dim, num_neighbors, scale, MOSAIC_KNN_ROUND_PRODUCTS, out, stream);
}

int mosaic_knn_interp_fwd_ex(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors, const float* rel_pos,
                             const void* w_q, const int32_t* target_order, const mosaic_knn_tiles* tiles,
                             int32_t num_from, int32_t num_to, int32_t batch, int32_t num_heads, int32_t head_dim,
                             int32_t num_neighbors, float scale, uint32_t flags, void* out, void* stream) {
    if (flags & ~MOSAIC_KNN_ROUND_PRODUCTS) return MOSAIC_ERR_MODE;
    const bool tiled = tiles != nullptr && !(flags & MOSAIC_KNN_ROUND_PRODUCTS);
    if (tiled) {
        if (tiles->start == nullptr || tiles->src == nullptr || tiles->nsrc == nullptr || tiles->slot == nullptr)
            return MOSAIC_ERR_NULL_POINTER;
        if (tiles->num_tiles <= 0 || tiles->max_rows <= 0 || tiles->max_rows % 8 || tiles->max_rows > kKnnTileRows)
            return MOSAIC_ERR_SHAPE;
        for (const void* t : {(const void*)tiles->start, (const void*)tiles->src, (const void*)tiles->nsrc,
                              (const void*)tiles->slot})
            if (reinterpret_cast<uintptr_t>(t) % 4) return MOSAIC_ERR_ALIGNMENT;
    }
    if (num_from <= 0 || num_to <= 0 || batch <= 0 || num_heads <= 0) return MOSAIC_ERR_SHAPE;
    if (head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (num_neighbors <= 0 || num_neighbors > 32) return MOSAIC_ERR_BLOCK_COUNT;
    if (int e = check_bnhd(k)) return e;
    if (int e = check_bnhd(v)) return e;
    if ((neighbors == nullptr && !tiled) || rel_pos == nullptr || w_q == nullptr || out == nullptr)
        return MOSAIC_ERR_NULL_POINTER;
    if (!aligned16(out) || !aligned16(w_q) || reinterpret_cast<uintptr_t>(rel_pos) % 4 ||
        reinterpret_cast<uintptr_t>(neighbors) % 4 || reinterpret_cast<uintptr_t>(target_order) % 4)
        return MOSAIC_ERR_ALIGNMENT;
    InterpParams p{};
    p.target_order = target_order;
    p.k = static_cast<const bf16_t*>(k.ptr); p.k_sn = k.stride_n; p.k_sb = k.stride_b; p.k_sh = k.stride_h;
    p.v = static_cast<const bf16_t*>(v.ptr); p.v_sn = v.stride_n; p.v_sb = v.stride_b; p.v_sh = v.stride_h;
    p.neighbors = neighbors;
    p.rel_pos = rel_pos;
    p.w_q = static_cast<const bf16_t*>(w_q);
    p.out = static_cast<bf16_t*>(out);
    p.S_from = num_from; p.S_to = num_to; p.B = batch; p.H = num_heads; p.K = num_neighbors;
    p.scale = resolve_scale(scale, head_dim);
    int exp2 = 0;
    p.scale_pow2 = std::isfinite(p.scale) && p.scale >= 0x1p-126f && std::frexp(p.scale, &exp2) == 0.5f;
    p.scale_log2e = p.scale * kLog2e;
    p.round_products = (flags & MOSAIC_KNN_ROUND_PRODUCTS) != 0;
    if (tiled && knn_tiled_supported(p)) {
        KnnTiles t{};
        t.start = tiles->start; t.src = tiles->src; t.nsrc = tiles->nsrc; t.slot = tiles->slot;
        t.n = tiles->num_tiles; t.rows = tiles->max_rows;
        return launch_status(launch_knn_attn_tiled(p, t, static_cast<hipStream_t>(stream)));
    }
    if (neighbors == nullptr) return MOSAIC_ERR_NULL_POINTER;  // tiles given, but not usable here
    return launch_status(launch_knn_attn(p, static_cast<hipStream_t>(stream)));
}

// scores [B, Hk, nb, nb_pad] bf16, then k_cmp in operand order [B, Hk, nb_pad, 64] bf16
size_t topk_scores_bytes(size_t batch, size_t num_blocks, size_t num_kv_heads) {
    const size_t nbp = (num_blocks + 31) / 32 * 32;
    return align_up(batch * num_kv_heads * num_blocks * nbp * 2);
}

size_t mosaic_attn_topk_workspace_size(int32_t batch, int32_t num_blocks, int32_t num_kv_heads) {
    if (batch <= 0 || num_blocks <= 0 || num_kv_heads <= 0) return 0;
    const size_t nbp = (size_t)(num_blocks + 31) / 32 * 32;
    return topk_scores_bytes(batch, num_blocks, num_kv_heads) + align_up((size_t)batch * num_kv_heads * nbp * kHeadDim * 2);
}

int mosaic_attn_topk_fwd(mosaic_bnhd q_cmp, mosaic_bnhd k_cmp, int32_t batch, int32_t num_blocks,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_count,
                         int64_t* indices_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (batch <= 0 || num_blocks <= 0) return MOSAIC_ERR_SHAPE;
    if (head_dim != kHeadDim) return MOSAIC_ERR_HEAD_DIM;
    if (int e = check_heads(num_q_heads, num_kv_heads)) return e;
    if (int e = check_bnhd(q_cmp)) return e;
    if (int e = check_bnhd(k_cmp)) return e;
    if (indices_out == nullptr) return MOSAIC_ERR_NULL_POINTER;
    if (block_count <= 0 || block_count > num_blocks) return MOSAIC_ERR_BLOCK_COUNT;
    if (num_blocks > kMaxBlocksTopk) return MOSAIC_ERR_UNSUPPORTED;
    const size_t need = mosaic_attn_topk_workspace_size(batch, num_blocks, num_kv_heads);
    if (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & (kAlign - 1)))
        return MOSAIC_ERR_WORKSPACE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nb_pad = (num_blocks + 31) / 32 * 32;
    // k_cmp into operand order: the pooling kernel with blocks of one token (an exact copy)
    bf16_t* kfr = reinterpret_cast<bf16_t*>(static_cast<char*>(workspace) + topk_scores_bytes(batch, num_blocks, num_kv_heads));
    PoolParams pp{};
    pp.x[1] = static_cast<const bf16_t*>(k_cmp.ptr);
    pp.sb[1] = k_cmp.stride_b; pp.sn[1] = k_cmp.stride_n; pp.sh[1] = k_cmp.stride_h; pp.heads[1] = num_kv_heads;
    pp.kfrag = kfr;
    pp.B = batch; pp.nb = num_blocks; pp.nb_pad = nb_pad; pp.bs = 1;
    if (int e = launch_status(launch_pool(pp, s))) return e;
    CmpParams cp{};
    cp.qc = static_cast<const bf16_t*>(q_cmp.ptr); cp.q_sb = q_cmp.stride_b; cp.q_sn = q_cmp.stride_n; cp.q_sh = q_cmp.stride_h;
    cp.kfr = kfr;
    cp.sbar = static_cast<bf16_t*>(workspace);
    cp.B = batch; cp.nb = num_blocks; cp.nb_pad = nb_pad; cp.Hq = num_q_heads; cp.Hk = num_kv_heads;
    cp.G = num_q_heads / num_kv_heads;
    cp.nsplit = choose_splits(batch, num_blocks, num_kv_heads);
    cp.ut_total = nb_pad / 32;
    if (int e = launch_status(launch_cmp(cp, true, false, s))) return e;
    TopkParams tp{};
    tp.sbar = cp.sbar; tp.idx64 = indices_out;
    tp.B = batch; tp.nb = num_blocks; tp.nb_pad = nb_pad; tp.Hk = num_kv_heads; tp.K = block_count;
    tp.rows = batch * num_kv_heads * num_blocks;
    tp.G = cp.G;
    return launch_status(launch_topk(tp, s));
}

const char* mosaic_bsa_strerror(int status) {
    switch (status) {
        case MOSAIC_OK: return "ok";
        case MOSAIC_ERR_NULL_POINTER: return "a required pointer is NULL";
        case MOSAIC_ERR_HEAD_DIM: return "head_dim must be 64";
        case MOSAIC_ERR_HEADS: return "num_q_heads must be a positive multiple of num_kv_heads";
        case MOSAIC_ERR_BLOCK_SIZE: return "block sizes must be positive multiples of 64 that divide seq_len";
        case MOSAIC_ERR_BLOCK_COUNT: return "sparse_block_count out of range";
        case MOSAIC_ERR_WORKSPACE: return "workspace missing, too small or not 256-byte aligned";
        case MOSAIC_ERR_ALIGNMENT: return "bf16 rows must be 16-byte aligned (pointer and strides multiples of 8 elements)";
        case MOSAIC_ERR_SHAPE: return "invalid sizes";
        case MOSAIC_ERR_LAUNCH: return "the HIP runtime rejected a kernel launch or call";
        case MOSAIC_ERR_MODE: return "unknown mode";
        case MOSAIC_ERR_UNSUPPORTED: return "outside the library's limits (query heads per kv head <= 16, blocks <= 8192, selected blocks <= 1024)";
        case MOSAIC_ERR_SCRATCH_LIMIT: return "the request needs more workspace than the static scratch of mosaic_bsa_fwd_noalloc (128 MiB)";
        default: return "unknown status";
    }
}

int mosaic_bsa_abi_version(void) { return MOSAIC_BSA_ABI_VERSION; }

}  // extern "C"
