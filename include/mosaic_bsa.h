/*
 * mosaic_bsa.h -- C ABI of the MI355X (gfx950) block-sparse attention library.
 *
 * The library computes Mosaic's three-branch block-sparse attention forward on HEALPix
 * nested-order sequences: local attention inside contiguous blocks, compressed attention
 * between mean-pooled blocks, top-k block selection with attention over the selected key
 * blocks, and the gated merge of the three.  All entry points are asynchronous on the given
 * HIP stream, allocate nothing, never synchronise the host, and validate their arguments
 * before any launch.  Tensors are device pointers; bf16 tensors of shape [B, N, H, d] are
 * described by element strides for the batch, token and head dimensions, with the head_dim
 * dimension contiguous.  head_dim must be 64.
 *
 * Every entry point returns a mosaic_status (0 = success); mosaic_bsa_strerror() names it.
 */
#ifndef MOSAIC_BSA_H
#define MOSAIC_BSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOSAIC_BSA_ABI_VERSION 10

#if defined(__GNUC__) || defined(__clang__)
#define MOSAIC_API __attribute__((visibility("default")))
#else
#define MOSAIC_API
#endif

typedef enum {
    MOSAIC_OK = 0,
    MOSAIC_ERR_NULL_POINTER = 1,   /* a required pointer is NULL                          */
    MOSAIC_ERR_HEAD_DIM = 2,       /* head_dim != 64                                      */
    MOSAIC_ERR_HEADS = 3,          /* num_q_heads not a positive multiple of num_kv_heads */
    MOSAIC_ERR_BLOCK_SIZE = 4,     /* block sizes not multiples of 64 / not dividing N    */
    MOSAIC_ERR_BLOCK_COUNT = 5,    /* sparse_block_count < 0 or > number of blocks        */
    MOSAIC_ERR_WORKSPACE = 6,      /* workspace missing, too small or misaligned          */
    MOSAIC_ERR_ALIGNMENT = 7,      /* bf16 rows not 16-byte aligned                       */
    MOSAIC_ERR_SHAPE = 8,          /* non-positive or too large sizes                     */
    MOSAIC_ERR_LAUNCH = 9,         /* the HIP runtime rejected a kernel launch            */
    MOSAIC_ERR_MODE = 10,          /* unknown mode                                        */
    MOSAIC_ERR_UNSUPPORTED = 11,   /* valid request outside the library's limits          */
    MOSAIC_ERR_SCRATCH_LIMIT = 12  /* mosaic_bsa_fwd_noalloc: workspace > static scratch  */
} mosaic_status;

/* Branch combination, matching mosaic_attn_func (primitives.py:54-89). */
typedef enum {
    MOSAIC_BSA_FULL = 0,           /* o_ba*w0 + o_cmp*w1 + o_slc*w2           (:86-89) */
    MOSAIC_BSA_LOCAL_ONLY = 1,     /* block_attn_only: o_ba                  (:62-63) */
    MOSAIC_BSA_NO_COMPRESSION = 2, /* (o_ba*w0 + o_slc*w2) / (w0+w2+1e-8)    (:68-74) */
    MOSAIC_BSA_NO_SELECTION = 3    /* sparse_block_count == 0:
                                      (o_ba*w0 + o_cmp*w1) / (w0+w1+1e-8)    (:80-84) */
} mosaic_bsa_mode;

/* Element types of the model-level elementwise entry points. */
typedef enum {
    MOSAIC_DTYPE_F32 = 0,
    MOSAIC_DTYPE_BF16 = 1
} mosaic_dtype;

/* A bf16 [B, N, H, 64] tensor: element strides of b, n and h; head_dim stride is 1. */
typedef struct {
    const void* ptr;
    int64_t stride_b, stride_n, stride_h;
} mosaic_bnhd;

/*
 * Arguments of the full forward.  Replaces the Python function
 *   mosaic_attn_func(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size,
 *                    sparse_block_count, block_attn_only, no_compression)
 * (primitives.py:54-89) including the helpers it calls: block_attention (:28-32), the
 * einops mean pooling (:65-66,76), flash_attn_func on the pooled blocks (:77-78), attn_topk
 * (:35-51) and mosaic_sparse_attn (ops.py:557-566).
 */
typedef struct {
    int32_t batch, seq_len, num_q_heads, num_kv_heads, head_dim;
    int32_t block_attn_size;       /* local block (multiple of 64, divides seq_len)          */
    int32_t sparse_block_size;     /* pooling / selection block (multiple of 64, divides N)  */
    int32_t sparse_block_count;    /* top-k blocks per query block                           */
    int32_t mode;                  /* mosaic_bsa_mode                                        */
    float softmax_scale;           /* <= 0 selects head_dim^-0.5 (flash-attn / ops.py:565)   */
    mosaic_bnhd q, k, v;
    /* weight_ba_cmp_slc, bf16 [3, B, N, Hq(, 1)] with arbitrary element strides; unused
       (may be NULL) in MOSAIC_BSA_LOCAL_ONLY mode. */
    const void* weights;
    int64_t w_stride_s, w_stride_b, w_stride_n, w_stride_h;
    void* out;                     /* bf16 [B, N, Hq, 64]; heads and head_dim contiguous     */
    int64_t* block_indices_out;    /* optional: int64 [B, N/bs, Hk, K] selected blocks       */
    /* Element strides of out's batch and token dimensions; 0 selects the contiguous
       N*Hq*64 / Hq*64.  A caller whose next step wants sequence-first rows ([N, B, Hq*64],
       the reference's 'b s h d -> s b (h d)' before to_o, primitives.py:207) passes
       out_stride_b = Hq*64 and out_stride_n = B*Hq*64.  Multiples of 8, 16-byte rows. */
    int64_t out_stride_b, out_stride_n;
} mosaic_bsa_args;

/* Bytes of device workspace mosaic_bsa_fwd needs for these arguments (256-byte aligned). */
MOSAIC_API size_t mosaic_bsa_workspace_size(const mosaic_bsa_args* args);

/* Full forward (primitives.py:54-89).  workspace: device memory of at least
   mosaic_bsa_workspace_size(args) bytes, 256-byte aligned.  stream: hipStream_t. */
MOSAIC_API int mosaic_bsa_fwd(const mosaic_bsa_args* args, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Size of the static device scratch that mosaic_bsa_fwd_noalloc uses as its workspace. */
#define MOSAIC_BSA_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

/* mosaic_bsa_fwd without a workspace argument, for callers that cannot allocate device memory
   (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
   counterpart in the reference.  The caller still passes inputs and outputs; the workspace is
   a static device array of MOSAIC_BSA_NOALLOC_SCRATCH_BYTES, one copy per GPU, held from the
   library's load until the process ends.  Its address is resolved once per device, on the
   first call with that device current; the call runs on the current device, and stream must
   belong to it.  Nothing is allocated and nothing synchronises the host.  A request whose
   mosaic_bsa_workspace_size() exceeds the scratch returns MOSAIC_ERR_SCRATCH_LIMIT before any
   launch (128 MiB covers e.g. N = 196608 with 12/3 heads and 64-token blocks, or 24 members of
   N = 12288 with 16/4 heads).  Every call on one GPU shares that GPU's array, which keeps the
   last call's contents: calls that overlap on one GPU (unordered streams, or threads) race
   and corrupt each other's results.  HIP loads the library's code object on a device (and
   places the static array there) at the first launch of any library kernel on it: make one
   call on each device before capturing a HIP graph, so that the load and the address lookup
   do not happen under capture. */
MOSAIC_API int mosaic_bsa_fwd_noalloc(const mosaic_bsa_args* args, void* stream);

/* As mosaic_bsa_fwd, recording events[0..4] (hipEvent_t) on the stream before the pooling
   kernel, before the compressed/score kernel, before the top-k kernel, before the attention
   kernel and after it, so a caller can time each kernel.  No reference counterpart: it is
   the measurement hook of the benchmark. */
MOSAIC_API int mosaic_bsa_fwd_profiled(const mosaic_bsa_args* args, void* workspace,
                            size_t workspace_bytes, void* stream, void* const* events);

/* Stages of the full forward, in launch order (mosaic_bsa_fwd_stage). */
typedef enum {
    MOSAIC_BSA_STAGE_POOL = 0,   /* pooling (with RoPE where the entry fuses it) */
    MOSAIC_BSA_STAGE_CMP = 1,    /* compressed attention partials + selection scores */
    MOSAIC_BSA_STAGE_TOPK = 2,   /* top-k selection + split combine (combine alone without selection) */
    MOSAIC_BSA_STAGE_ATTN = 3    /* fused local + selected attention with the merge */
} mosaic_bsa_stage;

/* One stage of mosaic_bsa_fwd alone: the same validation, then only that stage's launch,
   reading what the earlier stages left in the workspace.  The workspace must hold the
   results of a complete mosaic_bsa_fwd with the same args (and the same inputs, for the
   outputs to be the op's); each stage rewrites exactly what it wrote in that call, so
   repeating a stage is idempotent.  A stage the mode does not run returns MOSAIC_OK and
   launches nothing.  No reference counterpart: it lets a caller time each kernel on its own
   with plain launches (no events between the kernels of a call). */
MOSAIC_API int mosaic_bsa_fwd_stage(const mosaic_bsa_args* args, void* workspace, size_t workspace_bytes,
                                    void* stream, int stage);

/* Full forward with the input side's 2-D RoPE fused into the pooling pass: q and k are
   rotated as the caller's RoPE modules rotate them (primitives.py:125-135, applied at
   :193-195) and the op (primitives.py:54-89) runs on the rotated tensors.
   rope_cos, rope_sin: fp32 [seq_len, 32], the reference's cos_freqs / sin_freqs buffers
   (primitives.py:115-123: 16 longitude then 16 latitude frequencies per position); pair
   (2m, 2m+1) of every head is rotated by angle m.  q_rot, k_rot: caller-allocated bf16
   [batch, seq_len, H, 64] contiguous outputs holding the rotated q and k.  In the FULL and
   NO_COMPRESSION modes the attention kernel rotates q itself and q_rot may be null (then
   the rotated q is not written).  Same workspace as mosaic_bsa_fwd. */
MOSAIC_API int mosaic_bsa_fwd_rope(const mosaic_bsa_args* args, const float* rope_cos, const float* rope_sin,
                                   void* q_rot, void* k_rot, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* Input side of mosaic_bsa_fwd_proj: the attention block's input x and its stacked projection
   weight.  x: bf16 rows of model dimension dim (contiguous), token n of member b at
   x + n * x_stride_n + b * x_stride_b (elements; the model's sequence-first [N, B, dim]
   activations have x_stride_n = B * dim, x_stride_b = dim).  weight: bf16 [weight_rows, dim],
   the nn.Linear weights to_q (Hq * 64 rows), to_k (Hk * 64), to_v (Hk * 64) and, unless the
   mode is LOCAL_ONLY, to_strategy_combine_mlp (3 * Hq rows, channel 3 h + branch), each block
   starting at a multiple of 64 rows: q at 0, k at 64 Hq, v at 64 (Hq + Hk), gates at
   64 (Hq + 2 Hk); every other row zero; weight_rows = 256 * ceil(groups / 4) with
   groups = Hq + 2 Hk (+ 1 with gates).  rope_cos / rope_sin: fp32 [seq_len, 32] as for
   mosaic_bsa_fwd_rope, or both NULL for no rotation.  Outputs (caller-allocated, 16-byte
   aligned): q, k, v bf16 [B, N, H, 64] contiguous (q and k rotated); weights bf16
   [B, N, Hq, 3], the softmax of each head's three gate logits (NULL in LOCAL_ONLY mode). */
typedef struct {
    const void* x;
    int64_t x_stride_n, x_stride_b;
    int32_t dim;
    int32_t weight_rows;
    const void* weight;
    const float* rope_cos;
    const float* rope_sin;
    void* q;
    void* k;
    void* v;
    void* weights;
} mosaic_proj_args;

/* The attention block from its input rows: the q / k / v / gate projection
   (primitives.py:182-195, one GEMM over the stacked weights), the 2-D RoPE of q and k
   (:125-135, :193-195), the gate softmax (:171-180) and then the op (primitives.py:54-89) --
   with the projection, RoPE, gate softmax and the block pooling of q, k and v (:65-66, 76) in
   one kernel, so q, k and v are written once and the op does not read them back to pool them.
   args as for mosaic_bsa_fwd, except that q, k, v, weights and their strides are ignored (the
   projection's outputs take their place).  Requirements beyond mosaic_bsa_fwd's: dim a
   positive multiple of 128; seq_len a multiple of 256; sparse_block_size 64 or 128 unless
   LOCAL_ONLY; 3 * Hq <= 64.  Same workspace (mosaic_bsa_workspace_size of the same args). */
MOSAIC_API int mosaic_bsa_fwd_proj(const mosaic_bsa_args* args, const mosaic_proj_args* proj, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* k-nearest-neighbour cross-attention between two grids: the gather-attention of
   CrossAttentionInterpolate.forward (primitives.py:265-283), from the kv projection to the
   input of to_o.  Target s attends to the num_neighbors source points neighbors[s, :]
   (int32 [num_to, num_neighbors]) of k and v, with queries to_q(rel_pos[s, j]) formed
   inside the kernel from rel_pos (fp32 [num_to, num_neighbors, 3]) and w_q (bf16
   [num_heads * 64, 3], the to_q weight); softmax over the neighbours in fp32.
   k, v: bf16 [num_from, batch, num_heads, 64] given by strides (stride_n: source point,
   stride_b: batch member, stride_h: head).  out: bf16 [num_to, batch, num_heads, 64]
   contiguous.  num_neighbors <= 32; scale <= 0 selects head_dim^-0.5.  Neighbour indices
   outside [0, num_from) are clamped.  w_q and out 16-byte aligned. */
MOSAIC_API int mosaic_knn_interp_fwd(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors,
                                     const float* rel_pos, const void* w_q, int32_t num_from,
                                     int32_t num_to, int32_t batch, int32_t num_heads,
                                     int32_t head_dim, int32_t num_neighbors, float scale,
                                     void* out, void* stream);

/* mosaic_knn_interp_fwd with the targets taken in a given order: target_order (int32
   [num_to], 4-byte aligned) is a permutation of 0..num_to-1, or NULL for index order.  The
   output is the same in any order (each target's row is computed alone); the order decides
   which targets run at the same time, so an order along a space-filling curve of the target
   positions keeps the neighbour rows they share in L2.  Entries outside [0, num_to) are
   clamped; an order that is not a permutation leaves some rows of out unwritten.  Same
   replacement as mosaic_knn_interp_fwd (primitives.py:265-283); the order is computed once
   per grid pair with the neighbours (primitives.py:250-263). */
MOSAIC_API int mosaic_knn_interp_fwd_ordered(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors,
                                             const float* rel_pos, const void* w_q,
                                             const int32_t* target_order, int32_t num_from,
                                             int32_t num_to, int32_t batch, int32_t num_heads,
                                             int32_t head_dim, int32_t num_neighbors, float scale,
                                             void* out, void* stream);

/* Flags of mosaic_knn_interp_fwd_ex. */
#define MOSAIC_KNN_ROUND_PRODUCTS 1u /* round every q*k and w*v product to bf16 before summing */

/* Tiles of targets for mosaic_knn_interp_fwd_ex (int32 device arrays, 4-byte aligned).  Tile i
   holds the targets at positions [start[i], start[i+1]) of the target order (at most 16;
   start[0] = 0, start[num_tiles] = num_to); src[i, 0 .. nsrc[i]-1] are the distinct source
   points its targets use (at most max_rows; src is [num_tiles, max_rows]); slot[pos, j] is the
   row of that list holding neighbour j of the target at order position pos (slot is
   [num_to, num_neighbors]).  Static per grid pair and order: built once with the neighbours.
   Entries out of range are clamped; tiles that do not partition the order leave rows of out
   unwritten. */
typedef struct {
    const int32_t* start;
    const int32_t* src;
    const int32_t* nsrc;
    const int32_t* slot;
    int32_t num_tiles;
    int32_t max_rows; /* a multiple of 8, at most 128 */
} mosaic_knn_tiles;

/* mosaic_knn_interp_fwd_ordered with a choice of product rounding and optional target tiles
   (same replacement, primitives.py:265-283).  With MOSAIC_KNN_ROUND_PRODUCTS every product of
   (q * k).sum(-1) and (w * v).sum(1) is rounded to bf16 before the fp32 sum, as the
   reference's eager bf16 elementwise ops do (mosaic_knn_interp_fwd and _ordered are this
   form).  Without it the products are exact and summed in fp32, as the reference's default
   inference path computes them (its torch.compile'd model, inference.py:470-473, fuses each
   product into its reduction); the roundings of the score, the scaled score, the weights and
   the output are the same in both.  tiles (optional, fp32 products only; ignored with
   MOSAIC_KNN_ROUND_PRODUCTS): each tile's distinct source rows are staged once per member and
   head for all its targets; the output is the same bit for bit (neighbors is then not read;
   the tiles were built from it).  Unknown flag bits return MOSAIC_ERR_MODE. */
MOSAIC_API int mosaic_knn_interp_fwd_ex(mosaic_bnhd k, mosaic_bnhd v, const int32_t* neighbors,
                                        const float* rel_pos, const void* w_q,
                                        const int32_t* target_order, const mosaic_knn_tiles* tiles,
                                        int32_t num_from, int32_t num_to, int32_t batch,
                                        int32_t num_heads, int32_t head_dim, int32_t num_neighbors,
                                        float scale, uint32_t flags, void* out, void* stream);

/*
 * Selected-branch attention given block indices.  Replaces mosaic_sparse_attn /
 * MosaicAttnFunction.forward / mosaic_attn_fwd (ops.py:557-566, 510-538, 137-176):
 * for query token n of block i = n / block_size, query head j and kv head c = j / (Hq/Hk),
 * attend to the tokens of blocks block_indices[b, i, c, 0..K-1].  out: bf16 [B, N, Hq, 64]
 * contiguous; lse (optional): fp32 [B, N, Hq] base-2 log-sum-exp of the scaled logits.
 * block_indices: int64 [B, N/block_size, Hk, K] contiguous; entries outside [0, N/bs) are
 * skipped (a row whose entries are all invalid yields NaN).
 */
MOSAIC_API int mosaic_sparse_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v,
                           const int64_t* block_indices, int32_t batch, int32_t seq_len,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t block_size, int32_t block_count, float softmax_scale,
                           void* out, float* lse, void* stream);

/* As mosaic_sparse_attn_fwd, with a workspace of mosaic_sparse_attn_fwd_workspace_size()
   bytes (16-byte aligned) for the key-norm bounds of k's blocks ([B, N/block_size, Hk, 8]
   fp32, a pass over k): query tiles whose logits all lie within the bound then take the
   bounded-logit path of the fused forward (reference 0, row sums on the matrix pipe) instead
   of the running maximum.  Same outputs, to fp32 rounding. */
MOSAIC_API size_t mosaic_sparse_attn_fwd_workspace_size(int32_t batch, int32_t seq_len, int32_t num_kv_heads,
                                                        int32_t block_size);
MOSAIC_API int mosaic_sparse_attn_fwd_ws(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v,
                                         const int64_t* block_indices, int32_t batch, int32_t seq_len,
                                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                         int32_t block_size, int32_t block_count, float softmax_scale,
                                         void* out, float* lse, void* workspace, size_t workspace_bytes,
                                         void* stream);

/*
 * Backward of the selected-branch attention.  Replaces MosaicAttnFunction.backward /
 * mosaic_attn_bwd (ops.py:541-554, 437-507) and its grad-q, block-mask and grad-k/v kernels
 * (ops.py:179-273, 276-297, 300-434): given the forward's inputs, its output out (bf16
 * [B, N, Hq, 64] contiguous), its lse (fp32 [B, N, Hq], base 2) and grad_out (strided like q),
 * writes grad_q (bf16 [B, N, Hq, 64]), grad_k and grad_v (bf16 [B, N, Hk, 64]), all
 * contiguous.  Keys that no query block selected get zero gradients.  block_indices as for
 * mosaic_sparse_attn_fwd (entries outside [0, N/bs) are skipped); N / block_size <= 4096.
 * workspace: mosaic_sparse_attn_bwd_workspace_size() bytes (the per-row -lse and
 * -delta = -(o . do) and the pre-scaled q' = bf16((q * scale) * log2 e) the two gradient
 * kernels share).
 */
MOSAIC_API size_t mosaic_sparse_attn_bwd_workspace_size(int32_t batch, int32_t seq_len, int32_t num_q_heads);
MOSAIC_API int mosaic_sparse_attn_bwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, const void* out,
                                      const float* lse, mosaic_bnhd grad_out, const int64_t* block_indices,
                                      int32_t batch, int32_t seq_len, int32_t num_q_heads,
                                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                      int32_t block_count, float softmax_scale, void* grad_q, void* grad_k,
                                      void* grad_v, void* workspace, size_t workspace_bytes, void* stream);

/* Local attention inside contiguous blocks.  Replaces block_attention (primitives.py:28-32),
   i.e. flash_attn_func on [(B*N/bs), bs, H, d] views.  out: bf16 [B, N, Hq, 64] contiguous. */
MOSAIC_API int mosaic_block_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, int32_t batch,
                          int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t block_size, float softmax_scale, void* out,
                          void* stream);

/* Dense (full-sequence) attention: the baseline the sparse op is compared with.  Same
   contract as mosaic_block_attn_fwd with block_size = seq_len (flash_attn_func on the whole
   sequence, primitives.py:31 with one block). */
MOSAIC_API int mosaic_dense_attn_fwd(mosaic_bnhd q, mosaic_bnhd k, mosaic_bnhd v, int32_t batch,
                          int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, float softmax_scale, void* out, void* stream);

/* Mean over runs of block_size tokens, rounded to bf16.  Replaces the einops
   reduce(x, 'b (nb bs) h d -> b nb h d', 'mean') of primitives.py:65-66,76.
   out: bf16 [B, N/block_size, H, 64] contiguous. */
MOSAIC_API int mosaic_pool_mean_fwd(mosaic_bnhd x, int32_t batch, int32_t seq_len, int32_t num_heads,
                         int32_t head_dim, int32_t block_size, void* out, void* stream);

/* Top-k block selection from pooled queries/keys.  Replaces attn_topk (primitives.py:35-51):
   scores[b, h, t, u] = mean over g of bf16(q_cmp[b, t, g*Hk + h] . k_cmp[b, u, (g*Hk+h)/G]),
   rounded to bf16; indices_out[b, t, h, :] = the block_count largest u, in descending score
   order (ties: lower u first).  q_cmp/k_cmp: bf16 [B, nb, H, 64]; indices_out: int64
   [B, nb, Hk, K] contiguous.  workspace: mosaic_attn_topk_workspace_size() bytes. */
MOSAIC_API size_t mosaic_attn_topk_workspace_size(int32_t batch, int32_t num_blocks, int32_t num_kv_heads);
MOSAIC_API int mosaic_attn_topk_fwd(mosaic_bnhd q_cmp, mosaic_bnhd k_cmp, int32_t batch,
                         int32_t num_blocks, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_count, int64_t* indices_out,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Row-wise RMSNorm, optionally after a residual add.  Replaces torch.nn.RMSNorm as the model
   calls it (MosaicBlock.norm1 / norm2, primitives.py:220-226; the U-Net's pre/post-processing
   and resampling norms, mosaic.py:163-217, primitives.py:313-359) and, with residual != NULL,
   the add in front of it (x + attention(...), primitives.py:225):
     y = x + residual      rounded to dtype (written to sum_out, contiguous [rows, cols], when
                           sum_out != NULL)
     out = y * rsqrt(mean(y^2) + eps) * weight      fp32 statistics, rounded once to out_dtype
   x, residual: dtype rows of cols contiguous elements, rows x_row_stride / residual_row_stride
   elements apart; out: out_dtype [rows, cols] contiguous; weight: optional fp32 [cols].
   cols a multiple of 8, at most 4096; pointers 16-byte aligned. */
MOSAIC_API int mosaic_rms_norm_fwd(const void* x, const void* residual, int32_t dtype, int64_t rows,
                                   int32_t cols, int64_t x_row_stride, int64_t residual_row_stride,
                                   const float* weight, float eps, void* sum_out, void* out,
                                   int32_t out_dtype, void* stream);

/* The epilogue of HEALPixUpsample / HEALPixDownsample.forward (primitives.py:313-359): the
   split of the projection P, the broadcast position term, the skip connection and the RMSNorm
   in one pass.  Output row R = (n factor + j) members + b of out ([coarse_rows * factor *
   members, dim] bf16 contiguous, the sequence-first [(n f), B, d] layout) is
     y = bf16(P[n members + b, j dim + c] + pos[n, j dim + c])        c < dim
     y = bf16(y + shortcut[R, c])                                     (shortcut != NULL)
     out = y * rsqrt(mean(y^2) + eps) * weight                        fp32 statistics
   P: bf16 rows of factor * dim elements, p_row_stride apart; pos: bf16 [coarse_rows, factor *
   dim] contiguous; shortcut: optional bf16 like out; weight: optional fp32 [dim].  factor = 1
   without a shortcut is the downsampling epilogue (norm(proj_x(x) + proj_pos(rel_pos))).  dim a
   multiple of 8, at most 4096; pointers 16-byte aligned.  No counterpart entry point in the
   reference, which runs these as eager tensor ops. */
MOSAIC_API int mosaic_resample_norm_fwd(const void* p, int64_t p_row_stride, const void* pos,
                                        const void* shortcut, const float* weight, float eps,
                                        int64_t coarse_rows, int32_t members, int32_t factor,
                                        int32_t dim, void* out, void* stream);

/* The end of an encoder stage and the input of HEALPixDownsample (mosaic.py:318-321,
   primitives.py:322-326): sum_out = bf16(x + residual) (bf16 [coarse_rows * factor * members,
   dim] contiguous, the sequence-first [(n f), B, d] rows; the skip connection) and merged_out
   = the same sums as [coarse_rows, members, factor * dim] ('(n f) b c -> n b (f c)'), the
   downsampling projection's input.  x, residual: bf16 like sum_out.  dim a multiple of 8;
   pointers 16-byte aligned.  No counterpart entry point in the reference. */
MOSAIC_API int mosaic_add_merge_fwd(const void* x, const void* residual, int64_t coarse_rows,
                                    int32_t members, int32_t factor, int32_t dim, void* sum_out,
                                    void* merged_out, void* stream);

/* MosaicAttention.generate_strategy_weights (primitives.py:173-180) on a bf16 logits slice:
   w[s, b, n, h] = bf16(softmax_s(fp32 logits[n, b, 3 h + s])) for s < 3, the softmax computed
   as torch.softmax(..., dim=0) computes it (max, exp of the differences, divided by their sum).
   logits: bf16 rows (n, b) of 3 * heads elements, row n * members + b at logits_row_stride
   elements (the sequence-first [seq, members, .] gate slice of a wider projection); w: bf16
   [3, members, seq, heads] contiguous, the layout mosaic_bsa_args.weights takes with strides
   (members seq heads, seq heads, heads, 1).  No counterpart entry point in the reference. */
MOSAIC_API int mosaic_gate_softmax_fwd(const void* logits, int64_t logits_row_stride, int64_t seq,
                                       int32_t members, int32_t heads, void* w, void* stream);

/* The SwiGLU gate of cSwiGLU.forward (primitives.py:102-105): with x1 = h[:, :hidden] and
   x3 = h[:, hidden:2*hidden], out = silu(x1 + noise[row % noise_rows]) * x3, each of the
   add, the silu and the product rounded to dtype as the reference's eager ops round.
   h: dtype [rows, >= 2*hidden] with row stride h_row_stride; noise: optional dtype
   [noise_rows, hidden] contiguous (the noise_bias(z) rows, one per batch member of a
   sequence-first [S, B, .] activation); out: dtype [rows, hidden] contiguous.  hidden a
   multiple of 8; pointers 16-byte aligned. */
MOSAIC_API int mosaic_swiglu_fwd(const void* h, int32_t dtype, int64_t rows, int32_t hidden,
                                 int64_t h_row_stride, const void* noise, int32_t noise_rows, void* out,
                                 void* stream);

/* cSwiGLU's first projection and gate in one kernel (primitives.py:92-105, w13 then the gate
   of mosaic_swiglu_fwd): out = silu(x1 + noise[row % noise_rows]) * x3 with h = x w13^T
   rounded to bf16 (fp32 accumulation) and x1, x3 its two halves, so h is never stored.
   x: bf16 [rows, dim] with row stride x_row_stride; weight: bf16 [2*hidden, dim] contiguous,
   w13 with its rows permuted in 64-row groups -- group t holds rows 32t..32t+31 of the x1 half
   (w13 rows 32t..) then of the x3 half (w13 rows hidden+32t..); noise: optional bf16
   [noise_rows, hidden] contiguous; out: bf16 [rows, hidden] contiguous.  rows a multiple of
   256, dim of 128, hidden of 128; pointers 16-byte aligned, x_row_stride a multiple of 8.
   No reference counterpart as one function: it fuses the Linear and the gate the reference
   runs as separate ops. */
MOSAIC_API int mosaic_swiglu_linear_fwd(const void* x, int64_t rows, int32_t dim, int64_t x_row_stride,
                                        const void* weight, int32_t hidden, const void* noise,
                                        int32_t noise_rows, void* out, void* stream);

/* Name of a status code (static storage). */
MOSAIC_API const char* mosaic_bsa_strerror(int status);

/* MOSAIC_BSA_ABI_VERSION of the loaded library. */
MOSAIC_API int mosaic_bsa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MOSAIC_BSA_H */
