"""Block-sparse attention primitives: the MI355X drop-in for the reference's primitives.py op.

Same names, arguments and branch logic as the reference:
  * ``block_attention(q, k, v, block_size)``                       primitives.py:28-32
  * ``attn_topk(q, k, block_count)``                               primitives.py:35-51
  * ``mosaic_attn_func(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size,
    sparse_block_count, block_attn_only, no_compression=False)``   primitives.py:54-89
  * ``RoPE`` and ``MosaicAttention`` modules (primitives.py:108-209), the op's caller, with
    the reference's parameter and buffer names so its state dicts load unchanged.

Every op runs as HIP kernels through the C ABI of libmosaic_bsa.so on the current stream;
there is no CPU path.  Extras beyond the reference: ``pool_mean`` (the einops mean pooling of
:65-66 as one kernel), ``dense_attention`` (full-sequence baseline), and the keyword-only
``return_block_indices`` of ``mosaic_attn_func``.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _lib, fused
from .healpix import rope_tables
from .ops import _as_bf16_bnhd, _check_gqa, bnhd, forward_only, mosaic_sparse_attn, stream_of

__all__ = [
    "block_attention", "dense_attention", "pool_mean", "attn_topk", "mosaic_attn_func",
    "mosaic_attn_func_rope", "mosaic_attn_proj", "stack_projection_weight", "mosaic_sparse_attn", "RoPE",
    "MosaicAttention",
]


def _out_like(q: torch.Tensor) -> torch.Tensor:
    return torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)


def block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_size: int) -> torch.Tensor:
    """Attention inside contiguous blocks of ``block_size`` tokens (primitives.py:28-32)."""
    forward_only("block_attention", q, k, v)
    dtype = q.dtype
    q, k, v = (_as_bf16_bnhd(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    _check_gqa(q, k, v)
    B, N, Hq, d = q.shape
    out = _out_like(q)
    st = _lib.lib().mosaic_block_attn_fwd(bnhd(q), bnhd(k), bnhd(v), B, N, Hq, k.shape[2], d, int(block_size),
                                          0.0, out.data_ptr(), stream_of(q))
    _lib.check(st, "mosaic_block_attn_fwd")
    return out.to(dtype)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Full-sequence attention (flash_attn_func defaults), the dense baseline."""
    forward_only("dense_attention", q, k, v)
    dtype = q.dtype
    q, k, v = (_as_bf16_bnhd(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    _check_gqa(q, k, v)
    B, N, Hq, d = q.shape
    out = _out_like(q)
    st = _lib.lib().mosaic_dense_attn_fwd(bnhd(q), bnhd(k), bnhd(v), B, N, Hq, k.shape[2], d, 0.0,
                                          out.data_ptr(), stream_of(q))
    _lib.check(st, "mosaic_dense_attn_fwd")
    return out.to(dtype)


def pool_mean(x: torch.Tensor, block_size: int) -> torch.Tensor:
    """reduce(x, 'b (nb bs) h d -> b nb h d', 'mean', bs=block_size) in bf16 (primitives.py:65)."""
    forward_only("pool_mean", x)
    x = _as_bf16_bnhd(x, "x")
    B, N, H, d = x.shape
    if N % block_size:
        raise ValueError("sequence length must be a multiple of block_size")
    out = torch.empty(B, N // block_size, H, d, dtype=torch.bfloat16, device=x.device)
    st = _lib.lib().mosaic_pool_mean_fwd(bnhd(x), B, N, H, d, int(block_size), out.data_ptr(), stream_of(x))
    _lib.check(st, "mosaic_pool_mean_fwd")
    return out


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    ws = torch.empty(max(int(nbytes), 256) + 256, dtype=torch.uint8, device=device)
    off = (-ws.data_ptr()) % 256
    return ws[off:off + max(int(nbytes), 256)]


@torch.no_grad()
def attn_topk(q: torch.Tensor, k: torch.Tensor, block_count: int) -> torch.Tensor:
    """Top-``block_count`` key blocks per query block and kv head (primitives.py:35-51).

    q, k are the pooled tensors [B, nb, Hq, d] / [B, nb, Hk, d]; returns int64 [B, nb, Hk, K]
    sorted by descending score.
    """
    q = _as_bf16_bnhd(q, "q")
    k = _as_bf16_bnhd(k, "k")
    B, nb, Hq, d = q.shape
    Hk = k.shape[2]
    if k.shape[0] != B or k.shape[1] != nb or k.shape[3] != d:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if not 0 < block_count <= nb:
        raise ValueError(f"block_count must be in [1, {nb}], got {block_count}")
    L = _lib.lib()
    ws = _workspace(L.mosaic_attn_topk_workspace_size(B, nb, Hk), q.device)
    idx = torch.empty(B, nb, Hk, block_count, dtype=torch.int64, device=q.device)
    st = L.mosaic_attn_topk_fwd(bnhd(q), bnhd(k), B, nb, Hq, Hk, d, int(block_count), idx.data_ptr(),
                                ws.data_ptr(), ws.numel(), stream_of(q))
    _lib.check(st, "mosaic_attn_topk_fwd")
    return idx


def _bsa_args(q, k, v, w, out, block_attn_size, sparse_block_size, sparse_block_count, mode, idx_out):
    B, N, Hq, d = q.shape
    a = _lib.BsaArgs()
    a.batch, a.seq_len, a.num_q_heads, a.num_kv_heads, a.head_dim = B, N, Hq, k.shape[2], d
    a.block_attn_size = int(block_attn_size)
    a.sparse_block_size = int(sparse_block_size)
    a.sparse_block_count = int(sparse_block_count)
    a.mode = mode
    a.softmax_scale = 0.0
    a.q, a.k, a.v = bnhd(q), bnhd(k), bnhd(v)
    if w is not None:
        a.weights = w.data_ptr()
        a.w_stride_s, a.w_stride_b, a.w_stride_n, a.w_stride_h = (w.stride(i) for i in range(4))
    a.out = out.data_ptr()
    a.block_indices_out = idx_out.data_ptr() if idx_out is not None else None
    return a


def _weights_view(w: torch.Tensor, B: int, N: int, Hq: int, device) -> torch.Tensor:
    if w is None:
        raise ValueError("weight_ba_cmp_slc is required unless block_attn_only")
    if w.dim() == 5:
        if w.shape[-1] != 1:
            raise ValueError("weight_ba_cmp_slc must be [3, B, N, Hq, 1]")
        w = w[..., 0]
    if tuple(w.shape) != (3, B, N, Hq):
        raise ValueError(f"weight_ba_cmp_slc shape {tuple(w.shape)} != (3, {B}, {N}, {Hq}, 1)")
    if w.device != device:
        raise ValueError("weight_ba_cmp_slc must be on the same device as q")
    if w.dtype != torch.bfloat16:
        w = w.to(torch.bfloat16)
    return w


def mosaic_attn_func(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size, sparse_block_count,
                     block_attn_only, no_compression=False, *, return_block_indices=False, out=None):
    """Three-branch block-sparse attention forward (primitives.py:54-89).

    Branch logic as in the reference: ``block_attn_only`` returns the local branch; with
    ``no_compression`` the local and selected branches are merged with renormalised weights;
    ``sparse_block_count == 0`` merges local and compressed with renormalised weights;
    otherwise ``o_ba*w0 + o_cmp*w1 + o_slc*w2``.  With ``return_block_indices`` the selected
    block indices (int64 [B, N/sparse_block_size, Hk, K]) are returned as well.  ``out``
    (keyword-only) is an optional preallocated bf16 [B, N, Hq, 64] destination whose head and
    head_dim strides are 64 and 1 (e.g. the transposed view of a sequence-first buffer); the
    kernel writes it in place.
    """
    out, idx, _ = _bsa_forward(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size, sparse_block_count,
                               block_attn_only, no_compression, return_block_indices, None, out=out)
    return (out, idx) if return_block_indices else out


def mosaic_attn_func_rope(q, k, v, weight_ba_cmp_slc, rope_cos, rope_sin, block_attn_size, sparse_block_size,
                          sparse_block_count, block_attn_only, no_compression=False, *, return_rotated=False,
                          return_block_indices=False, out=None):
    """mosaic_attn_func on q and k rotated by the 2-D RoPE, with the rotation fused into the
    op's pooling pass (primitives.py:193-195 followed by :54-89): q and k are read once,
    rotated, pooled and written rotated for the attention kernel.

    ``rope_cos`` / ``rope_sin`` are the RoPE module's ``cos_freqs`` / ``sin_freqs`` ([N, 32]
    fp32, primitives.py:115-123).  The result equals ``mosaic_attn_func(RoPE(q), RoPE(k), v,
    ...)``.  With ``return_rotated`` the rotated q and k ([B, N, H, 64] bf16) are returned
    after the output (and before the indices, when those are asked for too).  ``out`` as for
    ``mosaic_attn_func``.
    """
    out, idx, rot = _bsa_forward(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size,
                                 sparse_block_count, block_attn_only, no_compression, return_block_indices,
                                 (rope_cos, rope_sin), return_rotated, out=out)
    res = (out,) + (rot if return_rotated else ()) + ((idx,) if return_block_indices else ())
    return res[0] if len(res) == 1 else res


def stack_projection_weight(w_q, w_k, w_v, w_gate, num_q_heads, num_kv_heads):
    """The stacked bf16 weight of ``mosaic_attn_proj``: the rows of to_q, to_k, to_v and (unless
    None) to_strategy_combine_mlp at row offsets 0, 64 Hq, 64 (Hq + Hk) and 64 (Hq + 2 Hk), zero
    rows up to a multiple of 256 (one 64-row group per head, then one for the gate logits)."""
    groups = num_q_heads + 2 * num_kv_heads + (1 if w_gate is not None else 0)
    rows = 256 * ((groups + 3) // 4)
    dim = w_q.shape[1]
    out = torch.zeros(rows, dim, dtype=torch.bfloat16, device=w_q.device)
    r = 0
    for w, n in ((w_q, 64 * num_q_heads), (w_k, 64 * num_kv_heads), (w_v, 64 * num_kv_heads)):
        if tuple(w.shape) != (n, dim):
            raise ValueError(f"projection weight shape {tuple(w.shape)} != ({n}, {dim})")
        out[r:r + n] = w
        r += n
    if w_gate is not None:
        if tuple(w_gate.shape) != (3 * num_q_heads, dim):
            raise ValueError(f"gate weight shape {tuple(w_gate.shape)} != ({3 * num_q_heads}, {dim})")
        out[r:r + 3 * num_q_heads] = w_gate
    return out


def _bsa_mode(block_attn_only, no_compression, sparse_block_count):
    if block_attn_only:
        return _lib.MODE_LOCAL_ONLY
    if no_compression:
        if sparse_block_count <= 0:
            raise ValueError("no_compression needs sparse_block_count >= 1")
        return _lib.MODE_NO_COMPRESSION
    return _lib.MODE_NO_SELECTION if sparse_block_count == 0 else _lib.MODE_FULL


def mosaic_attn_proj(x, weight, num_q_heads, num_kv_heads, block_attn_size, sparse_block_size, sparse_block_count,
                     block_attn_only, no_compression=False, *, rope_cos=None, rope_sin=None,
                     return_projections=False, return_block_indices=False, out=None):
    """The attention block from its input rows: the q / k / v / gate projection
    (primitives.py:182-195), RoPE of q and k (:125-135, :193-195), the gate softmax (:171-180)
    and mosaic_attn_func (:54-89), with the projection, rotation, gate softmax and the block
    pooling of q, k and v in one kernel (q, k and v are written once, not read back to pool).

    x: sequence-first rows [S, B, dim] (the model's layout; bf16, or converted as autocast
    would).  weight: ``stack_projection_weight(...)``.  ``rope_cos`` / ``rope_sin``: the RoPE
    module's [S, 32] tables, or None.  Returns the op output [B, S, Hq, 64] (``out`` as for
    ``mosaic_attn_func``), then with ``return_projections`` the rotated q, rotated k, v
    ([B, S, H, 64]) and the branch weights [B, S, Hq, 3], then with ``return_block_indices``
    the selected blocks.  Needs S % 256 == 0, dim % 128 == 0, sparse_block_size 64 or 128
    (unless block_attn_only) and 3 Hq <= 64; ``ValueError`` otherwise.
    """
    forward_only("mosaic_attn_proj", x, weight)
    if x.dim() != 3:
        raise ValueError(f"x must be [S, B, dim], got shape {tuple(x.shape)}")
    if x.device.type != "cuda":
        raise ValueError(f"x must be on a ROCm device, got {x.device}")
    S, B, dim = x.shape
    Hq, Hk = num_q_heads, num_kv_heads
    mode = _bsa_mode(block_attn_only, no_compression, sparse_block_count)
    local = mode == _lib.MODE_LOCAL_ONLY
    if S % 256 or dim % 128 or (not local and (sparse_block_size not in (64, 128) or 3 * Hq > 64)):
        raise ValueError("mosaic_attn_proj needs S % 256 == 0, dim % 128 == 0, sparse_block_size 64 or 128 "
                         "and 3 * num_q_heads <= 64")
    dtype = x.dtype
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if x.stride(2) != 1 or x.data_ptr() % 16 or x.stride(0) % 8 or x.stride(1) % 8:
        x = x.contiguous()
    groups = Hq + 2 * Hk + (0 if local else 1)
    if weight.dtype != torch.bfloat16 or tuple(weight.shape) != (256 * ((groups + 3) // 4), dim):
        raise ValueError("weight must be stack_projection_weight(...) for these heads (bf16 "
                         f"[{256 * ((groups + 3) // 4)}, {dim}])")
    weight = weight.contiguous()
    dev = x.device
    q = torch.empty(B, S, Hq, 64, dtype=torch.bfloat16, device=dev)
    k = torch.empty(B, S, Hk, 64, dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    w = None if local else torch.empty(B, S, Hq, 3, dtype=torch.bfloat16, device=dev)
    rope = None
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError("rope_cos and rope_sin go together")
    if rope_cos is not None:
        rope = tuple(t.to(device=dev, dtype=torch.float32).contiguous() for t in (rope_cos, rope_sin))
        if any(tuple(t.shape) != (S, 32) for t in rope):
            raise ValueError(f"RoPE tables must be [seq_len, 32] = [{S}, 32]")
    selects = mode in (_lib.MODE_FULL, _lib.MODE_NO_COMPRESSION)
    idx = None
    if return_block_indices and selects:
        idx = torch.empty(B, S // sparse_block_size, Hk, sparse_block_count, dtype=torch.int64, device=dev)
    if out is None:
        out = torch.empty(B, S, Hq, 64, dtype=torch.bfloat16, device=dev)
    elif (tuple(out.shape) != (B, S, Hq, 64) or out.dtype != torch.bfloat16 or out.device != dev
          or out.stride(3) != 1 or out.stride(2) != 64 or out.stride(0) % 8 or out.stride(1) % 8
          or out.data_ptr() % 16):
        raise ValueError("out must be a bf16 [B, N, Hq, 64] view with contiguous heads and 16-byte rows")
    a = _lib.BsaArgs()
    a.batch, a.seq_len, a.num_q_heads, a.num_kv_heads, a.head_dim = B, S, Hq, Hk, 64
    a.block_attn_size, a.sparse_block_size, a.sparse_block_count = block_attn_size, sparse_block_size, sparse_block_count
    a.mode, a.softmax_scale = mode, 0.0
    a.out = out.data_ptr()
    a.block_indices_out = idx.data_ptr() if idx is not None else None
    a.out_stride_b, a.out_stride_n = out.stride(0), out.stride(1)
    j = _lib.ProjArgs()
    j.x, j.x_stride_n, j.x_stride_b, j.dim = x.data_ptr(), x.stride(0), x.stride(1), dim
    j.weight_rows, j.weight = weight.shape[0], weight.data_ptr()
    j.rope_cos = rope[0].data_ptr() if rope else None
    j.rope_sin = rope[1].data_ptr() if rope else None
    j.q, j.k, j.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    j.weights = w.data_ptr() if w is not None else None
    # the op's workspace: the same as mosaic_bsa_fwd's for these shapes (q/k/v/weights stand-ins
    # only carry shapes and strides for the size query)
    qa = _lib.BsaArgs.from_buffer_copy(a)
    qa.q = _lib.Bnhd(q.data_ptr(), q.stride(0), q.stride(1), q.stride(2))
    qa.k = _lib.Bnhd(k.data_ptr(), k.stride(0), k.stride(1), k.stride(2))
    qa.v = _lib.Bnhd(v.data_ptr(), v.stride(0), v.stride(1), v.stride(2))
    if w is not None:
        qa.weights = w.data_ptr()
        qa.w_stride_s, qa.w_stride_b, qa.w_stride_n, qa.w_stride_h = 1, S * Hq * 3, Hq * 3, 3
    L = _lib.lib()
    nbytes = L.mosaic_bsa_workspace_size(ctypes.byref(qa))
    if nbytes == 0 and not local:
        _lib.check(L.mosaic_bsa_fwd_proj(ctypes.byref(a), ctypes.byref(j), None, 0, stream_of(x)), "mosaic_bsa_fwd_proj")
    ws = _workspace(nbytes, dev) if nbytes else None
    _lib.check(L.mosaic_bsa_fwd_proj(ctypes.byref(a), ctypes.byref(j), ws.data_ptr() if ws is not None else None,
                                     ws.numel() if ws is not None else 0, stream_of(x)), "mosaic_bsa_fwd_proj")
    res = (out.to(dtype),)
    if return_projections:
        res += (q, k, v, w)
    if return_block_indices:
        res += (idx,)
    return res[0] if len(res) == 1 else res


def _bsa_forward(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size, sparse_block_count,
                 block_attn_only, no_compression, return_block_indices, rope, return_rotated=False, out=None):
    forward_only("mosaic_attn_func", q, k, v, weight_ba_cmp_slc, *(rope or ()))
    dtype = q.dtype
    q, k, v = (_as_bf16_bnhd(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    _check_gqa(q, k, v)
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    if block_attn_only:
        mode = _lib.MODE_LOCAL_ONLY
    elif no_compression:
        if sparse_block_count <= 0:
            raise ValueError("no_compression needs sparse_block_count >= 1")
        mode = _lib.MODE_NO_COMPRESSION
    elif sparse_block_count == 0:
        mode = _lib.MODE_NO_SELECTION
    else:
        mode = _lib.MODE_FULL
    w = None if block_attn_only else _weights_view(weight_ba_cmp_slc, B, N, Hq, q.device)
    selects = mode in (_lib.MODE_FULL, _lib.MODE_NO_COMPRESSION)
    idx = None
    if return_block_indices and selects:
        idx = torch.empty(B, N // sparse_block_size, Hk, sparse_block_count, dtype=torch.int64, device=q.device)
    if out is None:
        out = _out_like(q)
    elif (tuple(out.shape) != (B, N, Hq, d) or out.dtype != torch.bfloat16 or out.device != q.device
          or out.stride(3) != 1 or out.stride(2) != d or out.stride(0) % 8 or out.stride(1) % 8
          or out.data_ptr() % 16):
        raise ValueError("out must be a bf16 [B, N, Hq, 64] view with contiguous heads and 16-byte rows")
    a = _bsa_args(q, k, v, w, out, block_attn_size, sparse_block_size, sparse_block_count, mode, idx)
    a.out_stride_b, a.out_stride_n = out.stride(0), out.stride(1)
    L = _lib.lib()
    rot = ()
    if rope is not None:
        cos, sin = (t.to(device=q.device, dtype=torch.float32).contiguous() for t in rope)
        if tuple(cos.shape) != (N, d // 2) or tuple(sin.shape) != (N, d // 2):
            raise ValueError(f"RoPE tables must be [seq_len, head_dim/2] = [{N}, {d // 2}]")
        # the full and no-compression modes rotate q inside the attention kernel: the rotated q
        # is only written when asked for
        want_q = return_rotated or mode not in (_lib.MODE_FULL, _lib.MODE_NO_COMPRESSION)
        q_rot = torch.empty(B, N, Hq, d, dtype=torch.bfloat16, device=q.device) if want_q else None
        k_rot = torch.empty(B, N, Hk, d, dtype=torch.bfloat16, device=q.device)
        rot = (q_rot, k_rot)

        def run(ws_ptr, nbytes):
            return L.mosaic_bsa_fwd_rope(ctypes.byref(a), cos.data_ptr(), sin.data_ptr(),
                                         q_rot.data_ptr() if q_rot is not None else None, k_rot.data_ptr(),
                                         ws_ptr, nbytes, stream_of(q))
        name = "mosaic_bsa_fwd_rope"
    else:
        def run(ws_ptr, nbytes):
            return L.mosaic_bsa_fwd(ctypes.byref(a), ws_ptr, nbytes, stream_of(q))
        name = "mosaic_bsa_fwd"
    nbytes = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    if nbytes == 0 and mode != _lib.MODE_LOCAL_ONLY:
        # invalid arguments: let the entry point report which
        _lib.check(run(None, 0), name)
    ws = _workspace(nbytes, q.device) if nbytes else None
    _lib.check(run(ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0), name)
    return out.to(dtype), idx, tuple(t.to(dtype) if t is not None else None for t in rot)


class RoPE(nn.Module):
    """2-D (lon, lat) rotary embedding with the reference's buffers (primitives.py:108-135)."""

    def __init__(self, dim, theta=10000):
        super().__init__()
        assert dim % 2 == 0
        self.dim = dim
        self.theta = theta

    def initialize_rope(self, positions):
        cos, sin = rope_tables(positions, self.dim, self.theta)
        self.register_buffer("cos_freqs", cos, persistent=True)
        self.register_buffer("sin_freqs", sin, persistent=True)

    def forward(self, x):
        xf = x.float()
        c = self.cos_freqs.unsqueeze(0).unsqueeze(2)
        s = self.sin_freqs.unsqueeze(0).unsqueeze(2)
        x_even, x_odd = xf[..., 0::2], xf[..., 1::2]
        out = torch.empty_like(xf)
        out[..., 0::2] = x_even * c - x_odd * s
        out[..., 1::2] = x_odd * c + x_even * s
        return out.to(x.dtype)


class MosaicAttention(nn.Module):
    """The op's caller (primitives.py:138-209): projections, gates, RoPE, block-sparse attention.

    ``config`` needs: block_attn_size, sparse_block_size, sparse_block_count, num_heads,
    gqa_ratio, dim, qkv_compress_ratio, rope, rope_theta.  x is sequence-first [S, B, dim].
    """

    def __init__(self, config, block_attn_only: bool, no_compression: bool = False):
        super().__init__()
        self.block_attn_only = block_attn_only
        self.no_compression = no_compression
        self.block_attn_size = config.block_attn_size
        self.sparse_block_size = config.sparse_block_size
        self.sparse_block_count = config.sparse_block_count
        q_heads = config.num_heads
        kv_heads = q_heads // config.gqa_ratio
        head_dim = int(config.dim // q_heads // config.qkv_compress_ratio)
        self.q_heads, self.kv_heads = q_heads, kv_heads
        self.to_q = nn.Linear(config.dim, q_heads * head_dim, bias=False)
        self.to_k = nn.Linear(config.dim, kv_heads * head_dim, bias=False)
        self.to_v = nn.Linear(config.dim, kv_heads * head_dim, bias=False)
        self.to_o = nn.Linear(q_heads * head_dim, config.dim, bias=False)
        self.q_rope = RoPE(head_dim, config.rope_theta) if config.rope else None
        self.k_rope = RoPE(head_dim, config.rope_theta) if config.rope else None
        self.to_strategy_combine_mlp = None if block_attn_only else nn.Linear(config.dim, 3 * q_heads, bias=False)
        # a list to append each call's selected block indices to (int64 [B, N/bs, Hk, K], None
        # without selection), or None; tests use it to evaluate a checker on the same selection
        self.record_block_indices = None

    def generate_strategy_weights(self, x):
        """Softmax over the 3 branch logits per head, channel index h*3 + s (primitives.py:173-180)."""
        if self.block_attn_only:
            return None
        logits = self.to_strategy_combine_mlp(x)                      # [S, B, Hq*3]
        S_, B_ = logits.shape[:2]
        logits = logits.view(S_, B_, self.q_heads, 3).permute(3, 1, 0, 2)   # [3, B, S, Hq]
        return torch.softmax(logits.float(), dim=0).type_as(x).unsqueeze(-1)

    def _shared_rope_tables(self):
        """True when the q and k RoPE modules hold equal tables (the model initialises both
        from the same grid, mosaic.py:268-270); the comparison is cached per table version."""
        tabs = (self.q_rope.cos_freqs, self.q_rope.sin_freqs, self.k_rope.cos_freqs, self.k_rope.sin_freqs)
        key = tuple((t.data_ptr(), t._version) for t in tabs)
        if getattr(self, "_rope_key", None) != key:
            self._rope_key = key
            self._rope_shared = bool(torch.equal(tabs[0], tabs[2]) and torch.equal(tabs[1], tabs[3]))
        return self._rope_shared

    def _proj_modules(self):
        mods = [self.to_q, self.to_k, self.to_v]
        if not self.block_attn_only:
            mods.append(self.to_strategy_combine_mlp)
        return mods

    def _weights_key(self):
        return tuple((m.weight.data_ptr(), m.weight._version, m.weight.dtype) for m in self._proj_modules())

    def _projections(self, x):
        """q, k, v and the gate logits from ONE GEMM over x: the four weights stacked, instead of
        four GEMMs that each read x (the gate projection alone, 36-60 outputs wide, ran ~10x
        slower than its bytes allow as a separate skinny GEMM).  Zero rows pad the width to a
        multiple of 256 (of 64 below 512 outputs): every slice starts 16-byte aligned, and the
        library GEMM runs its fast tiles (768 -> 1216 outputs took 2.79 ms on 1.18 M rows,
        768 -> 1280 2.04 ms).  The stacked weight is built once per weight version (the op has
        no backward, so it carries no graph)."""
        mods = self._proj_modules()
        sizes = [m.out_features for m in mods]
        key = self._weights_key()
        if getattr(self, "_cat_key", None) != key:
            total = sum(sizes)
            pad = -total % (256 if total >= 512 else 64)
            with torch.no_grad():
                ws = [m.weight for m in mods]
                if pad:
                    ws.append(ws[0].new_zeros(pad, ws[0].shape[1]))
                self._cat_weight = torch.cat(ws, 0)
            self._cat_key, self._cat_pad = key, pad
        pad = self._cat_pad
        y = torch.nn.functional.linear(x, self._cat_weight)
        parts = y.split(sizes + ([pad] if pad else []), dim=-1)
        return parts[0], parts[1], parts[2], (parts[3] if not self.block_attn_only else None)

    def _stacked_weight(self):
        """The bf16 weight of mosaic_attn_proj, built once per weight version."""
        key = self._weights_key()
        if getattr(self, "_stack_key", None) != key:
            with torch.no_grad():
                self._stack_weight = stack_projection_weight(
                    self.to_q.weight, self.to_k.weight, self.to_v.weight,
                    None if self.block_attn_only else self.to_strategy_combine_mlp.weight, self.q_heads, self.kv_heads)
            self._stack_key = key
        return self._stack_weight

    # class-wide switch of the fused input side (mosaic_attn_proj).  Off by default: on the
    # shipped stage-1 shape (1.18 M rows, 768 -> 1280, 24 members) a whole attention block
    # measures 18.0 ms with the library GEMM and the RoPE pooling pass against 18.2 ms with the
    # fused kernel (3.09 ms: its GEMM core is slower than the library's, and every workgroup
    # re-reads its tokens' RoPE tables); set True (or per instance) to take it.
    fused_input_side = False

    def _fused_input_side(self, x):
        """Whether mosaic_attn_proj can run this call: bf16 arithmetic (bf16 autocast, or bf16
        input and weights), q and k rotated by equal tables (or no RoPE), and its shape limits."""
        if not self.fused_input_side:
            return False
        if x.device.type != "cuda" or x.dim() != 3 or self.to_q.out_features != 64 * self.q_heads:
            return False
        bf16 = ((torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16)
                or (x.dtype == torch.bfloat16 and self.to_q.weight.dtype == torch.bfloat16))
        S_, _, dim = x.shape
        if not bf16 or S_ % 256 or dim % 128:
            return False
        if not self.block_attn_only and (self.sparse_block_size not in (64, 128) or 3 * self.q_heads > 64):
            return False
        return self.q_rope is None or self._shared_rope_tables()

    def forward(self, x):
        S_, B_ = x.shape[:2]
        forward_only("MosaicAttention", x, *self.parameters())
        if self._fused_input_side(x):
            # projection, RoPE, gate softmax and pooling in one kernel, then the op
            o = torch.empty(S_, B_, 64 * self.q_heads, dtype=torch.bfloat16, device=x.device)
            o_view = o.view(S_, B_, self.q_heads, -1).transpose(0, 1)
            record = self.record_block_indices is not None
            rope = {} if self.q_rope is None else dict(rope_cos=self.q_rope.cos_freqs, rope_sin=self.q_rope.sin_freqs)
            res = mosaic_attn_proj(x, self._stacked_weight(), self.q_heads, self.kv_heads, self.block_attn_size,
                                   self.sparse_block_size, self.sparse_block_count, self.block_attn_only,
                                   self.no_compression, out=o_view, return_block_indices=record, **rope)
            if record:
                self.record_block_indices.append(res[1])
            return self.to_o(o)
        q, k, v, logits = self._projections(x)
        q = q.unflatten(-1, (self.q_heads, -1)).transpose(0, 1)
        k = k.unflatten(-1, (self.kv_heads, -1)).transpose(0, 1)
        v = v.unflatten(-1, (self.kv_heads, -1)).transpose(0, 1)
        w = None
        if logits is not None:      # generate_strategy_weights on the fused GEMM's slice
            if logits.is_cuda and logits.dtype == torch.bfloat16 and x.dtype == torch.bfloat16:
                w = fused.gate_softmax(logits, self.q_heads).unsqueeze(-1)   # one pass, same values
            else:
                logits = logits.unflatten(-1, (self.q_heads, 3)).permute(3, 1, 0, 2)
                w = torch.softmax(logits.float(), dim=0).type_as(x).unsqueeze(-1)
        args = dict(block_attn_size=self.block_attn_size, sparse_block_size=self.sparse_block_size,
                    sparse_block_count=self.sparse_block_count, block_attn_only=self.block_attn_only,
                    no_compression=self.no_compression)
        # the kernel writes sequence-first rows ('b s h d -> s b (h d)', primitives.py:207), so
        # to_o reads one contiguous [S*B, Hq*64] matrix (a transposed view would make the GEMM
        # a batch of S tiny products)
        o = torch.empty(S_, B_, self.q_heads * q.shape[-1], dtype=torch.bfloat16, device=x.device)
        o_view = o.view(S_, B_, self.q_heads, -1).transpose(0, 1)
        record = self.record_block_indices is not None
        if self.q_rope is not None and self._shared_rope_tables():
            # the rotation runs inside the op's pooling pass (one read of q and k)
            res = mosaic_attn_func_rope(q, k, v, w, self.q_rope.cos_freqs, self.q_rope.sin_freqs, **args,
                                        out=o_view, return_block_indices=record)
        else:
            if self.q_rope is not None:
                q = self.q_rope(q)
                k = self.k_rope(k)
            res = mosaic_attn_func(q=q, k=k, v=v, weight_ba_cmp_slc=w, **args, out=o_view,
                                   return_block_indices=record)
        if record:
            self.record_block_indices.append(res[1])
        return self.to_o(o.to(q.dtype))
