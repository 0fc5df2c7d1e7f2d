"""Selected-branch attention: the MI355X drop-in for the reference's ops.py.

Same names and arguments as the reference:
  * ``mosaic_sparse_attn(q, k, v, block_indices, block_size, softmax_scale=None)``
    (ops.py:557-566): ``softmax_scale`` defaults to ``head_dim ** -0.5``.
  * ``MosaicAttnFunction`` (ops.py:510-554): forward and backward run HIP kernels.
  * ``mosaic_attn_fwd(q, k, v, block_indices, block_size, softmax_scale)`` (ops.py:137-176)
    returns ``(output, lse)`` with lse the base-2 log-sum-exp, fp32 [B, N, Hq].
  * ``mosaic_attn_bwd(q, k, v, output, lse, grad_o, softmax_scale, block_indices,
    block_size)`` (ops.py:437-507) returns ``(grad_q, grad_k, grad_v)``.

q [B, N, Hq, 64], k/v [B, N, Hk, 64] on a ROCm device; block_indices int64 [B, N/bs, Hk, K].
Work is enqueued on the current stream.  The computation is bf16 (like the reference kernel,
which casts q/k/v to bf16, ops.py:92,115-116); fp16 and fp32 inputs are converted to bf16 and
the output is returned in q's dtype (ops.py:538).  As in the reference, ``MosaicAttnFunction``
is marked ``torch.amp.custom_fwd`` / ``custom_bwd`` (ops.py:513, 541), so its backward runs
under the forward's autocast state.
"""

from __future__ import annotations

import torch

from . import _lib


def forward_only(what: str, *tensors) -> None:
    """Raise where autograd would need a backward that ``what`` does not have.

    The three-branch op, the local / dense / pooling pieces, the fused norm and gate and the
    k-NN interpolation have no backward here (the reference differentiates them through
    flash-attn and eager torch); only the selected branch (``mosaic_sparse_attn``) does.  Rather
    than return outputs cut off from the graph, these ops refuse inputs that require grad while
    grad mode is on.
    """
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        raise RuntimeError(
            f"{what} has no backward in mosaic_amd: call it under torch.no_grad() or "
            "torch.inference_mode(), or on tensors that do not require grad (the selected branch, "
            "mosaic_sparse_attn, is differentiable)")


def _as_bf16_bnhd(t: torch.Tensor, name: str, allow_fp16: bool = False) -> torch.Tensor:
    """t as a bf16 [B, N, H, d] device tensor with 16-byte rows (copying only if needed).

    float16 is refused unless ``allow_fp16``: the kernels compute in bf16, and where the
    reference computes in fp16 (flash-attn under fp16 autocast) converting would silently drop
    three mantissa bits.  The selected branch converts fp16 to bf16 as the reference's own
    kernel does (ops.py:92, 115-116), so it allows it.
    """
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, N, H, d], got shape {tuple(t.shape)}")
    if t.dtype == torch.float16 and not allow_fp16:
        raise TypeError(f"{name} is float16: these kernels compute in bfloat16 (run the model under "
                        "torch.autocast(..., dtype=torch.bfloat16), or convert the inputs)")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm device, got {t.device}")
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
        t = t.contiguous()
    return t


def bnhd(t: torch.Tensor) -> _lib.Bnhd:
    return _lib.Bnhd(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree on batch/seq/head_dim")


def mosaic_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                    block_size: int, softmax_scale: float):
    """(output bf16 [B, N, Hq, d], lse fp32 [B, N, Hq]) of the selected-branch attention."""
    q, k, v = (_as_bf16_bnhd(t, n, allow_fp16=True) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    _check_gqa(q, k, v)
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    if block_indices.dim() != 4:
        raise ValueError("block_indices must be [B, N/block_size, Hk, K]")
    idx = block_indices.to(device=q.device, dtype=torch.int64).contiguous()
    if N % block_size == 0 and tuple(idx.shape[:3]) != (B, N // block_size, Hk):
        raise ValueError(f"block_indices shape {tuple(idx.shape)} != {(B, N // block_size, Hk, '*')}")
    out = torch.empty(B, N, Hq, d, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, N, Hq, dtype=torch.float32, device=q.device)
    L = _lib.lib()
    # workspace for the key-norm bounds of k's blocks (lets query tiles take the bounded path)
    nbytes = L.mosaic_sparse_attn_fwd_workspace_size(B, N, Hk, int(block_size))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    st = L.mosaic_sparse_attn_fwd_ws(
        bnhd(q), bnhd(k), bnhd(v), idx.data_ptr(), B, N, Hq, Hk, d, int(block_size), int(idx.shape[-1]),
        float(softmax_scale), out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(q))
    _lib.check(st, "mosaic_sparse_attn_fwd_ws")
    return out, lse


def mosaic_attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, output: torch.Tensor, lse: torch.Tensor,
                    grad_o: torch.Tensor, softmax_scale: float, block_indices: torch.Tensor, block_size: int):
    """(grad_q, grad_k, grad_v) of the selected-branch attention (ops.py:437-507), in q's / k's /
    v's dtypes; keys no query block selected get zero gradients."""
    dtypes = (q.dtype, k.dtype, v.dtype)
    q, k, v = (_as_bf16_bnhd(t, n, allow_fp16=True) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    go = _as_bf16_bnhd(grad_o, "grad_o", allow_fp16=True)
    _check_gqa(q, k, v)
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    if tuple(go.shape) != (B, N, Hq, d):
        raise ValueError(f"grad_o shape {tuple(go.shape)} != {(B, N, Hq, d)}")
    # the kernels index these as contiguous [B, N, Hq, 64], [B, N, Hq] and [B, N/bs, Hk, K]
    if tuple(output.shape) != (B, N, Hq, d):
        raise ValueError(f"output shape {tuple(output.shape)} != {(B, N, Hq, d)}")
    if tuple(lse.shape) != (B, N, Hq):
        raise ValueError(f"lse shape {tuple(lse.shape)} != {(B, N, Hq)}")
    if block_size <= 0 or N % block_size:
        raise ValueError(f"block_size {block_size} must divide the sequence length {N}")
    if block_indices.dim() != 4 or tuple(block_indices.shape[:3]) != (B, N // block_size, Hk):
        raise ValueError(f"block_indices shape {tuple(block_indices.shape)} != {(B, N // block_size, Hk, '*')}")
    o = output.to(device=q.device, dtype=torch.bfloat16).contiguous()
    lse = lse.to(device=q.device, dtype=torch.float32).contiguous()
    idx = block_indices.to(device=q.device, dtype=torch.int64).contiguous()
    gq = torch.empty(B, N, Hq, d, dtype=torch.bfloat16, device=q.device)
    gk = torch.empty(B, N, Hk, d, dtype=torch.bfloat16, device=q.device)
    gv = torch.empty(B, N, Hk, d, dtype=torch.bfloat16, device=q.device)
    L = _lib.lib()
    nbytes = L.mosaic_sparse_attn_bwd_workspace_size(B, N, Hq)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    st = L.mosaic_sparse_attn_bwd(bnhd(q), bnhd(k), bnhd(v), o.data_ptr(), lse.data_ptr(), bnhd(go), idx.data_ptr(),
                                  B, N, Hq, Hk, d, int(block_size), int(idx.shape[-1]), float(softmax_scale),
                                  gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), ws.data_ptr(), ws.numel(),
                                  stream_of(q))
    _lib.check(st, "mosaic_sparse_attn_bwd")
    return gq.to(dtypes[0]), gk.to(dtypes[1]), gv.to(dtypes[2])


class MosaicAttnFunction(torch.autograd.Function):
    """Autograd function of the selected-branch attention (ops.py:510-554): the forward saves
    q, k, v, the output, its LSE and the indices; the backward runs the HIP backward."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, q, k, v, block_indices, block_size, softmax_scale):
        dtype = q.dtype
        output, lse = mosaic_attn_fwd(q, k, v, block_indices, block_size, softmax_scale)
        ctx.save_for_backward(q, k, v, output, lse, block_indices)
        ctx.block_size = block_size
        ctx.softmax_scale = softmax_scale
        return output.to(dtype)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_o):
        q, k, v, output, lse, block_indices = ctx.saved_tensors
        gq, gk, gv = mosaic_attn_bwd(q, k, v, output, lse, grad_o.contiguous(), ctx.softmax_scale,
                                     block_indices, ctx.block_size)
        return gq, gk, gv, None, None, None


def mosaic_sparse_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                       block_size: int, softmax_scale: float | None = None) -> torch.Tensor:
    """Attention of each query block over its selected key blocks (ops.py:557-566)."""
    softmax_scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    return MosaicAttnFunction.apply(q, k, v, block_indices, block_size, softmax_scale)
