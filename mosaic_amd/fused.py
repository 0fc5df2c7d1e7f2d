"""The model's row-wise elementwise work as single HIP passes (libmosaic_bsa.so).

* ``rms_norm(x, weight, eps, out_dtype, residual=None)``: torch.nn.RMSNorm over the last
  dimension, optionally after ``x + residual`` (returned too), as MosaicBlock applies them
  (primitives.py:220-226).
* ``RMSNorm``: ``torch.nn.RMSNorm`` (same parameters) running ``rms_norm`` on a ROCm device,
  with ``add_forward`` for the residual-add variant.
* ``swiglu(h, noise)``: the gate ``silu(x1 + noise) * x3`` of cSwiGLU (primitives.py:102-105).
* ``add_merge(x, residual, factor)``: an encoder stage's last residual add and the merge of each
  coarse pixel's children for the downsampling projection (mosaic.py:318-321), one pass.
* ``gate_softmax(logits, heads)``: MosaicAttention's branch weights, the softmax over the three
  logits of each head (primitives.py:173-180), from the projection's gate slice.
* ``resample_norm(p, pos, weight, eps, factor, shortcut)``: the epilogue of the HEALPix
  up/downsampling layers (primitives.py:313-359): split, position term, skip connection and
  RMSNorm in one pass.
* ``swiglu_linear(x, w13_perm, noise)``: cSwiGLU's ``w13`` projection and that gate in one
  kernel (h is never stored); ``permute_w13`` lays out the weight it takes.

Inputs must be on a ROCm device; there is no CPU path.  ``autocast_dtype`` reports the dtype
torch's own RMSNorm returns under the current autocast state, so the fused norm's output has
the dtype the reference's module would have.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .ops import forward_only, stream_of

__all__ = ["RMSNorm", "rms_norm", "swiglu", "swiglu_linear", "permute_w13", "swiglu_linear_ok", "autocast_dtype",
           "resample_norm", "gate_softmax", "add_merge"]

_DT = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}
_autocast_out: dict = {}

# torch's rms_norm with eps=None adds the epsilon of its fp32 accumulation type for fp32 and
# bf16 inputs alike (the statistics are always computed in fp32)
DEFAULT_EPS = torch.finfo(torch.float32).eps


def autocast_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype ``torch.nn.functional.rms_norm`` returns for an input like ``x`` under the
    current autocast state (probed once per state on a 1x8 tensor, then cached)."""
    on = torch.is_autocast_enabled(x.device.type)
    key = (x.dtype, x.device.type, on, torch.get_autocast_dtype(x.device.type) if on else None)
    dt = _autocast_out.get(key)
    if dt is None:
        probe = torch.zeros(1, 8, dtype=x.dtype, device=x.device)
        dt = torch.nn.functional.rms_norm(probe, (8,)).dtype
        _autocast_out[key] = dt
    return dt


def _on_device(t: torch.Tensor) -> bool:
    return t.is_cuda


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """t as [rows, cols] with a unit last stride and one row stride (copying if needed)."""
    t2 = t.reshape(-1, t.shape[-1])
    align = 4 if t.dtype == torch.float32 else 8
    if t2.stride(-1) != 1 or t2.stride(0) % align or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2, t2.stride(0)


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float | None,
             out_dtype: torch.dtype | None = None, residual: torch.Tensor | None = None,
             return_sum: bool = True):
    """RMSNorm of ``x`` (or of ``x + residual``) over its last dimension.

    Returns ``out`` (dtype ``out_dtype``, default x's), or ``(x + residual, out)`` when a
    residual is given; the sum has x's dtype, rounded as torch's add rounds.  With a residual
    and ``return_sum=False`` only ``out`` is returned and the sum is never stored.
    """
    forward_only("fused.rms_norm", x, weight, residual)
    if not _on_device(x):
        raise ValueError("fused.rms_norm needs a ROCm device tensor")
    if residual is not None and (residual.dtype != x.dtype or x.dtype not in _DT):
        # mixed dtypes, or a pair the kernel does not read (fp16, fp64): torch's add with its
        # promotion and rounding, then the plain norm of the sum
        x = x + residual
        out = rms_norm(x, weight, eps, out_dtype)
        return (x, out) if return_sum else out
    out_dtype = out_dtype or x.dtype
    if x.dtype not in _DT:
        x = x.float()                         # statistics in fp32 either way
    if out_dtype not in _DT:                  # the kernel writes fp32, then torch's cast
        return rms_norm(x, weight, eps, torch.float32).to(out_dtype)
    shape = x.shape
    C = shape[-1]
    x2, xs = _rows(x)
    rows = x2.shape[0]
    out = torch.empty(shape, dtype=out_dtype, device=x.device)
    w = None
    if weight is not None:
        w = weight.to(device=x.device, dtype=torch.float32).contiguous()
    r2, rs, s_out = None, 0, None
    if residual is not None:
        r2, rs = _rows(residual.expand(shape))
        if return_sum:
            s_out = torch.empty(shape, dtype=x.dtype, device=x.device)
    st = _lib.lib().mosaic_rms_norm_fwd(
        x2.data_ptr(), r2.data_ptr() if r2 is not None else None, _DT[x.dtype], rows, C, xs, rs,
        w.data_ptr() if w is not None else None, float(DEFAULT_EPS if eps is None else eps),
        s_out.data_ptr() if s_out is not None else None, out.data_ptr(), _DT[out_dtype], stream_of(x))
    _lib.check(st, "mosaic_rms_norm_fwd")
    return (s_out, out) if residual is not None and return_sum else out


def swiglu(h: torch.Tensor, noise: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(x1 + noise) * x3`` for ``x1, x3 = h.chunk(2, -1)``; h is ``[S, B, 2*hidden]``
    (sequence-first) and noise, if given, ``[B, hidden]`` (one row per batch member)."""
    forward_only("fused.swiglu", h, noise)
    if not h.is_cuda:
        raise ValueError("fused.swiglu needs a ROCm device tensor")
    if h.dtype not in _DT:
        raise ValueError(f"unsupported dtype {h.dtype}")
    hidden = h.shape[-1] // 2
    h2, hs = _rows(h)
    rows = h2.shape[0]
    n = None
    if noise is not None:
        n = noise.to(h.dtype).reshape(-1, hidden).contiguous()
        if h.dim() < 2 or h.shape[-2] != n.shape[0]:
            raise ValueError("noise must hold one row per batch member (h.shape[-2])")
    out = torch.empty(*h.shape[:-1], hidden, dtype=h.dtype, device=h.device)
    st = _lib.lib().mosaic_swiglu_fwd(h2.data_ptr(), _DT[h.dtype], rows, hidden, hs,
                                      n.data_ptr() if n is not None else None,
                                      n.shape[0] if n is not None else 0, out.data_ptr(), stream_of(h))
    _lib.check(st, "mosaic_swiglu_fwd")
    return out


def permute_w13(w13: torch.Tensor) -> torch.Tensor:
    """w13 ``[2*hidden, dim]`` with its rows in the order ``swiglu_linear`` takes: 64-row group
    t holds rows 32t..32t+31 of the x1 half, then the same rows of the x3 half."""
    two_h, dim = w13.shape
    hidden = two_h // 2
    if two_h % 2 or hidden % 32:
        raise ValueError(f"w13 rows {two_h} must be 2 * a multiple of 32")
    a = w13[:hidden].reshape(hidden // 32, 32, dim)
    b = w13[hidden:].reshape(hidden // 32, 32, dim)
    return torch.stack([a, b], dim=1).reshape(two_h, dim).contiguous()


def swiglu_linear_ok(x: torch.Tensor, hidden: int) -> bool:
    """Whether ``swiglu_linear`` takes this input: bf16 on a ROCm device, unit stride in the
    last dimension, rows a multiple of 256, dim and hidden multiples of 128."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or x.dim() < 2 or x.stride(-1) != 1:
        return False
    rows = x.numel() // x.shape[-1]
    return rows > 0 and rows % 256 == 0 and x.shape[-1] % 128 == 0 and hidden % 128 == 0


def swiglu_linear(x: torch.Tensor, w13_perm: torch.Tensor, noise: torch.Tensor | None = None) -> torch.Tensor:
    """``swiglu(x @ w13^T, noise)`` in one kernel: the projection (bf16 operands, fp32
    accumulation, rounded to bf16 as a bf16 Linear) and the gate with its rounding points.
    x: bf16 ``[..., dim]`` (rows sequence-first ``[S, B]`` when noise is given); w13_perm:
    ``permute_w13(w13)`` in bf16; noise: ``[B, hidden]`` or None.  Returns ``[..., hidden]``."""
    forward_only("fused.swiglu_linear", x, w13_perm, noise)
    two_h, dim = w13_perm.shape
    hidden = two_h // 2
    if x.shape[-1] != dim:
        raise ValueError(f"x has {x.shape[-1]} features, the weight {dim}")
    if not swiglu_linear_ok(x, hidden):
        raise ValueError("swiglu_linear needs bf16 ROCm input with rows % 256 == 0, dim % 128 == 0, hidden % 128 == 0")
    if w13_perm.dtype != torch.bfloat16 or not w13_perm.is_contiguous() or w13_perm.device != x.device:
        raise ValueError("w13_perm must be a contiguous bf16 tensor on x's device")
    x2 = x.reshape(-1, dim)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    n = None
    if noise is not None:
        n = noise.to(torch.bfloat16).reshape(-1, hidden).contiguous()
        if x.dim() < 2 or x.shape[-2] != n.shape[0]:
            raise ValueError("noise must hold one row per batch member (x.shape[-2])")
    out = torch.empty(*x.shape[:-1], hidden, dtype=torch.bfloat16, device=x.device)
    st = _lib.lib().mosaic_swiglu_linear_fwd(x2.data_ptr(), rows, dim, x2.stride(0), w13_perm.data_ptr(), hidden,
                                             n.data_ptr() if n is not None else None,
                                             n.shape[0] if n is not None else 0, out.data_ptr(), stream_of(x))
    _lib.check(st, "mosaic_swiglu_linear_fwd")
    return out


class RMSNorm(nn.RMSNorm):
    """``torch.nn.RMSNorm`` (same parameters and eps rule) whose forward on a ROCm device is
    one fused kernel: fp32 statistics, output in the autocast dtype when autocast is on (the
    module's output dtype under the reference's bf16 autocast), else in the input's dtype.
    Forward-only on the device: with grad mode on and an input or the weight requiring grad it
    raises rather than return an output without a graph."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda:
            return rms_norm(x, self.weight, self.eps, out_dtype=autocast_dtype(x))
        return super().forward(x)

    def add_forward(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``(x + residual, self(x + residual))``; on a ROCm device one kernel reads x and the
        residual once and writes both results."""
        if x.is_cuda and x.dtype == residual.dtype:
            y, out = rms_norm(x, self.weight, self.eps, out_dtype=autocast_dtype(x), residual=residual)
            return y, out
        y = x + residual
        return y, self(y)

    def add_norm(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """``self(x + residual)`` without storing the sum; on a ROCm device one kernel."""
        if x.is_cuda and x.dtype == residual.dtype:
            return rms_norm(x, self.weight, self.eps, out_dtype=autocast_dtype(x), residual=residual,
                            return_sum=False)
        return self(x + residual)


def resample_norm(p: torch.Tensor, pos: torch.Tensor, weight: torch.Tensor | None, eps: float | None,
                  factor: int, shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """The epilogue of HEALPixUpsample / HEALPixDownsample (primitives.py:313-359) in one kernel:
    ``rms_norm(split(p + pos[:, None]) (+ shortcut))`` where ``split`` is the
    ``'n b (f d) -> (n f) b d'`` rearrangement.  p: bf16 ``[n, B, factor * d]`` (unit last
    stride), pos: bf16 ``[n, factor * d]``, shortcut: bf16 ``[n * factor, B, d]`` or None.  The
    adds round to bf16 as torch's bf16 adds do; the norm is ``rms_norm``'s.  Returns bf16
    ``[n * factor, B, d]``."""
    forward_only("fused.resample_norm", p, pos, shortcut, weight)
    if p.dim() != 3 or p.dtype != torch.bfloat16 or not p.is_cuda:
        raise ValueError("resample_norm needs a bf16 ROCm tensor p of shape [n, B, factor * d]")
    n, B, fd = p.shape
    if fd % factor:
        raise ValueError(f"p's last dimension {fd} is not a multiple of factor {factor}")
    d = fd // factor
    if pos.shape != (n, fd) or pos.dtype != torch.bfloat16:
        raise ValueError(f"pos must be bf16 [{n}, {fd}], got {tuple(pos.shape)} {pos.dtype}")
    p2 = p.reshape(n * B, fd)
    if p2.stride(-1) != 1 or p2.stride(0) % 8 or p2.data_ptr() % 16:
        p2 = p2.contiguous()
    pos = pos.contiguous()
    sc = None
    if shortcut is not None:
        if shortcut.shape != (n * factor, B, d) or shortcut.dtype != torch.bfloat16:
            raise ValueError(f"shortcut must be bf16 [{n * factor}, {B}, {d}], got {tuple(shortcut.shape)}")
        sc = shortcut.contiguous()
    w = None
    if weight is not None:
        w = weight.to(device=p.device, dtype=torch.float32).contiguous()
    out = torch.empty(n * factor, B, d, dtype=torch.bfloat16, device=p.device)
    st = _lib.lib().mosaic_resample_norm_fwd(p2.data_ptr(), p2.stride(0), pos.data_ptr(),
                                             sc.data_ptr() if sc is not None else None,
                                             w.data_ptr() if w is not None else None,
                                             float(DEFAULT_EPS if eps is None else eps), n, B, factor, d,
                                             out.data_ptr(), stream_of(p))
    _lib.check(st, "mosaic_resample_norm_fwd")
    return out


def gate_softmax(logits: torch.Tensor, heads: int) -> torch.Tensor:
    """``torch.softmax(logits.unflatten(-1, (heads, 3)).permute(3, 1, 0, 2).float(), dim=0)``
    rounded to bf16, in one kernel: logits bf16 ``[S, B, 3 * heads]`` sequence-first (a slice
    of a wider projection is fine); returns bf16 ``[3, B, S, heads]``."""
    forward_only("fused.gate_softmax", logits)
    if logits.dim() != 3 or logits.dtype != torch.bfloat16 or not logits.is_cuda or logits.shape[-1] != 3 * heads:
        raise ValueError(f"gate_softmax needs bf16 ROCm logits [S, B, {3 * heads}], got {tuple(logits.shape)}")
    S, B, _ = logits.shape
    if logits.stride(-1) != 1 or logits.stride(0) != B * logits.stride(1):
        logits = logits.contiguous()
    w = torch.empty(3, B, S, heads, dtype=torch.bfloat16, device=logits.device)
    st = _lib.lib().mosaic_gate_softmax_fwd(logits.data_ptr(), logits.stride(1), S, B, heads, w.data_ptr(),
                                            stream_of(logits))
    _lib.check(st, "mosaic_gate_softmax_fwd")
    return w


def add_merge(x: torch.Tensor, residual: torch.Tensor, factor: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``s = x + residual`` (bf16, rounded as torch's add) and ``s`` merged per coarse pixel,
    ``s.view(n, f, B, C).transpose(1, 2).reshape(n, B, f * C)``, in one kernel.  x, residual:
    bf16 ``[n * factor, B, C]``; returns ``(s, merged)``."""
    forward_only("fused.add_merge", x, residual)
    if x.dim() != 3 or x.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("add_merge needs bf16 ROCm tensors [n * factor, B, C]")
    if residual.shape != x.shape:
        raise ValueError(f"residual {tuple(residual.shape)} does not match x {tuple(x.shape)}")
    S, B, C = x.shape
    if S % factor:
        raise ValueError(f"{S} rows are not a multiple of factor {factor}")
    x, residual = x.contiguous(), residual.contiguous()
    s = torch.empty_like(x)
    merged = torch.empty(S // factor, B, factor * C, dtype=torch.bfloat16, device=x.device)
    st = _lib.lib().mosaic_add_merge_fwd(x.data_ptr(), residual.data_ptr(), S // factor, B, factor, C,
                                         s.data_ptr(), merged.data_ptr(), stream_of(x))
    _lib.check(st, "mosaic_add_merge_fwd")
    return s, merged
