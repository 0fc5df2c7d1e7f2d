"""Host-side behaviour of the Python boundary that needs no GPU (CPU only).

* Ops without a backward refuse inputs that require grad while grad mode is on, instead of
  returning outputs cut off from the autograd graph; the check runs before any device check,
  so CPU tensors show it.
* float16 is refused where the reference computes in fp16 (flash-attn branches, the k-NN
  interpolation under fp16 autocast) and accepted by the selected branch, whose reference
  kernel converts to bf16 itself (ops.py:92, 115-116).
* MosaicAttnFunction carries the reference's autocast decorators (ops.py:513, 541).
* mosaic_attn_bwd validates the shapes of output, lse and block_indices before any launch.
"""

import pytest
import torch

import mosaic_amd as M
from mosaic_amd import fused, ops
from mosaic_amd.interp import knn_attention


def t(*shape, grad=False, dtype=torch.bfloat16):
    x = torch.zeros(*shape, dtype=dtype)
    return x.requires_grad_() if grad else x


Q, KV = (1, 256, 4, 64), (1, 256, 1, 64)
W = (3, 1, 256, 4, 1)


@pytest.mark.parametrize("call", [
    lambda g: M.mosaic_attn_func(t(*Q, grad=g), t(*KV), t(*KV), t(*W), 64, 64, 2, False),
    lambda g: M.mosaic_attn_func(t(*Q), t(*KV), t(*KV), t(*W, grad=g), 64, 64, 2, False),
    lambda g: M.primitives.mosaic_attn_func_rope(t(*Q), t(*KV, grad=g), t(*KV), t(*W), t(256, 32, dtype=torch.float32),
                                                 t(256, 32, dtype=torch.float32), 64, 64, 2, False),
    lambda g: M.block_attention(t(*Q), t(*KV), t(*KV, grad=g), 64),
    lambda g: M.dense_attention(t(*Q, grad=g), t(*KV), t(*KV)),
    lambda g: M.pool_mean(t(*Q, grad=g), 64),
    lambda g: fused.rms_norm(t(4, 64, grad=g), None, None),
    lambda g: fused.rms_norm(t(4, 64), t(64, grad=g, dtype=torch.float32), None),
    lambda g: fused.swiglu(t(4, 2, 128, grad=g)),
    lambda g: knn_attention(t(10, 1, 1, 64, grad=g), t(10, 1, 1, 64), torch.zeros(5, 3, dtype=torch.long),
                            t(5, 3, 3, dtype=torch.float32), t(64, 3)),
], ids=["attn_q", "attn_weights", "attn_rope", "block_attention", "dense_attention", "pool_mean", "rms_norm",
        "rms_norm_weight", "swiglu", "knn_attention"])
def test_forward_only_ops_refuse_grad(call):
    with pytest.raises(RuntimeError, match="no backward"):
        call(True)
    # without grad the op gets past the guard (and then needs a device tensor)
    with torch.no_grad(), pytest.raises(ValueError, match="ROCm|device"):
        call(True)
    with pytest.raises(ValueError, match="ROCm|device"):
        call(False)


def test_rms_norm_module_with_trainable_weight_refuses_grad_on_device_path():
    m = fused.RMSNorm(64)
    x = t(4, 64)
    # the CPU path is torch's own differentiable RMSNorm
    assert m(x.float().requires_grad_()).requires_grad
    with pytest.raises(RuntimeError, match="no backward"):
        fused.rms_norm(x, m.weight, m.eps)


@pytest.mark.parametrize("call", [
    lambda: M.mosaic_attn_func(t(*Q, dtype=torch.float16), t(*KV), t(*KV), t(*W), 64, 64, 2, False),
    lambda: M.block_attention(t(*Q, dtype=torch.float16), t(*KV), t(*KV), 64),
    lambda: M.dense_attention(t(*Q, dtype=torch.float16), t(*KV), t(*KV)),
    lambda: knn_attention(t(10, 1, 1, 64, dtype=torch.float16), t(10, 1, 1, 64, dtype=torch.float16),
                          torch.zeros(5, 3, dtype=torch.long), t(5, 3, 3, dtype=torch.float32), t(64, 3)),
], ids=["mosaic_attn_func", "block_attention", "dense_attention", "knn_attention"])
def test_fp16_is_refused_where_the_reference_computes_in_fp16(call):
    with pytest.raises(TypeError, match="bfloat16"):
        call()


def test_selected_branch_accepts_fp16_as_the_reference_kernel_does():
    idx = torch.zeros(1, 4, 1, 2, dtype=torch.long)
    # gets past the dtype check and stops at the device check
    with pytest.raises(ValueError, match="ROCm"):
        ops.mosaic_attn_fwd(t(*Q, dtype=torch.float16), t(*KV, dtype=torch.float16), t(*KV, dtype=torch.float16),
                            idx, 64, 0.125)


def test_autograd_function_has_the_reference_autocast_decorators():
    # torch.amp.custom_fwd / custom_bwd wrap the staticmethods (functools.wraps keeps __wrapped__)
    assert hasattr(ops.MosaicAttnFunction.forward, "__wrapped__")
    assert hasattr(ops.MosaicAttnFunction.backward, "__wrapped__")


@pytest.mark.parametrize("change", ["output", "lse", "indices_nb", "indices_heads", "block_size"])
def test_backward_validates_shapes(change, monkeypatch):
    # device tensors are not available here: skip the device conversion to reach the checks
    monkeypatch.setattr(ops, "_as_bf16_bnhd", lambda x, name, allow_fp16=False: x)
    B, N, Hq, Hk, bs, K = 1, 256, 4, 1, 64, 2
    q, k, v, go = t(B, N, Hq, 64), t(B, N, Hk, 64), t(B, N, Hk, 64), t(B, N, Hq, 64)
    o, lse = t(B, N, Hq, 64), t(B, N, Hq, dtype=torch.float32)
    idx = torch.zeros(B, N // bs, Hk, K, dtype=torch.long)
    if change == "output":
        o = t(B, N, Hk, 64)
    elif change == "lse":
        lse = t(B, Hq, N, dtype=torch.float32)
    elif change == "indices_nb":
        idx = torch.zeros(B, N // bs - 1, Hk, K, dtype=torch.long)
    elif change == "indices_heads":
        idx = torch.zeros(B, N // bs, Hk + 1, K, dtype=torch.long)
    else:
        bs = 96
    with pytest.raises(ValueError):
        ops.mosaic_attn_bwd(q, k, v, o, lse, go, 0.125, idx, bs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float64])
@pytest.mark.parametrize("return_sum", [True, False])
def test_rms_norm_residual_pairs_the_kernel_does_not_read_never_reach_it(dtype, return_sum, monkeypatch):
    # x and residual share a dtype the kernel does not take: the kernel must only ever see
    # buffers whose dtype matches the dtype code it is given (an fp16 residual passed as fp32
    # would be read past its end).  The launch is recorded instead of run.
    calls = []

    class FakeLib:
        def mosaic_rms_norm_fwd(self, x, r, dt, rows, C, xs, rs, w, eps, s_out, out, out_dt, stream):
            calls.append(dict(x=x, r=r, dt=dt, out_dt=out_dt, rows=rows, C=C, xs=xs, rs=rs))
            return 0

    monkeypatch.setattr(fused, "_on_device", lambda x: True)
    monkeypatch.setattr(fused, "stream_of", lambda x: 0)
    monkeypatch.setattr(fused._lib, "lib", lambda: FakeLib())
    x = torch.randn(4, 64).to(dtype)
    res = torch.randn(4, 64).to(dtype)
    out = fused.rms_norm(x, None, None, residual=res, return_sum=return_sum)
    assert len(calls) == 1
    call = calls[0]
    assert call["r"] is None                   # the sum was formed by torch, not by the kernel
    assert call["dt"] == fused._lib.DTYPE_F32  # the kernel read an fp32 copy of the sum
    assert call["xs"] == 64 and call["rows"] == 4 and call["C"] == 64
    if return_sum:
        s, out = out
        assert s.dtype == dtype and torch.equal(s, x + res)
    assert out.dtype == dtype                  # torch.nn.RMSNorm's output dtype for this input
