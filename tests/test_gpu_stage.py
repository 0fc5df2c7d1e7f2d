"""mosaic_bsa_fwd_stage: each kernel of the forward alone reproduces the whole call (GPU).

The stages re-run on the workspace a complete forward left must rewrite exactly what that call
wrote, so the output after the stages, in order or the attention kernel alone again, is
bit-identical to the call's (the benchmark times the kernels this way).
"""

import ctypes

import pytest
import torch

from mosaic_amd import _lib
from mosaic_amd.inputs import BOTTLENECK_NSIDE16, make_inputs
from mosaic_amd.ops import bnhd

DEV = "cuda"


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [_lib.MODE_FULL, _lib.MODE_NO_SELECTION, _lib.MODE_LOCAL_ONLY])
def test_stages_alone_reproduce_the_call(mode):
    print(f"stage entry, mode {mode}", flush=True)
    q, k, v, w = (t.to(DEV) for t in make_inputs(BOTTLENECK_NSIDE16, seed=3))
    w4 = w[..., 0]
    B, N, Hq, d = q.shape
    L = _lib.lib()
    a = _lib.BsaArgs()
    a.batch, a.seq_len, a.num_q_heads, a.num_kv_heads, a.head_dim = B, N, Hq, k.shape[2], d
    a.block_attn_size, a.sparse_block_size, a.sparse_block_count = 64, 64, 4
    a.mode, a.softmax_scale = mode, 0.0
    a.q, a.k, a.v = bnhd(q), bnhd(k), bnhd(v)
    a.weights = w4.data_ptr() if mode != _lib.MODE_LOCAL_ONLY else None
    a.w_stride_s, a.w_stride_b, a.w_stride_n, a.w_stride_h = (w4.stride(i) for i in range(4))
    out = torch.empty_like(q)
    a.out = out.data_ptr()
    n = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    ws = torch.empty(n + 256, dtype=torch.uint8, device=DEV)
    wp = (ws.data_ptr() + 255) // 256 * 256 if n else None
    sp = torch.cuda.current_stream().cuda_stream
    assert L.mosaic_bsa_fwd(ctypes.byref(a), wp, n, sp) == 0
    ref = out.clone()
    out.fill_(float("nan"))
    for stage in (_lib.STAGE_POOL, _lib.STAGE_CMP, _lib.STAGE_TOPK, _lib.STAGE_ATTN):
        assert L.mosaic_bsa_fwd_stage(ctypes.byref(a), wp, n, sp, stage) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    out.fill_(float("nan"))
    for _ in range(3):
        assert L.mosaic_bsa_fwd_stage(ctypes.byref(a), wp, n, sp, _lib.STAGE_ATTN) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
