"""The allocation-free forward, mosaic_bsa_fwd_noalloc, against mosaic_bsa_fwd (GPU).

Both entry points run the same kernels; the no-allocation one takes its workspace from the
library's static per-device scratch instead of a caller buffer.  Two calls in a row, the second
on a smaller problem, must each reproduce mosaic_bsa_fwd bit for bit (output and selected
indices), so stale scratch contents from the first call cannot leak into the second.
"""

import ctypes

import pytest
import torch

from mosaic_amd import _lib
from mosaic_amd.inputs import Workload, make_inputs
from mosaic_amd.ops import stream_of
from mosaic_amd.primitives import _bsa_args, _workspace

pytestmark = pytest.mark.gpu

CALLS = [
    # name, nside, batch, Hq, Hk, bs_l, bs, K
    Workload("nside16_h20kv5_bs64_top4", 16, 1, 20, 5, 64, 64, 64, 4, False),
    Workload("nside8_b2_h12kv3_bl128_top8", 8, 2, 12, 3, 64, 128, 64, 8, False),
]


def _run(wl, mode, noalloc):
    q, k, v, w = (t.cuda() for t in make_inputs(wl, seed=3))
    B, N, Hq, _ = q.shape
    Hk = k.shape[2]
    nb = N // wl.sparse_block_size
    out = torch.full((B, N, Hq, 64), float("nan"), dtype=torch.bfloat16, device="cuda")
    selects = mode in (_lib.MODE_FULL, _lib.MODE_NO_COMPRESSION)
    idx = torch.full((B, nb, Hk, wl.sparse_block_count), -7, dtype=torch.int64, device="cuda") if selects else None
    K = wl.sparse_block_count if mode != _lib.MODE_NO_SELECTION else 0
    a = _bsa_args(q, k, v, w[..., 0], out, wl.block_attn_size, wl.sparse_block_size, K, mode, idx)
    L = _lib.lib()
    if noalloc:
        st = L.mosaic_bsa_fwd_noalloc(ctypes.byref(a), stream_of(q))
    else:
        ws = _workspace(L.mosaic_bsa_workspace_size(ctypes.byref(a)), q.device)
        st = L.mosaic_bsa_fwd(ctypes.byref(a), ws.data_ptr(), ws.numel(), stream_of(q))
    torch.cuda.synchronize()
    assert st == 0, _lib.strerror(st)
    return out.cpu(), (idx.cpu() if idx is not None else None)


@pytest.mark.parametrize("mode", [_lib.MODE_FULL, _lib.MODE_NO_COMPRESSION, _lib.MODE_NO_SELECTION],
                         ids=["full", "no_compression", "no_selection"])
def test_noalloc_matches_workspace_entry_two_calls(mode):
    for wl in CALLS:   # the second call is smaller than the first
        print(f"noalloc {wl.name} mode {mode}", flush=True)
        ref_out, ref_idx = _run(wl, mode, noalloc=False)
        got_out, got_idx = _run(wl, mode, noalloc=True)
        assert torch.isfinite(got_out.float()).all()
        assert torch.equal(got_out, ref_out)
        if ref_idx is not None:
            assert torch.equal(got_idx, ref_idx)


def test_noalloc_rejects_requests_beyond_scratch():
    # N = 393216 with 12/3 heads and 64-token blocks needs ~260 MB of workspace
    q = torch.empty(1, 393216, 12, 64, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(1, 393216, 3, 64, dtype=torch.bfloat16, device="cuda")
    w = torch.empty(3, 1, 393216, 12, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    a = _bsa_args(q, k, k, w, out, 64, 64, 16, _lib.MODE_FULL, None)
    L = _lib.lib()
    assert L.mosaic_bsa_workspace_size(ctypes.byref(a)) > _lib.NOALLOC_SCRATCH_BYTES
    assert L.mosaic_bsa_fwd_noalloc(ctypes.byref(a), stream_of(q)) == _lib.ERR_SCRATCH_LIMIT
