"""C-ABI checks that need no GPU: the library loads, exports every declared symbol, and rejects
invalid arguments on the host before any launch (CPU only)."""

import ctypes
import os
import re

import pytest

from mosaic_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mosaic_bsa.h")

pytestmark = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH),
                                reason="libmosaic_bsa.so not built (python -m mosaic_amd.build)")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"MOSAIC_API\s+[\w\s\*]+?\b(mosaic_\w+)\s*\(", text)))


def test_header_declarations_match_binding_list():
    assert declared_symbols() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(handle, name), name


def test_abi_version_and_strerror():
    L = _lib.lib()
    assert L.mosaic_bsa_abi_version() == _lib.ABI_VERSION
    assert _lib.strerror(0) == "ok"
    for code in range(1, 13):
        assert _lib.strerror(code) not in ("ok", "unknown status")
    assert _lib.strerror(999) == "unknown status"


FAKE = 1 << 20  # non-null, 16-byte aligned host address; never dereferenced (validation fails first)


def _args(**kw):
    a = _lib.BsaArgs()
    a.batch, a.seq_len, a.num_q_heads, a.num_kv_heads, a.head_dim = 1, 3072, 20, 5, 64
    a.block_attn_size, a.sparse_block_size, a.sparse_block_count = 64, 64, 4
    a.mode = _lib.MODE_FULL
    for name in ("q", "k", "v"):
        setattr(a, name, _lib.Bnhd(FAKE, 3072 * 20 * 64, 20 * 64, 64))
    a.weights, a.out = FAKE, FAKE
    a.w_stride_s, a.w_stride_b, a.w_stride_n, a.w_stride_h = 3072 * 20, 3072 * 20, 20, 1
    for key, val in kw.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("change,status", [
    (dict(head_dim=32), 2),
    (dict(num_q_heads=21), 3),
    (dict(num_q_heads=5 * 17), 11),
    (dict(sparse_block_size=96), 4),
    (dict(block_attn_size=100), 4),
    (dict(sparse_block_count=49), 5),
    (dict(sparse_block_count=0), 5),
    (dict(mode=7), 10),
    (dict(batch=0), 8),
    (dict(out=None), 1),
    (dict(weights=None), 1),
    (dict(q=_lib.Bnhd(FAKE + 2, 0, 1280, 64)), 7),
    (dict(q=_lib.Bnhd(FAKE, 0, 1281, 64)), 7),
])
def test_bsa_fwd_validation(change, status):
    L = _lib.lib()
    a = _args(**change)
    assert L.mosaic_bsa_workspace_size(ctypes.byref(a)) == 0
    assert L.mosaic_bsa_fwd(ctypes.byref(a), None, 0, None) == status


def test_workspace_size_and_missing_workspace():
    L = _lib.lib()
    a = _args()
    n = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    # q_cmp + k_cmp + v_cmp^T + compressed partials + scores + indices, each 256-aligned
    nb, nbp, Hq, Hk, K = 48, 64, 20, 5, 4
    assert n >= nb * Hq * 64 * 2 + nb * Hk * 64 * 2 + Hk * 64 * nbp * 2 + nb * Hq * 64 * 4 + Hk * nb * nbp * 2 + nb * Hk * K * 4
    assert n % 256 == 0
    assert L.mosaic_bsa_fwd(ctypes.byref(a), None, 0, None) == 6
    assert L.mosaic_bsa_fwd(ctypes.byref(a), FAKE + 16, n, None) == 6   # misaligned
    assert L.mosaic_bsa_fwd(ctypes.byref(a), FAKE, n - 1, None) == 6    # too small
    local = _args(mode=_lib.MODE_LOCAL_ONLY, weights=None)
    assert L.mosaic_bsa_workspace_size(ctypes.byref(local)) == 0


def test_noalloc_entry_validates_before_touching_the_device():
    L = _lib.lib()
    assert L.mosaic_bsa_fwd_noalloc(ctypes.byref(_args(head_dim=32)), None) == 2
    assert L.mosaic_bsa_fwd_noalloc(ctypes.byref(_args(out=None)), None) == 1
    # N = 393216 in 64-token blocks: the selection scores alone are 5 * 6144 * 6144 * 2 bytes
    big = _args(seq_len=393216)
    assert L.mosaic_bsa_workspace_size(ctypes.byref(big)) > _lib.NOALLOC_SCRATCH_BYTES
    assert L.mosaic_bsa_fwd_noalloc(ctypes.byref(big), None) == _lib.ERR_SCRATCH_LIMIT
    assert "static scratch" in _lib.strerror(_lib.ERR_SCRATCH_LIMIT)


def test_stage_entry_validates_before_any_launch():
    L = _lib.lib()
    a = _args()
    n = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    for stage in (_lib.STAGE_POOL, _lib.STAGE_CMP, _lib.STAGE_TOPK, _lib.STAGE_ATTN):
        # the forward's own validation runs first, whatever the stage
        assert L.mosaic_bsa_fwd_stage(ctypes.byref(_args(head_dim=32)), FAKE, n, None, stage) == 2
        assert L.mosaic_bsa_fwd_stage(ctypes.byref(a), None, 0, None, stage) == 6
    assert L.mosaic_bsa_fwd_stage(ctypes.byref(a), FAKE, n, None, -1) == 11
    assert L.mosaic_bsa_fwd_stage(ctypes.byref(a), FAKE, n, None, 4) == 11


def test_fused_rope_entry_validates():
    L = _lib.lib()
    a = _args()
    n = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(a), None, FAKE, FAKE, FAKE, FAKE, n, None) == 1
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(a), FAKE, FAKE, FAKE, None, FAKE, n, None) == 1   # k_rot
    # the rotated q is optional only where the attention kernel rotates q itself
    local = _args(mode=_lib.MODE_LOCAL_ONLY, weights=None)
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(local), FAKE, FAKE, None, FAKE, None, 0, None) == 1
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(a), FAKE + 4, FAKE, FAKE, FAKE, FAKE, n, None) == 7
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(a), FAKE, FAKE, FAKE, FAKE + 2, FAKE, n, None) == 7
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(_args(head_dim=32)), FAKE, FAKE, FAKE, FAKE, FAKE, n, None) == 2
    assert L.mosaic_bsa_fwd_rope(ctypes.byref(a), FAKE, FAKE, FAKE, FAKE, None, 0, None) == 6


def _proj(**kw):
    j = _lib.ProjArgs()
    j.x, j.x_stride_n, j.x_stride_b, j.dim = FAKE, 768, 768, 768
    # groups 20 + 10 + 1 = 31: eight 256-row tiles
    j.weight_rows, j.weight = 2048, FAKE
    j.q, j.k, j.v, j.weights = FAKE, FAKE, FAKE, FAKE
    for key, val in kw.items():
        setattr(j, key, val)
    return j


@pytest.mark.parametrize("args_change,proj_change,status", [
    ({}, dict(x=None), 1),
    ({}, dict(weights=None), 1),
    ({}, dict(rope_cos=FAKE), 1),                       # cos without sin
    ({}, dict(v=FAKE + 2), 7),
    ({}, dict(x_stride_b=770), 7),
    ({}, dict(dim=704), 11),                            # not a multiple of 128
    (dict(seq_len=3072 + 64 * 5), {}, 11),              # not a multiple of 256 (valid for the op)
    (dict(sparse_block_size=256), {}, 11),
    ({}, dict(weight_rows=1792), 8),
    (dict(head_dim=32), {}, 2),
    (dict(num_q_heads=21), {}, 3),
    (dict(num_q_heads=25, num_kv_heads=25), dict(weight_rows=256 * 19), 11),   # 3 Hq > 64 gate logits
])
def test_fused_projection_entry_validates(args_change, proj_change, status):
    L = _lib.lib()
    a = _args(**args_change)
    assert L.mosaic_bsa_fwd_proj(ctypes.byref(a), ctypes.byref(_proj(**proj_change)), FAKE, 1 << 30, None) == status


def test_fused_projection_local_only_needs_no_weights_output():
    L = _lib.lib()
    a = _args(mode=_lib.MODE_LOCAL_ONLY, weights=None)
    # local only: groups 20 + 10 = 30 -> eight tiles; a wrong size is reported, not the missing gates
    assert L.mosaic_bsa_fwd_proj(ctypes.byref(a), ctypes.byref(_proj(weights=None, weight_rows=256)), None, 0, None) == 8


def test_other_entry_points_validate():
    L = _lib.lib()
    t = _lib.Bnhd(FAKE, 0, 64 * 4, 64)
    assert L.mosaic_sparse_attn_fwd(t, t, t, FAKE, 1, 256, 4, 1, 64, 64, 0, 0.0, FAKE, None, None) == 5
    assert L.mosaic_sparse_attn_fwd(t, t, t, FAKE, 1, 256, 4, 3, 64, 64, 1, 0.0, FAKE, None, None) == 3
    assert L.mosaic_sparse_attn_fwd(t, t, t, None, 1, 256, 4, 1, 64, 64, 1, 0.0, FAKE, None, None) == 1
    # the workspace variant: key-norm bounds [B, N/bs, Hk, 8] fp32
    assert L.mosaic_sparse_attn_fwd_workspace_size(2, 256, 3, 64) == 2 * 4 * 3 * 8 * 4
    assert L.mosaic_sparse_attn_fwd_workspace_size(1, 250, 1, 64) == 0
    ws = L.mosaic_sparse_attn_fwd_workspace_size(1, 256, 1, 64)
    assert L.mosaic_sparse_attn_fwd_ws(t, t, t, FAKE, 1, 256, 4, 1, 64, 64, 1, 0.0, FAKE, None, None, ws, None) == 6
    assert L.mosaic_sparse_attn_fwd_ws(t, t, t, FAKE, 1, 256, 4, 1, 64, 64, 1, 0.0, FAKE, None, FAKE, ws - 4,
                                       None) == 6
    assert L.mosaic_sparse_attn_fwd_ws(t, t, t, FAKE, 1, 256, 4, 1, 64, 64, 0, 0.0, FAKE, None, FAKE, ws, None) == 5
    assert L.mosaic_block_attn_fwd(t, t, t, 1, 256, 4, 1, 64, 96, 0.0, FAKE, None) == 4
    assert L.mosaic_dense_attn_fwd(t, t, t, 1, 100, 4, 1, 64, 0.0, FAKE, None) == 4
    assert L.mosaic_pool_mean_fwd(t, 1, 256, 4, 48, 64, FAKE, None) == 2
    assert L.mosaic_attn_topk_fwd(t, t, 1, 48, 4, 1, 64, 49, FAKE, FAKE, 1 << 20, None) == 5
    assert L.mosaic_attn_topk_fwd(t, t, 1, 48, 4, 1, 64, 4, FAKE, FAKE, 16, None) == 6
    assert L.mosaic_attn_topk_fwd(t, t, 1, 9000, 4, 1, 64, 4, FAKE, FAKE, 1 << 30, None) == 11
    # scores [1, 5, 48, 64] bf16, then k_cmp in operand order [1, 5, 64 (padded blocks), 64] bf16
    align = lambda n: (n + 255) // 256 * 256
    assert L.mosaic_attn_topk_workspace_size(1, 48, 5) == align(5 * 48 * 64 * 2) + align(5 * 64 * 64 * 2)


def test_knn_interp_entry_validates():
    L = _lib.lib()
    t = _lib.Bnhd(FAKE, 3 * 64, 2 * 3 * 64, 64)   # [S_from, B=2, H=3, 64]
    ok = dict(num_from=84, num_to=48, batch=2, heads=3, d=64, K=24)

    def call(kk=t, nb=FAKE, rel=FAKE, wq=FAKE, out=FAKE, **kw):
        a = {**ok, **kw}
        return L.mosaic_knn_interp_fwd(kk, t, nb, rel, wq, a["num_from"], a["num_to"], a["batch"], a["heads"],
                                       a["d"], a["K"], 0.0, out, None)
    assert call(nb=None) == 1 and call(rel=None) == 1 and call(wq=None) == 1 and call(out=None) == 1
    assert call(d=32) == 2
    assert call(K=0) == 5 and call(K=33) == 5
    assert call(num_to=0) == 8 and call(batch=-1) == 8
    assert call(wq=FAKE + 8) == 7 and call(out=FAKE + 2) == 7 and call(rel=FAKE + 2) == 7
    assert call(kk=_lib.Bnhd(FAKE + 2, 3 * 64, 2 * 3 * 64, 64)) == 7

    def ordered(order=None, **kw):
        a = {**ok, **kw}
        return L.mosaic_knn_interp_fwd_ordered(t, t, FAKE, FAKE, FAKE, order, a["num_from"], a["num_to"], a["batch"],
                                               a["heads"], a["d"], a["K"], 0.0, FAKE, None)
    assert ordered(order=FAKE + 2) == 7                  # the order's int32 entries need 4-byte alignment
    assert ordered(order=FAKE, d=32) == 2 and ordered(order=FAKE, K=33) == 5


def test_backward_entry_validates():
    L = _lib.lib()
    t = _lib.Bnhd(FAKE, 0, 64 * 4, 64)
    ws = L.mosaic_sparse_attn_bwd_workspace_size(1, 256, 4)
    assert ws == 2 * ((256 * 4 * 4 + 255) // 256 * 256) + (256 * 4 * 64 * 2 + 255) // 256 * 256   # -lse, -delta, q'

    def call(q=t, out=FAKE, lse=FAKE, idx=FAKE, N=256, Hq=4, Hk=1, d=64, bs=64, K=2, gq=FAKE, w=FAKE, wsb=ws):
        return L.mosaic_sparse_attn_bwd(q, t, t, out, lse, t, idx, 1, N, Hq, Hk, d, bs, K, 0.0, gq, FAKE, FAKE,
                                        w, wsb, None)
    assert call(d=32) == 2
    assert call(Hq=4, Hk=3) == 3
    assert call(bs=96) == 4 and call(N=200) == 4
    assert call(K=0) == 5
    assert call(N=64 * 5000) == 11                       # more query blocks than the LDS marks hold
    assert call(out=None) == 1 and call(lse=None) == 1 and call(idx=None) == 1 and call(gq=None) == 1
    assert call(q=_lib.Bnhd(FAKE + 2, 0, 256, 64)) == 7 and call(gq=FAKE + 4) == 7
    assert call(w=None) == 6 and call(wsb=ws - 1) == 6


def test_fused_elementwise_entries_validate():
    L = _lib.lib()
    F32, BF = _lib.DTYPE_F32, _lib.DTYPE_BF16
    # rms_norm(x, residual, dtype, rows, cols, x_stride, r_stride, weight, eps, sum_out, out, out_dtype, stream)
    assert L.mosaic_rms_norm_fwd(FAKE, None, BF, 0, 768, 768, 0, None, 0.0, None, FAKE, BF, None) == 8
    assert L.mosaic_rms_norm_fwd(FAKE, None, 5, 4, 768, 768, 0, None, 0.0, None, FAKE, BF, None) == 11
    assert L.mosaic_rms_norm_fwd(FAKE, None, BF, 4, 770, 770, 0, None, 0.0, None, FAKE, BF, None) == 11
    assert L.mosaic_rms_norm_fwd(FAKE, None, BF, 4, 8192, 8192, 0, None, 0.0, None, FAKE, BF, None) == 11
    # a residual without sum_out is valid (the sum is not stored): a misaligned residual still fails
    assert L.mosaic_rms_norm_fwd(FAKE, FAKE + 2, BF, 4, 768, 768, 768, None, 0.0, None, FAKE, BF, None) == 7
    assert L.mosaic_rms_norm_fwd(None, None, BF, 4, 768, 768, 0, None, 0.0, None, FAKE, BF, None) == 1
    assert L.mosaic_rms_norm_fwd(FAKE + 2, None, BF, 4, 768, 768, 0, None, 0.0, None, FAKE, BF, None) == 7
    assert L.mosaic_rms_norm_fwd(FAKE, None, BF, 4, 768, 772, 0, None, 0.0, None, FAKE, F32, None) == 7
    # resample_norm(p, p_stride, pos, shortcut, weight, eps, coarse_rows, members, factor, dim, out, stream)
    rn = L.mosaic_resample_norm_fwd
    assert rn(FAKE, 3072, FAKE, FAKE, None, 0.0, 0, 24, 4, 768, FAKE, None) == 8
    assert rn(FAKE, 3072, FAKE, FAKE, None, 0.0, 16, 24, 4, 770, FAKE, None) == 11      # dim % 8
    assert rn(FAKE, 32768, FAKE, None, None, 0.0, 16, 24, 1, 8192, FAKE, None) == 11    # dim > 4096
    assert rn(FAKE, 3000, FAKE, FAKE, None, 0.0, 16, 24, 4, 768, FAKE, None) == 8       # stride < factor * dim
    assert rn(None, 3072, FAKE, FAKE, None, 0.0, 16, 24, 4, 768, FAKE, None) == 1
    assert rn(FAKE, 3072, None, FAKE, None, 0.0, 16, 24, 4, 768, FAKE, None) == 1
    assert rn(FAKE, 3072, FAKE, FAKE, None, 0.0, 16, 24, 4, 768, None, None) == 1
    assert rn(FAKE, 3076, FAKE, FAKE, None, 0.0, 16, 24, 4, 768, FAKE, None) == 7       # stride % 8
    assert rn(FAKE, 3072, FAKE, FAKE + 4, None, 0.0, 16, 24, 4, 768, FAKE, None) == 7
    # add_merge(x, residual, coarse_rows, members, factor, dim, sum_out, merged_out, stream)
    am = L.mosaic_add_merge_fwd
    assert am(FAKE, FAKE, 0, 24, 4, 768, FAKE, FAKE, None) == 8
    assert am(FAKE, FAKE, 16, 24, 4, 770, FAKE, FAKE, None) == 11
    assert am(FAKE, None, 16, 24, 4, 768, FAKE, FAKE, None) == 1
    assert am(FAKE, FAKE, 16, 24, 4, 768, FAKE, None, None) == 1
    assert am(FAKE, FAKE, 16, 24, 4, 768, FAKE + 8, FAKE, None) == 7
    # gate_softmax(logits, row_stride, seq, members, heads, w, stream)
    gs = L.mosaic_gate_softmax_fwd
    assert gs(FAKE, 1280, 0, 24, 12, FAKE, None) == 8
    assert gs(FAKE, 30, 100, 24, 12, FAKE, None) == 8          # row stride < 3 * heads
    assert gs(None, 1280, 100, 24, 12, FAKE, None) == 1
    assert gs(FAKE, 1280, 100, 24, 12, None, None) == 1
    assert gs(FAKE + 1, 1280, 100, 24, 12, FAKE, None) == 7
    # swiglu(h, dtype, rows, hidden, h_stride, noise, noise_rows, out, stream)
    assert L.mosaic_swiglu_fwd(FAKE, BF, 0, 3072, 6144, None, 0, FAKE, None) == 8
    assert L.mosaic_swiglu_fwd(FAKE, BF, 4, 3070, 6140, None, 0, FAKE, None) == 11
    assert L.mosaic_swiglu_fwd(FAKE, BF, 4, 3072, 6000, None, 0, FAKE, None) == 8
    assert L.mosaic_swiglu_fwd(FAKE, BF, 4, 3072, 6144, FAKE, 0, FAKE, None) == 8
    assert L.mosaic_swiglu_fwd(None, BF, 4, 3072, 6144, None, 0, FAKE, None) == 1
    assert L.mosaic_swiglu_fwd(FAKE, BF, 4, 3072, 6144, FAKE + 8, 2, FAKE, None) == 7
    # swiglu_linear(x, rows, dim, x_stride, weight, hidden, noise, noise_rows, out, stream)
    sl = L.mosaic_swiglu_linear_fwd
    assert sl(FAKE, 0, 768, 768, FAKE, 3072, None, 0, FAKE, None) == 8
    assert sl(FAKE, 300, 768, 768, FAKE, 3072, None, 0, FAKE, None) == 11      # rows % 256
    assert sl(FAKE, 512, 700, 704, FAKE, 3072, None, 0, FAKE, None) == 11      # dim % 128
    assert sl(FAKE, 512, 768, 768, FAKE, 3000, None, 0, FAKE, None) == 11      # hidden % 128
    assert sl(FAKE, 512, 768, 760, FAKE, 3072, None, 0, FAKE, None) == 7       # stride < dim
    assert sl(FAKE, 512, 768, 772, FAKE, 3072, None, 0, FAKE, None) == 7       # stride % 8
    assert sl(FAKE + 8, 512, 768, 768, FAKE, 3072, None, 0, FAKE, None) == 7
    assert sl(FAKE, 512, 768, 768, FAKE, 3072, FAKE + 8, 2, FAKE, None) == 7
    assert sl(FAKE, 512, 768, 768, FAKE, 3072, FAKE, 0, FAKE, None) == 8       # noise rows
    assert sl(None, 512, 768, 768, FAKE, 3072, None, 0, FAKE, None) == 1
    assert sl(FAKE, 512, 768, 768, None, 3072, None, 0, FAKE, None) == 1
    assert sl(FAKE, 512, 768, 1 << 26, FAKE, 3072, None, 0, FAKE, None) == 11  # 32-bit offsets


def test_permute_w13_layout():
    import torch
    from mosaic_amd import fused
    w = torch.arange(2 * 96 * 4, dtype=torch.float32).view(2 * 96, 4)
    p = fused.permute_w13(w)
    for t in range(3):
        assert torch.equal(p[64 * t:64 * t + 32], w[32 * t:32 * t + 32])          # x1 rows
        assert torch.equal(p[64 * t + 32:64 * t + 64], w[96 + 32 * t:96 + 32 * t + 32])   # x3 rows
    with pytest.raises(ValueError):
        fused.permute_w13(torch.zeros(2 * 40, 4))


def test_bsa_fwd_output_strides_validate():
    L = _lib.lib()
    a = _args()
    a.out_stride_n = 20 * 64 + 4                       # rows must stay 16-byte aligned
    assert L.mosaic_bsa_fwd(ctypes.byref(a), None, 0, None) == 7
