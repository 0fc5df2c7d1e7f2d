"""GPU parity of the fused input side (mosaic_attn_proj / mosaic_bsa_fwd_proj): projection GEMM,
RoPE, gate softmax and block pooling in one kernel, then the op (needs an MI355X; marked ``gpu``).

Checks, from the strongest down:
  * exact-arithmetic inputs (integer x, weights in multiples of 1/8: every fp32 sum of the GEMM
    is exact, so the bf16 results cannot depend on summation order): q / k / v bit-exact to
    torch's bf16 Linear, q / k rotated bit-exact to the RoPE module applied to them, and the op
    output and selected blocks bit-exact to mosaic_attn_func on the projections (the pooled
    sums of integer-valued rows are exact in any order as well);
  * the gate weights within one bf16 ulp of torch's fp32 softmax of the same logits;
  * random inputs with RoPE: the pooled q (read from the op's workspace) within one bf16 ulp of
    pool_mean of the rotated q, the op output within the usual bar of mosaic_attn_func on the
    projections;
  * the U-Net attention block: the fused path against the unfused one under bf16 autocast.
"""

import ctypes

import pytest
import torch

import mosaic_amd as M
from mosaic_amd import _lib
from mosaic_amd.primitives import MosaicAttention, RoPE, mosaic_attn_proj, stack_projection_weight
from mosaic_amd.healpix import get_healpix_grid, rope_tables

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_ABS = 2e-2
REL_L2 = 1e-2


def gen(seed):
    return torch.Generator().manual_seed(seed)


def exact_inputs(S, B, dim, Hq, Hk, gates, seed=0):
    """Integer x in [-2, 2] and weights in multiples of 1/8 in [-1/4, 1/4]: exact fp32 GEMM sums."""
    g = gen(seed)
    x = torch.randint(-2, 3, (S, B, dim), generator=g).to(torch.bfloat16)
    ws = [torch.randint(-2, 3, (n, dim), generator=g).float() / 8 for n in (64 * Hq, 64 * Hk, 64 * Hk)]
    wg = torch.randint(-2, 3, (3 * Hq, dim), generator=g).float() / 64 if gates else None
    return x, ws, wg


def random_inputs(S, B, dim, Hq, Hk, gates, seed=0):
    g = gen(seed)
    x = torch.randn(S, B, dim, generator=g).to(torch.bfloat16)
    sc = dim ** -0.5
    ws = [torch.randn(n, dim, generator=g) * sc for n in (64 * Hq, 64 * Hk, 64 * Hk)]
    wg = torch.randn(3 * Hq, dim, generator=g) * sc if gates else None
    return x, ws, wg


def reference_projections(x, ws, wg, Hq, Hk, rope):
    """torch: bf16 Linear per weight, RoPE module arithmetic, fp32 softmax of the gate logits."""
    S, B, _ = x.shape
    xd = x.to(DEV)
    outs = [torch.nn.functional.linear(xd, w.to(DEV, torch.bfloat16)) for w in ws]
    q = outs[0].view(S, B, Hq, 64).transpose(0, 1)
    k = outs[1].view(S, B, Hk, 64).transpose(0, 1)
    v = outs[2].view(S, B, Hk, 64).transpose(0, 1)
    if rope is not None:
        r = RoPE(64)
        r.register_buffer("cos_freqs", rope[0].to(DEV))
        r.register_buffer("sin_freqs", rope[1].to(DEV))
        q, k = r(q), r(k)
    w = None
    if wg is not None:
        logits = torch.nn.functional.linear(xd, wg.to(DEV, torch.bfloat16)).view(S, B, Hq, 3)
        w = torch.softmax(logits.float(), dim=-1).to(torch.bfloat16).transpose(0, 1)   # [B, S, Hq, 3]
    return q.contiguous(), k.contiguous(), v.contiguous(), w


def tables(S, nside):
    return rope_tables(get_healpix_grid(nside), 64, 10000)


def run_proj(x, ws, wg, Hq, Hk, mode_kw, rope=None, record=True):
    W = stack_projection_weight(*[w.to(DEV) for w in ws], wg.to(DEV) if wg is not None else None, Hq, Hk)
    kw = {} if rope is None else dict(rope_cos=rope[0].to(DEV), rope_sin=rope[1].to(DEV))
    return mosaic_attn_proj(x.to(DEV), W, Hq, Hk, **mode_kw, return_projections=True,
                            return_block_indices=record, **kw)


MODES = {
    "full": dict(block_attn_size=256, sparse_block_size=64, sparse_block_count=4, block_attn_only=False),
    "full_bs128": dict(block_attn_size=256, sparse_block_size=128, sparse_block_count=3, block_attn_only=False),
    "no_compression": dict(block_attn_size=128, sparse_block_size=64, sparse_block_count=4, block_attn_only=False,
                           no_compression=True),
    "no_selection": dict(block_attn_size=256, sparse_block_size=128, sparse_block_count=0, block_attn_only=False),
    "local_only": dict(block_attn_size=256, sparse_block_size=64, sparse_block_count=4, block_attn_only=True),
}


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("use_rope", [False, True])
def test_projection_outputs_exact(mode, use_rope):
    S, B, dim, Hq, Hk = 768, 2, 256, 8, 2
    print(f"proj exact mode={mode} rope={use_rope}", flush=True)
    kw = MODES[mode]
    gates = not kw["block_attn_only"]
    x, ws, wg = exact_inputs(S, B, dim, Hq, Hk, gates, seed=1)
    rope = tables(S, 8) if use_rope else None
    res = run_proj(x, ws, wg, Hq, Hk, kw, rope)
    q, k, v, w = res[1:5]
    rq, rk, rv, rw = reference_projections(x, ws, wg, Hq, Hk, rope)
    assert torch.equal(q, rq) and torch.equal(k, rk) and torch.equal(v, rv)
    if gates:
        assert w.shape == rw.shape
        assert ((w.float() - rw.float()).abs() <= 2 ** -9).all()
    else:
        assert w is None


@pytest.mark.parametrize("mode", list(MODES))
def test_op_exact_against_unfused(mode):
    """Integer inputs, no RoPE: the fused op equals mosaic_attn_func on its own projections."""
    S, B, dim, Hq, Hk = 1024, 2, 384, 12, 3
    print(f"proj op exact mode={mode}", flush=True)
    kw = MODES[mode]
    x, ws, wg = exact_inputs(S, B, dim, Hq, Hk, not kw["block_attn_only"], seed=2)
    res = run_proj(x, ws, wg, Hq, Hk, kw)
    out, q, k, v, w, idx = res
    wv = None if w is None else w.permute(3, 0, 1, 2).unsqueeze(-1)
    ref = M.mosaic_attn_func(q, k, v, wv, **kw, return_block_indices=True)
    ref_out, ref_idx = ref
    assert torch.equal(out, ref_out)
    if idx is not None or ref_idx is not None:
        assert torch.equal(idx, ref_idx)


@pytest.mark.parametrize("bs", [64, 128])
def test_pooled_q_and_op_with_rope(bs):
    """Random inputs with RoPE: pooled q from the workspace within one bf16 ulp of pool_mean of
    the rotated q; the op output within the bar of mosaic_attn_func on the projections."""
    S, B, dim, Hq, Hk = 3072, 2, 768, 12, 3
    print(f"proj rope random bs={bs}", flush=True)
    x, ws, wg = random_inputs(S, B, dim, Hq, Hk, True, seed=3)
    rope = tables(S, 16)
    kw = dict(block_attn_size=1024, sparse_block_size=bs, sparse_block_count=6, block_attn_only=False)
    # through the C ABI with a workspace of our own, to read the pooled q (the first region)
    W = stack_projection_weight(*[t.to(DEV) for t in ws], wg.to(DEV), Hq, Hk)
    xd = x.to(DEV)
    cos, sin = (t.to(DEV).contiguous() for t in rope)
    q = torch.empty(B, S, Hq, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(B, S, Hk, 64, dtype=torch.bfloat16, device=DEV)
    v = torch.empty_like(k)
    w = torch.empty(B, S, Hq, 3, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(B, S, Hq, 64, dtype=torch.bfloat16, device=DEV)
    a = _lib.BsaArgs()
    a.batch, a.seq_len, a.num_q_heads, a.num_kv_heads, a.head_dim = B, S, Hq, Hk, 64
    a.block_attn_size, a.sparse_block_size, a.sparse_block_count = 1024, bs, 6
    a.mode, a.out = _lib.MODE_FULL, out.data_ptr()
    for name, t in (("q", q), ("k", k), ("v", v)):
        setattr(a, name, _lib.Bnhd(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)))
    a.weights = w.data_ptr()
    a.w_stride_s, a.w_stride_b, a.w_stride_n, a.w_stride_h = 1, S * Hq * 3, Hq * 3, 3
    L = _lib.lib()
    nbytes = L.mosaic_bsa_workspace_size(ctypes.byref(a))
    assert nbytes > 0
    ws_t = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    j = _lib.ProjArgs()
    j.x, j.x_stride_n, j.x_stride_b, j.dim = xd.data_ptr(), xd.stride(0), xd.stride(1), dim
    j.weight_rows, j.weight = W.shape[0], W.data_ptr()
    j.rope_cos, j.rope_sin = cos.data_ptr(), sin.data_ptr()
    j.q, j.k, j.v, j.weights = q.data_ptr(), k.data_ptr(), v.data_ptr(), w.data_ptr()
    _lib.check(L.mosaic_bsa_fwd_proj(ctypes.byref(a), ctypes.byref(j), ws_t.data_ptr(), nbytes,
                                     torch.cuda.current_stream().cuda_stream), "mosaic_bsa_fwd_proj")
    torch.cuda.synchronize()
    nb = S // bs
    qc = ws_t[: B * nb * Hq * 64 * 2].view(torch.bfloat16).view(B, nb, Hq, 64)
    ref_qc = M.pool_mean(q, bs)
    diff = (qc.float() - ref_qc.float()).abs()
    assert (diff <= 2 ** -7 * ref_qc.float().abs() + 1e-30).all(), diff.max().item()
    assert (diff > 0).float().mean().item() < 1e-2
    # the projections themselves against torch within rounding (random data: order-dependent sums)
    rq, rk, rv, rw = reference_projections(x, ws, wg, Hq, Hk, rope)
    for got, ref in ((q, rq), (k, rk), (v, rv)):
        d = (got.float() - ref.float()).abs()
        assert (d <= 2 ** -6 * ref.float().abs() + 1e-3).all()
        assert (d > 0).float().mean().item() < 2e-2
    ref_out = M.mosaic_attn_func(q, k, v, w.permute(3, 0, 1, 2).unsqueeze(-1), 1024, bs, 6, False)
    g, r = out.float(), ref_out.float()
    err = (g - r).abs().max().item()
    rel = ((g - r).norm() / r.norm()).item()
    assert err <= MAX_ABS and rel <= REL_L2, (err, rel)


def test_mosaic_attention_fused_matches_unfused():
    """The U-Net attention block (stage-1 heads) under bf16 autocast: the fused input side
    against the unfused path (library GEMM, pooling pass with RoPE) on the same module."""
    from types import SimpleNamespace
    cfg = SimpleNamespace(block_attn_size=1024, sparse_block_size=128, sparse_block_count=8, num_heads=12,
                          gqa_ratio=4, dim=768, qkv_compress_ratio=1, rope=True, rope_theta=10000)
    torch.manual_seed(0)
    m = MosaicAttention(cfg, block_attn_only=False).to(DEV)
    m.fused_input_side = True
    S, B = 3072, 3
    cos, sin = tables(S, 16)
    m.q_rope.register_buffer("cos_freqs", cos.to(DEV))
    m.q_rope.register_buffer("sin_freqs", sin.to(DEV))
    m.k_rope.register_buffer("cos_freqs", cos.to(DEV))
    m.k_rope.register_buffer("sin_freqs", sin.to(DEV))
    x = torch.randn(S, B, 768, device=DEV)
    with torch.no_grad(), torch.autocast(DEV, dtype=torch.bfloat16):
        assert m._fused_input_side(x)
        fused = m(x).float()
        m._fused_input_side = lambda x: False
        unfused = m(x).float()
    err = (fused - unfused).abs().max().item()
    rel = ((fused - unfused).norm() / unfused.norm()).item()
    assert rel <= REL_L2, (err, rel)


def test_fused_path_refuses_grad():
    from types import SimpleNamespace
    cfg = SimpleNamespace(block_attn_size=256, sparse_block_size=64, sparse_block_count=2, num_heads=4,
                          gqa_ratio=4, dim=256, qkv_compress_ratio=1, rope=False, rope_theta=10000)
    m = MosaicAttention(cfg, block_attn_only=False).to(DEV)
    m.fused_input_side = True
    x = torch.randn(256, 1, 256, device=DEV)
    with torch.autocast(DEV, dtype=torch.bfloat16):
        assert m._fused_input_side(x)
        with pytest.raises(RuntimeError, match="no backward"):
            m(x)
