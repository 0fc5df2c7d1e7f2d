"""The HEALPix resampling epilogue (fused.resample_norm, fused.hip) against the eager form of
HEALPixUpsample / HEALPixDownsample.forward (primitives.py:313-359): the bf16 add of the
position term, the '(f d)' split, the skip add and the RMSNorm.  The eager adds run as torch
bf16 ops and the norm as fused.rms_norm, so the fused kernel must match bit for bit; torch's
own fp32 rms_norm of the same sums anchors the norm within bf16 rounding."""
import pytest
import torch
import torch.nn.functional as F

from mosaic_amd import fused
from mosaic_amd.model import HEALPixDownsample, HEALPixUpsample

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def inputs(n, B, f, d, seed, shortcut=True):
    g = torch.Generator().manual_seed(seed)
    p = torch.randn(n, B, f * d, generator=g).to(torch.bfloat16)
    pos = torch.randn(n, f * d, generator=g).to(torch.bfloat16)
    sc = torch.randn(n * f, B, d, generator=g).to(torch.bfloat16) if shortcut else None
    w = torch.rand(d, generator=g) + 0.5
    return [t.to(DEV) if t is not None else None for t in (p, pos, sc, w)]


def eager_sum(p, pos, sc, f):
    n, B, fd = p.shape
    x = p + pos.unsqueeze(1)
    x = x.view(n, B, f, fd // f).transpose(1, 2).reshape(n * f, B, fd // f)
    return x + sc if sc is not None else x


@pytest.mark.parametrize("n,B,f,d,shortcut", [
    (64, 4, 4, 768, True),       # upsampling, the stage-1 width
    (32, 3, 4, 1024, True),      # upsampling into stage 2
    (16, 2, 1, 1280, False),     # downsampling into the bottleneck (f = 1, no skip)
    (96, 24, 1, 1024, False),    # downsampling, 24 members
    (8, 24, 4, 96, True),        # one 8-element chunk per lane, partial wave
])
def test_resample_norm_matches_eager(n, B, f, d, shortcut):
    print(f"resample_norm n={n} B={B} f={f} d={d} shortcut={shortcut}", flush=True)
    p, pos, sc, w = inputs(n, B, f, d, seed=n + d, shortcut=shortcut)
    with torch.no_grad():
        got = fused.resample_norm(p, pos, w, 1e-6, f, sc)
        y = eager_sum(p, pos, sc, f)
        ref = fused.rms_norm(y, w, 1e-6, out_dtype=torch.bfloat16)
        anchor = F.rms_norm(y.float(), (d,), w, 1e-6)
    torch.cuda.synchronize()
    assert got.shape == (n * f, B, d) and got.dtype == torch.bfloat16
    assert torch.equal(got, ref), f"max diff {(got.float() - ref.float()).abs().max().item():.3e}"
    err = (got.float() - anchor).abs() - 2.0 ** -7 * anchor.abs()
    assert err.max().item() <= 1e-6, f"beyond one bf16 rounding of the fp32 norm by {err.max().item():.3e}"


def test_resample_norm_strided_p():
    """p as a view with a row stride wider than factor * d (a slice of a wider projection)."""
    n, B, f, d = 16, 3, 4, 128
    g = torch.Generator().manual_seed(3)
    wide = torch.randn(n, B, f * d + 64, generator=g).to(torch.bfloat16).to(DEV)
    p = wide[..., : f * d]
    _, pos, sc, w = inputs(n, B, f, d, seed=4)
    with torch.no_grad():
        got = fused.resample_norm(p, pos, w, None, f, sc)
        ref = fused.rms_norm(eager_sum(p, pos, sc, f), w, None, out_dtype=torch.bfloat16)
    assert torch.equal(got, ref)


def test_resampling_modules_fused_equal_eager():
    """HEALPixUpsample / HEALPixDownsample under bf16 autocast (the fused epilogue) against the
    same modules' eager formula on their own projections."""
    torch.manual_seed(0)
    up = HEALPixUpsample(256, 128, 8, 16).to(DEV)      # f = 4
    down = HEALPixDownsample(128, 256, 16, 8).to(DEV)  # f = 4 children merged
    B = 3
    x = torch.randn(12 * 8 * 8, B, 256, device=DEV).to(torch.bfloat16)
    skip = torch.randn(12 * 16 * 16, B, 128, device=DEV).to(torch.bfloat16)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        u = up(x, skip)
        pu, qu = up.proj_x(x), up.proj_pos(up.rel_pos)
        ru = up.norm(eager_sum(pu, qu, skip, up.factor))
        dn = down(u)
        S = u.shape[0]
        xd = u.view(S // 4, 4, B, 128).transpose(1, 2).reshape(S // 4, B, 512)
        rd = down.norm(down.proj_x(xd) + down.proj_pos(down.rel_pos).unsqueeze(1))
    assert u.dtype == torch.bfloat16 and torch.equal(u, ru)
    assert dn.dtype == torch.bfloat16 and torch.equal(dn, rd)


def test_add_norm_equals_add_forward():
    torch.manual_seed(1)
    m = fused.RMSNorm(768).to(DEV)
    x = torch.randn(1000, 3, 768, device=DEV).to(torch.bfloat16)
    r = torch.randn(1000, 3, 768, device=DEV).to(torch.bfloat16)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        a = m.add_norm(x, r)
        _, b = m.add_forward(x, r)
    assert torch.equal(a, b)


def test_resample_norm_refuses_grad():
    p, pos, sc, w = inputs(8, 2, 4, 64, seed=5)
    w.requires_grad_(True)
    with pytest.raises(RuntimeError, match="no backward"):
        fused.resample_norm(p, pos, w, None, 4, sc)


@pytest.mark.parametrize("n,B,f,C", [(192, 24, 4, 768), (48, 3, 4, 1024), (7, 5, 1, 96)])
def test_add_merge_matches_eager(n, B, f, C):
    """An encoder stage's last residual add and the merge of the children
    ('(n f) b c -> n b (f c)') for the downsampling projection."""
    print(f"add_merge n={n} B={B} f={f} C={C}", flush=True)
    g = torch.Generator().manual_seed(n + C)
    x = torch.randn(n * f, B, C, generator=g).to(torch.bfloat16).to(DEV)
    r = torch.randn(n * f, B, C, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        s, merged = fused.add_merge(x, r, f)
        ref = x + r
        ref_m = ref.view(n, f, B, C).transpose(1, 2).reshape(n, B, f * C)
    assert torch.equal(s, ref) and torch.equal(merged, ref_m)
