"""cSwiGLU's w13 projection and gate as one kernel (fused.swiglu_linear, ffn.hip) against the
reference's two steps (primitives.py:92-105): h = x w13^T as a bf16 Linear (fp32
accumulation, rounded to bf16), then the gate with the eager bf16 rounding points."""
import pytest
import torch
import torch.nn.functional as F

from mosaic_amd import fused
from mosaic_amd.model import cSwiGLU

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def reference(x, w13, noise):
    """fp32-accumulated projection rounded to bf16, then the gate in eager bf16 ops."""
    h = (x.float() @ w13.float().t()).to(torch.bfloat16)
    x1, x3 = h.chunk(2, dim=-1)
    if noise is not None:
        x1 = x1 + noise.to(torch.bfloat16)          # [S, B, H] + [B, H], rounded to bf16
    return F.silu(x1) * x3


def check(got, ref, name):
    g, r = got.float().cpu(), ref.float().cpu()
    assert torch.isfinite(g).all(), f"{name}: non-finite"
    rel = ((g - r).norm() / r.norm().clamp_min(1e-30)).item()
    err = (g - r).abs().max().item()
    bound = 2e-2 * max(1.0, r.abs().max().item())
    print(f"  {name}: rel_l2 {rel:.2e} max_abs {err:.2e} (bound {bound:.2e})", flush=True)
    assert rel <= 1e-2 and err <= bound, f"{name}: rel_l2 {rel:.3e} max_abs {err:.3e}"


@pytest.mark.parametrize("S,B,dim,hidden,noise", [
    (128, 4, 256, 256, True),
    (256, 1, 128, 384, False),
    (64, 24, 768, 3072, True),      # stage-1 widths of the era5 preset, 24 members
    (64, 12, 1024, 4096, True),     # stage-2 widths
    (32, 8, 1280, 5120, False),     # bottleneck widths
])
def test_swiglu_linear_matches_reference(S, B, dim, hidden, noise):
    print(f"swiglu_linear S={S} B={B} dim={dim} hidden={hidden} noise={noise}", flush=True)
    g = torch.Generator().manual_seed(S + dim + hidden)
    x = torch.randn(S, B, dim, generator=g).to(torch.bfloat16)
    w13 = (torch.randn(2 * hidden, dim, generator=g) * dim ** -0.5).to(torch.bfloat16)
    nz = torch.randn(B, hidden, generator=g).to(torch.bfloat16) if noise else None
    xd, wd = x.to(DEV), w13.to(DEV)
    nd = nz.to(DEV) if nz is not None else None
    with torch.no_grad():
        got = fused.swiglu_linear(xd, fused.permute_w13(wd), nd)
        two_step = fused.swiglu((xd @ wd.t()), nd)      # library GEMM, then the gate kernel
    torch.cuda.synchronize()
    assert got.shape == (S, B, hidden) and got.dtype == torch.bfloat16
    check(got, reference(x, w13, nz), "vs fp32-accumulate reference")
    check(got, two_step, "vs library GEMM + gate kernel")


def test_swiglu_linear_strided_rows():
    """x as a row-strided view (a slice of a wider activation)."""
    g = torch.Generator().manual_seed(7)
    xw = torch.randn(512, 384, generator=g).to(torch.bfloat16)
    x = xw[:, :256]                                     # row stride 384
    w13 = (torch.randn(512, 256, generator=g) * 256 ** -0.5).to(torch.bfloat16)
    with torch.no_grad():
        got = fused.swiglu_linear(x.to(DEV), fused.permute_w13(w13.to(DEV)))
    check(got, reference(x, w13, None), "strided x")


def test_cswiglu_module_fused_equals_unfused():
    """cSwiGLU.forward through the fused kernel and through w13 + gate kernel + w2."""
    torch.manual_seed(0)
    m = cSwiGLU(768, 3072, 64).to(DEV)
    x = torch.randn(64, 24, 768, device=DEV).to(torch.bfloat16)
    z = torch.randn(24, 64, device=DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        m.fused_linear_gate = True
        a = m(x, z)
        m.fused_linear_gate = False
        b = m(x, z)
    check(a, b, "module fused vs unfused")
    # the permuted weight is rebuilt when the weight changes
    with torch.no_grad():
        m.w13.weight.mul_(0.5)
        m.fused_linear_gate = True
        with torch.autocast("cuda", dtype=torch.bfloat16):
            c = m(x, z)
            m.fused_linear_gate = False
            d = m(x, z)
    check(c, d, "after a weight update")


@pytest.mark.parametrize("fused_gate", [True, False])
def test_cswiglu_refuses_grad(fused_gate):
    """With grad mode on and weights that require grad, both paths raise rather than return an
    output cut off from the graph."""
    m = cSwiGLU(256, 256, 0).to(DEV).to(torch.bfloat16)
    m.fused_linear_gate = fused_gate
    x = torch.randn(256, 1, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no backward"):
        m(x)
