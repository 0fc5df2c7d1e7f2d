"""MosaicAttention's branch weights (generate_strategy_weights, primitives.py:173-180) from the
gate slice of the stacked projection: fused.gate_softmax against the eager form the module
runs otherwise, torch.softmax(logits.float(), dim=0).type_as(x), bit for bit."""
import pytest
import torch

from mosaic_amd import fused

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def eager(logits, heads):
    lg = logits.unflatten(-1, (heads, 3)).permute(3, 1, 0, 2)
    return torch.softmax(lg.float(), dim=0).to(torch.bfloat16)


@pytest.mark.parametrize("S,B,heads,width,offset,scale", [
    (4096, 24, 12, 1280, 1152, 1.0),    # stage 1: the gate slice after q, k, v (768 + 192 + 192)
    (1024, 24, 16, 1792, 1536, 4.0),    # stage 2, larger logits
    (333, 1, 20, 1536, 1280, 30.0),     # bottleneck heads, one member, logits far apart
    (64, 3, 4, 12, 0, 1.0),             # contiguous logits
])
def test_gate_softmax_matches_torch(S, B, heads, width, offset, scale):
    print(f"gate_softmax S={S} B={B} heads={heads}", flush=True)
    g = torch.Generator().manual_seed(S + heads)
    y = (torch.randn(S, B, width, generator=g) * scale).to(torch.bfloat16).to(DEV)
    y[:5, :, offset:offset + 3 * heads] = 0.25     # exact ties
    logits = y[..., offset:offset + 3 * heads]
    with torch.no_grad():
        got = fused.gate_softmax(logits, heads)
        ref = eager(logits, heads)
    torch.cuda.synchronize()
    assert got.shape == (3, B, S, heads) and got.dtype == torch.bfloat16
    assert torch.equal(got, ref), f"max diff {(got.float() - ref.float()).abs().max().item():.3e}"


def test_gate_softmax_refuses_grad():
    lg = torch.randn(8, 2, 12, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(RuntimeError, match="no backward"):
        fused.gate_softmax(lg, 4)
