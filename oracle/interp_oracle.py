"""CPU oracle of the k-nearest-neighbour cross-attention interpolation (test infrastructure).

Restates CrossAttentionInterpolate.forward's gather-attention (primitives.py:265-283) with
the reference's own torch operations, on the CPU, in the precision the model runs it under
bf16 autocast: q = to_q(rel_pos) as a bf16 matmul with fp32 accumulation, bf16 elementwise
q * k, the sum over the head dimension rounded to bf16, scaled in bf16, softmax over the
neighbours in fp32 and cast to bf16, bf16 elementwise weights * v summed over the neighbours.
``products="fp32"`` keeps the products of the two sums exact (fp32 products, fp32 sums), as
the reference's torch.compile'd inference path computes them (inference.py:470-473); every
other rounding is the same.
Only tests and the benchmark's CPU baseline use it; the product path never does.

Pinned in tests/test_interp_oracle.py by: a single neighbour returning that neighbour's v;
zero queries giving uniform weights (a closed-form mean); a float64 dense attention masked to
each target's neighbour set; invariance under permuting the neighbour order; the two product
forms equal bit for bit on inputs whose products are exact in bf16 (and apart on general
inputs); and, for the neighbour search, a brute-force great-circle k-NN.
"""

from __future__ import annotations

import torch


def knn_attention(k: torch.Tensor, v: torch.Tensor, neighbors: torch.Tensor, rel_pos: torch.Tensor,
                  w_q: torch.Tensor, scale: float, products: str = "bf16") -> torch.Tensor:
    """k, v [S_from, B, H, d] bf16; neighbors [S_to, K]; rel_pos [S_to, K, 3]; w_q [H*d, 3]
    -> [S_to, B, H, d] bf16 (primitives.py:265-280).  products: "bf16" (eager elementwise
    products) or "fp32" (exact products, as the compiled path fuses them into the sums)."""
    if products not in ("bf16", "fp32"):
        raise ValueError(products)
    S_from, B, H, d = k.shape
    q = (rel_pos.to(torch.bfloat16).float() @ w_q.to(torch.bfloat16).float().t()).to(torch.bfloat16)  # :266
    q = q.view(*q.shape[:2], 1, H, d)                                                                  # :267
    nb = neighbors.long()
    kg, vg = k[nb], v[nb]                                                                              # :274
    if products == "fp32":
        scores = (q.float() * kg.float()).sum(dim=-1, keepdim=True).to(torch.bfloat16) * scale        # :276
        w = torch.softmax(scores, dim=1, dtype=torch.float32).type_as(kg)                              # :277
        return (w.float() * vg.float()).sum(dim=1).to(torch.bfloat16)                                  # :278
    scores = (q * kg).sum(dim=-1, keepdim=True) * scale                                                # :276
    w = torch.softmax(scores, dim=1, dtype=torch.float32).type_as(kg)                                  # :277
    return (w * vg).sum(dim=1)                                                                         # :278


def great_circle_knn(pos_from: torch.Tensor, pos_to: torch.Tensor, k: int) -> torch.Tensor:
    """Brute-force k nearest neighbours by great-circle distance ((lon, lat) radians), nearest
    first, ties by index."""
    def xyz(p):
        lon, lat = p[:, 0].double(), p[:, 1].double()
        return torch.stack([lat.cos() * lon.cos(), lat.cos() * lon.sin(), lat.sin()], -1)
    ang = torch.acos((xyz(pos_to) @ xyz(pos_from).t()).clamp(-1, 1))
    return torch.sort(ang, dim=1, stable=True).indices[:, :k]
