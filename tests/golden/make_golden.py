"""Write the small golden fixtures under tests/golden/.

``topk_scores_small.pt``: selection scores and indices for a tiny (q_cmp, k_cmp) pair, built
by evaluating the reference's expression (primitives.py:37-50: repeat_interleave of the kv
heads, bf16 matmul, einops ``reduce(..., 'b (g h) t k -> b h t k', 'mean')``, topk) with
einops 0.8.2 and torch directly -- not through the oracle -- so that the oracle's own
restatement is checked against it.  Shapes: B=2, nb=48 blocks, 20 query / 5 kv heads, d=64,
block_count 4 (the Nside-16 bottleneck head layout), values ~ N(0, 1/64) like pooled N(0,1).

Run: python tests/golden/make_golden.py
"""

import os

import einops
import torch


def main():
    g = torch.Generator().manual_seed(1234)
    B, nb, Hq, Hk, d, K = 2, 48, 20, 5, 64, 4
    q_cmp = (torch.randn(B, nb, Hq, d, generator=g) / 8).to(torch.bfloat16)
    k_cmp = (torch.randn(B, nb, Hk, d, generator=g) / 8).to(torch.bfloat16)
    G = Hq // Hk
    k = k_cmp.repeat_interleave(G, dim=2)
    scores = torch.matmul(einops.rearrange(q_cmp, "b t h d -> b h t d"),
                          einops.rearrange(k, "b t h d -> b h d t"))
    scores = einops.reduce(scores, "b (g h) t k -> b h t k", "mean", g=G)
    idx = einops.rearrange(scores, "b h t k -> b t h k").topk(k=K, dim=-1, largest=True)[1]
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "topk_scores_small.pt")
    torch.save({"q_cmp": q_cmp, "k_cmp": k_cmp, "scores": scores, "indices": idx,
                "block_count": torch.tensor(K)}, out)
    print("wrote", out, tuple(scores.shape), tuple(idx.shape))


if __name__ == "__main__":
    main()
