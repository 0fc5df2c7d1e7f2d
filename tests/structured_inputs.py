"""Block-structured inputs under which the compressed branch's logits matter.

With i.i.d. N(0,1) tokens the pooled q and k have std 1/8 per element, so the pooled logits
q_cmp . k_cmp * d^-0.5 have std ~1/64 and the compressed softmax is almost uniform: a
compressed branch that ignored its logits would still pass the output bar.  Here every token of
block i and head h is ``sigma * u[b, i, h] + e`` with u, e ~ N(0, 1): the pooled tensors keep
sigma * u, and the pooled logits have std ~sigma^2 (2.25 at sigma = 1.5).  v uses a smaller
sigma_v so that the outputs stay below 2 in magnitude, where one bf16 spacing (2^-7 .. 2^-6) is
inside the 2e-2 absolute bar.
"""

from __future__ import annotations

import torch


def block_structured(B, N, H, bs, sigma, generator):
    u = torch.randn(B, N // bs, 1, H, 64, generator=generator)
    e = torch.randn(B, N // bs, bs, H, 64, generator=generator)
    return (sigma * u + e).reshape(B, N, H, 64).to(torch.bfloat16)


def compressed_only_inputs(B, N, Hq, Hk, bs, sigma=1.5, sigma_v=0.5, seed=0):
    """(q, k, v, w) with block-structured q, k, v and gates (0, 1, 0): the full op's output is
    then exactly the compressed branch broadcast over each block's tokens."""
    g = torch.Generator().manual_seed(seed)
    q = block_structured(B, N, Hq, bs, sigma, g)
    k = block_structured(B, N, Hk, bs, sigma, g)
    v = block_structured(B, N, Hk, bs, sigma_v, g)
    w = torch.zeros(3, B, N, Hq, 1, dtype=torch.bfloat16)
    w[1] = 1.0
    return q, k, v, w


def pooled_logit_std(q_cmp, k_cmp):
    """Std of the scaled pooled logits q_cmp . k_cmp * d^-0.5 over all (head, query, key)."""
    Hq, Hk = q_cmp.shape[2], k_cmp.shape[2]
    kr = k_cmp.float().repeat_interleave(Hq // Hk, dim=2)
    s = torch.einsum("bthd,buhd->bhtu", q_cmp.float(), kr) * q_cmp.shape[-1] ** -0.5
    return s.std().item()
