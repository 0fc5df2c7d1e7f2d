"""Seeded synthetic inputs for the block-sparse attention workloads.

Draw order (CPU generator, one seed): q [B,N,Hq,d], k [B,N,Hk,d], v [B,N,Hk,d] ~ N(0,1) in
bf16, then gate logits [3,B,N,Hq] ~ N(0,1) -> sigmoid -> bf16 -> [3,B,N,Hq,1].  With
``rope=True`` q and k are rotated by the 2-D RoPE of the HEALPix (lon, lat) pixel centres of
the workload's nside (primitives.py:108-135, utils.py:19-30).  Inputs are made on the CPU so
that a CPU checker and the device see identical tensors.
"""

from __future__ import annotations

from dataclasses import dataclass, asdict

import torch

from .healpix import apply_rope, get_healpix_grid, rope_tables


@dataclass(frozen=True)
class Workload:
    name: str
    nside: int
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_attn_size: int
    sparse_block_size: int
    sparse_block_count: int
    rope: bool

    @property
    def seq_len(self) -> int:
        return 12 * self.nside * self.nside

    @property
    def num_blocks(self) -> int:
        return self.seq_len // self.sparse_block_size

    def describe(self) -> dict:
        d = asdict(self)
        d["seq_len"] = self.seq_len
        return d


# Single attention forward at the bottleneck: Nside 16, 20/5 heads, top-4.
BOTTLENECK_NSIDE16 = Workload("bsa_nside16_b1_h20kv5_bs64_top4", 16, 1, 20, 5, 64, 64, 64, 4, False)
# Stage-1 attention forward: Nside 64 (N = 49152), 12/3 heads, top-16, RoPE.
STAGE1_NSIDE64 = Workload("bsa_nside64_b1_h12kv3_bs64_top16", 64, 1, 12, 3, 64, 64, 64, 16, True)
# Stage-1 attention forward with the shipped model's block settings (inference.py:71-88):
# local blocks of 1024 tokens, selection blocks of 128, top-24.
STAGE1_NSIDE64_MODEL = Workload("bsa_nside64_b1_h12kv3_bl1024_bs128_top24", 64, 1, 12, 3, 64, 1024, 128, 24, True)
# Stage-2 attention forward, ensemble-batched: Nside 32, 24 members, 16/4 heads, top-16, RoPE.
STAGE2_NSIDE32_B24 = Workload("bsa_nside32_b24_h16kv4_bs64_top16", 32, 24, 16, 4, 64, 64, 64, 16, True)


def scaling_workload(nside: int) -> Workload:
    """Attention-only scaling sweep point: 12/3 heads, block 64, top-16, no RoPE."""
    return Workload(f"bsa_nside{nside}_b1_h12kv3_bs64_top16", nside, 1, 12, 3, 64, 64, 64, 16, False)


WORKLOADS = {w.name: w for w in (BOTTLENECK_NSIDE16, STAGE1_NSIDE64, STAGE2_NSIDE32_B24)}


def make_inputs(wl: Workload, seed: int = 0, batch: int | None = None):
    """(q, k, v, w) CPU bf16 tensors for ``wl``; ``batch`` overrides the batch size."""
    B = wl.batch if batch is None else batch
    N, Hq, Hk, d = wl.seq_len, wl.q_heads, wl.kv_heads, wl.head_dim
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, N, Hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(B, N, Hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, N, Hk, d, generator=g).to(torch.bfloat16)
    w = torch.sigmoid(torch.randn(3, B, N, Hq, generator=g)).to(torch.bfloat16).unsqueeze(-1)
    if wl.rope:
        cos, sin = rope_tables(get_healpix_grid(wl.nside), d)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
    return q, k, v, w
