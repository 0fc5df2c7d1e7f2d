"""mosaic_amd: Mosaic's block-sparse attention on the HEALPix mesh, as HIP kernels for MI355X.

Drop-in Python surface of the reference op (primitives.py / ops.py):
``mosaic_attn_func``, ``block_attention``, ``attn_topk``, ``mosaic_sparse_attn``,
``MosaicAttnFunction``, ``RoPE``, ``MosaicAttention``; ``mosaic_attn_func_rope`` runs the op
with the input side's RoPE fused into its pooling pass.  All compute runs in libmosaic_bsa.so
(built with ``python -m mosaic_amd.build``) through its C ABI (include/mosaic_bsa.h).
"""

from .ops import MosaicAttnFunction, mosaic_attn_bwd, mosaic_attn_fwd, mosaic_sparse_attn
from .primitives import (
    MosaicAttention,
    RoPE,
    attn_topk,
    block_attention,
    dense_attention,
    mosaic_attn_func,
    mosaic_attn_func_rope,
    mosaic_attn_proj,
    pool_mean,
    stack_projection_weight,
)
from .healpix import get_healpix_grid, pix2ang_nest

__all__ = [
    "MosaicAttnFunction", "mosaic_attn_bwd", "mosaic_attn_fwd", "mosaic_sparse_attn", "MosaicAttention", "RoPE",
    "attn_topk", "block_attention", "dense_attention", "mosaic_attn_func", "mosaic_attn_func_rope", "mosaic_attn_proj",
    "stack_projection_weight", "pool_mean",
    "get_healpix_grid", "pix2ang_nest",
]
