"""The Mosaic U-Net forecast model around the block-sparse attention op.

Mirrors mosaic.py (``Transformer``, ``UNetStage``, the stage / model configs) and the
building blocks of primitives.py it composes (``MosaicBlock``, ``cSwiGLU``,
``NoiseGenerator``, ``HEALPixDownsample``, ``HEALPixUpsample``), with the reference's module
and parameter names, so a reference state dict loads unchanged.  Every attention layer runs
``MosaicAttention`` (the op in libmosaic_bsa.so, RoPE fused into its pooling pass) and both
grid interpolations run ``CrossAttentionInterpolate`` (the k-NN gather-attention kernel).  The
projections are library GEMMs; the RMSNorms and the SwiGLU gate run as the fused HIP kernels of
``mosaic_amd.fused`` when their inputs are on a ROCm device.

Activations are sequence-first ``[S, B, C]`` (S pixels, B = members x noise samples), as in
the reference.  The model runs under ``torch.autocast('cuda', torch.bfloat16)``.  The
reference's inference autocasts to ``DTYPE = torch.float16`` (inference.py:59, 379); the
attention op and the interpolation kernel here compute in bf16 only and refuse fp16 inputs
with a ``TypeError``, so a caller keeps bf16 autocast.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn

from . import fused
from .fused import RMSNorm
from .healpix import get_healpix_grid
from .interp import CrossAttentionInterpolate, rad_to_xyz
from .ops import forward_only
from .primitives import MosaicAttention

__all__ = [
    "StageConfig", "BottleneckConfig", "ModelConfig", "era5_config", "RMSNorm", "cSwiGLU", "MosaicBlock",
    "NoiseGenerator", "HEALPixDownsample", "HEALPixUpsample", "UNetStage", "Transformer", "model_flops",
]


@dataclass
class StageConfig:
    """An encoder/decoder stage (mosaic.py:28-40)."""
    nside: int
    dim: int
    num_heads: int
    block_attn_size: int
    sparse_block_size: int
    sparse_block_count: int
    encoder_depth: int
    decoder_depth: int
    mlp_ratio: float
    gqa_ratio: int


@dataclass
class BottleneckConfig:
    """The bottleneck stage (mosaic.py:43-54)."""
    nside: int
    dim: int
    num_heads: int
    block_attn_size: int
    sparse_block_size: int
    sparse_block_count: int
    depth: int
    mlp_ratio: float
    gqa_ratio: int


@dataclass
class ModelConfig:
    """Model-wide settings (mosaic.py:57-76)."""
    dim: int
    num_heads: int
    k_neighbors: int
    qk_norm: bool
    rope: bool
    rope_theta: int
    sparse_every: int
    variables: list
    static_variables: list
    qkv_compress_ratio: int
    cg_stage_cfgs: list
    bottleneck_cfg: BottleneckConfig
    num_history_steps: int = 1
    noise_dim: int = 32
    ortho_init: bool = False
    rmsnorm_elementwise_affine: bool = True
    no_compression: bool = False


@dataclass
class _MergedStageConfig:
    """What a MosaicBlock reads: the stage's settings plus the model-wide ones (mosaic.py:79-110)."""
    dim: int
    num_heads: int
    block_attn_size: int
    sparse_block_size: int
    sparse_block_count: int
    gqa_ratio: int
    qkv_compress_ratio: int
    rope: bool
    rope_theta: int
    mlp_ratio: float
    noise_dim: int
    rmsnorm_elementwise_affine: bool


def _merge_configs(config: ModelConfig, stage_cfg) -> _MergedStageConfig:
    return _MergedStageConfig(
        dim=stage_cfg.dim, num_heads=stage_cfg.num_heads, block_attn_size=stage_cfg.block_attn_size,
        sparse_block_size=stage_cfg.sparse_block_size, sparse_block_count=stage_cfg.sparse_block_count,
        gqa_ratio=stage_cfg.gqa_ratio, qkv_compress_ratio=config.qkv_compress_ratio, rope=config.rope,
        rope_theta=config.rope_theta, mlp_ratio=stage_cfg.mlp_ratio, noise_dim=config.noise_dim,
        rmsnorm_elementwise_affine=config.rmsnorm_elementwise_affine)


def era5_config(num_variables: int = 82, num_static: int = 3) -> ModelConfig:
    """The shipped ``era5`` preset (inference.py:71-103, 286-302): stages nside 64/32 with
    dims 768/1024 and 12/16 heads, bottleneck nside 16 / 1280 / 20 heads, GQA 4, local blocks
    of 1024, sparse blocks of 128 with top-24/12/4, 2 history states, 24 neighbours."""
    stages = [
        StageConfig(nside=64, dim=768, num_heads=12, block_attn_size=1024, sparse_block_size=128,
                    sparse_block_count=24, encoder_depth=4, decoder_depth=2, mlp_ratio=4.0, gqa_ratio=4),
        StageConfig(nside=32, dim=1024, num_heads=16, block_attn_size=1024, sparse_block_size=128,
                    sparse_block_count=12, encoder_depth=4, decoder_depth=2, mlp_ratio=4.0, gqa_ratio=4),
    ]
    bottleneck = BottleneckConfig(nside=16, dim=1280, num_heads=20, block_attn_size=1024, sparse_block_size=128,
                                  sparse_block_count=4, depth=2, mlp_ratio=4.0, gqa_ratio=4)
    return ModelConfig(
        dim=768, num_heads=12, k_neighbors=24, qk_norm=False, rope=True, rope_theta=10000, sparse_every=1,
        variables=[f"v{i}" for i in range(num_variables)], static_variables=[f"s{i}" for i in range(num_static)],
        qkv_compress_ratio=1, cg_stage_cfgs=stages, bottleneck_cfg=bottleneck, num_history_steps=2,
        noise_dim=32, rmsnorm_elementwise_affine=False)


class cSwiGLU(nn.Module):
    """SwiGLU feed-forward with an additive noise bias on the gate (primitives.py:92-105):
    ``w2(silu(x1 + noise_bias(z)) * x3)`` with ``x1, x3 = w13(x).chunk(2)``."""

    def __init__(self, dim: int, hidden_dim: int, noise_dim: int):
        super().__init__()
        self.w13 = nn.Linear(dim, 2 * hidden_dim, bias=False)
        self.w2 = nn.Linear(hidden_dim, dim, bias=False)
        self.act_fn = nn.SiLU()
        if noise_dim > 0:
            self.noise_bias = nn.Linear(noise_dim, hidden_dim, bias=False)

    # With this set (and on a ROCm device with bf16 input of qualifying shape), w13 and the gate
    # run as one kernel (fused.swiglu_linear) on a row-permuted bf16 copy of w13, so h is never
    # stored.  Off by default: at the era5 stage-1 shape (1,179,648 rows, 768 -> 2 x 3072, 24
    # members) the fused kernel takes 15.3 ms against 14.1 ms for the library GEMM (9.4 ms)
    # followed by the gate kernel; its GEMM core alone (epilogue arithmetic removed) takes
    # 12.8 ms, slower than the library's.
    fused_linear_gate = False

    def _w13_perm(self) -> torch.Tensor:
        wt = self.w13.weight
        key = (wt.data_ptr(), wt._version, wt.device, wt.dtype)
        if getattr(self, "_w13_perm_key", None) != key:
            with torch.no_grad():
                self._w13_perm_cache = fused.permute_w13(wt.detach().to(torch.bfloat16))
            self._w13_perm_key = key
        return self._w13_perm_cache

    def forward(self, x: torch.Tensor, z: torch.Tensor | None = None) -> torch.Tensor:
        noise = self.noise_bias(z) if z is not None else None      # [B, hidden]
        if self.fused_linear_gate and fused.swiglu_linear_ok(x, self.w2.in_features):
            forward_only("cSwiGLU", x, self.w13.weight, noise)
            return self.w2(fused.swiglu_linear(x, self._w13_perm(), noise))
        h = self.w13(x)
        if h.is_cuda:
            g = fused.swiglu(h, noise)
        else:
            x1, x3 = h.chunk(2, dim=-1)
            g = self.act_fn(x1 + (noise.unsqueeze(0) if noise is not None else 0)) * x3
        return self.w2(g)


class MosaicBlock(nn.Module):
    """Pre-norm transformer block: attention then SwiGLU, each residual (primitives.py:212-227)."""

    def __init__(self, config, block_attn_only: bool, no_compression: bool = False):
        super().__init__()
        dim = config.dim
        self.attention = MosaicAttention(config, block_attn_only, no_compression)
        self.norm1 = RMSNorm(dim, elementwise_affine=config.rmsnorm_elementwise_affine)
        self.norm2 = RMSNorm(dim, elementwise_affine=config.rmsnorm_elementwise_affine)
        self.ffn = cSwiGLU(dim, int(dim * config.mlp_ratio), config.noise_dim)

    def forward(self, x: torch.Tensor, z: torch.Tensor | None = None) -> torch.Tensor:
        x, f = self.forward_deferred(x, None, z)
        return x + f

    def forward_deferred(self, x: torch.Tensor, pending: torch.Tensor | None, z: torch.Tensor | None = None):
        """The block on ``x + pending`` with its own last residual add left undone: returns
        ``(y, f)`` with the block's output equal to ``y + f``.  A stage passes ``f`` on to the
        next block, whose norm1 adds it in the same pass that normalises (each add then costs
        no separate read and write of the activations)."""
        if pending is None:
            h = self.norm1(x)
        else:
            x, h = self.norm1.add_forward(x, pending)
        # x + attention(norm1(x)), then norm2 of that sum, in one pass over the activations
        x, h = self.norm2.add_forward(x, self.attention(h))
        return x, self.ffn(h, z)


class NoiseGenerator(nn.Module):
    """Per-sample noise vectors ``to_noise(randn(n, noise_dim))`` from a seeded device generator
    (primitives.py:286-302)."""

    def __init__(self, noise_dim: int, seed: int):
        super().__init__()
        self.seed = seed
        self.to_noise = nn.Linear(noise_dim, noise_dim, bias=False)
        self.generator = None

    def forward(self, num_samples: int, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        if self.generator is None:
            self.generator = torch.Generator(device=device)
            self.generator.manual_seed(self.seed)
        noise = torch.randn((num_samples, self.to_noise.in_features), generator=self.generator,
                            device=device, dtype=dtype)
        return self.to_noise(noise)


def _child_offsets(nside_fine: int, nside_coarse: int) -> torch.Tensor:
    """Standardised xyz offsets of each coarse pixel's children, ``[n_coarse, f*3]``
    (primitives.py:315-322, 338-345).  In NESTED order the f = (nside_fine/nside_coarse)^2
    children of coarse pixel p are the fine pixels p*f .. p*f+f-1."""
    fine = rad_to_xyz(torch.deg2rad(get_healpix_grid(nside_fine)))
    coarse = rad_to_xyz(torch.deg2rad(get_healpix_grid(nside_coarse)))
    f = fine.shape[0] // coarse.shape[0]
    rel = (fine.view(coarse.shape[0], f, 3) - coarse[:, None]).reshape(coarse.shape[0], f * 3)
    return ((rel - rel.mean(dim=0, keepdim=True)) / (rel.std(dim=0, keepdim=True) + 1e-6)).contiguous()


def _bf16_epilogue(*ts: torch.Tensor) -> bool:
    """Whether a resampling epilogue runs as fused.resample_norm: bf16 ROCm tensors whose
    RMSNorm output would be bf16 too (the model under bf16 autocast)."""
    return (all(t.is_cuda and t.dtype == torch.bfloat16 for t in ts)
            and fused.autocast_dtype(ts[0]) == torch.bfloat16)


class HEALPixDownsample(nn.Module):
    """Merge each coarse pixel's f children: ``norm(proj_x(concat children) + proj_pos(rel_pos))``
    (primitives.py:305-329).  The concat is a view of the NESTED sequence-first activations."""

    space_dim: int = 3

    def __init__(self, in_dim, out_dim, nside_before, nside_after, rmsnorm_elementwise_affine=True):
        super().__init__()
        self.factor = (nside_before // nside_after) ** 2
        self.proj_x = nn.Linear(self.factor * in_dim, out_dim, bias=False)
        self.proj_pos = nn.Linear(self.factor * self.space_dim, out_dim, bias=False)
        self.norm = RMSNorm(out_dim, elementwise_affine=rmsnorm_elementwise_affine)
        self.register_buffer("rel_pos", _child_offsets(nside_before, nside_after), persistent=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        S, B, C = x.shape
        # '(n f) b c -> n b (f c)': pixel n*f + j, member b lands at [n, b, j*C:(j+1)*C]
        x = x.view(S // self.factor, self.factor, B, C).transpose(1, 2).reshape(S // self.factor, B, self.factor * C)
        return self.forward_merged(x)

    def forward_merged(self, x: torch.Tensor) -> torch.Tensor:
        """forward on the children already merged per coarse pixel, ``[n, B, f * C]``."""
        p, pos = self.proj_x(x), self.proj_pos(self.rel_pos)
        if _bf16_epilogue(p, pos):  # the add and the norm in one pass
            return fused.resample_norm(p, pos, self.norm.weight, self.norm.eps, 1)
        return self.norm(p + pos.unsqueeze(1))


class HEALPixUpsample(nn.Module):
    """Split each coarse pixel into its f children and add the skip connection:
    ``norm(split(proj_x(x) + proj_pos(rel_pos)) + shortcut)`` (primitives.py:332-359)."""

    space_dim: int = 3

    def __init__(self, in_dim, out_dim, nside_before, nside_after, rmsnorm_elementwise_affine=True):
        super().__init__()
        self.factor = (nside_after // nside_before) ** 2
        self.proj_x = nn.Linear(in_dim, out_dim * self.factor, bias=False)
        self.proj_pos = nn.Linear(self.factor * self.space_dim, out_dim * self.factor, bias=False)
        self.norm = RMSNorm(out_dim, elementwise_affine=rmsnorm_elementwise_affine)
        self.register_buffer("rel_pos", _child_offsets(nside_after, nside_before), persistent=True)

    def forward(self, x: torch.Tensor, shortcut: torch.Tensor) -> torch.Tensor:
        n, B, _ = x.shape
        p, pos = self.proj_x(x), self.proj_pos(self.rel_pos)
        if _bf16_epilogue(p, pos, shortcut):  # add, split, skip add and norm in one pass
            return fused.resample_norm(p, pos, self.norm.weight, self.norm.eps, self.factor, shortcut)
        x = p + pos.unsqueeze(1)
        # 'n b (f d) -> (n f) b d'
        x = x.view(n, B, self.factor, -1).transpose(1, 2).reshape(n * self.factor, B, -1)
        return self.norm(x + shortcut)


class UNetStage(nn.Module):
    """``depth`` MosaicBlocks at one resolution (mosaic.py:116-133); with sparse_every = 1 every
    block runs all three attention branches."""

    def __init__(self, config: ModelConfig, stage_cfg, depth: int):
        super().__init__()
        self.nside = stage_cfg.nside
        merged = _merge_configs(config, stage_cfg)
        self.blocks = nn.ModuleList([
            MosaicBlock(merged,
                        block_attn_only=(config.sparse_every <= 0) or not (i % config.sparse_every == 0),
                        no_compression=config.no_compression)
            for i in range(depth)])

    def forward(self, x: torch.Tensor, z: torch.Tensor | None = None) -> torch.Tensor:
        x, pending = self.forward_pending(x, z)
        return x if pending is None else x + pending

    def forward_pending(self, x: torch.Tensor, z: torch.Tensor | None = None):
        """The stage with its last residual add left undone: ``(x, pending)``, the output being
        ``x + pending`` (pending None for a stage without blocks)."""
        pending = None
        for block in self.blocks:
            x, pending = block.forward_deferred(x, pending, z)
        return x, pending


class Transformer(nn.Module):
    """The U-Net forecast backbone (mosaic.py:136-337): lat-lon features -> preprocess MLP ->
    interpolation to HEALPix -> encoder stages with downsampling -> bottleneck -> decoder
    stages with upsampling and skips -> interpolation back to lat-lon -> postprocess MLP."""

    space_dim = 3
    time_dim = 4

    def __init__(self, config: ModelConfig, seed: int = 42):
        super().__init__()
        self.config = config
        self.nside = config.cg_stage_cfgs[0].nside
        self.noise_dim = config.noise_dim
        d0 = config.dim
        affine = config.rmsnorm_elementwise_affine
        feature_dim = (len(config.variables) * config.num_history_steps + len(config.static_variables)
                       + self.space_dim + self.time_dim)
        if self.noise_dim > 0:
            self.noise_generator = NoiseGenerator(self.noise_dim, seed)
        self.preprocess = nn.Sequential(
            nn.Linear(feature_dim, d0, bias=False), RMSNorm(d0, elementwise_affine=affine), nn.SiLU(),
            nn.Linear(d0, d0, bias=False), RMSNorm(d0, elementwise_affine=affine))
        self.interp_to_hp = CrossAttentionInterpolate(config)
        self.interp_to_ll = CrossAttentionInterpolate(config)

        stages = [*config.cg_stage_cfgs, config.bottleneck_cfg]
        self.encoder_stages = nn.ModuleList()
        self.downsample_layers = nn.ModuleList()
        for i in range(len(config.cg_stage_cfgs)):
            cur, nxt = stages[i], stages[i + 1]
            self.encoder_stages.append(UNetStage(config, cur, cur.encoder_depth))
            self.downsample_layers.append(HEALPixDownsample(cur.dim, nxt.dim, cur.nside, nxt.nside, affine))
        self.bottleneck = UNetStage(config, config.bottleneck_cfg, config.bottleneck_cfg.depth)
        self.decoder_stages = nn.ModuleList()
        self.upsample_layers = nn.ModuleList()
        for i in reversed(range(len(config.cg_stage_cfgs))):
            prev, cur = stages[i + 1], stages[i]
            self.upsample_layers.append(HEALPixUpsample(prev.dim, cur.dim, prev.nside, cur.nside, affine))
            self.decoder_stages.append(UNetStage(config, cur, cur.decoder_depth))
        self.norm_before_interp_ll = RMSNorm(d0, elementwise_affine=affine)
        self.postprocess = nn.Sequential(
            RMSNorm(d0, elementwise_affine=affine), nn.Linear(d0, d0, bias=False), nn.SiLU(),
            nn.Linear(d0, len(config.variables), bias=False))

        self.apply(self._initialize_weights)
        self._zero_init_residual_layers()
        self.initialize_rope()

    def _initialize_weights(self, module):
        """N(0, std) with std = min(1, sqrt(fan_out/fan_in)) / sqrt(fan_in) (mosaic.py:224-236)."""
        if module is self or not isinstance(module, nn.Linear):
            return
        fan_in, fan_out = module.weight.size(1), module.weight.size(0)
        std = 1.0 / math.sqrt(fan_in) * min(1.0, math.sqrt(fan_out / fan_in))
        if self.config.ortho_init:
            nn.init.orthogonal_(module.weight)
            module.weight.data.mul_(std)
        else:
            nn.init.normal_(module.weight, mean=0.0, std=std)
        if module.bias is not None:
            nn.init.zeros_(module.bias)

    def _zero_init_residual_layers(self):
        """Residual outputs, upsampling projections and the noise map start near zero (mosaic.py:238-264)."""
        def small(w):
            if self.config.ortho_init:
                nn.init.orthogonal_(w)
                w.data.mul_(0.01)
            else:
                nn.init.normal_(w, mean=0.0, std=0.01)
        for stage in [*self.encoder_stages, self.bottleneck, *self.decoder_stages]:
            for block in stage.blocks:
                small(block.attention.to_o.weight)
                small(block.ffn.w2.weight)
                if self.noise_dim > 0:
                    nn.init.normal_(block.ffn.noise_bias.weight, mean=0.0, std=0.01)
        for up in self.upsample_layers:
            small(up.proj_x.weight)
            small(up.proj_pos.weight)
        if self.noise_dim > 0:
            nn.init.normal_(self.noise_generator.to_noise.weight, mean=0.0, std=0.01)

    def initialize_rope(self):
        """RoPE tables of every attention layer from its stage's HEALPix grid (mosaic.py:266-274)."""
        if not self.config.rope:
            return
        for stage in [*self.encoder_stages, self.bottleneck, *self.decoder_stages]:
            grid = get_healpix_grid(stage.nside)
            for block in stage.blocks:
                if block.attention.q_rope is not None:
                    block.attention.q_rope.initialize_rope(grid)
                    block.attention.k_rope.initialize_rope(grid)

    def initialize_interpolation(self, longitude: torch.Tensor, latitude: torch.Tensor):
        """k-NN schemes lat-lon -> HEALPix and back (mosaic.py:276-280); lon-major meshgrid."""
        ll = torch.deg2rad(torch.stack(torch.meshgrid(longitude, latitude, indexing="ij"), -1).reshape(-1, 2))
        hp = torch.deg2rad(get_healpix_grid(self.nside)).to(longitude.device)
        self.interp_to_hp.initialize_interpolation_scheme(ll, hp)
        self.interp_to_ll.initialize_interpolation_scheme(hp, ll)

    @torch.no_grad()
    def initialize_static_vars(self, static_vars: torch.Tensor, longitude: torch.Tensor, latitude: torch.Tensor):
        """Static fields [lon, lat, c] plus the grid's xyz, standardised per channel, stored as
        ``[(lon lat), 1, c+3]`` (mosaic.py:282-291)."""
        ll = torch.deg2rad(torch.stack(torch.meshgrid(longitude, latitude, indexing="ij"), -1))
        s = torch.cat([static_vars, rad_to_xyz(ll)], dim=-1)
        s = (s - s.mean(dim=(0, 1), keepdim=True)) / (s.std(dim=(0, 1), keepdim=True) + 1e-6)
        self.register_buffer("static_vars", s.reshape(-1, 1, s.shape[-1]).contiguous(), persistent=True)

    @torch.no_grad()
    def time_embedding(self, day_year_time: torch.Tensor) -> torch.Tensor:
        """[sin, cos] of the day and year phases (mosaic.py:293-302)."""
        day, year = day_year_time[:, 0:1], day_year_time[:, 1:2]
        return torch.cat([torch.sin(2 * math.pi * day), torch.cos(2 * math.pi * day),
                          torch.sin(2 * math.pi * year), torch.cos(2 * math.pi * year)], dim=-1)

    def forward(self, x: torch.Tensor, day_year_time: torch.Tensor, num_noise_samples: int) -> torch.Tensor:
        """x [b, n, t, lon, lat, c] -> [b, n*s, lon, lat, len(variables)] (mosaic.py:304-337)."""
        b, n, t, lon, lat, c = x.shape
        s = num_noise_samples
        batch = b * s * n
        z = self.noise_generator(batch, x.device, x.dtype) if self.noise_dim > 0 else None
        # 'b n t lon lat c -> (lon lat) (b s n) (t c)'
        xs = x.permute(3, 4, 0, 1, 2, 5).reshape(lon * lat, b, 1, n, t * c).expand(-1, -1, s, -1, -1)
        xs = xs.reshape(lon * lat, batch, t * c)
        dyt = day_year_time.unsqueeze(1).expand(-1, s, -1, -1).reshape(batch, -1)
        xs = torch.cat([xs, self.static_vars.expand(-1, batch, -1),
                        self.time_embedding(dyt).unsqueeze(0).expand(xs.shape[0], -1, -1)], dim=-1)

        h = self.preprocess(xs)
        h = self.interp_to_hp(h)
        skips = []
        for stage, down in zip(self.encoder_stages, self.downsample_layers):
            h, pending = stage.forward_pending(h, z)
            if pending is not None and _bf16_epilogue(h, pending):
                # the stage's last add and the merge of the children in one pass
                h, merged = fused.add_merge(h, pending, down.factor)
                skips.append(h)
                h = down.forward_merged(merged)
            else:
                h = h if pending is None else h + pending
                skips.append(h)
                h = down(h)
        h = self.bottleneck(h, z)
        pending = None
        for i, (stage, up, skip) in enumerate(zip(self.decoder_stages, self.upsample_layers, reversed(skips))):
            h = up(h, skip)
            if i + 1 < len(self.decoder_stages):
                h = stage(h, z)
            else:  # the last stage's residual add goes into the norm after it
                h, pending = stage.forward_pending(h, z)
        h = self.norm_before_interp_ll(h) if pending is None else self.norm_before_interp_ll.add_norm(h, pending)
        h = self.interp_to_ll(h)
        h = self.postprocess(h)
        # '(lon lat) (b n s) c -> b (n s) lon lat c'
        return h.view(lon, lat, b, n * s, -1).permute(2, 3, 0, 1, 4)


def model_flops(config: ModelConfig, batch: int, n_ll: int) -> dict:
    """Algorithmic FLOPs of one forward for ``batch`` samples on an ``n_ll``-point lat-lon grid:
    2*M*N*K per projection, the attention op's per-config formula per layer, and the k-NN
    interpolations' q.k and p.v products (elementwise work is not counted)."""
    d0 = config.dim
    H0 = config.num_heads
    feat = len(config.variables) * config.num_history_steps + len(config.static_variables) + 7
    gemm = 2 * n_ll * batch * (feat * d0 + d0 * d0)                  # preprocess
    gemm += 2 * n_ll * batch * (d0 * d0 + d0 * len(config.variables))  # postprocess
    npix0 = 12 * config.cg_stage_cfgs[0].nside ** 2
    gemm += 2 * npix0 * batch * (2 * d0 * d0 + d0 * d0)                 # interp to_hp: to_kv + to_o
    gemm += 2 * npix0 * batch * 2 * d0 * d0 + 2 * n_ll * batch * d0 * d0  # interp to_ll
    interp = 4 * batch * config.k_neighbors * d0 * (n_ll + npix0)
    attn = 0
    stages = [*config.cg_stage_cfgs, config.bottleneck_cfg]
    for i, st in enumerate(stages):
        depth = st.depth if i == len(stages) - 1 else st.encoder_depth + st.decoder_depth
        N = 12 * st.nside ** 2
        D = st.dim
        Hq = st.num_heads
        Hk = Hq // st.gqa_ratio
        hd = D // Hq // config.qkv_compress_ratio
        hid = int(D * st.mlp_ratio)
        per_tok = 2 * D * (Hq * hd + 2 * Hk * hd + Hq * hd) + 2 * D * 3 * Hq + 2 * D * 2 * hid + 2 * hid * D
        gemm += depth * per_tok * N * batch
        nb = N // st.sparse_block_size
        attn += depth * (4 * batch * Hq * hd * (N * st.block_attn_size + N * st.sparse_block_count
                                                * st.sparse_block_size + nb * nb) + 2 * batch * Hq * hd * nb * nb)
        if i < len(stages) - 1:
            nxt = stages[i + 1]
            f = (st.nside // nxt.nside) ** 2
            n_c = 12 * nxt.nside ** 2
            gemm += 2 * n_c * batch * f * D * nxt.dim                   # downsample proj_x
            gemm += 2 * n_c * batch * nxt.dim * f * D                   # upsample proj_x
    return {"gemm": gemm, "attention": attn, "interp": interp, "total": gemm + attn + interp}
