"""CPU checks of the U-Net's structure (mosaic.py, primitives.py:286-359) without a GPU.

* The shipped era5 preset has 214,184,448 parameters, the count read off the reference's
  module definitions, and the reference's parameter names.
* The FLOP model of one forward reproduces the per-layer attention totals of the op's own
  formula and the whole-step total.
* The HEALPix resampling modules group pixels as the reference's einops patterns do
  (evaluated by einops itself), and their child offsets are standardised per column.
* The oracle's autocast Linear rounds once, from fp32 accumulation.
"""

import math

import torch
from einops import rearrange

from mosaic_amd.model import (HEALPixDownsample, HEALPixUpsample, Transformer, _child_offsets, era5_config,
                              model_flops)
from oracle import bsa_oracle, unet_oracle


def test_era5_parameter_count_and_names():
    m = Transformer(era5_config())
    assert sum(p.numel() for p in m.parameters()) == 214_184_448
    names = set(dict(m.named_parameters()))
    for n in ["noise_generator.to_noise.weight", "preprocess.0.weight", "preprocess.3.weight",
              "interp_to_hp.to_kv.weight", "interp_to_ll.to_q.weight",
              "encoder_stages.0.blocks.3.attention.to_strategy_combine_mlp.weight",
              "encoder_stages.1.blocks.0.ffn.w13.weight", "encoder_stages.1.blocks.0.ffn.noise_bias.weight",
              "downsample_layers.0.proj_x.weight", "downsample_layers.1.proj_pos.weight",
              "bottleneck.blocks.1.attention.to_o.weight", "upsample_layers.0.proj_x.weight",
              "decoder_stages.1.blocks.1.ffn.w2.weight", "postprocess.3.weight"]:
        assert n in names, n
    # stage dims: downsample 0 maps 4 x 768 -> 1024, upsample 0 maps 1280 -> 4 x 1024
    assert tuple(m.downsample_layers[0].proj_x.weight.shape) == (1024, 4 * 768)
    assert tuple(m.upsample_layers[0].proj_x.weight.shape) == (4 * 1024, 1280)
    assert tuple(m.preprocess[0].weight.shape) == (768, 82 * 2 + 3 + 3 + 4)
    # zero-ish init of the residual outputs (mosaic.py:238-264)
    assert m.encoder_stages[0].blocks[0].attention.to_o.weight.std().item() < 0.02


def test_model_flops():
    cfg = era5_config()
    f = model_flops(cfg, 24, 240 * 121)
    # per member and layer: stage 1 619.2, stage 2 128.9, bottleneck 24.2 GFLOP of attention
    per_member = (6 * bsa_oracle.flops(1, 49152, 12, 64, 1024, 128, 24)
                  + 6 * bsa_oracle.flops(1, 12288, 16, 64, 1024, 128, 12)
                  + 2 * bsa_oracle.flops(1, 3072, 20, 64, 1024, 128, 4))
    assert f["attention"] == 24 * per_member
    assert abs(bsa_oracle.flops(1, 49152, 12, 64, 1024, 128, 24) / 1e9 - 619.2) < 0.1
    assert 300e12 < f["total"] < 315e12          # ~307 TFLOP per 24-member step


def test_resampling_layouts_match_einops():
    torch.manual_seed(0)
    down = HEALPixDownsample(16, 24, 4, 2, rmsnorm_elementwise_affine=False)
    x = torch.randn(192, 3, 16)
    ref_in = rearrange(x, "(n f) b c -> n b (f c)", f=4)
    ref = torch.nn.functional.rms_norm(down.proj_x(ref_in) + down.proj_pos(down.rel_pos).unsqueeze(1), (24,))
    assert torch.allclose(down(x), ref, atol=1e-5)
    up = HEALPixUpsample(24, 16, 2, 4, rmsnorm_elementwise_affine=False)
    y = torch.randn(48, 3, 24)
    skip = torch.randn(192, 3, 16)
    t = rearrange(up.proj_x(y) + up.proj_pos(up.rel_pos).unsqueeze(1), "n b (f d) -> (n f) b d", f=4)
    assert torch.allclose(up(y, skip), torch.nn.functional.rms_norm(t + skip, (16,)), atol=1e-5)


def test_child_offsets():
    off = _child_offsets(8, 4)               # 192 coarse pixels, 4 children each
    assert off.shape == (192, 12)
    assert torch.allclose(off.mean(0), torch.zeros(12), atol=1e-5)
    # unit std per column, except the z offsets of children 1 and 2, which share their
    # parent's ring height: those columns are ~0 after the +1e-6 guarded standardisation
    sd = off.std(0)
    flat = torch.tensor([i in (5, 8) for i in range(12)])
    assert torch.allclose(sd[~flat], torch.ones(10), atol=1e-3) and (sd[flat] < 0.05).all()
    # nested children surround their parent: the raw offsets of the 4 children sum to ~0
    from mosaic_amd.healpix import get_healpix_grid
    from mosaic_amd.interp import rad_to_xyz
    fine = rad_to_xyz(torch.deg2rad(get_healpix_grid(8))).view(192, 4, 3)
    parent = rad_to_xyz(torch.deg2rad(get_healpix_grid(4)))
    centroid = fine.mean(1)
    assert (centroid - parent).norm(dim=-1).max() < 0.02
    assert ((fine - parent[:, None]).norm(dim=-1) < 0.25).all()


def test_oracle_linear_rounds_once():
    x = torch.randn(7, 33)
    w = torch.randn(5, 33)
    got = unet_oracle.linear(x, w)
    exact = x.bfloat16().double() @ w.bfloat16().double().t()
    assert got.dtype == torch.bfloat16
    # one rounding of the (nearly exact) fp32 sum: within half a bf16 spacing plus fp32 noise
    assert ((got.double() - exact).abs() <= exact.abs() * 2 ** -8 + 1e-4).all()
    assert math.isclose(unet_oracle.rms_norm(torch.full((1, 4), 3.0), {torch.float32: torch.float32})[0, 0].item(),
                        1.0, rel_tol=1e-6)


def _tiny_unet_cpu(seed=0):
    """The tiny three-resolution U-Net of the GPU model tests (nside 16 / 8 / 4, head_dim 64),
    random init with the residual outputs at full scale, on the CPU, as a state dict."""
    from mosaic_amd.model import BottleneckConfig, ModelConfig, StageConfig
    stages = [StageConfig(nside=16, dim=256, num_heads=4, block_attn_size=256, sparse_block_size=64,
                          sparse_block_count=6, encoder_depth=1, decoder_depth=1, mlp_ratio=2.0, gqa_ratio=4),
              StageConfig(nside=8, dim=512, num_heads=8, block_attn_size=256, sparse_block_size=64,
                          sparse_block_count=4, encoder_depth=1, decoder_depth=1, mlp_ratio=2.0, gqa_ratio=4)]
    bottleneck = BottleneckConfig(nside=4, dim=512, num_heads=8, block_attn_size=192, sparse_block_size=64,
                                  sparse_block_count=2, depth=1, mlp_ratio=2.0, gqa_ratio=4)
    cfg = ModelConfig(dim=256, num_heads=4, k_neighbors=8, qk_norm=False, rope=True, rope_theta=10000,
                      sparse_every=1, variables=[f"v{i}" for i in range(5)], static_variables=["a", "b", "c"],
                      qkv_compress_ratio=1, cg_stage_cfgs=stages, bottleneck_cfg=bottleneck,
                      num_history_steps=2, noise_dim=32, rmsnorm_elementwise_affine=False)
    torch.manual_seed(seed)
    model = Transformer(cfg, seed=11)
    g = torch.Generator().manual_seed(seed + 1)
    for name, p in model.named_parameters():
        if name.endswith(("to_o.weight", "w2.weight", "proj_x.weight", "proj_pos.weight")) and "interp" not in name:
            p.data = torch.randn(p.shape, generator=g) / math.sqrt(p.shape[1])
    lon, lat = torch.linspace(0, 345, 24), torch.linspace(-90, 90, 13)
    model.initialize_interpolation(lon, lat)
    model.initialize_static_vars(torch.randn(24, 13, 3, generator=g), lon, lat)
    probe = {dt: torch.nn.functional.rms_norm(torch.zeros(1, 8, dtype=dt), (8,)).dtype
             for dt in (torch.bfloat16, torch.float32)}
    return cfg, model.state_dict(), probe


def test_unet_oracle_members_are_independent_and_ordered():
    """The oracle's composition of the whole forward keeps ensemble members apart (mosaic.py:
    301-309: each member is the same input with its own noise row): two members at once give
    each member's one-member forecast, and swapping the noise rows swaps the members.  A
    rearrange that mixed the member and pixel axes anywhere in the chain (the einops patterns
    of the stages, the attention, the interpolation) would fail; so does a planted one."""
    cfg, P, probe = _tiny_unet_cpu()
    # the noise projection at a scale where the members' forecasts differ clearly (it is
    # initialised at std 0.01)
    P = dict(P)
    P["noise_generator.to_noise.weight"] = P["noise_generator.to_noise.weight"] * 100
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 1, 2, 24, 13, 5, generator=g)
    dyt = torch.rand(1, 1, 2, generator=g)
    noise = torch.randn(2, cfg.noise_dim, generator=g)
    both = unet_oracle.forward(P, cfg, x, dyt, 2, noise, probe).float()
    one = [unet_oracle.forward(P, cfg, x, dyt, 1, noise[i:i + 1], probe).float() for i in range(2)]
    swapped = unet_oracle.forward(P, cfg, x, dyt, 2, noise.flip(0), probe).float()
    assert both.shape == (1, 2, 24, 13, 5)
    # the members differ by ~45% (relative L2); one member alone or in the pair agrees to ~1%
    # (the CPU products sum in another order for another batch size, and bf16 roundings
    # propagate through the layers)
    assert ((both[:, 0] - both[:, 1]).norm() / both[:, 0].norm()).item() > 0.2
    for i in range(2):
        rel = ((both[:, i] - one[i][:, 0]).norm() / one[i].norm()).item()
        assert rel <= 3e-2, (i, rel)
    assert ((swapped.flip(1) - both).norm() / both.norm()).item() <= 3e-2

    # planted: the attention output of every layer rolled by one member
    real = unet_oracle.mosaic_attention
    try:
        unet_oracle.mosaic_attention = lambda *a, **k: real(*a, **k).roll(1, dims=1)
        mixed = unet_oracle.forward(P, cfg, x, dyt, 2, noise, probe).float()
    finally:
        unet_oracle.mosaic_attention = real
    assert ((mixed[:, 0] - one[0][:, 0]).norm() / one[0].norm()).item() > 6e-2   # ~12%
