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
