"""GPU parity of the k-nearest-neighbour cross-attention (CrossAttentionInterpolate's
gather-attention, primitives.py:265-283) against the CPU oracle (marked ``gpu``).

Both product forms are tested: exact products summed in fp32 (the default, as the reference's
compiled inference path fuses them into the sums) against the oracle's ``products="fp32"``,
and products rounded to bf16 (``round_products=True``, the reference's eager elementwise ops)
against its ``products="bf16"``.  Bars: max-abs 2e-2 and relative L2 1e-2 (bf16 in, fp32
accumulate); the kernel rounds where its oracle form rounds, so nearly every output is
bit-equal to it (sums in another order and the exponential's last fp32 bits aside): at least
97% of the elements must be.  Against the eager form the fp32 form is held to relative L2
1e-2 (the two differ by up to two bf16 spacings where the softmax is sharp), and against a
float64 evaluation of the same formula it must be at least as accurate as the eager form.
"""

import pytest
import torch

from mosaic_amd.healpix import get_healpix_grid
from mosaic_amd.interp import CrossAttentionInterpolate, get_neighbors, knn_attention, rad_to_xyz, spatial_order
from oracle import interp_oracle as IO

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_ABS = 2e-2
REL_L2 = 1e-2


def close(got, ref, min_equal=0.97):
    g, r = got.float().cpu(), ref.float().cpu()
    assert g.shape == r.shape, (g.shape, r.shape)
    assert torch.isfinite(g).all(), "non-finite output"
    err = (g - r).abs().max().item()
    rel = ((g - r).norm() / r.norm().clamp_min(1e-30)).item()
    eq = (got.cpu() == ref.cpu()).float().mean().item()
    assert err <= MAX_ABS and rel <= REL_L2 and eq >= min_equal, f"max_abs {err:.3e} rel_l2 {rel:.3e} equal {eq:.4f}"


FORMS = pytest.mark.parametrize("round_products", [False, True], ids=["fp32_products", "bf16_products"])


def oracle(k, v, nb, rel, w_q, scale, round_products):
    return IO.knn_attention(k, v, nb, rel, w_q, scale, products="bf16" if round_products else "fp32")


def exact(k, v, nb, rel, w_q, scale):
    """The gather-attention in float64 from the bf16 queries (to_q's bf16 output)."""
    H = k.shape[2]
    q = (rel.to(torch.bfloat16).float() @ w_q.float().t()).to(torch.bfloat16).double()
    q = q.view(*q.shape[:2], 1, H, 64)
    kg, vg = k.double()[nb], v.double()[nb]
    p = torch.softmax((q * kg).sum(-1, keepdim=True) * scale, dim=1)
    return (p * vg).sum(dim=1)


def lonlat_grid(n_lon, n_lat):
    lon = torch.linspace(0, 360 - 360 / n_lon, n_lon)
    lat = torch.linspace(-90, 90, n_lat)
    return torch.deg2rad(torch.stack(torch.meshgrid(lon, lat, indexing="ij"), -1).reshape(-1, 2))


def scheme(pos_from, pos_to, K):
    nb = torch.from_numpy(get_neighbors(pos_from.numpy(), pos_to.numpy(), k=K)).long()
    rel = rad_to_xyz(pos_to).unsqueeze(1) - rad_to_xyz(pos_from)[nb]
    return nb, torch.nn.functional.normalize(rel, dim=-1)


def rand(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@FORMS
@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
@pytest.mark.parametrize("K", [32, 29, 24, 20, 7, 1])
def test_knn_attention_matches_oracle(direction, K, round_products):
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))    # 312 and 192 points
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    nb, rel = scheme(src, dst, K)
    B, H = 2, 3
    k, v = rand(len(src), B, H, 64, seed=K), rand(len(src), B, H, 64, seed=K + 100)
    w_q = rand(H * 64, 3, seed=K + 200, scale=2.0)
    ref = oracle(k, v, nb, rel, w_q, 0.125, round_products)
    got = knn_attention(k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125,
                        round_products=round_products)
    torch.cuda.synchronize()
    if K == 1:
        assert torch.equal(got.cpu(), v[nb[:, 0]])
    close(got, ref)
    if not round_products:   # the fp32 form against the eager form and against float64
        eager = IO.knn_attention(k, v, nb, rel, w_q, 0.125).double()
        g = got.cpu().double()
        assert ((g - eager).norm() / eager.norm()).item() <= REL_L2
        x = exact(k, v, nb, rel, w_q, 0.125)
        err_got, err_eager = ((g - x).norm() / x.norm()).item(), ((eager - x).norm() / x.norm()).item()
        assert err_got <= 1.05 * err_eager, (err_got, err_eager)


@FORMS
def test_knn_attention_zero_queries_and_large_scores(round_products):
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(ll, hp, 24)
    k, v = rand(len(ll), 1, 4, 64, seed=1, scale=3.0), rand(len(ll), 1, 4, 64, seed=2)
    for w_q, scale in ((torch.zeros(4 * 64, 3, dtype=torch.bfloat16), 0.125), (rand(4 * 64, 3, seed=3, scale=4.0), 1.0)):
        ref = oracle(k, v, nb, rel, w_q, scale, round_products)
        got = knn_attention(k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), scale,
                            round_products=round_products)
        close(got, ref)


@FORMS
def test_knn_attention_strided_views_equal_contiguous(round_products):
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(hp, ll, 20)
    S, B, H = len(hp), 3, 2
    kv = rand(S, B, 2 * H * 64, seed=4).to(DEV)              # the to_kv output layout
    k = kv[..., :H * 64].unflatten(-1, (H, 64))
    v = kv[..., H * 64:].unflatten(-1, (H, 64))
    w_q = rand(H * 64, 3, seed=5).to(DEV)
    a = knn_attention(k, v, nb.to(DEV), rel.to(DEV), w_q, 0.125, round_products=round_products)
    b = knn_attention(k.contiguous(), v.contiguous(), nb.to(DEV), rel.to(DEV), w_q, 0.125,
                      round_products=round_products)
    assert torch.equal(a, b)
    close(a, oracle(k.cpu(), v.cpu(), nb, rel, w_q.cpu(), 0.125, round_products))


@FORMS
@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
def test_knn_attention_full_size_sampled(direction, round_products):
    """Model grids: 121 x 240 lat-lon (29040 points) and HEALPix nside 64 (49152), K 24,
    12 heads; every target computed on the device, a sample of targets against the oracle."""
    ll, hp = lonlat_grid(240, 121), torch.deg2rad(get_healpix_grid(64))
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    K, B, H = 24, 2, 12
    nb, rel = scheme(src, dst, K)
    k, v = rand(len(src), B, H, 64, seed=7), rand(len(src), B, H, 64, seed=8)
    w_q = rand(H * 64, 3, seed=9)
    got = knn_attention(k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125,
                        round_products=round_products).cpu()
    g = torch.Generator().manual_seed(10)
    sample = torch.cat([torch.arange(64), len(dst) - 64 + torch.arange(64),
                        torch.randint(0, len(dst), (1024,), generator=g)])
    ref = oracle(k, v, nb[sample], rel[sample], w_q, 0.125, round_products)
    close(got[sample], ref)


@FORMS
def test_knn_attention_deterministic(round_products):
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = [t.to(DEV) for t in scheme(ll, hp, 24)]
    k, v = rand(len(ll), 2, 3, 64, seed=11).to(DEV), rand(len(ll), 2, 3, 64, seed=12).to(DEV)
    w_q = rand(3 * 64, 3, seed=13).to(DEV)
    a = knn_attention(k, v, nb, rel, w_q, 0.125, round_products=round_products)
    assert all(torch.equal(a, knn_attention(k, v, nb, rel, w_q, 0.125, round_products=round_products))
               for _ in range(3))


@FORMS
def test_cross_attention_interpolate_module(round_products):
    from types import SimpleNamespace
    cfg = SimpleNamespace(k_neighbors=20, dim=192, num_heads=3, rmsnorm_elementwise_affine=True)
    torch.manual_seed(0)
    m = CrossAttentionInterpolate(cfg)
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    m.initialize_interpolation_scheme(ll, hp)
    m = m.to(DEV).to(torch.bfloat16)
    m.round_products = round_products
    x = torch.randn(len(ll), 2, 192, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="no backward"):   # parameters require grad
        m(x)
    with torch.no_grad():
        y = m(x)
    # the same torch projections around the oracle's gather-attention
    with torch.no_grad():
        kv = m.to_kv(m.kv_norm(x))
        k = kv[..., :192].unflatten(-1, (3, 64)).cpu()
        v = kv[..., 192:].unflatten(-1, (3, 64)).cpu()
        att = oracle(k, v, m.neighbors.cpu(), m.rel_pos.float().cpu(), m.to_q.weight.cpu(), m.scale, round_products)
        ref = m.to_o(att.to(DEV).flatten(-2))
    assert y.shape == (len(hp), 2, 192)
    close(y, ref, min_equal=0.9)


@FORMS
def test_knn_attention_random_neighbour_lists(round_products):
    """Neighbour lists with no spatial structure (repeats allowed), K = 13 (a partial slot)."""
    S_from, S_to, K = 2000, 160, 13
    g = torch.Generator().manual_seed(30)
    nb = torch.randint(0, S_from, (S_to, K), generator=g)
    rel = torch.nn.functional.normalize(torch.randn(S_to, K, 3, generator=g), dim=-1)
    k, v = rand(S_from, 2, 2, 64, seed=31), rand(S_from, 2, 2, 64, seed=32)
    w_q = rand(2 * 64, 3, seed=33)
    got = knn_attention(k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125,
                        round_products=round_products)
    close(got, oracle(k, v, nb, rel, w_q, 0.125, round_products))


@FORMS
@pytest.mark.parametrize("scale", [0.1, 0.3])
def test_knn_attention_scale_not_a_power_of_two(scale, round_products):
    """A scale that is not a power of two rounds bf16(score) * scale to bf16 again (the
    kernel's other path; 0.125 = 64^-0.5 skips that exact rounding)."""
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(ll, hp, 24)
    k, v = rand(len(ll), 2, 3, 64, seed=40, scale=2.0), rand(len(ll), 2, 3, 64, seed=41)
    w_q = rand(3 * 64, 3, seed=42, scale=2.0)
    got = knn_attention(k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), scale,
                        round_products=round_products)
    close(got, oracle(k, v, nb, rel, w_q, scale, round_products))


@FORMS
def test_knn_attention_negative_point_stride_equals_forward_order(round_products):
    """k / v handed over through the C ABI as views with a negative point stride over copies
    stored in reverse row order (point n is still k[n]): the kernel's 64-bit offset path,
    which must give the same output as the forward-order call (32-bit offsets)."""
    from mosaic_amd import _lib
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(hp, ll, 24)
    S, B, H = len(hp), 2, 3
    k, v = rand(S, B, H, 64, seed=50).to(DEV), rand(S, B, H, 64, seed=51).to(DEV)
    w_q = rand(H * 64, 3, seed=52).to(DEV)
    nb_d, rel_d = nb.to(DEV), rel.to(DEV)
    fwd = knn_attention(k, v, nb_d, rel_d, w_q, 0.125, round_products=round_products)
    kr, vr = k.flip(0).contiguous(), v.flip(0).contiguous()      # row S-1-n holds point n

    def reversed_view(t):     # starts at row S-1 (point 0) and steps back one row per point
        last = t[S - 1]
        return _lib.Bnhd(last.data_ptr(), t.stride(1), -t.stride(0), t.stride(2))
    nb32 = nb_d.to(torch.int32).contiguous()
    out = torch.empty_like(fwd)
    flags = _lib.KNN_ROUND_PRODUCTS if round_products else 0
    st = _lib.lib().mosaic_knn_interp_fwd_ex(reversed_view(kr), reversed_view(vr), nb32.data_ptr(),
                                             rel_d.float().contiguous().data_ptr(), w_q.data_ptr(), None, None,
                                             S, len(ll), B, H, 64, 24, 0.125, flags, out.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "mosaic_knn_interp_fwd_ex")
    torch.cuda.synchronize()
    assert torch.equal(out, fwd)


@FORMS
@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
def test_knn_attention_target_order_leaves_the_output_unchanged(direction, round_products):
    """The targets taken in the spatial order, in a random order and in index order: the same
    output bit for bit (each target's row is computed alone)."""
    ll, hp = lonlat_grid(48, 25), torch.deg2rad(get_healpix_grid(8))
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    nb, rel = [t.to(DEV) for t in scheme(src, dst, 24)]
    k, v = rand(len(src), 3, 2, 64, seed=60).to(DEV), rand(len(src), 3, 2, 64, seed=61).to(DEV)
    w_q = rand(2 * 64, 3, seed=62).to(DEV)
    base = knn_attention(k, v, nb, rel, w_q, 0.125, round_products=round_products)
    g = torch.Generator().manual_seed(63)
    for order in (spatial_order(dst), torch.randperm(len(dst), generator=g)):
        assert torch.equal(knn_attention(k, v, nb, rel, w_q, 0.125, target_order=order.to(DEV),
                                         round_products=round_products), base)
    with pytest.raises(ValueError, match="target_order"):
        knn_attention(k, v, nb, rel, w_q, 0.125, target_order=torch.arange(3, device=DEV))


def test_knn_attention_legacy_entry_points_round_products():
    """mosaic_knn_interp_fwd / _ordered are the rounded-product form; unknown flag bits are
    refused before any launch."""
    from mosaic_amd import _lib
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(ll, hp, 24)
    S, B, H = len(ll), 2, 2
    k, v = rand(S, B, H, 64, seed=70).to(DEV), rand(S, B, H, 64, seed=71).to(DEV)
    w_q = rand(H * 64, 3, seed=72).to(DEV)
    nb32, rel32 = nb.to(DEV, torch.int32).contiguous(), rel.to(DEV).float().contiguous()
    want = knn_attention(k, v, nb.to(DEV), rel.to(DEV), w_q, 0.125, round_products=True)
    out = torch.empty_like(want)
    kv = [_lib.Bnhd(t.data_ptr(), t.stride(1), t.stride(0), t.stride(2)) for t in (k, v)]
    stream = torch.cuda.current_stream().cuda_stream
    st = _lib.lib().mosaic_knn_interp_fwd(kv[0], kv[1], nb32.data_ptr(), rel32.data_ptr(), w_q.data_ptr(),
                                          S, len(hp), B, H, 64, 24, 0.125, out.data_ptr(), stream)
    _lib.check(st, "mosaic_knn_interp_fwd")
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    st = _lib.lib().mosaic_knn_interp_fwd_ex(kv[0], kv[1], nb32.data_ptr(), rel32.data_ptr(), w_q.data_ptr(), None,
                                             None, S, len(hp), B, H, 64, 24, 0.125, 2, out.data_ptr(), stream)
    assert st == _lib.ERR_MODE


def tiles_on(nb, order, max_targets=16, max_rows=None):
    from mosaic_amd.interp import knn_tiles
    t = knn_tiles(nb, order, max_targets, max_rows)
    return {n: (x.to(DEV) if torch.is_tensor(x) else x) for n, x in t.items()}


@pytest.mark.parametrize("max_targets,max_rows", [(16, 64), (16, 128), (5, 32), (1, 32)])
@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
@pytest.mark.parametrize("K", [32, 24, 20, 13, 7, 1])
def test_knn_attention_tiled_equals_direct(direction, K, max_targets, max_rows):
    """The LDS-staged kernel (tiles of targets sharing staged source rows) against the
    per-target kernel in the fp32-product form: the same output bit for bit, at any tile
    limits, K (one to four neighbour slots per lane) and direction."""
    if K > max_rows:
        pytest.skip("tiles hold at least K rows")
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    nb, rel = scheme(src, dst, K)
    B, H = 3, 2
    k, v = rand(len(src), B, H, 64, seed=K + 300), rand(len(src), B, H, 64, seed=K + 400)
    w_q = rand(H * 64, 3, seed=K + 500, scale=2.0)
    order = spatial_order(dst)
    args = (k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125)
    direct = knn_attention(*args, target_order=order.to(DEV))
    tiled = knn_attention(*args, target_order=order.to(DEV), tiles=tiles_on(nb, order, max_targets, max_rows))
    torch.cuda.synchronize()
    assert torch.equal(tiled, direct)
    close(tiled, oracle(k, v, nb, rel, w_q, 0.125, False))


@pytest.mark.parametrize("scale", [0.125, 0.3])
def test_knn_attention_tiled_random_lists_and_members(scale):
    """Neighbour lists without spatial structure (repeats allowed: a tile's source list holds
    each once), K 24, an odd member count (the member loop runs two members per pass) and a
    scale that is not a power of two."""
    S_from, S_to, K = 3000, 200, 24
    g = torch.Generator().manual_seed(80)
    nb = torch.randint(0, S_from, (S_to, K), generator=g)
    rel = torch.nn.functional.normalize(torch.randn(S_to, K, 3, generator=g), dim=-1)
    for B in (1, 5):
        k, v = rand(S_from, B, 3, 64, seed=81), rand(S_from, B, 3, 64, seed=82)
        w_q = rand(3 * 64, 3, seed=83)
        order = torch.randperm(S_to, generator=g)
        args = (k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), scale)
        direct = knn_attention(*args, target_order=order.to(DEV))
        tiled = knn_attention(*args, target_order=order.to(DEV), tiles=tiles_on(nb, order, 16, 128))
        assert torch.equal(tiled, direct)
        close(tiled, oracle(k, v, nb, rel, w_q, scale, False))


@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
def test_knn_attention_tiled_full_size(direction):
    """Model grids (121 x 240 lat-lon, HEALPix nside 64), K 24, 12 heads, 2 members, the
    module's tiles: equal to the per-target kernel everywhere, sampled targets against the
    oracle."""
    ll, hp = lonlat_grid(240, 121), torch.deg2rad(get_healpix_grid(64))
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    K, B, H = 24, 2, 12
    nb, rel = scheme(src, dst, K)
    k, v = rand(len(src), B, H, 64, seed=90), rand(len(src), B, H, 64, seed=91)
    w_q = rand(H * 64, 3, seed=92)
    order = spatial_order(dst)
    args = (k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125)
    direct = knn_attention(*args, target_order=order.to(DEV))
    tiled = knn_attention(*args, target_order=order.to(DEV), tiles=tiles_on(nb, order))
    torch.cuda.synchronize()
    assert torch.equal(tiled, direct)
    g = torch.Generator().manual_seed(93)
    sample = torch.randint(0, len(dst), (512,), generator=g)
    close(tiled.cpu()[sample], oracle(k, v, nb[sample], rel[sample], w_q, 0.125, False))


def test_knn_attention_tiles_argument_checks():
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(ll, hp, 24)
    k = rand(len(ll), 1, 2, 64, seed=95).to(DEV)
    w_q = rand(2 * 64, 3, seed=96).to(DEV)
    order = spatial_order(hp)
    tiles = tiles_on(nb, order)
    with pytest.raises(ValueError, match="target_order"):
        knn_attention(k, k, nb.to(DEV), rel.to(DEV), w_q, 0.125, tiles=tiles)
    bad = dict(tiles, max_rows=60)
    with pytest.raises(RuntimeError):
        knn_attention(k, k, nb.to(DEV), rel.to(DEV), w_q, 0.125, target_order=order.to(DEV), tiles=bad)


def test_module_rebuilds_tiles_when_neighbours_change():
    """The module's tile tables follow its neighbours: after load_state_dict copies other
    neighbour lists (and relative positions) into the buffers, the output equals the
    per-target kernel on the new lists."""
    from types import SimpleNamespace
    cfg = SimpleNamespace(k_neighbors=16, dim=128, num_heads=2, rmsnorm_elementwise_affine=True)
    torch.manual_seed(1)
    m = CrossAttentionInterpolate(cfg)
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    m.initialize_interpolation_scheme(ll, hp)
    m = m.to(DEV).to(torch.bfloat16)
    x = torch.randn(len(ll), 2, 128, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        m(x)                                          # tiles built for the first lists
        sd = m.state_dict()
        g = torch.Generator().manual_seed(2)
        sd["neighbors"] = torch.randint(0, len(ll), sd["neighbors"].shape, generator=g).to(DEV)
        sd["rel_pos"] = torch.nn.functional.normalize(torch.randn(sd["rel_pos"].shape, generator=g), dim=-1).to(DEV)
        m.load_state_dict(sd)
        y = m(x)
        kv = m.to_kv(m.kv_norm(x))
        k = kv[..., :128].unflatten(-1, (2, 64))
        v = kv[..., 128:].unflatten(-1, (2, 64))
        att = knn_attention(k, v, m.neighbors, m.rel_pos, m.to_q.weight, m.scale)   # per-target kernel
        ref = m.to_o(att.to(x.dtype).flatten(-2))
    assert torch.equal(y, ref)


def test_knn_attention_tiles_fall_back_with_64_bit_offsets():
    """Tiles given for k / v views the tiled kernel cannot address with 32-bit offsets (a
    negative point stride): the per-target kernel runs instead, with the same result as the
    tiled call on the forward-order copy."""
    from mosaic_amd import _lib
    from mosaic_amd.interp import knn_tiles
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(hp, ll, 24)
    S, B, H = len(hp), 2, 3
    k, v = rand(S, B, H, 64, seed=110).to(DEV), rand(S, B, H, 64, seed=111).to(DEV)
    w_q = rand(H * 64, 3, seed=112).to(DEV)
    order = spatial_order(ll)
    tiles = tiles_on(nb, order)
    fwd = knn_attention(k, v, nb.to(DEV), rel.to(DEV), w_q, 0.125, target_order=order.to(DEV), tiles=tiles)
    kr, vr = k.flip(0).contiguous(), v.flip(0).contiguous()

    def reversed_view(t):
        last = t[S - 1]
        return _lib.Bnhd(last.data_ptr(), t.stride(1), -t.stride(0), t.stride(2))
    parts = [tiles[n] for n in ("start", "src", "nsrc", "slot")]
    tl = _lib.KnnTiles(*(t.data_ptr() for t in parts), parts[0].numel() - 1, tiles["max_rows"])
    import ctypes
    nb32 = nb.to(DEV, torch.int32).contiguous()
    out = torch.empty_like(fwd)
    st = _lib.lib().mosaic_knn_interp_fwd_ex(reversed_view(kr), reversed_view(vr), nb32.data_ptr(),
                                             rel.to(DEV).float().contiguous().data_ptr(), w_q.data_ptr(),
                                             order.to(DEV, torch.int32).data_ptr(), ctypes.byref(tl), S, len(ll), B,
                                             H, 64, 24, 0.125, 0, out.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "mosaic_knn_interp_fwd_ex")
    torch.cuda.synchronize()
    assert torch.equal(out, fwd)


@pytest.mark.parametrize("H,B", [(1, 1), (1, 3), (5, 2)])
def test_knn_attention_tiled_head_and_member_counts(H, B):
    ll, hp = lonlat_grid(24, 13), torch.deg2rad(get_healpix_grid(4))
    nb, rel = scheme(ll, hp, 24)
    k, v = rand(len(ll), B, H, 64, seed=120 + H), rand(len(ll), B, H, 64, seed=130 + B)
    w_q = rand(H * 64, 3, seed=140)
    order = spatial_order(hp)
    args = (k.to(DEV), v.to(DEV), nb.to(DEV), rel.to(DEV), w_q.to(DEV), 0.125)
    direct = knn_attention(*args, target_order=order.to(DEV))
    tiled = knn_attention(*args, target_order=order.to(DEV), tiles=tiles_on(nb, order))
    assert torch.equal(tiled, direct)
    close(tiled, oracle(k, v, nb, rel, w_q, 0.125, False))
