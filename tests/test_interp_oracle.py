"""Pinning of the k-NN cross-attention oracle (CPU): closed forms, a float64 brute force, an
invariance, and the neighbour search against a brute-force great-circle search."""

import math

import numpy as np
import pytest
import torch

from mosaic_amd.healpix import get_healpix_grid
from mosaic_amd.interp import get_neighbors, rad_to_xyz
from oracle import interp_oracle as IO


def _grids():
    hp = torch.deg2rad(get_healpix_grid(2))                               # 48 points
    lon = torch.linspace(0, 330, 12)
    lat = torch.linspace(-90, 90, 7)
    ll = torch.deg2rad(torch.stack(torch.meshgrid(lon, lat, indexing="ij"), -1).reshape(-1, 2))   # 84 points
    return ll, hp


def _scheme(pos_from, pos_to, K):
    nb = torch.from_numpy(get_neighbors(pos_from.numpy(), pos_to.numpy(), k=K)).long()
    rel = rad_to_xyz(pos_to).unsqueeze(1) - rad_to_xyz(pos_from)[nb]
    return nb, torch.nn.functional.normalize(rel, dim=-1)


def _kv(S, B, H, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(S, B, H, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(S, B, H, 64, generator=g).to(torch.bfloat16)
    return k, v


def test_rad_to_xyz_known_points():
    pts = torch.tensor([[0.0, 0.0], [math.pi / 2, 0.0], [0.3, math.pi / 2], [math.pi, -math.pi / 2]])
    xyz = rad_to_xyz(pts)
    ref = torch.tensor([[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0], [0.0, 0.0, -1.0]])
    torch.testing.assert_close(xyz, ref, atol=1e-6, rtol=0)
    ll, _ = _grids()
    torch.testing.assert_close(rad_to_xyz(ll).norm(dim=-1), torch.ones(len(ll)), atol=1e-6, rtol=0)


@pytest.mark.parametrize("direction", ["ll_to_hp", "hp_to_ll"])
def test_neighbours_match_brute_force(direction):
    ll, hp = _grids()
    src, dst = (ll, hp) if direction == "ll_to_hp" else (hp, ll)
    K = 8
    got = torch.from_numpy(get_neighbors(src.numpy(), dst.numpy(), k=K)).long()
    ref = IO.great_circle_knn(src, dst, K + 1)

    def ang(idx):
        a = rad_to_xyz(dst.double()).unsqueeze(1)
        b = rad_to_xyz(src.double())[idx]
        return torch.acos((a * b).sum(-1).clamp(-1, 1))
    # the same distances (equidistant points may be listed in another order), nearest first
    torch.testing.assert_close(ang(got), ang(ref[:, :K]), atol=1e-9, rtol=0)
    assert (ang(got).diff(dim=1) >= -1e-12).all()
    # where the k-th and (k+1)-th distances differ, the neighbour sets are equal
    clear = (ang(ref)[:, K] - ang(ref)[:, K - 1]) > 1e-9
    for r in torch.nonzero(clear).flatten().tolist():
        assert set(got[r].tolist()) == set(ref[r, :K].tolist())


def test_single_neighbour_returns_its_value():
    ll, hp = _grids()
    nb, rel = _scheme(ll, hp, 1)
    k, v = _kv(len(ll), 2, 3, seed=1)
    w_q = torch.randn(3 * 64, 3).to(torch.bfloat16)
    out = IO.knn_attention(k, v, nb, rel, w_q, 0.125)
    assert torch.equal(out, v[nb[:, 0]])


def test_zero_queries_give_the_mean():
    ll, hp = _grids()
    K = 20
    nb, rel = _scheme(ll, hp, K)
    k, v = _kv(len(ll), 2, 2, seed=2)
    out = IO.knn_attention(k, v, nb, rel, torch.zeros(2 * 64, 3), 0.125).double()
    mean = v.double()[nb].mean(dim=1)
    assert (out - mean).abs().max().item() <= 2 ** -7 * v.double().abs().max().item()


@pytest.mark.parametrize("products", ["bf16", "fp32"])
@pytest.mark.parametrize("K", [7, 24])
def test_matches_float64_brute_force(K, products):
    ll, hp = _grids()
    nb, rel = _scheme(ll, hp, K)
    H = 2
    k, v = _kv(len(ll), 2, H, seed=3)
    w_q = (torch.randn(H * 64, 3, generator=torch.Generator().manual_seed(4)) * 0.6).to(torch.bfloat16)
    scale = 64 ** -0.5
    out = IO.knn_attention(k, v, nb, rel, w_q, scale, products=products).double()
    ref = torch.zeros_like(out)
    W = w_q.double()
    for t in range(len(hp)):
        for h in range(H):
            q = rel[t].double() @ W[h * 64:(h + 1) * 64].t()                 # [K, 64]
            for b in range(2):
                s = (q * k.double()[nb[t], b, h]).sum(-1) * scale            # [K]
                p = torch.softmax(s, dim=0)
                ref[t, b, h] = (p[:, None] * v.double()[nb[t], b, h]).sum(0)
    err = (out - ref).abs().max().item()
    assert err <= 2e-2, err
    assert ((out - ref).norm() / ref.norm()).item() <= 1e-2


def test_product_forms_agree_where_products_are_exact_in_bf16():
    """Inputs whose products all fit bf16 (one-hot rel_pos, so q = a column of w_q in steps of
    1/4; integer k; v in {0, +-1/2, +-1, +-2}; a scale that keeps the weights within a factor
    e^2 of each other, so every fp32 sum is exact): rounding the products changes nothing, and
    the two forms must be equal bit for bit.  On general inputs they must differ somewhere."""
    ll, hp = _grids()
    K, B, H = 16, 2, 2
    nb, _ = _scheme(ll, hp, K)
    g = torch.Generator().manual_seed(11)
    rel = torch.nn.functional.one_hot(torch.randint(0, 3, (len(hp), K), generator=g), 3).float()
    w_q = (torch.randint(-8, 9, (H * 64, 3), generator=g) / 4).to(torch.bfloat16)
    k = torch.randint(-7, 8, (len(ll), B, H, 64), generator=g).to(torch.bfloat16)
    pow2 = torch.tensor([0.0, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0])
    v = pow2[torch.randint(0, len(pow2), (len(ll), B, H, 64), generator=g)].to(torch.bfloat16)
    scale = 1 / 2048                      # |q . k| <= 2 * 7 * 64: scaled scores within [-0.44, 0.44]
    a = IO.knn_attention(k, v, nb, rel, w_q, scale, products="bf16")
    b = IO.knn_attention(k, v, nb, rel, w_q, scale, products="fp32")
    assert torch.equal(a, b)
    assert (a != 0).float().mean() > 0.5   # not a degenerate all-zero case
    kr, vr = _kv(len(ll), B, H, seed=12)
    _, relr = _scheme(ll, hp, K)
    wr = torch.randn(H * 64, 3, generator=g).to(torch.bfloat16)
    assert not torch.equal(IO.knn_attention(kr, vr, nb, relr, wr, 0.125, products="bf16"),
                           IO.knn_attention(kr, vr, nb, relr, wr, 0.125, products="fp32"))


def test_neighbour_order_does_not_matter():
    ll, hp = _grids()
    K = 12
    nb, rel = _scheme(ll, hp, K)
    k, v = _kv(len(ll), 1, 2, seed=5)
    w_q = torch.randn(2 * 64, 3, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(7))
    a = IO.knn_attention(k, v, nb, rel, w_q, 0.125).float()
    b = IO.knn_attention(k, v, nb[:, perm], rel[:, perm], w_q, 0.125).float()
    # the fp32 sums add in another order: at most one bf16 spacing apart
    assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * 2 ** -7 + 1e-6).all()


def test_module_scheme_on_cpu():
    from types import SimpleNamespace
    from mosaic_amd.interp import CrossAttentionInterpolate
    m = CrossAttentionInterpolate(SimpleNamespace(k_neighbors=8, dim=128, num_heads=2, rmsnorm_elementwise_affine=True))
    with pytest.raises(ValueError):
        m(torch.zeros(84, 1, 128))
    ll, hp = _grids()
    m.initialize_interpolation_scheme(ll, hp)
    nb, rel = _scheme(ll, hp, 8)
    assert torch.equal(m.neighbors, nb) and torch.equal(m.rel_pos, rel)
    assert set(m.state_dict()) >= {"neighbors", "rel_pos"}
    assert "target_order" not in m.state_dict()          # derived, not a checkpoint entry
    assert sorted(m.target_order.tolist()) == list(range(len(hp)))
    with torch.no_grad(), pytest.raises(ValueError):   # the gather-attention runs on the device only
        m(torch.zeros(84, 1, 128))
    with pytest.raises(RuntimeError, match="no backward"):   # to_q / to_kv weights require grad
        m(torch.zeros(84, 1, 128))


def test_spatial_order_is_a_permutation_that_follows_the_sphere():
    """The k-NN kernel's target order: a permutation whose consecutive points are close (a
    shuffled HEALPix grid, nside 16: mean step < 2.5 grid spacings, against ~1.3 shuffled);
    identical positions keep their given order (stable)."""
    from mosaic_amd.interp import spatial_order
    hp = torch.deg2rad(get_healpix_grid(16))
    pts = hp[torch.randperm(len(hp), generator=torch.Generator().manual_seed(0))]
    o = spatial_order(pts)
    assert o.dtype == torch.int64 and sorted(o.tolist()) == list(range(len(pts)))
    xyz = rad_to_xyz(pts.double())
    step = lambda idx: (xyz[idx][1:] - xyz[idx][:-1]).norm(dim=-1).mean().item()
    spacing = math.sqrt(4 * math.pi / len(pts))
    assert step(o) < 2.5 * spacing and step(torch.arange(len(pts))) > 10 * spacing
    same = torch.zeros(5, 2)
    assert spatial_order(same).tolist() == [0, 1, 2, 3, 4]


@pytest.mark.parametrize("max_targets,max_rows", [(16, 64), (16, 128), (5, 32), (1, 32)])
def test_knn_tiles_partition_the_order(max_targets, max_rows):
    """knn_tiles: consecutive runs of the order, each within max_targets targets and max_rows
    distinct sources, taken greedily (the next target would break a limit), and every
    neighbour found at its slot of its tile's source list."""
    from mosaic_amd.interp import knn_tiles, spatial_order
    ll, hp = _grids()
    K = 20
    nb, _ = _scheme(ll, hp, K)
    order = spatial_order(hp)
    t = knn_tiles(nb, order, max_targets, max_rows)
    start, src, nsrc, slot = (t[n].long() for n in ("start", "src", "nsrc", "slot"))
    assert start[0] == 0 and start[-1] == len(hp) and bool((start[1:] > start[:-1]).all())
    assert src.shape == (len(start) - 1, max_rows) and slot.shape == (len(hp), K)
    nb_ord = nb[order]
    for i in range(len(start) - 1):
        a, b = start[i].item(), start[i + 1].item()
        n = nsrc[i].item()
        assert b - a <= max_targets and 0 < n <= max_rows
        uniq = torch.unique(nb_ord[a:b])
        assert torch.equal(src[i, :n], uniq)                       # ascending distinct sources
        assert torch.equal(src[i, n:], uniq[-1].expand(max_rows - n))
        assert torch.equal(src[i][slot[a:b]], nb_ord[a:b])          # every neighbour at its slot
        if b < len(hp) and b - a < max_targets:                     # greedy: the next target did not fit
            assert len(torch.unique(nb_ord[a:b + 1])) > max_rows


def test_knn_tiles_reject_bad_limits():
    from mosaic_amd.interp import knn_tiles
    nb = torch.zeros(4, 24, dtype=torch.long)
    order = torch.arange(4)
    for mt, mr in ((0, 64), (17, 64), (16, 60), (16, 136), (16, 16)):
        with pytest.raises(ValueError):
            knn_tiles(nb, order, mt, mr)
