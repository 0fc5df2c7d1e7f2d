"""HEALPix nested pixel centres and the 2-D rotary embedding used to build the inputs.

The geometry (reference: utils.py:19-30 via healpy, which is not installed) is pinned by
published known answers and invariants of the HEALPix scheme (Gorski et al. 2005):
base-pixel centres at Nside 1, the nested numbering inside a base pixel at Nside 2, ring
latitudes and pixel counts, equal spacing along rings, and the parent/child hierarchy.
RoPE (primitives.py:108-135) is pinned by the complex-rotation form, norm preservation and
the relative-position property.
"""

import math

import numpy as np
import pytest
import torch
from scipy.spatial import Delaunay

from mosaic_amd import healpix as H
from mosaic_amd.primitives import RoPE


def _z_phi(nside):
    theta, phi = H.pix2ang_nest(nside, np.arange(H.nside2npix(nside)))
    return np.cos(theta), phi


def test_nside1_base_pixel_centres():
    z, phi = _z_phi(1)
    p = np.arange(12)
    z_exp = np.where(p < 4, 2 / 3, np.where(p < 8, 0.0, -2 / 3))
    phi_exp = np.where(p < 4, math.pi / 4 * (2 * p + 1),
                       np.where(p < 8, math.pi / 2 * (p - 4), math.pi / 4 * (2 * (p - 8) + 1)))
    np.testing.assert_allclose(z, z_exp, atol=1e-12)
    np.testing.assert_allclose(phi, phi_exp, atol=1e-12)


def test_nside2_nested_order_inside_base_pixel():
    # base pixel 0 at Nside 2: sub-pixel 0 south, 1 east, 2 west, 3 north
    theta, phi = H.pix2ang_nest(2, np.arange(4))
    np.testing.assert_allclose(np.cos(theta), [1 / 3, 2 / 3, 2 / 3, 11 / 12], atol=1e-12)
    np.testing.assert_allclose(phi, [math.pi / 4, 3 * math.pi / 8, math.pi / 8, math.pi / 4], atol=1e-12)


@pytest.mark.parametrize("nside", [1, 2, 4, 8, 16])
def test_rings_latitudes_counts_and_spacing(nside):
    n = nside
    z, phi = _z_phi(n)
    # ring index i = 1 .. 4n-1 from the north pole, with its z and pixel count
    rings = []
    for i in range(1, 4 * n):
        if i < n:
            rings.append((1 - i * i / (3 * n * n), 4 * i, 0.5))
        elif i <= 3 * n:
            rings.append((4 / 3 - 2 * i / (3 * n), 4 * n, 0.5 if (i - n) % 2 == 0 else 0.0))
        else:
            j = 4 * n - i
            rings.append((-1 + j * j / (3 * n * n), 4 * j, 0.5))
    seen = np.zeros(len(z), dtype=bool)
    for zr, count, first in rings:
        sel = np.abs(z - zr) < 1e-9
        assert sel.sum() == count
        seen |= sel
        ph = np.sort(phi[sel])
        step = 2 * math.pi / count
        # equally spaced from half a step (polar rings, every other equatorial ring) or from 0
        np.testing.assert_allclose(np.diff(ph), step, atol=1e-9)
        assert ph[0] == pytest.approx(first * step, abs=1e-9)
    assert seen.all()
    # equal area: every pixel covers 4 pi / npix; z is uniform, so the mean of z is 0
    assert abs(z.mean()) < 1e-12


@pytest.mark.parametrize("nside", [1, 2, 4, 8])
def test_parent_centre_inside_children(nside):
    tp, pp = H.pix2ang_nest(nside, np.arange(H.nside2npix(nside)))
    tc, pc = H.pix2ang_nest(2 * nside, np.arange(H.nside2npix(2 * nside)))

    def vec(t, p):
        return np.stack([np.sin(t) * np.cos(p), np.sin(t) * np.sin(p), np.cos(t)], -1)

    vp, vc = vec(tp, pp), vec(tc, pc).reshape(-1, 4, 3)
    pix = math.sqrt(4 * math.pi / H.nside2npix(nside))
    for p in range(len(vp)):
        c = vp[p]
        # tangent-plane basis at the parent centre
        a = np.cross(c, [0.0, 0.0, 1.0]) if abs(c[2]) < 0.9 else np.cross(c, [1.0, 0.0, 0.0])
        a /= np.linalg.norm(a)
        b = np.cross(c, a)
        ch = vc[p]
        assert np.all(ch @ c > math.cos(pix)), p   # children lie within one parent pixel size
        pts = np.stack([ch @ a, ch @ b], -1)
        assert Delaunay(pts).find_simplex(np.zeros(2), tol=1e-9) >= 0, p


def test_grid_units_and_range():
    g = H.get_healpix_grid(4)
    assert g.shape == (192, 2) and g.dtype == torch.float32
    assert float(g[:, 0].min()) >= 0 and float(g[:, 0].max()) < 360
    assert float(g[:, 1].min()) > -90 and float(g[:, 1].max()) < 90
    # pixel 0 of Nside 1 is at lon 45 deg, lat asin(2/3)
    g1 = H.get_healpix_grid(1)
    assert float(g1[0, 0]) == pytest.approx(45.0)
    assert float(g1[0, 1]) == pytest.approx(math.degrees(math.asin(2 / 3)), abs=1e-5)


def _positions(n, seed=0):
    gen = torch.Generator().manual_seed(seed)
    return torch.stack([torch.rand(n, generator=gen) * 360, torch.rand(n, generator=gen) * 180 - 90], -1)


def test_rope_frequencies():
    pos = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    cos, sin = H.rope_tables(pos, 64)
    ang = torch.atan2(sin, cos).double()
    f = 10000.0 ** (-torch.arange(16, dtype=torch.float64) / 16)
    np.testing.assert_allclose(ang[0, :16], math.radians(1.0) * f, rtol=1e-5)
    np.testing.assert_allclose(ang[0, 16:], 0.0, atol=1e-7)
    np.testing.assert_allclose(ang[1, 16:], math.radians(1.0) * f, rtol=1e-5)


def test_rope_is_complex_rotation_and_preserves_norm():
    pos = _positions(32)
    cos, sin = H.rope_tables(pos, 64)
    x = torch.randn(2, 32, 3, 64, generator=torch.Generator().manual_seed(1))
    y = H.apply_rope(x, cos, sin)
    xc = torch.view_as_complex(x.reshape(2, 32, 3, 32, 2).contiguous())
    rot = torch.polar(torch.ones_like(cos), torch.atan2(sin, cos))[None, :, None, :]
    yc = torch.view_as_real(xc * rot).reshape(2, 32, 3, 64)
    torch.testing.assert_close(y, yc, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1), atol=1e-4, rtol=1e-5)


def test_rope_relative_position_property():
    # <R(p1) q, R(p2) k> depends on p1 - p2 only
    p1, p2 = _positions(16, 2), _positions(16, 3)
    shift = torch.tensor([[17.0, -5.0]])
    gen = torch.Generator().manual_seed(4)
    q, k = torch.randn(1, 16, 1, 64, generator=gen), torch.randn(1, 16, 1, 64, generator=gen)

    def dots(a, b):
        ca, sa = H.rope_tables(a, 64)
        cb, sb = H.rope_tables(b, 64)
        return (H.apply_rope(q, ca, sa) * H.apply_rope(k, cb, sb)).sum(-1)

    torch.testing.assert_close(dots(p1, p2), dots(p1 + shift, p2 + shift), atol=2e-4, rtol=1e-4)


def test_rope_module_matches_tables_and_keeps_dtype():
    pos = H.get_healpix_grid(2)
    m = RoPE(64)
    m.initialize_rope(pos)
    x = torch.randn(1, 48, 2, 64).bfloat16()
    cos, sin = H.rope_tables(pos, 64)
    y = m(x)
    assert y.dtype == torch.bfloat16
    torch.testing.assert_close(y, H.apply_rope(x, cos, sin), atol=0, rtol=0)
