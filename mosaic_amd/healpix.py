"""HEALPix nested-order geometry and the 2-D (lon, lat) rotary embedding.

Pixel centres follow the published HEALPix scheme (Gorski et al. 2005, ApJ 622:759,
sections 4-5): a pixel index in NESTED order is split into its base face and the
bit-interleaved (ix, iy) position inside the face; the ring number and the position
along the ring then give (z = cos theta, phi).  healpy is not available here, so
this module is the geometry used for RoPE positions.

Reference behaviour restated here:
  * ``get_healpix_grid`` -- utils.py:19-30 (lon = phi in degrees, lat = 90 - theta in
    degrees, float64 math, returned as float32 [npix, 2]).
  * ``rope_tables`` / ``apply_rope`` -- primitives.py:108-135 (base frequencies
    ``theta ** (-arange(0, d/2, 2) / (d/2))``, 16 lon + 16 lat angles for d = 64, each
    used for one interleaved (2m, 2m+1) pair, fp32 math, cast back to the input dtype).
"""

from __future__ import annotations

import numpy as np
import torch

# Row ("jr") and column ("jp") offsets of the 12 base faces, in units of nside.
_FACE_ROW = np.array([2, 2, 2, 2, 3, 3, 3, 3, 4, 4, 4, 4], dtype=np.int64)
_FACE_COL = np.array([1, 3, 5, 7, 0, 2, 4, 6, 1, 3, 5, 7], dtype=np.int64)


def nside2npix(nside: int) -> int:
    return 12 * nside * nside


def _deinterleave(v: np.ndarray) -> np.ndarray:
    """Collect the even-position bits of ``v`` into a compact integer."""
    out = np.zeros_like(v)
    bit = 0
    while True:
        src = v >> (2 * bit)
        if not np.any(src):
            break
        out |= (src & 1) << bit
        bit += 1
    return out


def pix2ang_nest(nside: int, ipix) -> tuple[np.ndarray, np.ndarray]:
    """Colatitude theta and longitude phi (radians, float64) of NESTED pixel centres."""
    if nside < 1 or (nside & (nside - 1)) != 0:
        raise ValueError(f"nside must be a power of two, got {nside}")
    ipix = np.asarray(ipix, dtype=np.int64)
    npface = nside * nside
    if np.any(ipix < 0) or np.any(ipix >= 12 * npface):
        raise ValueError("pixel index out of range")
    face = ipix // npface
    ipf = ipix % npface
    ix = _deinterleave(ipf)
    iy = _deinterleave(ipf >> 1)

    # ring index counted from the north pole, 1 .. 4*nside-1
    jr = _FACE_ROW[face] * nside - ix - iy - 1
    nr = np.where(jr < nside, jr, np.where(jr > 3 * nside, 4 * nside - jr, nside))
    z = np.where(
        jr < nside,
        1.0 - nr.astype(np.float64) ** 2 / (3.0 * npface),
        np.where(
            jr > 3 * nside,
            -1.0 + nr.astype(np.float64) ** 2 / (3.0 * npface),
            (2 * nside - jr).astype(np.float64) * 2.0 / (3.0 * nside),
        ),
    )
    # equatorial rings alternate between pixels starting at phi = 0 and at half a step
    kshift = np.where((jr >= nside) & (jr <= 3 * nside), (jr - nside) & 1, 0)
    jp = (_FACE_COL[face] * nr + ix - iy + 1 + kshift) // 2
    jp = np.where(jp > 4 * nside, jp - 4 * nside, jp)
    jp = np.where(jp < 1, jp + 4 * nside, jp)
    phi = (jp - (kshift + 1) * 0.5) * (0.5 * np.pi / nr)
    theta = np.arccos(np.clip(z, -1.0, 1.0))
    return theta, phi


def get_healpix_grid(nside: int) -> torch.Tensor:
    """[12*nside^2, 2] float32 (lon deg, lat deg) of NESTED pixel centres (utils.py:19-30)."""
    theta, phi = pix2ang_nest(nside, np.arange(nside2npix(nside)))
    lon = np.rad2deg(phi)
    lat = 90.0 - np.rad2deg(theta)
    return torch.stack((torch.from_numpy(lon), torch.from_numpy(lat)), dim=-1).float()


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float = 10000.0):
    """cos/sin tables [npix, head_dim/2] for (lon, lat) positions (primitives.py:115-123)."""
    if head_dim % 4 != 0:
        raise ValueError("head_dim must be a multiple of 4 for 2-D RoPE")
    half = head_dim // 2
    base = 1.0 / (theta ** (torch.arange(0, half, 2).float() / half))
    lon = torch.deg2rad(positions[:, 0:1].float())
    lat = torch.deg2rad(positions[:, 1:2].float())
    freqs = torch.cat([lon @ base.unsqueeze(0), lat @ base.unsqueeze(0)], dim=-1)
    return freqs.cos().contiguous(), freqs.sin().contiguous()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate interleaved pairs of ``x`` [B, N, H, d] (primitives.py:125-135).

    Pair m of a token: x'[2m] = x[2m] cos_m - x[2m+1] sin_m, x'[2m+1] = x[2m+1] cos_m + x[2m] sin_m.
    """
    xf = x.float()
    c = cos.to(xf.device).unsqueeze(0).unsqueeze(2)
    s = sin.to(xf.device).unsqueeze(0).unsqueeze(2)
    x_even, x_odd = xf[..., 0::2], xf[..., 1::2]
    out = torch.empty_like(xf)
    out[..., 0::2] = x_even * c - x_odd * s
    out[..., 1::2] = x_odd * c + x_even * s
    return out.to(x.dtype)
