"""k-nearest-neighbour cross-attention interpolation between grids.

Mirrors ``CrossAttentionInterpolate`` (primitives.py:230-283) and its helpers
``rad_to_xyz`` / ``get_neighbors`` (utils.py:7-17, 33-41).  The gather-attention in the
middle of the forward runs in libmosaic_bsa.so (``mosaic_knn_interp_fwd_ex``): the queries
``to_q(rel_pos)`` and the gathered keys / values are never materialised.  The RMSNorm and the
``to_kv`` / ``to_o`` projections stay torch modules (library GEMMs).  Precision is that of the
model under bf16 autocast: bf16 projections, fp32 softmax, bf16 output.  The products of
``(q * k).sum(-1)`` and ``(w * v).sum(1)`` are exact and summed in fp32, as the reference's
default inference path computes them (``torch.compile`` fuses each product into its reduction,
inference.py:470-473); ``round_products=True`` rounds each to bf16 first, as its eager
elementwise ops do.
"""

from __future__ import annotations

import ctypes
import weakref

import numpy as np
import torch
import torch.nn as nn

from . import _lib
from .fused import RMSNorm
from .ops import forward_only, stream_of


def rad_to_xyz(lonlat: torch.Tensor) -> torch.Tensor:
    """(lon, lat) in radians -> unit vectors (utils.py:7-17)."""
    lon, lat = lonlat[..., 0], lonlat[..., 1]
    return torch.stack([torch.cos(lat) * torch.cos(lon), torch.cos(lat) * torch.sin(lon), torch.sin(lat)], dim=-1)


def get_neighbors(pos_from: np.ndarray, pos_to: np.ndarray, k: int = 8) -> np.ndarray:
    """Indices [len(pos_to), k] of the k nearest points of ``pos_from`` (both (lon, lat) in
    radians) by great-circle distance, nearest first: scikit-learn's BallTree with the
    haversine metric on (lat, lon), as utils.py:33-41 builds it."""
    from sklearn.neighbors import BallTree
    tree = BallTree(np.ascontiguousarray(pos_from[:, ::-1]), metric="haversine")
    _, idx = tree.query(np.ascontiguousarray(pos_to[:, ::-1]), k=k)
    return idx


def spatial_order(pos_rad: torch.Tensor, bits: int = 10) -> torch.Tensor:
    """A processing order of points (lon, lat in radians) along a Z-order (Morton) curve of
    their unit vectors, each coordinate quantised to ``bits`` bits: int64 [len(pos_rad)], a
    permutation.  Points close on the sphere come close in the order, so the targets that run
    at the same time in the k-NN kernel share most of their neighbours."""
    xyz = rad_to_xyz(pos_rad.detach().double().cpu()).numpy()
    q = np.rint((xyz + 1.0) * 0.5 * ((1 << bits) - 1)).astype(np.int64)
    code = np.zeros(len(q), dtype=np.int64)
    for b in range(bits):
        for c in range(3):
            code |= ((q[:, c] >> b) & 1) << (3 * b + c)
    return torch.from_numpy(np.argsort(code, kind="stable"))


def knn_tiles(neighbors: torch.Tensor, order: torch.Tensor, max_targets: int = 16,
              max_rows: int | None = None) -> dict:
    """Tiles of consecutive targets of ``order`` for the LDS-staged k-NN kernel: each tile takes
    as many targets (at most ``max_targets``, 16 at most) as keep its distinct source points
    within ``max_rows`` (a multiple of 8, 128 at most).  Returns int32 CPU tensors ``start``
    [n + 1] (order positions), ``src`` [n, max_rows] (the distinct source points, ascending,
    padded with the last), ``nsrc`` [n] and ``slot`` [S_to, K] (the row of ``src`` holding
    neighbour j of the target at order position pos), and ``max_rows``.

    ``max_rows=None`` takes the smallest of 64, 96 and 128 whose tiles hold 12 targets or more
    on average: the staging buffers are 512 bytes per row, so fewer rows keep more workgroups
    on a compute unit, while fuller tiles stage each source row for more targets (on the
    model's grids: 64 for lat-lon -> HEALPix, 96 for HEALPix -> lat-lon)."""
    if max_rows is None:
        for rows in (64, 96, 128):
            t = knn_tiles(neighbors, order, max_targets, rows)
            if rows == 128 or len(order) >= 12 * (t["start"].numel() - 1):
                return t
    if not (0 < max_targets <= 16) or max_rows <= 0 or max_rows % 8 or max_rows > 128:
        raise ValueError("max_targets must be in 1..16 and max_rows a multiple of 8 in 8..128")
    nb = neighbors.detach().cpu().long().numpy()
    S_to, K = nb.shape
    if K > max_rows:
        raise ValueError(f"{K} neighbours do not fit tiles of {max_rows} rows")
    nb = nb[order.detach().cpu().long().numpy()]
    starts, srcs, nsrc = [0], [], []
    slot = np.empty((S_to, K), dtype=np.int32)
    pos = 0
    while pos < S_to:
        cand = nb[pos:pos + max_targets]
        _, first = np.unique(cand.ravel(), return_index=True)
        grown = np.cumsum(np.bincount(first // K, minlength=len(cand)))
        m = int(np.searchsorted(grown, max_rows, side="right"))   # targets whose union fits
        uniq, inv = np.unique(cand[:m].ravel(), return_inverse=True)
        slot[pos:pos + m] = inv.reshape(m, K)
        row = np.full(max_rows, uniq[-1], dtype=np.int64)
        row[:len(uniq)] = uniq
        srcs.append(row)
        nsrc.append(len(uniq))
        pos += m
        starts.append(pos)
    as32 = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a), dtype=np.int32))
    return {"start": as32(starts), "src": as32(np.stack(srcs)), "nsrc": as32(nsrc), "slot": as32(slot),
            "max_rows": max_rows}


def _snhd(t: torch.Tensor) -> _lib.Bnhd:
    # [S, B, H, 64] -> the ABI's (stride_b = member, stride_n = point, stride_h = head)
    return _lib.Bnhd(t.data_ptr(), t.stride(1), t.stride(0), t.stride(2))


def knn_attention(k: torch.Tensor, v: torch.Tensor, neighbors: torch.Tensor, rel_pos: torch.Tensor,
                  w_q: torch.Tensor, scale: float | None = None,
                  target_order: torch.Tensor | None = None, round_products: bool = False,
                  tiles: dict | None = None) -> torch.Tensor:
    """The gather-attention of CrossAttentionInterpolate.forward (primitives.py:265-283).

    k, v: [S_from, B, H, 64] (views of the kv projection are fine); neighbors: [S_to, K]
    source indices; rel_pos: [S_to, K, 3]; w_q: [H*64, 3] (``to_q.weight``).  Returns
    [S_to, B, H, 64] bf16: for each target, softmax over its K neighbours of
    ``to_q(rel_pos) . k * scale``, applied to v.  ``target_order`` ([S_to], a permutation,
    e.g. ``spatial_order`` of the target positions) changes only the order the targets are
    computed in, not the result.  ``round_products`` rounds every product of the two weighted
    sums to bf16 before it is added (the reference's eager elementwise ops); by default the
    products are exact and summed in fp32 (its compiled path).  ``tiles`` (``knn_tiles`` of
    the neighbours and ``target_order``, on k's device) selects the LDS-staged kernel for the
    fp32 form: the same output bit for bit.
    """
    forward_only("knn_attention", k, v, rel_pos, w_q)
    if k.dim() != 4 or k.shape != v.shape or k.shape[-1] != 64:
        raise ValueError(f"k and v must both be [S_from, B, H, 64], got {tuple(k.shape)} and {tuple(v.shape)}")
    if torch.float16 in (k.dtype, v.dtype):
        raise TypeError("k / v are float16: the kernel computes in bfloat16 (run the model under "
                        "torch.autocast(..., dtype=torch.bfloat16), or convert the inputs)")
    if k.device.type != "cuda":
        raise ValueError("k and v must be on a ROCm device")
    S_from, B, H, d = k.shape
    S_to, K = neighbors.shape
    if tuple(rel_pos.shape) != (S_to, K, 3) or tuple(w_q.shape) != (H * d, 3):
        raise ValueError("rel_pos must be [S_to, K, 3] and w_q [H*64, 3]")

    def prep(t):
        t = t.to(torch.bfloat16)
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
            t = t.contiguous()
        return t
    k, v = prep(k), prep(v)
    nb = neighbors.to(device=k.device, dtype=torch.int32).contiguous()
    rp = rel_pos.to(device=k.device, dtype=torch.float32).contiguous()
    wq = w_q.to(device=k.device, dtype=torch.bfloat16).contiguous()
    order = None
    if target_order is not None:
        if tuple(target_order.shape) != (S_to,):
            raise ValueError(f"target_order must be [S_to] = [{S_to}], got {tuple(target_order.shape)}")
        order = target_order.to(device=k.device, dtype=torch.int32).contiguous()
    out = torch.empty(S_to, B, H, d, dtype=torch.bfloat16, device=k.device)
    flags = _lib.KNN_ROUND_PRODUCTS if round_products else 0
    tl = None
    if tiles is not None:
        if order is None:
            raise ValueError("tiles are built over a target order: pass target_order as well")
        parts = [tiles[n].to(device=k.device, dtype=torch.int32).contiguous() for n in ("start", "src", "nsrc", "slot")]
        if tuple(parts[3].shape) != (S_to, K):
            raise ValueError(f"tiles['slot'] must be [S_to, K] = [{S_to}, {K}], got {tuple(parts[3].shape)}")
        tl = _lib.KnnTiles(*(t.data_ptr() for t in parts), parts[0].numel() - 1, int(tiles["max_rows"]))
    st = _lib.lib().mosaic_knn_interp_fwd_ex(_snhd(k), _snhd(v), nb.data_ptr(), rp.data_ptr(), wq.data_ptr(),
                                             None if order is None else order.data_ptr(),
                                             None if tl is None else ctypes.byref(tl),
                                             S_from, S_to, B, H, d, K, 0.0 if scale is None else float(scale),
                                             flags, out.data_ptr(), stream_of(k))
    _lib.check(st, "mosaic_knn_interp_fwd_ex")
    return out


class CrossAttentionInterpolate(nn.Module):
    """Cross-attention from one grid to another over k nearest neighbours (primitives.py:230-283).

    ``config`` needs: k_neighbors, dim, num_heads, rmsnorm_elementwise_affine.  x_from is
    sequence-first [S_from, B, dim]; the output is [S_to, B, dim].
    """

    space_dim = 3
    # products of the two weighted sums rounded to bf16 (the reference's eager ops) or exact
    # and summed in fp32 (its compiled inference path, the default here)
    round_products = False

    def __init__(self, config):
        super().__init__()
        self.k_neighbors = config.k_neighbors
        dim, num_heads = config.dim, config.num_heads
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.kv_norm = RMSNorm(dim, elementwise_affine=config.rmsnorm_elementwise_affine)
        self.to_q = nn.Linear(self.space_dim, dim, bias=False)
        self.to_kv = nn.Linear(dim, 2 * dim, bias=False)
        self.to_o = nn.Linear(dim, dim, bias=False)
        self.register_buffer("neighbors", None, persistent=True)
        self.register_buffer("rel_pos", None, persistent=True)
        # the kernel's target order (int32, not part of the state dict): derived from the
        # target positions with the neighbours
        self.register_buffer("target_order", None, persistent=False)
        # tiles of targets for the LDS-staged kernel (int32, derived from the neighbours and
        # the order); _tile_source identifies the neighbours tensor they were built from (a weak
        # reference and its in-place version counter), so a later change of it (a new tensor,
        # or load_state_dict copying into the buffer) rebuilds them
        self.knn_tile_rows = 64
        self._tile_source = None
        for n in ("start", "src", "nsrc", "slot"):
            self.register_buffer("knn_tile_" + n, None, persistent=False)

    @torch.no_grad()
    def initialize_interpolation_scheme(self, pos_from_rad: torch.Tensor, pos_to_rad: torch.Tensor):
        """Neighbours and normalised relative positions of every target (primitives.py:250-263)."""
        nbrs = get_neighbors(pos_from_rad.cpu().numpy(), pos_to_rad.cpu().numpy(), k=self.k_neighbors)
        neighbors = torch.from_numpy(nbrs).long().to(pos_from_rad.device).contiguous()
        to_xyz, from_xyz = rad_to_xyz(pos_to_rad), rad_to_xyz(pos_from_rad)
        rel = (to_xyz.unsqueeze(1) - from_xyz[neighbors]).contiguous()
        self.neighbors = neighbors
        self.rel_pos = torch.nn.functional.normalize(rel, dim=-1).contiguous()
        order = spatial_order(pos_to_rad)
        self.target_order = order.to(device=pos_from_rad.device, dtype=torch.int32)
        self._build_tiles()

    @torch.no_grad()
    def _build_tiles(self):
        tiles = knn_tiles(self.neighbors, self.target_order)
        for n in ("start", "src", "nsrc", "slot"):
            setattr(self, "knn_tile_" + n, tiles[n].to(self.neighbors.device))
        self.knn_tile_rows = tiles["max_rows"]
        self._tile_source = (weakref.ref(self.neighbors), self.neighbors._version)

    def _current_tiles(self):
        """The tile tables for the current neighbours (rebuilt if the neighbours tensor was
        replaced or modified in place since they were built), or None without an order."""
        if self.target_order is None:
            return None
        src = self._tile_source
        if self.knn_tile_start is None or src is None or src[0]() is not self.neighbors or \
                src[1] != self.neighbors._version:
            self._build_tiles()
        return {"start": self.knn_tile_start, "src": self.knn_tile_src, "nsrc": self.knn_tile_nsrc,
                "slot": self.knn_tile_slot, "max_rows": self.knn_tile_rows}

    def forward(self, x_from: torch.Tensor) -> torch.Tensor:
        if self.neighbors is None or self.rel_pos is None:
            raise ValueError("Interpolation scheme not initialized.")
        S_from, B, dim = x_from.shape
        kv = self.to_kv(self.kv_norm(x_from))
        k = kv[..., :dim].unflatten(-1, (self.num_heads, self.head_dim))
        v = kv[..., dim:].unflatten(-1, (self.num_heads, self.head_dim))
        tiles = self._current_tiles()
        out = knn_attention(k, v, self.neighbors, self.rel_pos, self.to_q.weight, self.scale, self.target_order,
                            round_products=self.round_products, tiles=tiles)
        return self.to_o(out.to(x_from.dtype).flatten(-2))
