"""nvdiffrast-convention adapter over the HIP kernels.

mlx-swift-diffrast differs from nvdiffrast in two conventions
(CONVENTIONS.md:17-72 of the reference):

  * image y: pixel (h=0, w=0) is NDC (-1, +1) here (top-left), (-1, -1) in
    nvdiffrast (bottom-left); images are vertical flips of each other, and
    the d/dy channels of the screen derivatives change sign;
  * barycentric layout of `rast`: (u, v) = (w1, w2) here, (w0, w1) in
    nvdiffrast, so nvdiffrast's (u, v) = (1 - u - v, u).

This module converts between the two (`rast_to_nvdiffrast`,
`rast_from_nvdiffrast`, differentiable torch ops) and exposes nvdiffrast's
functional API (`rasterize`, `interpolate`, `texture`, `antialias`,
`texture_construct_mip`, `antialias_construct_topology_hash`) in
nvdiffrast's conventions on top of the kernels, so nvdiffrast fixtures are
directly comparable and nvdiffrast code can call the library.  Only the
conventions change: the barycentrics remain the reference's screen-space
ones (nvdiffrast's are perspective-correct; they agree when every w is
equal), coverage keeps the reference's inclusive edges, and antialias keeps
the reference's silhouette rule.  `load_safetensors` / `save_safetensors`
read and write fixtures such as the reference's
Tests/MLXDiffRastTests/Fixtures/diffrast_fixtures.safetensors.
"""
from __future__ import annotations

from typing import Dict, Optional, Sequence, Tuple

import torch

from .ops import DiffRast


# ---------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------

def _covered(rast: torch.Tensor) -> torch.Tensor:
    return rast[..., 3:4] > 0


def rast_to_nvdiffrast(rast: torch.Tensor, rast_db: Optional[torch.Tensor] = None
                       ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """This library's (rast, rast_db) -> nvdiffrast's: y flipped, (u, v) ->
    (1 - u - v, u); rast_db (du/dx, du/dy, dv/dx, dv/dy) ->
    (-(du/dx + dv/dx), du/dy + dv/dy, du/dx, -du/dy).  Empty pixels stay 0."""
    cov = _covered(rast)
    u, v = rast[..., 0], rast[..., 1]
    nv = torch.stack([1.0 - u - v, u, rast[..., 2], rast[..., 3]], -1)
    nv = torch.where(cov, nv, torch.zeros_like(nv)).flip(1)
    if rast_db is None or rast_db.shape[-1] == 0:
        return nv, rast_db
    d = rast_db
    nd = torch.stack([-(d[..., 0] + d[..., 2]), d[..., 1] + d[..., 3], d[..., 0], -d[..., 1]], -1)
    nd = torch.where(cov, nd, torch.zeros_like(nd)).flip(1)
    return nv, nd


def rast_from_nvdiffrast(rast: torch.Tensor, rast_db: Optional[torch.Tensor] = None
                         ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """nvdiffrast's (rast, rast_db) -> this library's (the inverse of
    `rast_to_nvdiffrast`): (u, v) = (nv.v, 1 - nv.u - nv.v), rast_db =
    (nv.dv/dx, -nv.dv/dy, -(nv.du/dx + nv.dv/dx), nv.du/dy + nv.dv/dy)."""
    r = rast.flip(1)
    cov = _covered(r)
    mine = torch.stack([r[..., 1], 1.0 - r[..., 0] - r[..., 1], r[..., 2], r[..., 3]], -1)
    mine = torch.where(cov, mine, torch.zeros_like(mine))
    if rast_db is None or rast_db.shape[-1] == 0:
        return mine, rast_db
    d = rast_db.flip(1)
    md = torch.stack([d[..., 2], -d[..., 3], -(d[..., 0] + d[..., 2]), d[..., 1] + d[..., 3]], -1)
    return mine, torch.where(cov, md, torch.zeros_like(md))


def _flip_da(da: torch.Tensor) -> torch.Tensor:
    """Screen derivatives (d/dx, d/dy) pairs of an image: y flip and the sign
    of every d/dy."""
    sign = torch.ones(da.shape[-1], device=da.device, dtype=da.dtype)
    sign[1::2] = -1.0
    return da.flip(1) * sign


# ---------------------------------------------------------------------------
# nvdiffrast's functional API
# ---------------------------------------------------------------------------

class RasterizeContext:
    """Stands in for nvdiffrast's RasterizeCudaContext / RasterizeGLContext:
    the kernels need no context; it only records the device."""

    def __init__(self, device=None, output_db: bool = True):
        self.device = torch.device(device) if device is not None else \
            torch.device("cuda", torch.cuda.current_device())
        self.output_db = output_db


RasterizeCudaContext = RasterizeContext
RasterizeGLContext = RasterizeContext


def rasterize(glctx, pos: torch.Tensor, tri: torch.Tensor, resolution: Sequence[int],
              ranges: Optional[torch.Tensor] = None, grad_db: bool = True
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """nvdiffrast.torch.rasterize in nvdiffrast's conventions.  rast_db is
    [N, H, W, 0] when grad_db is False."""
    db = bool(grad_db) and (glctx is None or getattr(glctx, "output_db", True))
    rast, rast_db = DiffRast.rasterize(pos, tri, (int(resolution[0]), int(resolution[1])),
                                       gradDB=db, ranges=ranges)
    if not db:
        return rast_to_nvdiffrast(rast)[0], rast_db
    return rast_to_nvdiffrast(rast, rast_db)


def interpolate(attr: torch.Tensor, rast: torch.Tensor, tri: torch.Tensor,
                rast_db: Optional[torch.Tensor] = None, diff_attrs=None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """nvdiffrast.torch.interpolate on an nvdiffrast-convention rast."""
    mine, mdb = rast_from_nvdiffrast(rast, rast_db if diff_attrs is not None else None)
    out, out_da = DiffRast.interpolate(attr, mine, tri, rastDB=mdb, diffAttrs=diff_attrs)
    out = out.flip(1)
    if out_da.shape[-1] == 0:
        return out, out_da
    return out, _flip_da(out_da)


def texture_construct_mip(tex: torch.Tensor, max_mip_level: Optional[int] = None,
                          cube_mode: bool = False):
    """nvdiffrast.torch.texture_construct_mip: the pyramid as a list
    [tex, level1, ...] (2x2 box means); pass it back as `mip=`."""
    if cube_mode:
        raise ValueError("texture_construct_mip: a cube map's pyramid is built inside texture()")
    return DiffRast.textureConstructMip(tex, maxLevel=max_mip_level)


def texture(tex: torch.Tensor, uv: torch.Tensor, uv_da: Optional[torch.Tensor] = None,
            mip_level_bias: Optional[torch.Tensor] = None, mip=None, filter_mode: str = "auto",
            boundary_mode: str = "wrap", max_mip_level: Optional[int] = None) -> torch.Tensor:
    """nvdiffrast.torch.texture.  Texture coordinates have no image-y
    convention, so this is the library's texture.  'auto' picks
    'linear-mipmap-linear' when uv_da or mip_level_bias is given, else
    'linear'.  Mip filters need uv_da (the bias scales the footprint, as in
    the reference: Texture.swift:104-126)."""
    if filter_mode == "auto":
        filter_mode = "linear-mipmap-linear" if (uv_da is not None or
                                                 mip_level_bias is not None) else "linear"
    mipmapped = "mipmap" in filter_mode
    if mipmapped and mip is None and max_mip_level is not None:
        mip = DiffRast.textureConstructMip(tex, maxLevel=max_mip_level)
    return DiffRast.texture(tex, uv, uvDA=uv_da if mipmapped else None, filterMode=filter_mode,
                            boundaryMode=boundary_mode,
                            mipLevelBiasMap=mip_level_bias if mipmapped else None,
                            mip=mip if mipmapped else None)


def antialias_construct_topology_hash(tri: torch.Tensor) -> torch.Tensor:
    """nvdiffrast.torch.antialias_construct_topology_hash (this library's
    [T, 3] edge-neighbour table, not nvdiffrast's opaque hash)."""
    return DiffRast.antialiasConstructTopologyHash(tri)


class _ScaleGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, s):
        ctx.s = s
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        return g * ctx.s, None


def antialias(color: torch.Tensor, rast: torch.Tensor, pos: torch.Tensor, tri: torch.Tensor,
              topology_hash: Optional[torch.Tensor] = None,
              pos_gradient_boost: float = 1.0) -> torch.Tensor:
    """nvdiffrast.torch.antialias on nvdiffrast-convention images (the
    reference's silhouette rule).  A shared pos [V, 4] is broadcast over the
    batch; pos_gradient_boost scales the gradient to pos."""
    mine, _ = rast_from_nvdiffrast(rast.detach())
    if pos.ndim == 2:
        pos = pos[None].expand(color.shape[0], -1, -1)
    if pos_gradient_boost != 1.0:
        pos = _ScaleGrad.apply(pos, float(pos_gradient_boost))
    out = DiffRast.antialias(color.flip(1), mine, pos, tri, topologyHash=topology_hash)
    return out.flip(1)


# ---------------------------------------------------------------------------
# fixture I/O
# ---------------------------------------------------------------------------

def load_safetensors(path: str, device=None) -> Dict[str, torch.Tensor]:
    """Every tensor of a .safetensors file (no code is executed on load)."""
    from safetensors.torch import load_file
    out = load_file(path)
    if device is not None:
        out = {k: v.to(device) for k, v in out.items()}
    return out


def save_safetensors(tensors: Dict[str, torch.Tensor], path: str) -> None:
    from safetensors.torch import save_file
    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, path)
