"""`DiffRast`: the four differentiable rasterization ops on MI355X.

Mirrors the public API of mnmly/mlx-swift-diffrast (the `DiffRast` enum in
Sources/MLXDiffRast/*.swift): same op names, argument names and meanings,
output layouts and conventions (clip-space pos, rast = (u, v, z/w,
tri_id+1), rastDB, instanced / range modes, top-left pixel origin).  Each op
is a `torch.autograd.Function` whose forward and backward call the C ABI of
libdiffrast_mi355x.so, the counterpart of the reference's
`CustomFunction { Forward; VJP }` pairs.  Swift `precondition` failures
become `ValueError`.

Tensors live on the current ROCm device; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import weakref
import enum
from typing import List, Optional, Sequence, Tuple, Union

import torch

from . import _lib


class BoundaryMode(enum.IntEnum):
    """Texture.swift:8-17."""
    wrap = 0
    clamp = 1
    zero = 2
    cube = 3


class FilterMode(enum.IntEnum):
    """Texture.swift:35-40."""
    nearest = 0
    linear = 1
    linearMipmapNearest = 2
    linearMipmapLinear = 3


_FILTER_NAMES = {"nearest": 0, "linear": 1, "linear-mipmap-nearest": 2,
                 "linear-mipmap-linear": 3, "linearMipmapNearest": 2, "linearMipmapLinear": 3}
_BOUNDARY_NAMES = {"wrap": 0, "clamp": 1, "zero": 2, "cube": 3}


class DiffAttrs:
    """Interpolate.swift:15-18: `DiffAttrs.all` or `DiffAttrs.indices([...])`."""

    def __init__(self, indices: Optional[Sequence[int]] = None):
        self.idx = None if indices is None else [int(i) for i in indices]

    @classmethod
    def indices(cls, idx: Sequence[int]) -> "DiffAttrs":
        return cls(list(idx))

    def __eq__(self, other):
        return isinstance(other, DiffAttrs) and self.idx == other.idx

    def __repr__(self):
        return "DiffAttrs.all" if self.idx is None else f"DiffAttrs.indices({self.idx})"


DiffAttrs.all = DiffAttrs(None)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# The current stream's handle.  torch.cuda.current_stream() builds a Stream
# object per call (~10 us, several calls per op); the raw query returns the
# same handle directly.
if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    _raw_stream = torch._C._cuda_getCurrentRawStream
    _cur_device = torch._C._cuda_getDevice
else:
    def _raw_stream(index):
        return torch.cuda.current_stream(index).cuda_stream
    _cur_device = torch.cuda.current_device


def _stream():
    return ctypes.c_void_p(_raw_stream(_cur_device()))


def _dev_f32(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a tensor on a ROCm device")
    return t.detach().to(torch.float32).contiguous()


def _dev_i32(t, name: str, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    return t.detach().to(device=device, dtype=torch.int32).contiguous()


# ---------------------------------------------------------------------------
# rasterize (Rasterize.swift:44-157)
# ---------------------------------------------------------------------------

# The last rasterize call per (device, stream): the caller's pos and tri
# objects (weak references), read in place (no conversion copy), and their
# autograd versions.  A peel layer given the same objects, unchanged since
# (same versions), reuses that call's triangle setup and tile lists
# (dr_rasterize_fwd_again, which also checks every pointer and size itself).
_last_raster = {}
# The last rasterize forward per (device, stream): its pos and tri buffers
# (address, shape, strides) and pos's version.  A backward whose pos and tri
# are those buffers, pos at that version, differentiates a forward over the
# same data (autograd has checked that its saved pos is unchanged since its
# own forward; a later in-place change would have bumped the version), so it
# may reuse the per-triangle values the last forward stored
# (DR_RASTERIZE_BWD_REUSE; the peel layers of one pos all qualify).
_last_fwd = {}


def _fwd_key(pos, tri):
    return (pos.data_ptr(), tuple(pos.shape), pos.stride(), pos._version, tri.data_ptr(),
            tuple(tri.shape))


def _where(device):
    idx = device.index if device.index is not None else _cur_device()
    return idx, _raw_stream(idx)


def _grad_buf(t, zero=False):
    """A float32 tensor of t's shape with the standard contiguous strides,
    for a gradient returned to autograd: a size-1 dimension of the input
    may carry any stride, and autograd copies a returned gradient whose
    strides differ from the standard ones there instead of keeping it as
    the leaf's .grad."""
    return (torch.zeros if zero else torch.empty)(t.shape, device=t.device, dtype=torch.float32)


def _raster_key(pos, tri, N, H, W, max_per_tile, ranges_host):
    return (pos._version, tri._version, tuple(pos.shape), tuple(tri.shape), N, H, W,
            int(max_per_tile), None if ranges_host is None else ranges_host.tobytes())


class _RasterizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, tri, ranges_host, peel, H, W, grad_db, max_per_tile=0, again=False):
        lib = _lib.load()
        range_mode = ranges_host is not None
        N = ranges_host.shape[0] if range_mode else pos.shape[0]
        V = pos.shape[0] if range_mode else pos.shape[1]
        T = tri.shape[0]
        posc = pos.contiguous()
        rast = torch.empty((N, H, W, 4), device=pos.device, dtype=torch.float32)
        rast_db = torch.empty((N, H, W, 4), device=pos.device, dtype=torch.float32) \
            if grad_db else torch.empty((N, H, W, 0), device=pos.device, dtype=torch.float32)
        rng = ranges_host.ctypes.data_as(ctypes.c_void_p) if range_mode else None
        fwd = lib.dr_rasterize_fwd_again if again else lib.dr_rasterize_fwd_ex
        _lib.check(fwd(
            _ptr(posc), 0 if range_mode else V * 4, _ptr(tri), rng, _ptr(peel), N, V, T, H, W,
            _ptr(rast), _ptr(rast_db) if grad_db else None, int(max_per_tile), _stream()))
        ctx.save_for_backward(posc, tri, rast)
        ctx.meta = (range_mode, N, V, H, W, grad_db)
        _last_fwd[_where(posc.device)] = _fwd_key(posc, tri)
        return rast, rast_db

    @staticmethod
    def backward(ctx, d_rast, d_rast_db):
        lib = _lib.load()
        pos, tri, rast = ctx.saved_tensors
        range_mode, N, V, H, W, grad_db = ctx.meta
        if d_rast is None:
            d_rast = _grad_buf(rast, zero=True)
        d_rast = d_rast.to(torch.float32).contiguous()
        db = None
        if grad_db and d_rast_db is not None:
            db = d_rast_db.to(torch.float32).contiguous()
        d_pos = _grad_buf(pos)
        flags = _lib.DR_RASTERIZE_BWD_REUSE if _last_fwd.get(_where(pos.device)) == _fwd_key(pos, tri) \
            else 0
        _lib.check(lib.dr_rasterize_bwd(
            _ptr(pos), 0 if range_mode else V * 4, _ptr(tri), _ptr(rast), _ptr(d_rast), _ptr(db),
            N, V, tri.shape[0], H, W, _ptr(d_pos), flags, _stream()))
        return d_pos, None, None, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# interpolate (Interpolate.swift:43-132)
# ---------------------------------------------------------------------------

class _InterpolateFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, attr, rast, rast_db, tri, diff_idx, K, shared):
        lib = _lib.load()
        N, H, W, _ = rast.shape
        V, A = attr.shape[-2], attr.shape[-1]
        stride = 0 if shared else V * A
        out = torch.empty((N, H, W, A), device=rast.device, dtype=torch.float32)
        out_da = torch.empty((N, H, W, 2 * K), device=rast.device, dtype=torch.float32)
        _lib.check(lib.dr_interpolate_fwd(
            _ptr(attr), stride, _ptr(rast), _ptr(rast_db) if K else None, _ptr(tri),
            _ptr(diff_idx), K, N, H, W, V, tri.shape[0], A, _ptr(out), _ptr(out_da) if K else None,
            _stream()))
        ctx.save_for_backward(attr, rast, rast_db if K else None, tri, diff_idx)
        ctx.meta = (K, shared)
        return out, out_da

    @staticmethod
    def backward(ctx, d_out, d_out_da):
        lib = _lib.load()
        attr, rast, rast_db, tri, diff_idx = ctx.saved_tensors
        K, shared = ctx.meta
        N, H, W, _ = rast.shape
        V, A = attr.shape[-2], attr.shape[-1]
        stride = 0 if shared else V * A
        d_out = torch.zeros((N, H, W, A), device=rast.device) if d_out is None \
            else d_out.to(torch.float32).contiguous()
        if K:
            d_out_da = torch.zeros((N, H, W, 2 * K), device=rast.device) if d_out_da is None \
                else d_out_da.to(torch.float32).contiguous()
        d_attr = _grad_buf(attr)
        d_rast = _grad_buf(rast)
        d_rast_db = _grad_buf(rast) if K else None
        _lib.check(lib.dr_interpolate_bwd(
            _ptr(attr), stride, _ptr(rast), _ptr(rast_db), _ptr(tri), _ptr(diff_idx), K,
            _ptr(d_out), _ptr(d_out_da) if K else None, N, H, W, V, tri.shape[0], A, _ptr(d_attr),
            stride,
            _ptr(d_rast), _ptr(d_rast_db), 0, _stream()))
        return d_attr, d_rast, d_rast_db, None, None, None, None


# ---------------------------------------------------------------------------
# texture (Texture.swift:62-327)
# ---------------------------------------------------------------------------

def _bias_map(m, uv):
    """Texture.swift:104-108: [N, H_img, W_img] or [N, H_img, W_img, 1]."""
    if m is None:
        return None
    if tuple(m.shape[:3]) != tuple(uv.shape[:3]) or m.ndim not in (3, 4) or \
            (m.ndim == 4 and m.shape[3] != 1):
        raise ValueError("texture: mipLevelBiasMap must be [N, H_img, W_img] or "
                         f"[N, H_img, W_img, 1] (got {list(m.shape)})")
    return m.to(torch.float32).contiguous()


class MipPyramid(list):
    """What `textureConstructMip` returns: the list [tex, level1, ...] plus
    the identity and in-place version of `tex` when the levels were built,
    so that `texture(mip=...)` can refuse a pyramid whose texture has been
    changed since (an optimizer step updates it in place)."""

    def __init__(self, levels, tex):
        super().__init__(levels)
        self.source_ptr = tex.data_ptr()
        self.source_version = tex._version


def _packed_pyramid(levels, tex, tex_arg):
    """(L, packed levels 1..L-1) of a `textureConstructMip` list: its levels
    are views of one buffer in the library's packing, used as they are; any
    other list of [Nt, Hk, Wk, C] levels is packed by a copy.  A
    `MipPyramid` must still describe `tex_arg` as it is now."""
    if isinstance(levels, MipPyramid):
        if tex_arg.data_ptr() != levels.source_ptr:
            raise ValueError("texture: mip was built from another texture tensor "
                             "(textureConstructMip(tex) of the tex passed here)")
        if tex_arg._version != levels.source_version:
            raise ValueError("texture: tex was modified in place after textureConstructMip; "
                             "rebuild mip from the current texture")
    levels = list(levels)
    if not levels:
        raise ValueError("texture: mip must hold at least level 0")
    Nt, H, W, C = tex.shape
    if tuple(levels[0].shape) != (Nt, H, W, C):
        raise ValueError(f"texture: mip[0] must be the texture's shape {[Nt, H, W, C]}")
    h, w = H, W
    for k, lv in enumerate(levels[1:], 1):
        h, w = h // 2, w // 2
        if tuple(lv.shape) != (Nt, h, w, C) or not lv.is_cuda:
            raise ValueError(f"texture: mip[{k}] must be [{Nt}, {h}, {w}, {C}] on the device "
                             f"(got {list(lv.shape)})")
    L = len(levels)
    if L > 1 and h < 1:
        raise ValueError("texture: mip has more levels than the texture allows")
    if L == 1:
        return 1, torch.empty(1, device=tex.device, dtype=torch.float32)
    first = levels[1]
    packed = all(lv.dtype == torch.float32 and lv.is_contiguous() for lv in levels[1:])
    off = 0
    for lv in levels[1:]:
        if not packed or lv.data_ptr() != first.data_ptr() + 4 * off:
            packed = False
            break
        off += lv.numel()
    if packed:
        n = sum(lv.numel() for lv in levels[1:])
        return L, first.reshape(-1).as_strided((n,), (1,))
    return L, torch.cat([lv.detach().to(torch.float32).reshape(-1) for lv in levels[1:]])


class _TextureFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, tex, uv, uv_da, bias_map, filt, boundary, bias, cached, dir_grad=False):
        lib = _lib.load()
        cube = boundary == BoundaryMode.cube
        N, Hi, Wi = uv.shape[0], uv.shape[1], uv.shape[2]
        Nt = tex.shape[0]
        Ht, Wt, C = (tex.shape[2], tex.shape[3], tex.shape[4]) if cube else \
            (tex.shape[1], tex.shape[2], tex.shape[3])
        mip = filt >= FilterMode.linearMipmapNearest
        L, pyr = 1, None
        if mip and cached is not None:
            L, pyr = cached
        elif mip:
            nfaces = Nt * 6 if cube else Nt   # a cube map's pyramid: every face's
            L = lib.dr_texture_mip_levels(Ht, Wt, -1, None, None)
            size = lib.dr_texture_mip_size(nfaces, Ht, Wt, C, L)
            pyr = torch.empty(max(size, 1), device=tex.device, dtype=torch.float32)
            _lib.check(lib.dr_texture_build_mip(_ptr(tex), nfaces, Ht, Wt, C, L, _ptr(pyr),
                                                _stream()))
        out = torch.empty((N, Hi, Wi, C), device=uv.device, dtype=torch.float32)
        _lib.check(lib.dr_texture_fwd(
            _ptr(tex), _ptr(pyr), Nt, Ht, Wt, C, L, _ptr(uv), _ptr(uv_da), _ptr(bias_map),
            float(bias), int(filt), int(boundary), N, Hi, Wi, _ptr(out), _stream()))
        ctx.save_for_backward(tex, uv, uv_da, bias_map, pyr)
        ctx.meta = (int(filt), int(boundary), float(bias), L, Nt, Ht, Wt, C, bool(dir_grad))
        return out

    @staticmethod
    def backward(ctx, d_out):
        lib = _lib.load()
        tex, uv, uv_da, bias_map, pyr = ctx.saved_tensors
        filt, boundary, bias, L, Nt, Ht, Wt, C, dir_grad = ctx.meta
        N, Hi, Wi = uv.shape[0], uv.shape[1], uv.shape[2]
        d_out = d_out.to(torch.float32).contiguous()
        d_tex = _grad_buf(tex)
        d_uv = _grad_buf(uv) if ctx.needs_input_grad[1] else None
        d_uv_da = _grad_buf(uv_da) if (uv_da is not None and ctx.needs_input_grad[2]) else None
        d_bias = _grad_buf(bias_map) if (bias_map is not None and ctx.needs_input_grad[3]) \
            else None
        _lib.check(lib.dr_texture_bwd(
            _ptr(tex), _ptr(pyr), Nt, Ht, Wt, C, L, _ptr(uv), _ptr(uv_da), _ptr(bias_map),
            float(bias), filt, boundary, N, Hi, Wi, _ptr(d_out), _ptr(d_tex), _ptr(d_uv),
            _ptr(d_uv_da), _ptr(d_bias), _lib.DR_CUBE_DIR_GRAD if dir_grad else 0, _stream()))
        if d_uv_da is None and uv_da is not None and ctx.needs_input_grad[2]:
            d_uv_da = _grad_buf(uv_da, zero=True)
        return d_tex, d_uv, d_uv_da, d_bias, None, None, None, None, None


# ---------------------------------------------------------------------------
# antialias (Antialias.swift:90-131)
# ---------------------------------------------------------------------------

class _AntialiasFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, color, pos, rast, tri, topo):
        lib = _lib.load()
        N, H, W, C = color.shape
        V, T = pos.shape[1], tri.shape[0]
        out = torch.empty_like(color)
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            # the saved state (blend mask, edge records) spares the backward
            # the pixels without blends and the per-triangle setup
            saved = torch.empty(lib.dr_antialias_saved_bytes(N, H, W, T), dtype=torch.uint8,
                                device=color.device)
            _lib.check(lib.dr_antialias_fwd_save(_ptr(color), _ptr(rast), _ptr(pos), _ptr(tri),
                                                 _ptr(topo), N, H, W, C, V, T, _ptr(out),
                                                 _ptr(saved), _stream()))
        else:
            saved = None
            _lib.check(lib.dr_antialias_fwd(_ptr(color), _ptr(rast), _ptr(pos), _ptr(tri),
                                            _ptr(topo), N, H, W, C, V, T, _ptr(out), _stream()))
        ctx.save_for_backward(color, pos, rast, tri, topo, saved)
        return out

    @staticmethod
    def backward(ctx, d_out):
        lib = _lib.load()
        color, pos, rast, tri, topo, saved = ctx.saved_tensors
        N, H, W, C = color.shape
        V, T = pos.shape[1], tri.shape[0]
        d_out = d_out.to(torch.float32).contiguous()
        d_color = _grad_buf(color) if ctx.needs_input_grad[0] else None
        d_pos = _grad_buf(pos) if ctx.needs_input_grad[1] else None
        if saved is not None:
            _lib.check(lib.dr_antialias_bwd_saved(_ptr(color), _ptr(rast), _ptr(pos), _ptr(tri),
                                                  _ptr(topo), _ptr(d_out), _ptr(saved), N, H, W,
                                                  C, V, T, _ptr(d_color), _ptr(d_pos), 0,
                                                  _stream()))
        else:
            _lib.check(lib.dr_antialias_bwd(_ptr(color), _ptr(rast), _ptr(pos), _ptr(tri),
                                            _ptr(topo), _ptr(d_out), N, H, W, C, V, T,
                                            _ptr(d_color), _ptr(d_pos), 0, _stream()))
        return d_color, d_pos, None, None, None


# ---------------------------------------------------------------------------
# public API
# ---------------------------------------------------------------------------

class DiffRast:
    """Namespace of the ops (MLXDiffRast.swift:18)."""

    BoundaryMode = BoundaryMode
    FilterMode = FilterMode
    DiffAttrs = DiffAttrs

    @staticmethod
    def rasterize(pos: torch.Tensor, tri, resolution: Tuple[int, int], gradDB: bool = True,
                  ranges=None, peelLayer: Optional[torch.Tensor] = None, maxPerTile: int = 0
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Rasterize.swift:44-144.  Instanced pos [N,V,4], or range mode: pos
        [V,4] with ranges [N,2] (start, count) per image.  Returns (rast,
        rastDB); rastDB is [N,H,W,0] when gradDB is False.

        `ranges` is read on the host (a device tensor is copied back first,
        which waits for it).  `maxPerTile` (no counterpart argument in the
        reference): 0 keeps every triangle; 128 reproduces the reference's
        per-tile limit (MAX_PER_TILE, Rasterize.swift:164-171), each 16x16
        tile keeping its 128 lowest triangle indices (the reference keeps
        the first 128 of its atomic appends)."""
        H, W = int(resolution[0]), int(resolution[1])
        posf = _dev_f32(pos, "rasterize: pos") if not pos.requires_grad else pos.to(torch.float32)
        if not posf.is_cuda:
            raise ValueError("rasterize: pos must be on a ROCm device")
        tri32 = _dev_i32(tri, "tri", posf.device)
        if tri32.ndim != 2 or tri32.shape[1] != 3:
            raise ValueError(f"rasterize: tri must be [T, 3] (got {list(tri32.shape)})")
        ranges_host = None
        if ranges is not None:
            if posf.ndim != 2 or posf.shape[1] != 4:
                raise ValueError(f"rasterize: with `ranges`, pos must be [V, 4] (got {list(posf.shape)})")
            r = ranges.detach().cpu() if isinstance(ranges, torch.Tensor) else torch.as_tensor(ranges)
            ranges_host = r.to(torch.int32).contiguous().numpy()
            if ranges_host.ndim != 2 or ranges_host.shape[1] != 2:
                raise ValueError(f"rasterize: ranges must be [N, 2] (got {list(ranges_host.shape)})")
            N = ranges_host.shape[0]
        else:
            if posf.ndim != 3 or posf.shape[2] != 4:
                raise ValueError(f"rasterize: pos must be [N, V, 4] (got {list(posf.shape)})")
            N = posf.shape[0]
        peel = None
        if peelLayer is not None:
            peel = _dev_f32(peelLayer, "peelLayer")
            if tuple(peel.shape) != (N, H, W, 4):
                raise ValueError("rasterize: peelLayer must match rast shape [N, H, W, 4] "
                                 f"(got {list(peel.shape)})")
        if not 0 <= int(maxPerTile) <= 1024:
            raise ValueError("rasterize: maxPerTile must be in [0, 1024] (0: no limit)")
        posc = posf.contiguous()
        # Reuse (peel layers only): the same pos and tri objects as the
        # previous call on this stream, read in place and unchanged since.
        in_place = (isinstance(pos, torch.Tensor) and isinstance(tri, torch.Tensor)
                    and posc.data_ptr() == pos.data_ptr() and tri32.data_ptr() == tri.data_ptr())
        where = (posc.device.index, _raw_stream(posc.device.index))
        key = _raster_key(pos, tri, N, H, W, maxPerTile, ranges_host) if in_place else None
        last = _last_raster.get(where)
        again = (peel is not None and key is not None and last is not None
                 and last[0]() is pos and last[1]() is tri and last[2] == key)
        out = _RasterizeFn.apply(posc, tri32, ranges_host, peel, H, W, bool(gradDB),
                                 int(maxPerTile), again)
        if key is None:
            _last_raster.pop(where, None)
        else:
            _last_raster[where] = (weakref.ref(pos), weakref.ref(tri), key)
        return out

    @staticmethod
    def rasterizeTileCounts(pos: torch.Tensor, tri, resolution: Tuple[int, int],
                            ranges=None) -> torch.Tensor:
        """Binning report: per 16x16 tile, the number of triangles binned to
        it, [N, ceil(H/16), ceil(W/16)] int32 -- the reference's bin counts
        (Rasterize.swift:227-239).  Tiles above 128 are those where the
        reference drops triangles (MAX_PER_TILE, :164-171); rasterize here
        keeps them all.  Same layouts as `rasterize`."""
        H, W = int(resolution[0]), int(resolution[1])
        posf = _dev_f32(pos.detach() if isinstance(pos, torch.Tensor) else pos,
                        "rasterizeTileCounts: pos")
        tri32 = _dev_i32(tri, "tri", posf.device)
        if tri32.ndim != 2 or tri32.shape[1] != 3:
            raise ValueError(f"rasterizeTileCounts: tri must be [T, 3] (got {list(tri32.shape)})")
        rng = None
        if ranges is not None:
            if posf.ndim != 2 or posf.shape[1] != 4:
                raise ValueError("rasterizeTileCounts: with `ranges`, pos must be [V, 4]")
            r = ranges.detach().cpu() if isinstance(ranges, torch.Tensor) else torch.as_tensor(ranges)
            rng = r.to(torch.int32).contiguous().numpy()
            if rng.ndim != 2 or rng.shape[1] != 2:
                raise ValueError("rasterizeTileCounts: ranges must be [N, 2]")
            N, V = rng.shape[0], posf.shape[0]
        else:
            if posf.ndim != 3 or posf.shape[2] != 4:
                raise ValueError("rasterizeTileCounts: pos must be [N, V, 4]")
            N, V = posf.shape[0], posf.shape[1]
        lib = _lib.load()
        counts = torch.empty((N, (H + 15) // 16, (W + 15) // 16), device=posf.device,
                             dtype=torch.int32)
        _lib.check(lib.dr_rasterize_tile_counts(
            _ptr(posf), 0 if rng is not None else V * 4, _ptr(tri32),
            rng.ctypes.data_as(ctypes.c_void_p) if rng is not None else None, N, V,
            tri32.shape[0], H, W, _ptr(counts), None, _stream()))
        return counts

    @staticmethod
    def interpolate(attr: torch.Tensor, rast: torch.Tensor, tri, rastDB=None,
                    diffAttrs: Union[None, DiffAttrs, str, Sequence[int]] = None
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Interpolate.swift:43-132.  attr [V,A], [1,V,A] or [N,V,A]."""
        if rast.ndim != 4 or rast.shape[3] != 4:
            raise ValueError(f"interpolate: rast must be [N, H, W, 4] (got {list(rast.shape)})")
        if attr.ndim not in (2, 3):
            raise ValueError(f"interpolate: attr must be [V, A] or [N, V, A] (got {list(attr.shape)})")
        N = rast.shape[0]
        tri32 = _dev_i32(tri, "tri", rast.device)
        if tri32.ndim != 2 or tri32.shape[1] != 3:
            raise ValueError(f"interpolate: tri must be [T, 3] (got {list(tri32.shape)})")
        if attr.ndim == 3 and attr.shape[0] not in (1, N):
            raise ValueError(f"interpolate: attr batch dim {attr.shape[0]} incompatible with "
                             f"rast batch {N}")
        shared = attr.ndim == 2 or attr.shape[0] == 1
        if attr.ndim == 3 and attr.shape[0] == 1 and N == 1:
            shared = False
        A = attr.shape[-1]
        if isinstance(diffAttrs, str):
            if diffAttrs != "all":
                raise ValueError("interpolate: diffAttrs must be 'all' or indices")
            diffAttrs = DiffAttrs.all
        elif diffAttrs is not None and not isinstance(diffAttrs, DiffAttrs):
            diffAttrs = DiffAttrs.indices(diffAttrs)
        rastf = rast.to(torch.float32).contiguous()
        attrf = attr.to(torch.float32).contiguous()
        if diffAttrs is None:
            out, _ = _InterpolateFn.apply(attrf, rastf, None, tri32, None, 0, shared)
            return out, torch.zeros((N, rast.shape[1], rast.shape[2], 0), device=rast.device)
        if rastDB is None:
            raise ValueError("interpolate: rastDB is required when diffAttrs is set")
        if tuple(rastDB.shape) != tuple(rast.shape):
            raise ValueError(f"interpolate: rastDB must match rast shape (got {list(rastDB.shape)} "
                             f"vs {list(rast.shape)})")
        if diffAttrs.idx is None:
            K, didx = A, None
        else:
            if len(diffAttrs.idx) == 0:
                raise ValueError("interpolate: diffAttrs.indices must be non-empty")
            if any(i < 0 or i >= A for i in diffAttrs.idx):
                raise ValueError(f"interpolate: diffAttrs.indices values must be in [0, A) (A={A})")
            K = len(diffAttrs.idx)
            didx = torch.tensor(diffAttrs.idx, dtype=torch.int32, device=rast.device)
        return _InterpolateFn.apply(attrf, rastf, rastDB.to(torch.float32).contiguous(), tri32,
                                    didx, K, shared)

    @staticmethod
    def texture(tex: torch.Tensor, uv: torch.Tensor, uvDA: Optional[torch.Tensor] = None,
                filterMode: Union[FilterMode, str] = FilterMode.linear,
                boundaryMode: Union[BoundaryMode, str] = BoundaryMode.wrap,
                mipLevelBias: float = 0.0, mipLevelBiasMap: Optional[torch.Tensor] = None,
                mip: Optional[Sequence[torch.Tensor]] = None, dirGrad: bool = False
                ) -> torch.Tensor:
        """Texture.swift:62-131.

        `mip` (mip filters only; no counterpart argument in the reference):
        a pyramid `[tex, level1, ...]` from `textureConstructMip(tex)`, kept
        across calls with the same texture so it is not rebuilt
        (Texture.swift:141-143 suggests such caching).  Its levels are read
        as given (fewer levels cap the LOD); the gradient still flows to
        `tex` through the 2x2 box backward, as for a pyramid built in the
        call.  A pyramid from `textureConstructMip` raises ValueError once
        `tex` has been changed in place (or when another tensor is passed);
        a plain list of levels is taken as it is.

        Cube maps (boundaryMode cube) also take the mip filters, with uvDA
        the direction's screen derivatives [N, H_img, W_img, 6] (the layout
        `interpolate(..., diffAttrs=.all)` gives a 3-channel direction), and
        `dirGrad=True` returns the direction gradient instead of the
        reference's zeros (Texture.swift:196-198).  Both are extensions; the
        reference samples cube maps bilinearly only (:75-76)."""
        filt = FilterMode(_FILTER_NAMES[filterMode] if isinstance(filterMode, str) else filterMode)
        bnd = BoundaryMode(_BOUNDARY_NAMES[boundaryMode] if isinstance(boundaryMode, str)
                           else boundaryMode)
        texf = tex.to(torch.float32).contiguous()
        uvf = uv.to(torch.float32).contiguous()
        if not texf.is_cuda or not uvf.is_cuda:
            raise ValueError("texture: tensors must be on a ROCm device")
        if bnd == BoundaryMode.cube:
            if filt == FilterMode.nearest:
                raise ValueError("texture: cube textures support the linear and mipmap filterModes")
            if texf.ndim != 5 or texf.shape[1] != 6:
                raise ValueError(f"texture: cube tex must be [N, 6, H, W, C] (got {list(texf.shape)})")
            if uvf.ndim != 4 or uvf.shape[3] != 3:
                raise ValueError("texture: cube uv must be [N, H_img, W_img, 3] direction vector "
                                 f"(got {list(uvf.shape)})")
            if texf.shape[0] not in (1, uvf.shape[0]):
                raise ValueError("texture: tex batch dim incompatible with uv batch")
            if mip is not None:
                raise ValueError("texture: a prebuilt `mip` is for 2D textures")
            if filt == FilterMode.linear:
                return _TextureFn.apply(texf, uvf, None, None, filt, bnd, 0.0, None,
                                        bool(dirGrad))
            if uvDA is None or tuple(uvDA.shape) != tuple(uvf.shape[:3]) + (6,):
                raise ValueError("texture: cube mipmap filterModes require uvDA "
                                 "[N, H_img, W_img, 6] (direction derivatives)")
            bm = _bias_map(mipLevelBiasMap, uvf)
            return _TextureFn.apply(texf, uvf, uvDA.to(torch.float32).contiguous(), bm, filt, bnd,
                                    float(mipLevelBias), None, bool(dirGrad))
        if texf.ndim != 4:
            raise ValueError(f"texture: tex must be [N, H_tex, W_tex, C] (got {list(texf.shape)})")
        if uvf.ndim != 4 or uvf.shape[3] != 2:
            raise ValueError(f"texture: uv must be [N, H_img, W_img, 2] (got {list(uvf.shape)})")
        if texf.shape[0] not in (1, uvf.shape[0]):
            raise ValueError(f"texture: tex batch dim {texf.shape[0]} incompatible with uv batch "
                             f"{uvf.shape[0]}")
        if filt in (FilterMode.nearest, FilterMode.linear):
            return _TextureFn.apply(texf, uvf, None, None, filt, bnd, 0.0, None)
        if uvDA is None:
            raise ValueError("texture: mipmap filterModes require uvDA")
        if tuple(uvDA.shape) != tuple(uvf.shape[:3]) + (4,):
            raise ValueError(f"texture: uvDA must be [N, H_img, W_img, 4] (got {list(uvDA.shape)})")
        bm = _bias_map(mipLevelBiasMap, uvf)
        cached = None if mip is None else _packed_pyramid(mip, texf, tex)
        return _TextureFn.apply(texf, uvf, uvDA.to(torch.float32).contiguous(), bm, filt, bnd,
                                float(mipLevelBias), cached)

    @staticmethod
    def textureConstructMip(tex: torch.Tensor, maxLevel: Optional[int] = None) -> List[torch.Tensor]:
        """Texture.swift:144-161: [level0 = tex, level1, ...], 2x2 box means
        (a `MipPyramid`, which also records tex's in-place version)."""
        if tex.ndim != 4:
            raise ValueError(f"textureConstructMip: tex must be [N, H, W, C] (got {list(tex.shape)})")
        lib = _lib.load()
        Nt, H, W, C = tex.shape
        L = lib.dr_texture_mip_levels(H, W, -1 if maxLevel is None else int(maxLevel), None, None)
        texf = _dev_f32(tex, "textureConstructMip: tex")
        size = lib.dr_texture_mip_size(Nt, H, W, C, L)
        pyr = torch.empty(max(size, 1), device=texf.device, dtype=torch.float32)
        _lib.check(lib.dr_texture_build_mip(_ptr(texf), Nt, H, W, C, L, _ptr(pyr), _stream()))
        levels, off, h, w = [tex], 0, H, W
        for _ in range(1, L):
            h, w = h // 2, w // 2
            n = Nt * h * w * C
            levels.append(pyr[off:off + n].view(Nt, h, w, C))
            off += n
        return MipPyramid(levels, tex)

    @staticmethod
    def antialiasConstructTopologyHash(tri) -> torch.Tensor:
        """Antialias.swift:19-66, computed on the GPU."""
        tri32 = _dev_i32(tri, "tri", torch.device("cuda", torch.cuda.current_device())
                         if not isinstance(tri, torch.Tensor) or not tri.is_cuda else tri.device)
        if tri32.ndim != 2 or tri32.shape[1] != 3:
            raise ValueError("antialiasConstructTopologyHash: tri must be [T, 3] "
                             f"(got {list(tri32.shape)})")
        lib = _lib.load()
        topo = torch.empty_like(tri32)
        _lib.check(lib.dr_antialias_topology(_ptr(tri32), tri32.shape[0], _ptr(topo), _stream()))
        return topo

    @staticmethod
    def antialias(color: torch.Tensor, rast: torch.Tensor, pos: torch.Tensor, tri,
                  topologyHash: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Antialias.swift:90-131."""
        if color.ndim != 4:
            raise ValueError(f"antialias: color must be [N, H, W, C] (got {list(color.shape)})")
        if rast.ndim != 4 or rast.shape[3] != 4 or tuple(rast.shape[:3]) != tuple(color.shape[:3]):
            raise ValueError("antialias: rast must match color in [N, H, W] and have 4 channels")
        if pos.ndim != 3 or pos.shape[2] != 4:
            raise ValueError(f"antialias: pos must be [N, V, 4] (got {list(pos.shape)})")
        tri32 = _dev_i32(tri, "tri", color.device)
        if tri32.ndim != 2 or tri32.shape[1] != 3:
            raise ValueError(f"antialias: tri must be [T, 3] (got {list(tri32.shape)})")
        topo = DiffRast.antialiasConstructTopologyHash(tri32) if topologyHash is None else \
            _dev_i32(topologyHash, "topologyHash", color.device)
        return _AntialiasFn.apply(color.to(torch.float32).contiguous(),
                                  pos.to(torch.float32).contiguous(),
                                  rast.detach().to(torch.float32).contiguous(), tri32, topo)


rasterize = DiffRast.rasterize
interpolate = DiffRast.interpolate
texture = DiffRast.texture
textureConstructMip = DiffRast.textureConstructMip
antialiasConstructTopologyHash = DiffRast.antialiasConstructTopologyHash
antialias = DiffRast.antialias
