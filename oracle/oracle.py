"""numpy front end of the CPU restatement of mlx-swift-diffrast.

TEST INFRASTRUCTURE ONLY: the parity checker (and the CPU baseline) for the
HIP kernels.  Only tests, the smoke check and the benchmark's CPU-baseline
leg use it; the product path never imports it.

The functions below restate the reference's host layer (the public
`DiffRast.*` functions and the dispatchers in
Sources/MLXDiffRast/{Rasterize,Interpolate,Texture,Antialias}.swift): shape
normalisation, broadcasts (materialised, as MLX does), kernel sequencing and
the cotangent plumbing MLX autodiff performs (sums over broadcast batch
axes, the backward of the mip pyramid's `mean`).  The per-thread arithmetic
lives in diffrast_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i = ctypes.c_int
_i64 = ctypes.c_int64

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    sig = {
        "orc_set_threads": [_i],
        "orc_rast_precompute": [_f32p, _i64, _i32p, _i32p, _i, _i, _i, _f32p],
        "orc_rast_bin_count": [_f32p, _i, _i, _i, _i, _i32p],
        "orc_rast_bin_fill": [_f32p, _i, _i, _i, _i, _i64p, _i32p, _i32p],
        "orc_rast_fwd": [_f32p, _i64p, _i32p, _i32p, _f32p, _i, _i, _i, _i, _i, _f32p, _f32p],
        "orc_rast_bwd": [_f32p, _i64, _i32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _f32p],
        "orc_interp_fwd": [_f32p, _i64, _f32p, _i32p, _i, _i, _i, _i, _i, _f32p],
        "orc_interp_fwd_da": [_f32p, _i64, _f32p, _f32p, _i32p, _i32p, _i, _i, _i, _i, _i, _i,
                              _f32p, _f32p],
        "orc_interp_grad_attr": [_f32p, _i32p, _f32p, _i, _i, _i, _i, _i, _i64, _f32p],
        "orc_interp_grad_attr_da": [_f32p, _f32p, _i32p, _f32p, _f32p, _i32p, _i, _i, _i, _i, _i,
                                    _i, _i64, _f32p],
        "orc_interp_grad_rast": [_f32p, _i64, _f32p, _i32p, _f32p, _i, _i, _i, _i, _i, _f32p],
        "orc_interp_grad_rast_db": [_f32p, _i64, _f32p, _i32p, _f32p, _i32p, _i, _i, _i, _i, _i,
                                    _i, _f32p],
        "orc_tex_fwd": [_f32p, _i64, _f32p, _i, _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_grad_tex": [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _i64, _f32p],
        "orc_tex_grad_uv": [_f32p, _i64, _f32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_nearest_fwd": [_f32p, _i64, _f32p, _i, _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_nearest_grad_tex": [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _i64, _f32p],
        "orc_tex_cube_fwd": [_f32p, _i64, _f32p, _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_cube_grad_tex": [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _i64, _f32p],
        "orc_mip_levels": [_i, _i, _i, _i32p, _i32p],
        "orc_mip_build": [_f32p, _i, _i, _i, _i, _i, _i64p, _f32p],
        "orc_mip_collapse": [_f32p, _i, _i, _i, _i, _i, _i64p, _f32p],
        "orc_tex_mip_fwd": [_f32p, _i64, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i, _i, _i, _i,
                            _i, _i, _i, _i, _f32p],
        "orc_tex_mip_grad_pyramid": [_f32p, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i64, _i, _i,
                                     _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_mip_grad_uv": [_f32p, _i64, _f32p, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i,
                                _i, _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_mip_grad_uvda": [_f32p, _i64, _f32p, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i,
                                  _i, _i, _i, _i, _i, _i, _f32p],
        "orc_tex_cube_mip_fwd": [_f32p, _i64, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i, _i, _i,
                                 _i, _i, _f32p],
        "orc_tex_cube_mip_bwd": [_f32p, _i64, _f32p, _f32p, _f32p, _i64p, _i32p, _i32p, _i, _i,
                                 _i, _i, _i, _i, _f32p, _f32p, _f32p],
        "orc_aa_topology": [_i32p, _i, _i32p],
        "orc_aa_fwd": [_f32p, _f32p, _f32p, _i32p, _i32p, _i, _i, _i, _i, _i, _f32p],
        "orc_aa_bwd_color": [_f32p, _f32p, _i32p, _i32p, _f32p, _i, _i, _i, _i, _i, _f32p],
        "orc_aa_bwd_pos": [_f32p, _f32p, _f32p, _i32p, _i32p, _f32p, _i, _i, _i, _i, _i, _f32p],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = None
    L.orc_rast_bin_count.restype = _i64
    L.orc_mip_levels.restype = _i


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def c32(a):
    """Contiguous float32 array (None stays None)."""
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def ci32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def fp(a):
    """float* of an array that the caller keeps alive (None -> NULL)."""
    return None if a is None else a.ctypes.data_as(_f32p)


def ip(a):
    return None if a is None else a.ctypes.data_as(_i32p)


def lp(a):
    return a.ctypes.data_as(_i64p)


# ---------------------------------------------------------------------------
# rasterize (Rasterize.swift:44-157, 823-894)
# ---------------------------------------------------------------------------

TILE_SIZE = 16
MAX_PER_TILE = 128


def _raster_layout(pos, tri, ranges):
    """Rasterize.swift:61-88: instanced [N,V,4] or range [V,4] + ranges."""
    pos = np.asarray(pos, dtype=np.float32)
    tri = ci32(tri)
    if tri.ndim != 2 or tri.shape[1] != 3:
        raise ValueError(f"rasterize: tri must be [T, 3] (got {tri.shape})")
    T = tri.shape[0]
    if ranges is not None:
        ranges = ci32(ranges)
        if pos.ndim != 2 or pos.shape[1] != 4:
            raise ValueError("rasterize: with `ranges`, pos must be [V, 4]")
        if ranges.ndim != 2 or ranges.shape[1] != 2:
            raise ValueError("rasterize: ranges must be [N, 2]")
        N, V = ranges.shape[0], pos.shape[0]
        pos_n = c32(np.broadcast_to(pos[None], (N, V, 4)))
    else:
        if pos.ndim != 3 or pos.shape[2] != 4:
            raise ValueError("rasterize: pos must be [N, V, 4]")
        N, V = pos.shape[0], pos.shape[1]
        pos_n = c32(pos)
        ranges = ci32(np.tile(np.array([[0, T]], dtype=np.int32), (N, 1)))
    return pos_n, tri, ranges, N, V, T


def rasterize(pos, tri, resolution, gradDB=True, ranges=None, peelLayer=None,
              max_per_tile: int = MAX_PER_TILE, stats: Optional[dict] = None):
    """DiffRast.rasterize forward (Rasterize.swift:44-144, :823-894).

    max_per_tile=128 reproduces the reference's silent bin overflow (tile
    lists truncated after 128 entries, in ascending triangle order);
    max_per_tile=0 keeps every triangle.
    """
    H, W = resolution
    pos_n, tri, ranges, N, V, T = _raster_layout(pos, tri, ranges)
    L = lib()
    screen = np.empty((N, T, 10), np.float32)
    L.orc_rast_precompute(fp(pos_n), V * 4, ip(tri), ip(ranges), N, V, T, fp(screen))
    ntx = (W + TILE_SIZE - 1) // TILE_SIZE
    nty = (H + TILE_SIZE - 1) // TILE_SIZE
    counts = np.zeros((N, nty * ntx), np.int32)
    total = L.orc_rast_bin_count(fp(screen), N, T, H, W, ip(counts))
    offsets = np.zeros(counts.size + 1, np.int64)
    np.cumsum(counts.reshape(-1), out=offsets[1:])
    fill = np.zeros_like(counts)
    lst = np.zeros(max(int(total), 1), np.int32)
    L.orc_rast_bin_fill(fp(screen), N, T, H, W, lp(offsets), ip(fill), ip(lst))
    peel = None
    if peelLayer is not None:
        peel = c32(peelLayer)
        if peel.shape != (N, H, W, 4):
            raise ValueError("rasterize: peelLayer must match rast shape [N, H, W, 4]")
    rast = np.empty((N, H, W, 4), np.float32)
    rast_db = np.empty((N, H, W, 4), np.float32) if gradDB else None
    L.orc_rast_fwd(fp(screen), lp(offsets), ip(counts), ip(lst), fp(peel), N, T, H, W,
                   int(max_per_tile), fp(rast), fp(rast_db))
    if stats is not None:
        stats["max_tile_count"] = int(counts.max()) if counts.size else 0
        stats["pairs"] = int(total)
        stats["overflow_tiles"] = int((counts > MAX_PER_TILE).sum())
    if not gradDB:
        rast_db = np.zeros((N, H, W, 0), np.float32)
    return rast, rast_db


def rasterize_tile_counts(pos, tri, resolution, ranges=None):
    """The reference's bin counts bins[tile, 0] (Rasterize.swift:182-240,
    after the precompute :280-328) as [N, ceil(H/16), ceil(W/16)] int32."""
    H, W = resolution
    pos_n, tri, ranges, N, V, T = _raster_layout(pos, tri, ranges)
    L = lib()
    screen = np.empty((N, T, 10), np.float32)
    L.orc_rast_precompute(fp(pos_n), V * 4, ip(tri), ip(ranges), N, V, T, fp(screen))
    ntx = (W + TILE_SIZE - 1) // TILE_SIZE
    nty = (H + TILE_SIZE - 1) // TILE_SIZE
    counts = np.zeros((N, nty * ntx), np.int32)
    L.orc_rast_bin_count(fp(screen), N, T, H, W, ip(counts))
    return counts.reshape(N, nty, ntx)


def rasterize_vjp(pos, tri, rast, d_rast, d_rast_db=None, ranges=None):
    """VJP closure (Rasterize.swift:109-118, 129-139) -> d_pos, shaped like pos.

    In range mode the [N,V,4] gradient is summed over N (MLX's broadcast
    backward, Rasterize.swift:72-76)."""
    pos_n, tri, ranges, N, V, T = _raster_layout(pos, tri, ranges)
    rast = c32(rast)
    _, H, W, _ = rast.shape
    d_rast = c32(d_rast)
    db = None if d_rast_db is None or np.shape(d_rast_db)[-1] == 0 else c32(d_rast_db)
    d_pos = np.zeros((N, V, 4), np.float32)
    lib().orc_rast_bwd(fp(pos_n), V * 4, ip(tri), fp(rast), fp(d_rast), fp(db), N, V, H, W,
                       fp(d_pos))
    if np.ndim(pos) == 2:
        return d_pos.sum(axis=0, dtype=np.float32)
    return d_pos


# ---------------------------------------------------------------------------
# interpolate (Interpolate.swift:43-132, 475-541)
# ---------------------------------------------------------------------------

def _attr_n(attr, N):
    attr = np.asarray(attr, np.float32)
    if attr.ndim not in (2, 3):
        raise ValueError("interpolate: attr must be [V, A] or [N, V, A]")
    a = attr[None] if attr.ndim == 2 else attr
    if a.shape[0] == 1 and N > 1:
        a = np.broadcast_to(a, (N,) + a.shape[1:])
    if a.shape[0] != N:
        raise ValueError("interpolate: attr batch dim incompatible with rast batch")
    return c32(a)


def _diff_idx(diffAttrs, A):
    if diffAttrs is None:
        return None
    if isinstance(diffAttrs, str):
        if diffAttrs != "all":
            raise ValueError("diffAttrs must be 'all' or a list of indices")
        return np.arange(A, dtype=np.int32)
    idx = ci32(list(diffAttrs))
    if idx.size == 0:
        raise ValueError("interpolate: diffAttrs.indices must be non-empty")
    if (idx < 0).any() or (idx >= A).any():
        raise ValueError("interpolate: diffAttrs.indices values must be in [0, A)")
    return idx


def interpolate(attr, rast, tri, rastDB=None, diffAttrs=None):
    rast = c32(rast)
    tri = ci32(tri)
    N, H, W, _ = rast.shape
    a = _attr_n(attr, N)
    V, A = a.shape[1], a.shape[2]
    L = lib()
    out = np.empty((N, H, W, A), np.float32)
    idx = _diff_idx(diffAttrs, A)
    if idx is None:
        L.orc_interp_fwd(fp(a), V * A, fp(rast), ip(tri), N, H, W, V, A, fp(out))
        return out, np.zeros((N, H, W, 0), np.float32)
    if rastDB is None:
        raise ValueError("interpolate: rastDB is required when diffAttrs is set")
    db = c32(rastDB)
    K = idx.size
    out_da = np.empty((N, H, W, 2 * K), np.float32)
    L.orc_interp_fwd_da(fp(a), V * A, fp(rast), fp(db), ip(tri), ip(idx), N, H, W, V, A, K,
                        fp(out), fp(out_da))
    return out, out_da


def interpolate_vjp(attr, rast, tri, d_out, rastDB=None, diffAttrs=None, d_out_da=None):
    """VJP closures (Interpolate.swift:86-91, 120-127) -> (d_attr, d_rast,
    d_rast_db or None); d_attr is reduced to attr's own shape as MLX's
    broadcast backward does."""
    rast = c32(rast)
    tri = ci32(tri)
    N, H, W, _ = rast.shape
    attr = np.asarray(attr, np.float32)
    a = _attr_n(attr, N)
    V, A = a.shape[1], a.shape[2]
    L = lib()
    g = c32(d_out)
    d_attr = np.zeros((N, V, A), np.float32)
    d_rast = np.empty((N, H, W, 4), np.float32)
    idx = _diff_idx(diffAttrs, A)
    d_rast_db = None
    if idx is None:
        L.orc_interp_grad_attr(fp(rast), ip(tri), fp(g), N, H, W, V, A, V * A, fp(d_attr))
    else:
        K = idx.size
        db = c32(rastDB)
        gd = c32(d_out_da)
        L.orc_interp_grad_attr_da(fp(rast), fp(db), ip(tri), fp(g), fp(gd), ip(idx), N, H, W, V,
                                  A, K, V * A, fp(d_attr))
        d_rast_db = np.empty((N, H, W, 4), np.float32)
        L.orc_interp_grad_rast_db(fp(a), V * A, fp(rast), ip(tri), fp(gd), ip(idx), N, H, W, V,
                                  A, K, fp(d_rast_db))
    L.orc_interp_grad_rast(fp(a), V * A, fp(rast), ip(tri), fp(g), N, H, W, V, A, fp(d_rast))
    if attr.ndim == 2:
        d_attr = d_attr.sum(axis=0, dtype=np.float32)
    elif attr.shape[0] == 1 and N > 1:
        d_attr = d_attr.sum(axis=0, keepdims=True, dtype=np.float32)
    return d_attr, d_rast, d_rast_db


# ---------------------------------------------------------------------------
# texture (Texture.swift:62-327, 1141-1312)
# ---------------------------------------------------------------------------

BOUNDARY = {"wrap": 0, "clamp": 1, "zero": 2, "cube": 3}


def texture_mip_levels(H, W, maxLevel=None):
    lh = np.zeros(32, np.int32)
    lw = np.zeros(32, np.int32)
    n = lib().orc_mip_levels(H, W, -1 if maxLevel is None else int(maxLevel), ip(lh), ip(lw))
    return lh[:n].copy(), lw[:n].copy()


def _pack_offsets(Nt, lh, lw, C):
    sizes = Nt * lh.astype(np.int64) * lw.astype(np.int64) * C
    offsets = np.zeros(len(lh), np.int64)
    offsets[1:] = np.cumsum(sizes)[:-1]
    return offsets, int(sizes.sum())


def textureConstructMip(tex, maxLevel=None):
    """Texture.swift:144-161 -> list of levels [N, H/2^k, W/2^k, C]."""
    tex = c32(tex)
    if tex.ndim != 4:
        raise ValueError("textureConstructMip: tex must be [N, H, W, C]")
    Nt, H, W, C = tex.shape
    lh, lw = texture_mip_levels(H, W, maxLevel)
    offsets, total = _pack_offsets(Nt, lh, lw, C)
    packed = np.empty(total, np.float32)
    lib().orc_mip_build(fp(tex), Nt, H, W, C, len(lh), lp(offsets), fp(packed))
    return [packed[offsets[k]:offsets[k] + Nt * lh[k] * lw[k] * C].reshape(Nt, lh[k], lw[k], C)
            for k in range(len(lh))]


def _bias_fold(uvDA, mipLevelBias, mipLevelBiasMap):
    """Texture.swift:109-126: uvDA * (2^map * 2^bias), as MLX ops."""
    uvDA = c32(uvDA)
    two = np.float32(2.0)
    if mipLevelBiasMap is not None:
        m = c32(mipLevelBiasMap)
        if m.ndim == 3:
            m = m[..., None]
        scale = np.power(two, m).astype(np.float32)
        if mipLevelBias != 0:
            scale = (scale * np.power(two, np.float32(mipLevelBias))).astype(np.float32)
        return c32(uvDA * scale), scale
    if mipLevelBias != 0:
        s = np.float32(np.power(two, np.float32(mipLevelBias)))
        return c32(uvDA * s), s
    return uvDA, None


def texture(tex, uv, uvDA=None, filterMode="linear", boundaryMode="wrap",
            mipLevelBias=0.0, mipLevelBiasMap=None):
    """DiffRast.texture forward (Texture.swift:62-131)."""
    return _texture(tex, uv, uvDA, filterMode, boundaryMode, mipLevelBias, mipLevelBiasMap,
                    d_out=None)


def texture_vjp(tex, uv, d_out, uvDA=None, filterMode="linear", boundaryMode="wrap",
                mipLevelBias=0.0, mipLevelBiasMap=None, dirGrad=False):
    """-> (d_tex, d_uv, d_uvDA or None, d_biasMap or None).  dirGrad (cube
    maps): the direction gradient of the extension instead of the
    reference's zeros."""
    return _texture(tex, uv, uvDA, filterMode, boundaryMode, mipLevelBias, mipLevelBiasMap,
                    d_out=d_out, dir_grad=dirGrad)


def _cube_ext(tex, dirs, dd, mode, mipLevelBias, mipLevelBiasMap, g, dir_grad):
    """Cube maps with mip filters / the direction gradient (an extension; see
    orc_tex_cube_mip_fwd): the pyramid of the N-broadcast faces, packed."""
    L = lib()
    N, Hi, Wi, _ = dirs.shape
    Ht, Wt, C = tex.shape[2], tex.shape[3], tex.shape[4]
    faces = c32(np.broadcast_to(tex, (N,) + tex.shape[1:])).reshape(N * 6, Ht, Wt, C)
    if mode > 0:
        lh, lw = texture_mip_levels(Ht, Wt)
        eff, scale = _bias_fold(dd, mipLevelBias, mipLevelBiasMap)
    else:
        lh, lw = texture_mip_levels(Ht, Wt, maxLevel=0)
        eff, scale = None, None
    nl = len(lh)
    offsets, total = _pack_offsets(N * 6, lh, lw, C)
    packed = np.empty(total, np.float32)
    L.orc_mip_build(fp(faces), N * 6, Ht, Wt, C, nl, lp(offsets), fp(packed))
    if g is None:
        out = np.empty((N, Hi, Wi, C), np.float32)
        L.orc_tex_cube_mip_fwd(fp(packed), 1, fp(dirs), fp(eff), lp(offsets), ip(lh), ip(lw), nl,
                               N, Hi, Wi, C, mode, fp(out))
        return out
    d_packed = np.zeros(total, np.float32)
    d_dir = np.zeros((N, Hi, Wi, 3), np.float32)
    d_eff = np.zeros((N, Hi, Wi, 6), np.float32) if mode > 0 else None
    L.orc_tex_cube_mip_bwd(fp(packed), 1, fp(dirs), fp(eff), fp(g), lp(offsets), ip(lh), ip(lw),
                           nl, N, Hi, Wi, C, mode, fp(d_packed), fp(d_dir), fp(d_eff))
    d_faces = np.empty((N * 6, Ht, Wt, C), np.float32)
    L.orc_mip_collapse(fp(d_packed), N * 6, Ht, Wt, C, nl, lp(offsets), fp(d_faces))
    d_tex = d_faces.reshape(N, 6, Ht, Wt, C)
    if tex.shape[0] == 1 and N > 1:
        d_tex = d_tex.sum(axis=0, keepdims=True, dtype=np.float32)
    if not dir_grad:
        d_dir = np.zeros_like(d_dir)
    d_dd, d_map = None, None
    if mode > 0:
        d_dd = d_eff if scale is None else c32(d_eff * scale)
        if scale is not None and mipLevelBiasMap is not None:
            gm = (d_eff * dd).astype(np.float32).sum(axis=3, keepdims=True, dtype=np.float32)
            d_map = c32(gm * scale * np.float32(np.log(2.0)))
            if np.ndim(mipLevelBiasMap) == 3:
                d_map = d_map[..., 0]
    return d_tex, d_dir, d_dd, d_map


def _texture(tex, uv, uvDA, filterMode, boundaryMode, mipLevelBias, mipLevelBiasMap, d_out,
             dir_grad=False):
    L = lib()
    tex = c32(tex)
    uv = c32(uv)
    g = c32(d_out)
    b = BOUNDARY[boundaryMode]
    if b == 3 and filterMode in ("linear-mipmap-linear", "linear-mipmap-nearest"):
        if tex.ndim != 5 or tex.shape[1] != 6:
            raise ValueError("texture: cube tex must be [N, 6, H, W, C]")
        if uv.ndim != 4 or uv.shape[3] != 3:
            raise ValueError("texture: cube uv must be [N, H_img, W_img, 3]")
        if uvDA is None or c32(uvDA).shape != uv.shape[:3] + (6,):
            raise ValueError("texture: cube mip filters need uvDA [N, H_img, W_img, 6]")
        mode = 2 if filterMode == "linear-mipmap-linear" else 1
        return _cube_ext(tex, uv, c32(uvDA), mode, mipLevelBias, mipLevelBiasMap, g, dir_grad)
    if b == 3 and g is not None and dir_grad:
        if filterMode != "linear":
            raise ValueError("texture: cube textures support linear and mip filters")
        return _cube_ext(tex, uv, None, 0, 0.0, None, g, True)
    if b == 3:  # Texture.swift:74-82, 174-206
        if filterMode != "linear":
            raise ValueError("texture: cube textures currently support filterMode .linear only")
        if tex.ndim != 5 or tex.shape[1] != 6:
            raise ValueError("texture: cube tex must be [N, 6, H, W, C]")
        if uv.ndim != 4 or uv.shape[3] != 3:
            raise ValueError("texture: cube uv must be [N, H_img, W_img, 3]")
        N, Hi, Wi, _ = uv.shape
        Ht, Wt, C = tex.shape[2], tex.shape[3], tex.shape[4]
        texN = c32(np.broadcast_to(tex, (N,) + tex.shape[1:]))
        if g is None:
            out = np.empty((N, Hi, Wi, C), np.float32)
            L.orc_tex_cube_fwd(fp(texN), 6 * Ht * Wt * C, fp(uv), N, Hi, Wi, Ht, Wt, C, fp(out))
            return out
        d_tex = np.zeros((N, 6, Ht, Wt, C), np.float32)
        L.orc_tex_cube_grad_tex(fp(uv), fp(g), N, Hi, Wi, Ht, Wt, C, 6 * Ht * Wt * C,
                                fp(d_tex))
        if tex.shape[0] == 1 and N > 1:
            d_tex = d_tex.sum(axis=0, keepdims=True, dtype=np.float32)
        return d_tex, np.zeros_like(uv), None, None

    if tex.ndim != 4:
        raise ValueError("texture: tex must be [N, H_tex, W_tex, C]")
    if uv.ndim != 4 or uv.shape[3] != 2:
        raise ValueError("texture: uv must be [N, H_img, W_img, 2]")
    N, Hi, Wi, _ = uv.shape
    if tex.shape[0] not in (1, N):
        raise ValueError("texture: tex batch dim incompatible with uv batch")
    Ht, Wt, C = tex.shape[1], tex.shape[2], tex.shape[3]
    texN = c32(np.broadcast_to(tex, (N, Ht, Wt, C)))
    bstride = Ht * Wt * C

    def reduce_tex(d):
        if tex.shape[0] == 1 and N > 1:
            return d.sum(axis=0, keepdims=True, dtype=np.float32)
        return d

    if filterMode == "nearest":
        if g is None:
            out = np.empty((N, Hi, Wi, C), np.float32)
            L.orc_tex_nearest_fwd(fp(texN), bstride, fp(uv), N, Hi, Wi, Ht, Wt, C, b, fp(out))
            return out
        d_tex = np.zeros((N, Ht, Wt, C), np.float32)
        L.orc_tex_nearest_grad_tex(fp(uv), fp(g), N, Hi, Wi, Ht, Wt, C, b, bstride, fp(d_tex))
        return reduce_tex(d_tex), np.zeros_like(uv), None, None

    if filterMode == "linear":
        if g is None:
            out = np.empty((N, Hi, Wi, C), np.float32)
            L.orc_tex_fwd(fp(texN), bstride, fp(uv), N, Hi, Wi, Ht, Wt, C, b, fp(out))
            return out
        d_tex = np.zeros((N, Ht, Wt, C), np.float32)
        L.orc_tex_grad_tex(fp(uv), fp(g), N, Hi, Wi, Ht, Wt, C, b, bstride, fp(d_tex))
        d_uv = np.empty((N, Hi, Wi, 2), np.float32)
        L.orc_tex_grad_uv(fp(texN), bstride, fp(uv), fp(g), N, Hi, Wi, Ht, Wt, C, b, fp(d_uv))
        return reduce_tex(d_tex), d_uv, None, None

    if filterMode not in ("linear-mipmap-linear", "linear-mipmap-nearest"):
        raise ValueError(f"unknown filterMode {filterMode}")
    if uvDA is None:
        raise ValueError("texture: mipmap filterModes require uvDA")
    uvDA = c32(uvDA)
    if uvDA.shape != (N, Hi, Wi, 4):
        raise ValueError("texture: uvDA must be [N, H_img, W_img, 4]")
    mip_linear = 1 if filterMode == "linear-mipmap-linear" else 0
    eff, scale = _bias_fold(uvDA, mipLevelBias, mipLevelBiasMap)
    # Texture.swift:282-307: pyramid of the N-broadcast texture, packed.
    lh, lw = texture_mip_levels(Ht, Wt)
    nl = len(lh)
    offsets, total = _pack_offsets(N, lh, lw, C)
    packed = np.empty(total, np.float32)
    L.orc_mip_build(fp(texN), N, Ht, Wt, C, nl, lp(offsets), fp(packed))
    if g is None:
        out = np.empty((N, Hi, Wi, C), np.float32)
        L.orc_tex_mip_fwd(fp(packed), 1, fp(uv), fp(eff), lp(offsets), ip(lh), ip(lw), nl, N, Hi,
                          Wi, Ht, Wt, C, b, mip_linear, fp(out))
        return out
    d_packed = np.zeros(total, np.float32)
    L.orc_tex_mip_grad_pyramid(fp(uv), fp(eff), fp(g), lp(offsets), ip(lh), ip(lw), nl, 1, N,
                               Hi, Wi, Ht, Wt, C, b, mip_linear, fp(d_packed))
    d_uv = np.empty((N, Hi, Wi, 2), np.float32)
    L.orc_tex_mip_grad_uv(fp(packed), 1, fp(uv), fp(eff), fp(g), lp(offsets), ip(lh), ip(lw),
                          nl, N, Hi, Wi, Ht, Wt, C, b, mip_linear, fp(d_uv))
    d_eff = np.empty((N, Hi, Wi, 4), np.float32)
    L.orc_tex_mip_grad_uvda(fp(packed), 1, fp(uv), fp(eff), fp(g), lp(offsets), ip(lh), ip(lw),
                            nl, N, Hi, Wi, Ht, Wt, C, b, fp(d_eff))
    d_tex = np.empty((N, Ht, Wt, C), np.float32)
    L.orc_mip_collapse(fp(d_packed), N, Ht, Wt, C, nl, lp(offsets), fp(d_tex))
    # Backward of the bias fold (MLX autodiff of uvDA * scale, scale = 2^m).
    d_map = None
    if scale is None:
        d_uvDA = d_eff
    else:
        d_uvDA = c32(d_eff * scale)
        if mipLevelBiasMap is not None:
            gm = (d_eff * uvDA).astype(np.float32).sum(axis=3, keepdims=True, dtype=np.float32)
            d_map = c32(gm * scale * np.float32(np.log(2.0)))
            if np.ndim(mipLevelBiasMap) == 3:
                d_map = d_map[..., 0]
    return reduce_tex(d_tex), d_uv, d_uvDA, d_map


# ---------------------------------------------------------------------------
# antialias (Antialias.swift:19-131, 556-600)
# ---------------------------------------------------------------------------

def antialiasConstructTopologyHash(tri):
    tri = ci32(tri)
    if tri.ndim != 2 or tri.shape[1] != 3:
        raise ValueError("antialiasConstructTopologyHash: tri must be [T, 3]")
    T = tri.shape[0]
    out = np.empty((T, 3), np.int32)
    lib().orc_aa_topology(ip(tri), T, ip(out))
    return out


def _aa_args(color, rast, pos, tri, topologyHash):
    color, rast, pos, tri = c32(color), c32(rast), c32(pos), ci32(tri)
    if color.ndim != 4:
        raise ValueError("antialias: color must be [N, H, W, C]")
    if rast.ndim != 4 or rast.shape[3] != 4 or rast.shape[:3] != color.shape[:3]:
        raise ValueError("antialias: rast must match color in [N, H, W] and have 4 channels")
    if pos.ndim != 3 or pos.shape[2] != 4:
        raise ValueError("antialias: pos must be [N, V, 4]")
    topo = antialiasConstructTopologyHash(tri) if topologyHash is None else ci32(topologyHash)
    return color, rast, pos, tri, topo


def antialias(color, rast, pos, tri, topologyHash=None):
    color, rast, pos, tri, topo = _aa_args(color, rast, pos, tri, topologyHash)
    N, H, W, C = color.shape
    V = pos.shape[1]
    out = np.empty_like(color)
    lib().orc_aa_fwd(fp(color), fp(rast), fp(pos), ip(tri), ip(topo), N, H, W, C, V, fp(out))
    return out


def antialias_vjp(color, rast, pos, tri, d_out, topologyHash=None):
    """VJP closure (Antialias.swift:118-128) -> (d_color, d_pos)."""
    color, rast, pos, tri, topo = _aa_args(color, rast, pos, tri, topologyHash)
    N, H, W, C = color.shape
    V = pos.shape[1]
    L = lib()
    d_color = np.zeros_like(color)
    d_pos = np.zeros_like(pos)
    g = c32(d_out)
    L.orc_aa_bwd_color(fp(rast), fp(pos), ip(tri), ip(topo), fp(g), N, H, W, C, V, fp(d_color))
    L.orc_aa_bwd_pos(fp(color), fp(rast), fp(pos), ip(tri), ip(topo), fp(g), N, H, W, C, V,
                     fp(d_pos))
    return d_color, d_pos


# ---------------------------------------------------------------------------
# loss and optimizer of the inverse-rendering samples
# ---------------------------------------------------------------------------

def mse_loss(out, target):
    """The samples' `lossFn` (ColorFitExample/main.swift:62-66): mean of
    the fp32 squares of (out - target), summed in float64 here.  Returns
    (loss, d_out) with d_out the gradient MLX autodiff forms for it:
    g = (out - target) * (1/n) in fp32, then g + g (the product rule of
    diff * diff)."""
    o = c32(out).ravel()
    t = c32(target).ravel()
    n = o.size
    d = (o - t).astype(np.float32)
    sq = (d * d).astype(np.float32)
    inv_n = np.float32(1.0) / np.float32(n)
    loss = np.float32(np.float32(sq.astype(np.float64).sum()) * inv_n)
    g = (d * inv_n).astype(np.float32)
    return loss, (g + g).astype(np.float32).reshape(np.shape(out))


def _pow_f32(b, t):
    """b**t (b fp32, t a positive integer) correctly rounded to fp32: the
    exact rational power, rounded to the nearest fp32 (ties to even)."""
    from fractions import Fraction
    exact = Fraction(float(b)) ** int(t)
    x = np.float32(float(exact))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - exact)
        key = (err, int(np.frombuffer(np.float32(c).tobytes(), np.uint32)[0]) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def adam_step(param, grad, m, v, t, lr=1e-2, beta1=0.9, beta2=0.999, eps=1e-8, mask=None):
    """One step of `Adam.step` (MLXDiffRastExamples/Adam.swift:36-43) in
    fp32, each operation rounded in the order written there.  t is the step
    count after the increment (1 on the first call).  Returns
    (new_param, new_m, new_v)."""
    f = np.float32
    g = c32(grad)
    if mask is not None:
        g = (g * c32(mask)).astype(f)
    b1, b2, lr, eps = f(beta1), f(beta2), f(lr), f(eps)
    m = (b1 * c32(m) + (f(1) - b1) * g).astype(f)
    v = (b2 * c32(v) + (f(1) - b2) * (g * g)).astype(f)
    c1 = f(1) - _pow_f32(b1, t)
    c2 = f(1) - _pow_f32(b2, t)
    m_hat = (m / c1).astype(f)
    v_hat = (v / c2).astype(f)
    p = (c32(param) - lr * m_hat / (np.sqrt(v_hat) + eps)).astype(f)
    return p, m, v
