"""MI355X-native differentiable rasterization: rasterize, interpolate,
texture and antialias (forward and backward) as hand-written gfx950 HIP
kernels behind a C ABI, with the `DiffRast` API of mlx-swift-diffrast."""
from .ops import (BoundaryMode, DiffAttrs, DiffRast, FilterMode, antialias,
                  antialiasConstructTopologyHash, interpolate, rasterize, texture,
                  textureConstructMip)
from ._lib import LIB_PATH, load

__all__ = ["DiffRast", "BoundaryMode", "FilterMode", "DiffAttrs", "rasterize", "interpolate",
           "texture", "textureConstructMip", "antialiasConstructTopologyHash", "antialias",
           "load", "LIB_PATH"]
