"""Benchmark: the reference's five workloads, forward + backward, one GPU.

One "step" is one pass of the workload's chain over its batch, with every
input resident on the GPU before timing starts:

  --config 3 (default, the headline metric): rasterize (with rast_db) ->
      interpolate (UV, all derivatives) -> texture (trilinear mip, clamp) ->
      antialias -> MSE loss against a target image, then the backward to
      pos, the UV attribute and the texture; 8 images of 1024x1024 of a
      level-6 icosphere (40,962 vertices, 81,920 triangles; spherical UVs, a
      random rotation per image, fov 45 degrees, radius 1 at distance 3) and
      a 1024x1024 RGBA fp32 value-noise texture.
  --config 1: one triangle, 256x256: rasterize -> interpolate (RGB) -> MSE,
      backward to the attribute.
  --config 2: hexagonal pie (7 vertices, 6 triangles), 4 x 512x512:
      rasterize -> interpolate -> antialias -> MSE, backward to pos and the
      colour attribute.
  --config 4: displaced level-8 icosphere (655,362 vertices, 1,310,720
      triangles), 16 x 2048x2048: four depth-peeling layers, each
      interpolated (normal + RGB), backward from fixed cotangents to the
      attribute and through every layer's rasterize to pos.
  --config 5: 4096 meshes of 512 random triangles in one [V,4] buffer (range
      mode), 256x256 each: rasterize (with rast_db) -> interpolate (a
      direction and its screen derivatives) -> cube-map texture (6 x 512^2
      x 3, trilinear, per-pixel bias map, direction gradient), backward from
      fixed cotangents to the cube map, the directions and pos.

Options: `--graph` times replays of one step captured into a HIP graph
(the warm-up runs on the capturing stream); `--max-per-tile 128` rasterizes
with the reference's per-tile limit.  Prints one JSON line.  `--gpus N`
with N > 1 is not supported (one GPU).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "mlx-swift-diffrast_amd"), os.path.join(ROOT, "tests"),
          os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

METRIC = "fwd+bwd Mpix/s (8×1024², 80k tris, full chain); % HBM roofline"
HBM_PEAK = 8.0e12  # bytes/s, MI355X


def copy_calibration(mib=256, reps=3):
    """A plain device copy of known size (elementwise y = x * 1), launched
    before the workload so a counter run over this command also measures
    what FETCH_SIZE / WRITE_SIZE read for exactly `mib` MiB in and out."""
    import torch
    x = torch.rand(mib << 18, device="cuda")
    y = torch.empty_like(x)
    for _ in range(reps):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    del x, y


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run
    on, capped by OMP_NUM_THREADS when the host sets it (a one-GPU box
    allots its share of cores that way)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
# workloads: build the inputs, the GPU step, the algorithmic bytes per step
# of each kernel (name of its timing scope -> bytes) and of the chain, and
# the CPU baseline on a bounded sample
# ---------------------------------------------------------------------------

class Workload:
    name = ""
    images = 0
    height = width = 0
    triangles = 0  # drawn per step, over all images
    # rasterize's maxPerTile: 0 keeps every triangle (this build's default);
    # 128 is the reference's per-tile limit (Rasterize.swift:164-171)
    max_per_tile = 0

    def config(self):
        raise NotImplementedError

    def setup(self):
        raise NotImplementedError

    def step(self):
        raise NotImplementedError

    def kernel_bytes(self):
        """{timing-scope name: algorithmic HBM bytes per step} for the
        memory-bound kernels (per-pixel reads and writes of the op's
        inputs and outputs, plus fixed per-call bytes)."""
        return {}

    def chain_bytes(self):
        return sum(self.kernel_bytes().values())

    def cpu_baseline(self, threads):
        raise NotImplementedError


def _dev(a, grad=False):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(a)).cuda()
    return t.requires_grad_(True) if grad else t


def _mse_backward(out, target, loss, lib, _lib):
    """MSE loss and its gradient 2/n (out - target) in one kernel, then the
    backward from it."""
    import torch
    from diffrast.ops import _stream
    d_out = torch.empty_like(out)
    _lib.check(lib.dr_mse_loss(out.data_ptr(), target.data_ptr(), out.numel(), loss.data_ptr(),
                               d_out.data_ptr(), _stream()))
    out.backward(d_out)


class Tier1(Workload):
    name, images, height, width, triangles = "tier-1 colour fit fwd+bwd", 1, 256, 256, 1

    def config(self):
        return {"workload": self.name, "images": 1, "height": 256, "width": 256, "triangles": 1,
                "attributes": "RGB", "loss": "MSE", "grads": "d_attr"}

    def setup(self):
        import scenes
        import torch
        from diffrast import DiffRast, _lib
        self.sc = sc = scenes.tier1_triangle(H=256, W=256)
        self.pos, self.tri = _dev(sc["pos"]), _dev(sc["tri"])
        self.attr = _dev(sc["attr"], grad=True)
        r, _ = DiffRast.rasterize(self.pos, self.tri, (256, 256), gradDB=False,
                                  maxPerTile=self.max_per_tile)
        self.target = DiffRast.interpolate(_dev(sc["target_attr"]), r, self.tri)[0].detach()
        self.loss = torch.empty((), device="cuda")
        self.lib, self._lib = _lib.load(), _lib

    def step(self):
        from diffrast import DiffRast
        self.attr.grad = None
        rast, _ = DiffRast.rasterize(self.pos, self.tri, (256, 256), gradDB=False,
                                     maxPerTile=self.max_per_tile)
        out, _ = DiffRast.interpolate(self.attr, rast, self.tri)
        _mse_backward(out, self.target, self.loss, self.lib, self._lib)
        return self.loss

    def kernel_bytes(self):
        P = 256 * 256
        return {"k_raster": 16 * P, "k_interp_fwd": (16 + 12) * P,
                "k_interp_bwd": (16 + 12 + 16) * P}

    def cpu_baseline(self, threads):
        import oracle as O
        sc = self.sc
        mpt = self.max_per_tile
        target, _ = O.interpolate(sc["target_attr"], O.rasterize(sc["pos"], sc["tri"], (256, 256),
                                                                 gradDB=False, max_per_tile=mpt)[0],
                                  sc["tri"])

        def run():
            rast, _ = O.rasterize(sc["pos"], sc["tri"], (256, 256), gradDB=False, max_per_tile=mpt)
            out, _ = O.interpolate(sc["attr"], rast, sc["tri"])
            g = ((2.0 / out.size) * (out - target)).astype(np.float32)
            O.interpolate_vjp(sc["attr"], rast, sc["tri"], g)
        return _time_cpu(run, 256 * 256, threads, "the whole workload (1 image, 256x256)")


class HexPie(Workload):
    name, images, height, width, triangles = "hexagonal pie chain fwd+bwd", 4, 512, 512, 4 * 6

    def config(self):
        return {"workload": self.name, "images": 4, "height": 512, "width": 512, "vertices": 7,
                "triangles": 6, "loss": "MSE", "grads": "d_pos, d_attr"}

    def setup(self):
        import scenes
        import torch
        from diffrast import DiffRast, _lib
        self.sc = sc = scenes.hex_pie(N=4, H=512, W=512)
        self.pos, self.tri = _dev(sc["pos"], grad=True), _dev(sc["tri"])
        self.attr, self.target = _dev(sc["attr"], grad=True), _dev(sc["target"])
        self.topo = DiffRast.antialiasConstructTopologyHash(self.tri)
        self.loss = torch.empty((), device="cuda")
        self.lib, self._lib = _lib.load(), _lib

    def step(self):
        from diffrast import DiffRast
        self.pos.grad = self.attr.grad = None
        rast, _ = DiffRast.rasterize(self.pos, self.tri, (512, 512), gradDB=False,
                                     maxPerTile=self.max_per_tile)
        col, _ = DiffRast.interpolate(self.attr, rast, self.tri)
        out = DiffRast.antialias(col, rast, self.pos, self.tri, topologyHash=self.topo)
        _mse_backward(out, self.target, self.loss, self.lib, self._lib)
        return self.loss

    def kernel_bytes(self):
        P = 4 * 512 * 512
        return {"k_raster": 16 * P, "k_interp_fwd": (16 + 12) * P, "k_aa_fwd": (12 + 16 + 12) * P,
                "k_aa_bwd": (12 + 12 + 16 + 12) * P, "k_interp_bwd": (16 + 12 + 16) * P,
                "k_raster_bwd": (16 + 16) * P}

    def cpu_baseline(self, threads):
        import oracle as O
        sc = self.sc
        pos, tri, attr, target = sc["pos"][:1], sc["tri"], sc["attr"], sc["target"][:1]
        topo = O.antialiasConstructTopologyHash(tri)

        def run():
            rast, _ = O.rasterize(pos, tri, (512, 512), gradDB=False,
                                  max_per_tile=self.max_per_tile)
            col, _ = O.interpolate(attr, rast, tri)
            out = O.antialias(col, rast, pos, tri, topo)
            g = ((2.0 / (4 * out.size)) * (out - target)).astype(np.float32)
            d_col, _ = O.antialias_vjp(col, rast, pos, tri, g, topo)
            _, d_rast, _ = O.interpolate_vjp(attr, rast, tri, d_col)
            O.rasterize_vjp(pos, tri, rast, d_rast)
        return _time_cpu(run, 512 * 512, threads, "1 of 4 images (512x512), full chain fwd+bwd")


class Icosphere(Workload):
    name, images, height, width = "textured icosphere full chain fwd+bwd", 8, 1024, 1024
    triangles = 8 * 81920

    def config(self):
        return {"workload": self.name, "images": 8, "height": 1024, "width": 1024,
                "vertices": 40962, "triangles": 81920,
                "texture": "1024x1024x4 f32, 11 mip levels, clamp, linear-mipmap-linear"}

    def setup(self):
        import scenes
        import torch
        from diffrast import DiffRast, _lib
        self.sc = sc = scenes.textured_icosphere(N=8, H=1024, W=1024, level=6, tex_size=1024)
        self.pos, self.tri = _dev(sc["pos"], grad=True), _dev(sc["tri"])
        self.attr = _dev(sc["uv"], grad=True)      # shared [V,2]
        self.tex = _dev(sc["tex"], grad=True)      # shared [1,Ht,Wt,4]
        self.target = _dev(sc["target"])
        self.topo = DiffRast.antialiasConstructTopologyHash(self.tri)
        self.loss = torch.empty((), device="cuda")
        self.lib, self._lib = _lib.load(), _lib

    def step(self):
        from diffrast import DiffRast
        self.pos.grad = self.attr.grad = self.tex.grad = None
        rast, rast_db = DiffRast.rasterize(self.pos, self.tri, (1024, 1024), gradDB=True,
                                           maxPerTile=self.max_per_tile)
        uv, uv_da = DiffRast.interpolate(self.attr, rast, self.tri, rastDB=rast_db,
                                         diffAttrs="all")
        col = DiffRast.texture(self.tex, uv, uvDA=uv_da, filterMode="linear-mipmap-linear",
                               boundaryMode="clamp")
        out = DiffRast.antialias(col, rast, self.pos, self.tri, topologyHash=self.topo)
        _mse_backward(out, self.target, self.loss, self.lib, self._lib)
        return self.loss

    def kernel_bytes(self):
        P, V = 8 * 1024 * 1024, 40962
        pyr = 22.4e6  # the 1024^2 RGBA texture and its levels
        return {"k_raster": 32 * P, "k_interp_fwd": 56 * P, "k_tex_fwd": 40 * P + pyr,
                "k_aa_fwd": 48 * P, "k_aa_bwd": 64 * P, "k_tex_bwd": 64 * P + 2 * pyr,
                "k_interp_bwd": 88 * P + 2 * V * 8, "k_raster_bwd": 48 * P + 2 * 8 * V * 16}

    def chain_bytes(self):
        # 440 B per pixel (176 forward, 264 backward: each op reads its inputs
        # and writes its outputs once) plus ~140 MB per step of pyramid
        # build and reads, the pyramid gradient and its collapse, pos/d_pos
        # and the mesh tables; the MSE loss's 48 B/px are not counted
        return 440 * 8 * 1024 * 1024 + 140e6

    def cpu_baseline(self, threads):
        import oracle as O
        sc = self.sc
        pos = sc["pos"][:1]
        tri, uva, tex = sc["tri"], sc["uv"], sc["tex"]
        topo = O.antialiasConstructTopologyHash(tri)

        def run():
            rast, db = O.rasterize(pos, tri, (1024, 1024), max_per_tile=self.max_per_tile)
            uv, uvda = O.interpolate(uva, rast, tri, rastDB=db, diffAttrs="all")
            col = O.texture(tex, uv, uvDA=uvda, filterMode="linear-mipmap-linear",
                            boundaryMode="clamp")
            out = O.antialias(col, rast, pos, tri, topo)
            g = (2.0 / (8 * out.size)) * (out - sc["target"][:1])
            d_col, _ = O.antialias_vjp(col, rast, pos, tri, g, topo)
            _, d_uv, d_uvda, _ = O.texture_vjp(tex, uv, d_col, uvDA=uvda,
                                               filterMode="linear-mipmap-linear",
                                               boundaryMode="clamp")
            _, d_rast, d_db = O.interpolate_vjp(uva, rast, tri, d_uv, rastDB=db, diffAttrs="all",
                                                d_out_da=d_uvda)
            O.rasterize_vjp(pos, tri, rast, d_rast, d_db)
        return _time_cpu(run, 1024 * 1024, threads,
                         "1 of 8 images (1024x1024), full chain fwd+bwd")


class DisplacedSphere(Workload):
    name, images, height, width = "displaced sphere 4-layer peel fwd+bwd", 16, 2048, 2048
    triangles = 16 * 1310720
    layers = 4

    def config(self):
        return {"workload": self.name, "images": 16, "height": 2048, "width": 2048,
                "vertices": 655362, "triangles": 1310720, "peel_layers": 4,
                "attributes": "normal + RGB", "grads": "d_attr, d_pos (fixed cotangents)"}

    def setup(self):
        import scenes
        import torch
        self.sc = sc = scenes.displaced_sphere(N=16, H=2048, W=2048, level=8)
        self.pos, self.tri = _dev(sc["pos"], grad=True), _dev(sc["tri"])
        self.attr = _dev(sc["attr"], grad=True)    # shared [1,V,6]
        g = torch.Generator(device="cuda").manual_seed(4)
        self.gs = [torch.randn((16, 2048, 2048, 6), device="cuda", generator=g) * 1e-3
                   for _ in range(self.layers)]

    def step(self):
        import torch
        from diffrast import DiffRast
        self.pos.grad = self.attr.grad = None
        prev, outs = None, []
        for _ in range(self.layers):
            r, _ = DiffRast.rasterize(self.pos, self.tri, (2048, 2048), gradDB=False,
                                      peelLayer=prev, maxPerTile=self.max_per_tile)
            out, _ = DiffRast.interpolate(self.attr, r, self.tri)
            outs.append(out)
            prev = r.detach()
        torch.autograd.backward(outs, self.gs)
        return outs[0]

    def kernel_bytes(self):
        P, L, V, T = 16 * 2048 * 2048, self.layers, 655362, 1310720
        return {"k_raster": (16 * L + 16 * (L - 1)) * P,   # write rast; read the layer above
                "k_interp_fwd": L * (16 + 24) * P, "k_interp_bwd": L * (16 + 24 + 16) * P,
                # read rast and d_rast; read pos and the triangle table
                "k_raster_bwd": L * (32 * P + 16 * 16 * V + 12 * T)}

    def chain_bytes(self):
        P, L, V, T = 16 * 2048 * 2048, self.layers, 655362, 1310720
        per_px = 16 * L + 16 * (L - 1) + L * (16 + 24) + L * (16 + 24 + 16) + L * 32
        # pos and the triangle table read by each layer's setup and
        # backward, d_pos written once, attr / d_attr
        fixed = L * (16 * V * 16 + 12 * T) * 2 + 16 * V * 16 + 2 * V * 24
        return per_px * P + fixed

    def cpu_baseline(self, threads):
        import oracle as O
        sc = self.sc
        pos, tri, attr = sc["pos"][:1], sc["tri"], sc["attr"]
        g = np.full((1, 2048, 2048, 6), 1e-3, np.float32)

        def run():
            prev = None
            for _ in range(self.layers):
                r, _ = O.rasterize(pos, tri, (2048, 2048), gradDB=False, peelLayer=prev,
                                   max_per_tile=self.max_per_tile)
                O.interpolate(attr, r, tri)
                _, d_rast, _ = O.interpolate_vjp(attr, r, tri, g)
                O.rasterize_vjp(pos, tri, r, d_rast)
                prev = r
        return _time_cpu(run, 2048 * 2048, threads,
                         "1 of 16 images (2048x2048, all 1.31M triangles), 4 layers fwd+bwd",
                         max_reps=2)


class RangeCube(Workload):
    name, images, height, width = "range-mode cube-map batch fwd+bwd", 4096, 256, 256
    triangles = 4096 * 512

    def config(self):
        return {"workload": self.name, "images": 4096, "height": 256, "width": 256,
                "triangles_per_image": 512, "mode": "ranges over one [V,4] buffer",
                "texture": "cube 6x512x512x3 f32, linear-mipmap-linear, per-pixel bias map",
                "grads": "d_cube, d_dir (direction gradient), d_pos (fixed cotangents)"}

    def setup(self):
        import scenes
        import torch
        self.sc = sc = scenes.range_batch(N=4096, T_per=512, H=256, W=256)
        rng = np.random.default_rng(9)
        self.cube_np = rng.random((1, 6, 512, 512, 3)).astype(np.float32)
        self.bias_np = rng.uniform(-1, 1, size=(4096, 256, 256)).astype(np.float32)
        self.pos, self.tri = _dev(sc["pos"], grad=True), _dev(sc["tri"])
        self.dir = _dev(sc["dir"], grad=True)
        self.cube, self.bias = _dev(self.cube_np, grad=True), _dev(self.bias_np)
        self.ranges = torch.as_tensor(sc["ranges"])
        hw = (np.arange(256, dtype=np.float32) + 0.5) / 256
        env = np.stack([np.ones((256, 256), np.float32), np.repeat(1 - 2 * hw[:, None], 256, 1),
                        np.repeat(1 - 2 * hw[None, :], 256, 0)], -1)
        self.env = _dev(env)
        g = torch.Generator(device="cuda").manual_seed(5)
        self.g = torch.randn((4096, 256, 256, 3), device="cuda", generator=g) * 1e-3

    def _chain(self, DiffRast, pos, tri, dirs_attr, cube, bias, ranges, env):
        rast, db = DiffRast.rasterize(pos, tri, (256, 256), gradDB=True, ranges=ranges,
                                      maxPerTile=self.max_per_tile)
        dirs, dirs_da = DiffRast.interpolate(dirs_attr, rast, tri, rastDB=db, diffAttrs="all")
        # empty pixels interpolate to the zero vector, which has no cube face
        # (NaN in the reference too): they look up an environment direction
        dirs = dirs + (rast[..., 3:4] == 0).float() * env
        return DiffRast.texture(cube, dirs, uvDA=dirs_da, filterMode="linear-mipmap-linear",
                                boundaryMode="cube", mipLevelBiasMap=bias, dirGrad=True)

    def step(self):
        from diffrast import DiffRast
        self.pos.grad = self.dir.grad = self.cube.grad = None
        col = self._chain(DiffRast, self.pos, self.tri, self.dir, self.cube, self.bias,
                          self.ranges, self.env)
        col.backward(self.g)
        return col

    def kernel_bytes(self):
        P = 4096 * 256 * 256
        return {"k_raster": 32 * P, "k_interp_fwd": (32 + 12 + 24) * P,
                "k_cube_fwd": (12 + 24 + 4 + 12) * P, "k_cube_bwd": (12 + 24 + 4 + 12 + 12 + 24 + 4) * P,
                "k_interp_bwd": (32 + 12 + 24 + 32) * P, "k_raster_bwd": 48 * P}

    def chain_bytes(self):
        P, V = 4096 * 256 * 256, 4096 * 512 * 3
        # the ops' per-pixel reads and writes, the background fill (rast id,
        # dirs in and out), pos / d_pos and the direction table both ways
        return sum(self.kernel_bytes().values()) + (4 + 24) * P + 2 * 16 * V + 2 * 12 * V

    def cpu_baseline(self, threads):
        import oracle as O
        sc = self.sc
        nm = 16
        nt, nv = nm * 512, nm * 512 * 3
        pos, tri, d, ranges = sc["pos"][:nv], sc["tri"][:nt], sc["dir"][:nv], sc["ranges"][:nm]
        hw = (np.arange(256, dtype=np.float32) + 0.5) / 256
        env = np.stack([np.ones((256, 256), np.float32), np.repeat(1 - 2 * hw[:, None], 256, 1),
                        np.repeat(1 - 2 * hw[None, :], 256, 0)], -1)
        g = np.full((nm, 256, 256, 3), 1e-3, np.float32)
        kw = dict(filterMode="linear-mipmap-linear", boundaryMode="cube",
                  mipLevelBiasMap=self.bias_np[:nm])

        def run():
            rast, db = O.rasterize(pos, tri, (256, 256), gradDB=True, ranges=ranges,
                                   max_per_tile=self.max_per_tile)
            dirs, dda = O.interpolate(d, rast, tri, rastDB=db, diffAttrs="all")
            dirs = dirs + (rast[..., 3:4] == 0).astype(np.float32) * env
            O.texture(self.cube_np, dirs, uvDA=dda, **kw)
            _, d_dir, d_dda, _ = O.texture_vjp(self.cube_np, dirs, g, uvDA=dda, dirGrad=True, **kw)
            _, d_rast, d_db = O.interpolate_vjp(d, rast, tri, d_dir, rastDB=db, diffAttrs="all",
                                                d_out_da=d_dda)
            O.rasterize_vjp(pos, tri, rast, d_rast, d_db, ranges=ranges)
        return _time_cpu(run, nm * 256 * 256, threads,
                         f"{nm} of 4096 meshes (256x256 each), full chain fwd+bwd")


WORKLOADS = {1: Tier1, 2: HexPie, 3: Icosphere, 4: DisplacedSphere, 5: RangeCube}


def _time_cpu(run, pixels, threads, what, budget_s=12.0, max_reps=40):
    """The oracle (the CPU restatement of the reference) on a bounded sample
    of the workload, OpenMP over `threads` host threads."""
    import oracle as O
    O.set_threads(threads)
    reps, total = 0, 0.0
    while reps == 0 or (total < budget_s and reps < max_reps):
        t0 = time.perf_counter()
        run()
        total += time.perf_counter() - t0
        reps += 1
    O.set_threads(1)
    per = total / reps
    return {"value": round(pixels / per / 1e6, 3), "unit": "Mpix/s", "cores": threads,
            "kind": "port", "cpu": cpu_model(),
            "sample": f"{what}, {reps} rep(s), {per:.3f} s each"}


def gpu_run(wl, steps, warmup, graph=False):
    """Warm-up, an untimed per-kernel breakdown, then `steps` timed steps:
    eager calls, or (graph) replays of one step captured into a HIP graph
    (torch.cuda.graph over the op wrappers, on the stream the warm-up ran
    on, so the library's scratch for it is sized before capture)."""
    import torch
    from diffrast import _lib

    if graph:
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            return _gpu_run(wl, steps, warmup, s)
    return _gpu_run(wl, steps, warmup, None)


def _gpu_run(wl, steps, warmup, graph_stream):
    import torch
    from diffrast import _lib

    prof = _lib.load()
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    # Per-kernel breakdown (every launch bracketed by HIP events), untimed.
    prof.dr_profile_select(None)
    prof.dr_profile_reset()
    prof.dr_profile_enable(1)
    n_break = 3
    for _ in range(n_break):
        wl.step()
    torch.cuda.synchronize()
    prof.dr_profile_enable(0)
    rep = _lib.profile_report()
    breakdown = {k: v["total_ms"] / n_break for k, v in rep.items()}
    launches = {k: v["count"] // n_break for k, v in rep.items()}
    dominant = max(breakdown, key=breakdown.get)
    if graph_stream is not None:
        # one step captured; the timed region replays it (no events inside a
        # graph: the dominant kernel's time is the breakdown's)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=graph_stream):
            res = wl.step()
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dom = {"count": n_break * launches[dominant], "total_ms": breakdown[dominant] * n_break}
        assert bool(torch.isfinite(res).all().item())
        return (t1 - t0) * 1e3 / steps, dominant, dom, breakdown, launches
    # Timed region: only the dominant kernel carries events, on its stream.
    prof.dr_profile_select(dominant.encode())
    prof.dr_profile_reset()
    prof.dr_profile_enable(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        res = wl.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    prof.dr_profile_enable(0)
    dom = _lib.profile_report().get(dominant, {"count": 0, "total_ms": 0.0})
    prof.dr_profile_select(None)
    assert bool(torch.isfinite(res).all().item())
    return (t1 - t0) * 1e3 / steps, dominant, dom, breakdown, launches


def measured_traffic(kernel, cfg):
    """HBM bytes per launch of `kernel` at the 8 x 1024^2 workload, from the
    committed counter summary (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
    passes over this script, scaled by what the same counters read for a
    copy of known size).  None for other workloads or kernels."""
    path = os.path.join(ROOT, "profiles", "chain_8x1024_hbm_traffic.json")
    if cfg != 3 or not os.path.exists(path):
        return None
    with open(path) as f:
        table = json.load(f)["kernels"]
    for name, rec in table.items():
        if name.startswith(kernel):
            return int(rec["traffic_bytes"])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=sorted(WORKLOADS),
                    help="which of the reference's five workloads (3: the headline metric)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of one step captured into a HIP graph")
    ap.add_argument("--max-per-tile", type=int, default=0,
                    help="rasterize with the reference's per-tile triangle limit (128 in the "
                         "reference; 0, the default, keeps every triangle)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a 256 MiB copy kernel (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)

    wl = WORKLOADS[args.config]()
    wl.max_per_tile = args.max_per_tile
    wl.setup()
    if args.calibrate_copy:
        copy_calibration()
    ms, dom_name, dom, breakdown, launches = gpu_run(wl, args.steps, args.warmup, args.graph)
    P = wl.images * wl.height * wl.width
    kb = wl.kernel_bytes()
    if "k_raster" in kb:  # the forward runs as k_raster_px for large triangles
        kb["k_raster_px"] = kb["k_raster"]

    # Dominant kernel: its launches in the timed region carry HIP events on
    # the stream it runs on; roofline against HBM on its algorithmic bytes.
    roofline = None
    if dom["count"] and dom_name in kb:
        avg_ms = dom["total_ms"] / dom["count"]
        per_launch = kb[dom_name] / max(1, launches.get(dom_name, 1))
        ach = per_launch / (avg_ms * 1e-3)
        roofline = {"bound": "hbm", "achieved": round(ach / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK, 4),
                    "traffic": measured_traffic(dom_name, args.config),
                    "kernel": dom_name, "avg_ms": round(avg_ms, 4),
                    "algorithmic_bytes": int(per_launch)}
    if roofline is None:
        roofline = {"bound": "hbm", "achieved": None, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                    "frac": None, "traffic": None, "kernel": dom_name}
    chain = wl.chain_bytes()
    roofline["chain_bytes"] = int(chain)
    roofline["chain_frac"] = round(chain / (ms * 1e-3) / HBM_PEAK, 4)
    roofline["pass_frac"] = {k: round(kb[k] / (breakdown[k] * 1e-3) / HBM_PEAK, 4)
                             for k in sorted(kb) if breakdown.get(k)}

    line = {
        "metric": METRIC if args.config == 3 else
        f"fwd+bwd Mpix/s (config {args.config}: {wl.name}); % HBM roofline",
        "value": round(P / (ms * 1e-3) / 1e6, 2), "unit": "Mpix/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded scenes of the reference's workload shapes)",
        "config": dict(wl.config(), **({"max_per_tile": wl.max_per_tile} if wl.max_per_tile
                                           else {}), **({"hip_graph": True} if args.graph else {})),
        "us_per_step": round(ms * 1e3, 1),
        "tris_per_s": round(wl.triangles / (ms * 1e-3), 1),
        "roofline": roofline,
        "kernels_ms_per_step": {k: round(v, 4) for k, v in
                                sorted(breakdown.items(), key=lambda kv: -kv[1])},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = wl.cpu_baseline(cpu_threads())
    print(json.dumps(line))


if __name__ == "__main__":
    main()
