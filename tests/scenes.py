"""Seeded synthetic workloads for the parity tests and the benchmark.

Each builder returns plain numpy arrays (float32 / int32) in the reference's
layouts.  Seeds default to the workload index, so the GPU run and the CPU
baseline see identical inputs.
"""
from __future__ import annotations

import math

import numpy as np


def icosphere(level: int):
    """Unit icosphere: V = 10*4^level + 2 vertices, T = 20*4^level faces,
    counter-clockwise seen from outside."""
    t = (1.0 + 5.0 ** 0.5) / 2.0
    v = np.array([[-1, t, 0], [1, t, 0], [-1, -t, 0], [1, -t, 0],
                  [0, -1, t], [0, 1, t], [0, -1, -t], [0, 1, -t],
                  [t, 0, -1], [t, 0, 1], [-t, 0, -1], [-t, 0, 1]], np.float64)
    f = np.array([[0, 11, 5], [0, 5, 1], [0, 1, 7], [0, 7, 10], [0, 10, 11],
                  [1, 5, 9], [5, 11, 4], [11, 10, 2], [10, 7, 6], [7, 1, 8],
                  [3, 9, 4], [3, 4, 2], [3, 2, 6], [3, 6, 8], [3, 8, 9],
                  [4, 9, 5], [2, 4, 11], [6, 2, 10], [8, 6, 7], [9, 8, 1]], np.int64)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    for _ in range(level):
        e = np.concatenate([f[:, [0, 1]], f[:, [1, 2]], f[:, [2, 0]]], axis=0)
        e.sort(axis=1)
        key = e[:, 0] * (1 << 32) + e[:, 1]
        uk, inv = np.unique(key, return_inverse=True)
        a, b = uk >> 32, uk & 0xFFFFFFFF
        mid = v[a] + v[b]
        mid /= np.linalg.norm(mid, axis=1, keepdims=True)
        base = v.shape[0]
        v = np.concatenate([v, mid], axis=0)
        F = f.shape[0]
        m01 = base + inv[0:F]
        m12 = base + inv[F:2 * F]
        m20 = base + inv[2 * F:3 * F]
        f = np.concatenate([
            np.stack([f[:, 0], m01, m20], 1),
            np.stack([f[:, 1], m12, m01], 1),
            np.stack([f[:, 2], m20, m12], 1),
            np.stack([m01, m12, m20], 1)], axis=0)
    return v.astype(np.float64), f.astype(np.int32)


def random_rotations(n: int, rng: np.random.Generator):
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    w, x, y, z = q.T
    R = np.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
        2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
        2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], axis=1)
    return R.reshape(n, 3, 3)


def perspective(fov_deg=45.0, near=1.0, far=10.0):
    f = 1.0 / math.tan(math.radians(fov_deg) / 2)
    return np.array([[f, 0, 0, 0],
                     [0, f, 0, 0],
                     [0, 0, (far + near) / (near - far), 2 * far * near / (near - far)],
                     [0, 0, -1, 0]], np.float64)


def spherical_uv(v):
    u = 0.5 + np.arctan2(v[:, 2], v[:, 0]) / (2 * np.pi)
    w = 0.5 - np.arcsin(np.clip(v[:, 1], -1, 1)) / np.pi
    return np.stack([u, w], 1).astype(np.float32)


def value_noise(H, W, C, rng, octaves=(8, 32, 128)):
    """Sum of bilinearly upsampled random grids (seeded value noise)."""
    out = np.zeros((H, W, C), np.float64)
    amp = 1.0
    for g in octaves:
        grid = rng.random((g + 1, g + 1, C))
        ys = np.linspace(0, g, H, endpoint=False) + 0.5 * g / H
        xs = np.linspace(0, g, W, endpoint=False) + 0.5 * g / W
        y0 = np.floor(ys).astype(int)
        x0 = np.floor(xs).astype(int)
        fy = (ys - y0)[:, None, None]
        fx = (xs - x0)[None, :, None]
        y1 = np.minimum(y0 + 1, g)
        x1 = np.minimum(x0 + 1, g)
        a = grid[y0][:, x0]
        b = grid[y0][:, x1]
        c = grid[y1][:, x0]
        d = grid[y1][:, x1]
        out += amp * ((1 - fy) * ((1 - fx) * a + fx * b) + fy * ((1 - fx) * c + fx * d))
        amp *= 0.5
    out /= out.max()
    return out.astype(np.float32)


def project(verts, R, dist=3.0):
    """verts [V,3] -> clip-space pos [N,V,4] for rotations R [N,3,3]."""
    P = perspective()
    cam = np.einsum("nij,vj->nvi", R, verts)
    cam[..., 2] -= dist
    h = np.concatenate([cam, np.ones(cam.shape[:2] + (1,))], axis=2)
    return np.einsum("ij,nvj->nvi", P, h).astype(np.float32)


def tier1_triangle(seed=0, H=256, W=256):
    """One triangle, x,y ~ U[-0.8,0.8], z=0.5, w=1; RGB attributes; N=1."""
    rng = np.random.default_rng(seed)
    xy = rng.uniform(-0.8, 0.8, size=(3, 2))
    pos = np.concatenate([xy, np.full((3, 1), 0.5), np.ones((3, 1))], 1)[None].astype(np.float32)
    tri = np.array([[0, 1, 2]], np.int32)
    attr = rng.random((1, 3, 3)).astype(np.float32)
    target_attr = rng.random((1, 3, 3)).astype(np.float32)
    return dict(pos=pos, tri=tri, attr=attr, target_attr=target_attr, H=H, W=W)


def hex_pie(seed=1, N=4, H=512, W=512, radius=0.6, jitter=0.02):
    """Centre + 6 ring vertices, 6 fan triangles (MeshFitExample layout)."""
    rng = np.random.default_rng(seed)
    ang = np.arange(6) * np.pi / 3
    base = np.concatenate([[[0.0, 0.0]], np.stack([radius * np.cos(ang), radius * np.sin(ang)], 1)])
    xy = base[None] + rng.normal(scale=jitter, size=(N, 7, 2))
    pos = np.concatenate([xy, np.zeros((N, 7, 1)), np.ones((N, 7, 1))], 2).astype(np.float32)
    tri = np.array([[0, 1, 2], [0, 2, 3], [0, 3, 4], [0, 4, 5], [0, 5, 6], [0, 6, 1]], np.int32)
    attr = rng.random((1, 7, 3)).astype(np.float32)
    target = rng.random((N, H, W, 3)).astype(np.float32)
    return dict(pos=pos, tri=tri, attr=attr, target=target, H=H, W=W)


def textured_icosphere(seed=2, N=8, H=1024, W=1024, level=6, tex_size=1024):
    """Icosphere, spherical UV, random rotation per image, fov 45, radius 1 at
    distance 3 (z in [2, 4]); RGBA value-noise texture."""
    rng = np.random.default_rng(seed)
    verts, tri = icosphere(level)
    uv = spherical_uv(verts)
    R = random_rotations(N, rng)
    pos = project(verts, R)
    tex = value_noise(tex_size, tex_size, 4, rng)[None]
    target = rng.random((N, H, W, 4)).astype(np.float32)
    return dict(pos=pos, tri=tri, uv=uv, tex=tex, target=target, H=H, W=W)


def displaced_sphere(seed=3, N=16, H=2048, W=2048, level=8, amp=0.1):
    """Icosphere with seeded radial displacement; attributes normal + RGB."""
    rng = np.random.default_rng(seed)
    verts, tri = icosphere(level)
    k = rng.normal(size=(8, 3)) * 3.0
    ph = rng.uniform(0, 2 * np.pi, size=8)
    disp = np.sin(verts @ k.T + ph).mean(axis=1)
    v = verts * (1.0 + amp * disp)[:, None]
    fn = np.cross(v[tri[:, 1]] - v[tri[:, 0]], v[tri[:, 2]] - v[tri[:, 0]])
    vn = np.zeros_like(v)
    for j in range(3):
        np.add.at(vn, tri[:, j], fn)
    vn /= np.linalg.norm(vn, axis=1, keepdims=True)
    rgb = rng.random((v.shape[0], 3))
    attr = np.concatenate([vn, rgb], 1)[None].astype(np.float32)
    R = random_rotations(N, rng)
    pos = project(v, R)
    return dict(pos=pos, tri=tri, attr=attr, H=H, W=W)


def range_batch(seed=4, N=4096, T_per=512, H=256, W=256):
    """N independent meshes of T_per random triangles (vertices U[-1,1]^3,
    w=1) in one shared [V,4] buffer, selected by ranges."""
    rng = np.random.default_rng(seed)
    V = N * T_per * 3
    xyz = rng.uniform(-1, 1, size=(V, 3)).astype(np.float32)
    pos = np.concatenate([xyz, np.ones((V, 1), np.float32)], 1)
    tri = np.arange(V, dtype=np.int32).reshape(-1, 3)
    ranges = np.stack([np.arange(N) * T_per, np.full(N, T_per)], 1).astype(np.int32)
    d = rng.normal(size=(V, 3)).astype(np.float32)
    return dict(pos=pos, tri=tri, ranges=ranges, dir=d, H=H, W=W)


def straight_edges(H=64, W=64):
    """Four images, one triangle each, whose only on-screen edge is a
    straight line (the other two edges lie off screen).  Images 0 and 1
    cross every pixel row at x_e = x0 + s (row + 0.5) (s = 1/4 with the
    triangle on the left, s = -1/8 with it on the right); images 2 and 3 are
    the same lines with x and y exchanged, crossing every pixel column.
    Endpoints, crossings and blend weights are exact in fp32 (offsets in
    eighths of a pixel, a 256-pixel edge span): the crossings never meet a
    pixel centre or a pixel border on their own axis, and on the other axis
    they fall on pixel borders only, where the weight is 0.

    Returns pos [4,3,4], tri [1,3], the blend weight beta [4,H,W] that
    Antialias.swift:274-309 gives the pixel holding the crossing,
    0.5 - |x_e - (q + 0.5)| for q = floor(x_e) (float64), and the coverage
    the line implies (pixel centres on the triangle's side) [4,H,W]."""
    lines = [(16.25, 0.25, -1.0), (48.125, -0.125, 1.0)]  # x0, slope, side
    pos = np.zeros((4, 3, 4), np.float64)
    beta = np.zeros((4, H, W), np.float64)
    cov = np.zeros((4, H, W), np.float32)
    r = np.arange(H)[:, None] + 0.5
    c = np.arange(W)[None, :] + 0.5
    for i in range(4):
        x0, s, side = lines[i % 2]
        # pixel-space vertices (a along the crossing axis, t along the other)
        pts = [(x0 + s * -64.0, -64.0), (x0 + s * 192.0, 192.0), (x0 + side * 300.0, 64.0)]
        for v, (a, t) in enumerate(pts):
            X, Y = (a, t) if i < 2 else (t, a)
            pos[i, v] = (2.0 * X / W - 1.0, 1.0 - 2.0 * Y / H, 0.0, 1.0)
        for k in range(H if i < 2 else W):
            xe = x0 + s * (k + 0.5)
            q = int(math.floor(xe))
            b = 0.5 - abs(xe - (q + 0.5))
            if i < 2:
                beta[i, k, q] = b
            else:
                beta[i, q, k] = b
        a, t = (c, r) if i < 2 else (r, c)
        cov[i] = side * (a - (x0 + s * t)) > 0
    return dict(pos=pos.astype(np.float32), tri=np.array([[0, 1, 2]], np.int32), beta=beta,
                cov=cov)
