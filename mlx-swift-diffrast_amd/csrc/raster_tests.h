// Per-pixel coverage test and the pixel-parallel rasterizer's two
// conservative culls, shared by the kernels (rasterize.hip) and a host-side
// check that every culled candidate fails the per-pixel test at every pixel
// centre of its box (tests/raster_culls.cpp).  Rec is the kernels'
// per-triangle record (4 x float4, layout in rasterize.hip):
//   r0 = (sx0, sy0, sx1, sy1)  r1 = (sx2, sy2, sz0, sz1)
//   r2 = (sz2, area, 1/area, 0)  r3 = (X0, X1, Y0, Y1) as int bits.
// Build with -ffp-contract=off on both sides, as the library is.
#pragma once

#include <cmath>
#include <cstring>

#ifdef __HIPCC__
#define DR_RT_FN __host__ __device__ __attribute__((always_inline)) inline
#else
#define DR_RT_FN inline
#endif

namespace dr {

DR_RT_FN int rt_bits(float f) { return __builtin_bit_cast(int, f); }

struct Best {
  float z, u, v;
  int t;
};

// One candidate against one pixel (Rasterize.swift:417-462).
// (x, y): the centre of pixel (X, Y); the box test is the record's pixel box.
template <typename Rec>
DR_RT_FN void test_tri(const Rec& R, int t, float x, float y, int X, int Y, float peel_z,
                       Best& b) {
  const float sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
  const float sx2 = R.r1.x, sy2 = R.r1.y, sz0 = R.r1.z, sz1 = R.r1.w;
  const float sz2 = R.r2.x, area = R.r2.y, inv_area = R.r2.z;
  if (X < rt_bits(R.r3.x) || X > rt_bits(R.r3.y) || Y < rt_bits(R.r3.z) || Y > rt_bits(R.r3.w))
    return;
  const float e0 = (sx1 - x) * (sy2 - y) - (sx2 - x) * (sy1 - y);
  const float e1 = (sx2 - x) * (sy0 - y) - (sx0 - x) * (sy2 - y);
  const float e2 = (sx0 - x) * (sy1 - y) - (sx1 - x) * (sy0 - y);
  if ((e0 * area) < 0.0f || (e1 * area) < 0.0f || (e2 * area) < 0.0f) return;
  const float bw = e0 * inv_area;
  const float u = e1 * inv_area;
  const float v = e2 * inv_area;
  const float z = bw * sz0 + u * sz1 + v * sz2;
  if (z < -1.0f || z > 1.0f) return;
  if (z <= peel_z) return;
  if (z < b.z || (z == b.z && t < b.t)) {
    b.z = z;
    b.u = u;
    b.v = v;
    b.t = t;
  }
}

// Whether one edge of the triangle keeps every pixel centre of the box
// [xa, xb] x [ya, yb] outside: the edge function (sa - x)(sb - y) -
// (sc - x)(sd - y) is affine, (ab - cd) + (d - b) x + (c - a) y, so its
// largest value (times the sign of the area) over the box is at a corner;
// in fp64, with a margin above the rounding of the fp32 per-pixel
// expression (three roundings of products of terms below |s| + 1, pixel
// centres lying in [-1, 1]), so a rejected triangle fails the per-pixel
// test at every centre of the box.
template <typename Rec>
DR_RT_FN bool edge_excludes(const Rec& R, float xa, float xb, float ya, float yb) {
  const double sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
  const double sx2 = R.r1.x, sy2 = R.r1.y;
  const double sg = R.r2.y > 0.0f ? 1.0 : -1.0;
  const double e[3][4] = {{sx1, sy2, sx2, sy1}, {sx2, sy0, sx0, sy2}, {sx0, sy1, sx1, sy0}};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const double a = e[k][0], b = e[k][1], c = e[k][2], d = e[k][3];
    const double A = sg * (d - b), B = sg * (c - a), C = sg * (a * b - c * d);
    const double mx = C + fmax(A * (double)xa, A * (double)xb) + fmax(B * (double)ya, B * (double)yb);
    const double tol = 0x1p-20 * ((fabs(a) + 1.0) * (fabs(b) + 1.0) + (fabs(c) + 1.0) * (fabs(d) + 1.0));
    if (mx < -tol) return true;
  }
  return false;
}

// Whether the triangle's depth lies above zq at every pixel centre of the
// box [xa, xb] x [ya, yb], so that it cannot take a pixel whose best depth
// so far is at most zq (test_tri keeps the smaller depth, and the lower index
// only on equal depths).  The depth sum_k e_k(x, y) sz_k / area is affine in
// (x, y), so its smallest value over the box is at a corner; in fp64, less a
// margin over the rounding of the fp32 per-pixel expression (each edge
// function within 2^-22 of its two products' magnitudes, scaled by 1/area,
// then the products with the depths and their sum) of four times its bound.
template <typename Rec>
DR_RT_FN bool depth_excludes(const Rec& R, float xa, float xb, float ya, float yb,
                             float zq) {
  const double sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
  const double sx2 = R.r1.x, sy2 = R.r1.y;
  const double sz[3] = {R.r1.z, R.r1.w, R.r2.x};
  const double inv = 1.0 / (double)R.r2.y;
  const double e[3][4] = {{sx1, sy2, sx2, sy1}, {sx2, sy0, sx0, sy2}, {sx0, sy1, sx1, sy0}};
  double z0 = 0.0, zx = 0.0, zy = 0.0, m = 0.0, s = 0.0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const double a = e[k][0], b = e[k][1], c = e[k][2], d = e[k][3];
    z0 += sz[k] * (a * b - c * d);
    zx += sz[k] * (d - b);
    zy += sz[k] * (c - a);
    m = fmax(m, (fabs(a) + 1.0) * (fabs(b) + 1.0) + (fabs(c) + 1.0) * (fabs(d) + 1.0));
    s += fabs(sz[k]);
  }
  z0 *= inv;
  zx *= inv;
  zy *= inv;
  const double zmin = z0 + fmin(zx * (double)xa, zx * (double)xb) + fmin(zy * (double)ya, zy * (double)yb);
  const double tol = 0x1p-20 * (1.0 + s) * (1.0 + fabs(inv) * m);
  return zmin - tol > (double)zq;  // false for NaN
}

}  // namespace dr
