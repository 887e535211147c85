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
// largest value (times the sign of the area) over the box is at a corner.
// Evaluated in fp32 at the corners; the margin, 2^-19 of S = (|a| + 1)(|b| +
// 1) + (|c| + 1)(|d| + 1), is twice the sum of two bounds: the rounding of
// that corner evaluation (below 2^-21 S: the products, their difference and
// the three-term sum, each term below S) and that of the per-pixel fp32
// expression (below 2^-22 S: four differences, two products, one
// difference, pixel centres lying in [-1, 1]).  So a rejected triangle fails
// the per-pixel test at every centre of the box.  An overflow or NaN
// anywhere makes the comparison false (no cull).
template <typename Rec>
DR_RT_FN bool edge_excludes(const Rec& R, float xa, float xb, float ya, float yb) {
  const float sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
  const float sx2 = R.r1.x, sy2 = R.r1.y;
  const float sg = R.r2.y > 0.0f ? 1.0f : -1.0f;
  const float e[3][4] = {{sx1, sy2, sx2, sy1}, {sx2, sy0, sx0, sy2}, {sx0, sy1, sx1, sy0}};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float a = e[k][0], b = e[k][1], c = e[k][2], d = e[k][3];
    const float A = sg * (d - b), B = sg * (c - a), C = sg * (a * b - c * d);
    const float mx = C + fmaxf(A * xa, A * xb) + fmaxf(B * ya, B * yb);
    const float tol = 0x1p-19f * ((fabsf(a) + 1.0f) * (fabsf(b) + 1.0f) + (fabsf(c) + 1.0f) * (fabsf(d) + 1.0f));
    if (mx < -tol) return true;
  }
  return false;
}

// Whether the triangle's depth lies above zq at every pixel centre of the
// box [xa, xb] x [ya, yb], so that it cannot take a pixel whose best depth
// so far is at most zq (test_tri keeps the smaller depth, and the lower index
// only on equal depths).  The depth sum_k e_k(x, y) sz_k / area is affine in
// (x, y), so its smallest value over the box is at a corner.  Evaluated in
// fp32 at the corners, each edge's coefficients scaled by the record's
// 1/area first (as the per-pixel expression scales the edge functions);
// the margin, 2^-17 (1 + sum |sz_k|)(1 + |1/area| max_k S_k) with S_k as
// above, is at least four times the sum of the corner evaluation's rounding
// and the per-pixel expression's (each below 2^-20 of that product: edge
// functions within 2^-21 S_k, the scaling, the products with the depths and
// their sum).  An overflow or NaN anywhere makes the comparison false.
template <typename Rec>
DR_RT_FN bool depth_excludes(const Rec& R, float xa, float xb, float ya, float yb,
                             float zq) {
  const float sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
  const float sx2 = R.r1.x, sy2 = R.r1.y;
  const float sz[3] = {R.r1.z, R.r1.w, R.r2.x};
  const float inv = R.r2.z;
  const float e[3][4] = {{sx1, sy2, sx2, sy1}, {sx2, sy0, sx0, sy2}, {sx0, sy1, sx1, sy0}};
  float z0 = 0.0f, zx = 0.0f, zy = 0.0f, m = 0.0f, s = 0.0f;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float a = e[k][0], b = e[k][1], c = e[k][2], d = e[k][3];
    z0 += sz[k] * ((a * b - c * d) * inv);
    zx += sz[k] * ((d - b) * inv);
    zy += sz[k] * ((c - a) * inv);
    m = fmaxf(m, (fabsf(a) + 1.0f) * (fabsf(b) + 1.0f) + (fabsf(c) + 1.0f) * (fabsf(d) + 1.0f));
    s += fabsf(sz[k]);
  }
  const float zmin = z0 + fminf(zx * xa, zx * xb) + fminf(zy * ya, zy * yb);
  const float tol = 0x1p-17f * (1.0f + s) * (1.0f + fabsf(inv) * m);
  return zmin - tol > zq;  // false for NaN
}

}  // namespace dr
