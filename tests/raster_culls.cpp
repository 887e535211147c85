// Host-side check of the pixel-parallel rasterizer's two culls
// (edge_excludes, depth_excludes in raster_tests.h) against the per-pixel
// test they stand in for (test_tri, Rasterize.swift:417-462): a candidate a
// cull drops must fail the per-pixel test at every pixel centre of the 8x8
// quadrant box it was dropped for.  Built with -ffp-contract=off, so the
// fp32 per-pixel expressions round as the library's do.
//
// Adversarial inputs, seeded: random triangles, slivers (a vertex a tiny
// distance off the opposite edge), off-screen and huge vertices, w close to
// 0, edges through pixel centres of the box, long edges grazing a corner
// centre of the box, near-degenerate areas, and depth thresholds at and
// around the triangle's own smallest depth over the box.  Prints the
// counts; exits 1 on the first violation.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>

#include "raster_tests.h"

struct F4 {
  float x, y, z, w;
};
struct Rec {
  F4 r0, r1, r2, r3;
};

static float int_bits(int i) { return __builtin_bit_cast(float, i); }

// The record of k_setup (screen-space vertices and depths, area, 1/area)
// with a pixel box over the whole image, so only the edge functions and the
// depth decide the per-pixel test.
static bool make_rec(const F4 (&v)[3], int W, int H, Rec& r) {
  for (const F4& p : v)
    if (!(p.w > 0.0f)) return false;
  const float sx0 = v[0].x / v[0].w, sy0 = v[0].y / v[0].w, sz0 = v[0].z / v[0].w;
  const float sx1 = v[1].x / v[1].w, sy1 = v[1].y / v[1].w, sz1 = v[1].z / v[1].w;
  const float sx2 = v[2].x / v[2].w, sy2 = v[2].y / v[2].w, sz2 = v[2].z / v[2].w;
  const float area = (sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0);
  r.r0 = {sx0, sy0, sx1, sy1};
  r.r1 = {sx2, sy2, sz0, sz1};
  r.r2 = {sz2, area, 1.0f / area, 0.0f};
  r.r3 = {int_bits(0), int_bits(W - 1), int_bits(0), int_bits(H - 1)};
  return std::isfinite(sx0) && std::isfinite(sx1) && std::isfinite(sx2) && std::isfinite(sy0) &&
         std::isfinite(sy1) && std::isfinite(sy2) && std::fabs(area) > 1e-30f;
}

static float cx(int X, int W) { return 2.0f * ((float)X + 0.5f) / (float)W - 1.0f; }
static float cy(int Y, int H) { return 1.0f - 2.0f * ((float)Y + 0.5f) / (float)H; }

int main(int argc, char** argv) {
  const long cases = argc > 1 ? atol(argv[1]) : 400000;
  std::mt19937_64 rng(20261202);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  long edge_tested = 0, edge_culled = 0, depth_tested = 0, depth_culled = 0;
  long edge_through_centre = 0;
  for (long it = 0; it < cases; ++it) {
    const int W = 8 << (int)(U(rng) * 9), H = 8 << (int)(U(rng) * 9);  // 8 .. 2048
    const int qx0 = (int)(U(rng) * (W / 8)) * 8, qy0 = (int)(U(rng) * (H / 8)) * 8;
    const int qx1 = qx0 + 7, qy1 = qy0 + 7;
    const float xa = cx(qx0, W), xb = cx(qx1, W), ya = cy(qy1, H), yb = cy(qy0, H);
    const int kind = (int)(U(rng) * 7);
    // vertices around the box, at a scale from a pixel to far off screen
    const double span = std::pow(10.0, -3.0 + 7.0 * U(rng));
    const double mx = 0.5 * (xa + xb), my = 0.5 * (ya + yb);
    F4 v[3];
    for (auto& p : v)
      p = {(float)(mx + span * (2 * U(rng) - 1)), (float)(my + span * (2 * U(rng) - 1)),
           (float)(2 * U(rng) - 1), 1.0f};
    if (kind == 1) {  // sliver: v2 a tiny distance off the edge v0 v1
      const double t = U(rng) * 1.4 - 0.2, off = std::pow(10.0, -9.0 + 6.0 * U(rng));
      const double ex = v[1].x - v[0].x, ey = v[1].y - v[0].y;
      v[2].x = (float)(v[0].x + t * ex - off * ey);
      v[2].y = (float)(v[0].y + t * ey + off * ex);
    } else if (kind == 2) {  // an edge through two pixel centres of the box
      const int X0 = qx0 + (int)(U(rng) * 8), Y0 = qy0 + (int)(U(rng) * 8);
      const int X1 = qx0 + (int)(U(rng) * 8), Y1 = qy0 + (int)(U(rng) * 8);
      v[0].x = cx(X0, W), v[0].y = cy(Y0, H);
      v[1].x = cx(X1, W), v[1].y = cy(Y1, H);
      if (U(rng) < 0.5) {  // extended far beyond the box along the same line
        const float dx = v[1].x - v[0].x, dy = v[1].y - v[0].y;
        v[1].x = v[0].x + 64.0f * dx;
        v[1].y = v[0].y + 64.0f * dy;
      }
      ++edge_through_centre;
    } else if (kind == 6) {
      // a long edge grazing a corner centre of the box with the box on its
      // outer side (the fp32 edge function's rounding is largest here), the
      // triangle beyond it
      const int X = U(rng) < 0.5 ? qx0 : qx1, Y = U(rng) < 0.5 ? qy0 : qy1;
      const double px = cx(X, W), py = cy(Y, H);
      const double sxn = X == qx0 ? -1.0 : 1.0, syn = Y == qy1 ? -1.0 : 1.0;  // outward
      const double a = 0.1 + 1.4 * U(rng), L = std::pow(10.0, 3.0 * U(rng));
      const double dx = syn * std::cos(a), dy = -sxn * std::sin(a);  // along the edge
      const double nx = sxn * std::sin(a), ny = syn * std::cos(a);   // outward normal
      const double eps = (U(rng) - 0.5) * std::pow(10.0, -9.0 + 6.0 * U(rng));
      v[0] = {(float)(px - L * dx + eps * nx), (float)(py - L * dy + eps * ny), 0.5f, 1.0f};
      v[1] = {(float)(px + L * dx + eps * nx), (float)(py + L * dy + eps * ny), 0.5f, 1.0f};
      v[2] = {(float)(px + L * nx), (float)(py + L * ny), 0.5f, 1.0f};
    } else if (kind == 3) {  // a vertex with w close to 0
      const float w = (float)std::pow(10.0, -7.0 + 6.0 * U(rng));
      v[0].x *= w, v[0].y *= w, v[0].z *= w, v[0].w = w;
    } else if (kind == 4) {  // all three vertices with random w
      for (auto& p : v) {
        const float w = (float)(0.05 + 4.0 * U(rng));
        p.x *= w, p.y *= w, p.z *= w, p.w = w;
      }
    }
    Rec R;
    if (!make_rec(v, W, H, R)) continue;
    Rec R0 = R;  // depths 0: only the edge functions can reject a pixel
    R0.r1.z = R0.r1.w = R0.r2.x = 0.0f;
    ++edge_tested;
    if (dr::edge_excludes(R, xa, xb, ya, yb)) {
      ++edge_culled;
      for (int Y = qy0; Y <= qy1; ++Y)
        for (int X = qx0; X <= qx1; ++X) {
          dr::Best b = {1e30f, 0.0f, 0.0f, -1};
          dr::test_tri(R0, 0, cx(X, W), cy(Y, H), X, Y, -1e30f, b);
          if (b.t >= 0) {
            printf("edge cull violated: case %ld kind %d W %d H %d pixel (%d, %d)\n", it, kind, W,
                   H, X, Y);
            return 1;
          }
        }
      continue;
    }
    // smallest depth over the covered centres, then thresholds around it
    float zmin = 1e30f;
    for (int Y = qy0; Y <= qy1; ++Y)
      for (int X = qx0; X <= qx1; ++X) {
        dr::Best b = {1e30f, 0.0f, 0.0f, 1 << 30};
        dr::test_tri(R, 0, cx(X, W), cy(Y, H), X, Y, -1e30f, b);
        if (b.t == 0 && b.z < zmin) zmin = b.z;
      }
    float zqs[5] = {(float)(2 * U(rng) - 1), -1.0f, 1.0f, 0.0f, 0.0f};
    if (zmin <= 1.0f) {
      zqs[3] = zmin;
      zqs[4] = std::nextafter(zmin, -2.0f);
    }
    for (float zq : zqs) {
      ++depth_tested;
      if (!dr::depth_excludes(R, xa, xb, ya, yb, zq)) continue;
      ++depth_culled;
      for (int Y = qy0; Y <= qy1; ++Y)
        for (int X = qx0; X <= qx1; ++X) {
          // a pixel whose best depth is zq (held by the highest index): the
          // candidate takes it if it covers it at a depth <= zq
          dr::Best b = {zq, 0.0f, 0.0f, 1 << 30};
          dr::test_tri(R, 0, cx(X, W), cy(Y, H), X, Y, -1e30f, b);
          if (b.t == 0) {
            printf("depth cull violated: case %ld kind %d zq %.9g z %.9g pixel (%d, %d)\n", it,
                   kind, zq, b.z, X, Y);
            return 1;
          }
        }
    }
  }
  printf("edge: %ld tested, %ld culled (%ld with an edge through pixel centres); "
         "depth: %ld tested, %ld culled\n",
         edge_tested, edge_culled, edge_through_centre, depth_tested, depth_culled);
  return 0;
}
