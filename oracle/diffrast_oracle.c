/*
 * CPU restatement of the mlx-swift-diffrast hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP kernels and the
 * CPU baseline timed beside them.  The product path never links or calls it.
 *
 * Each function below restates one Metal kernel body of the reference as a
 * sequential loop over the kernel's threads (thread-index order), citing the
 * file:line it follows.  Paths are relative to the reference repository.
 *
 * Parity pins (what checks each function, beyond these restatements):
 *   - rasterize fwd / rast_db: RasterizeTests.swift known answers, a
 *     brute-force full-triangle scan, the nvdiffrast fixture after the
 *     convention remap; backward: central finite differences.
 *   - interpolate: InterpolateTests.swift known answers, the nvdiffrast
 *     fixture (interp_out, interp_out_da, d_attr) after the remap, finite
 *     differences.
 *   - texture: TextureTests.swift known answers, the nvdiffrast fixture
 *     (tex_bilinear, tex_trilinear, d_tex, d_uv), finite differences,
 *     partition of unity of d_tex.
 *   - antialias: AntialiasTests.swift known answers, an O(T^2) topology
 *     brute force, finite differences.
 *
 * Build: -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).
 */
#include "diffrast_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

/* Scatter-add.  Sequential order in the default single-thread mode; an
 * atomic add when the pixel loops run on several threads. */
static inline void sadd(float* p, float v) {
  if (g_threads > 1) {
#pragma omp atomic update
    *p += v;
  } else {
    *p += v;
  }
}

/* Float -> int conversion of `(int)floor(x)` in the Metal bodies.  Out of
 * range values saturate and NaN gives 0 (the conversion GPUs implement; C
 * leaves it undefined), so that the oracle and the HIP kernels agree on
 * every input. */
static inline int f2i(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT_MAX;
  if (x <= -2147483648.0f) return INT_MIN;
  return (int)x;
}

/* ===================================================================== */
/* rasterize                                                             */
/* ===================================================================== */

/* Rasterize.swift:280-328 (precompute): one thread per (batch, triangle),
 * 10-float record (sx0,sy0,sz0, sx1,sy1,sz1, sx2,sy2,sz2, area). */
void orc_rast_precompute(const float* pos, int64_t pos_batch_stride,
                         const int32_t* tri, const int32_t* ranges,
                         int N, int V, int T, float* screen) {
  (void)V;
  for (int pn = 0; pn < N; ++pn) {
    for (int t = 0; t < T; ++t) {
      float* out = screen + ((int64_t)pn * T + t) * 10;
      int range_start = ranges[pn * 2 + 0];
      int range_count = ranges[pn * 2 + 1];
      if (t < range_start || t >= range_start + range_count) {  /* :292 */
        for (int k = 0; k < 10; ++k) out[k] = 0.0f;
        continue;
      }
      int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
      const float* p = pos + (int64_t)pn * pos_batch_stride;
      float w0 = p[(int64_t)i0 * 4 + 3];
      float w1 = p[(int64_t)i1 * 4 + 3];
      float w2 = p[(int64_t)i2 * 4 + 3];
      if (w0 <= 0.0f || w1 <= 0.0f || w2 <= 0.0f) {  /* :307 */
        for (int k = 0; k < 10; ++k) out[k] = 0.0f;
        continue;
      }
      float sx0 = p[(int64_t)i0 * 4 + 0] / w0, sy0 = p[(int64_t)i0 * 4 + 1] / w0,
            sz0 = p[(int64_t)i0 * 4 + 2] / w0;
      float sx1 = p[(int64_t)i1 * 4 + 0] / w1, sy1 = p[(int64_t)i1 * 4 + 1] / w1,
            sz1 = p[(int64_t)i1 * 4 + 2] / w1;
      float sx2 = p[(int64_t)i2 * 4 + 0] / w2, sy2 = p[(int64_t)i2 * 4 + 1] / w2,
            sz2 = p[(int64_t)i2 * 4 + 2] / w2;
      float area = (sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0); /* :322 */
      out[0] = sx0; out[1] = sy0; out[2] = sz0;
      out[3] = sx1; out[4] = sy1; out[5] = sz1;
      out[6] = sx2; out[7] = sy2; out[8] = sz2;
      out[9] = area;
    }
  }
}

/* Rasterize.swift:191-223: the tile rectangle a triangle's AABB touches.
 * Returns 0 when the triangle is skipped. */
static int bin_rect(const float* rec, int H, int W, int* tx0, int* tx1,
                    int* ty0, int* ty1) {
  float area = rec[9];
  if (area == 0.0f) return 0;
  float sx0 = rec[0], sy0 = rec[1];
  float sx1 = rec[3], sy1 = rec[4];
  float sx2 = rec[6], sy2 = rec[7];
  float minx_ndc = fminf(sx0, fminf(sx1, sx2));
  float maxx_ndc = fmaxf(sx0, fmaxf(sx1, sx2));
  float miny_ndc = fminf(sy0, fminf(sy1, sy2));
  float maxy_ndc = fmaxf(sy0, fmaxf(sy1, sy2));
  float px_min = (minx_ndc + 1.0f) * (float)W * 0.5f - 0.5f;
  float px_max = (maxx_ndc + 1.0f) * (float)W * 0.5f - 0.5f;
  float py_min = (1.0f - maxy_ndc) * (float)H * 0.5f - 0.5f;
  float py_max = (1.0f - miny_ndc) * (float)H * 0.5f - 0.5f;
  int pxmin_i = f2i(floorf(px_min));
  int pxmax_i = f2i(floorf(px_max));
  int pymin_i = f2i(floorf(py_min));
  int pymax_i = f2i(floorf(py_max));
  if (pxmin_i < 0) pxmin_i = 0;
  if (pxmax_i >= W) pxmax_i = W - 1;
  if (pymin_i < 0) pymin_i = 0;
  if (pymax_i >= H) pymax_i = H - 1;
  if (pxmin_i > pxmax_i || pymin_i > pymax_i) return 0;
  *tx0 = pxmin_i / ORC_TILE_SIZE;
  *tx1 = pxmax_i / ORC_TILE_SIZE;
  *ty0 = pymin_i / ORC_TILE_SIZE;
  *ty1 = pymax_i / ORC_TILE_SIZE;
  return 1;
}

/* Rasterize.swift:182-240 (bin), first half: the per-tile counts that the
 * `atomic_fetch_add` on bins[tile,0] accumulates.  counts: [N, tiles]. */
int64_t orc_rast_bin_count(const float* screen, int N, int T, int H, int W,
                           int32_t* counts) {
  int ntx = (W + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int nty = (H + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int64_t tiles = (int64_t)ntx * nty;
  memset(counts, 0, sizeof(int32_t) * (size_t)(N * tiles));
  int64_t total = 0;
  for (int pn = 0; pn < N; ++pn) {
    for (int t = 0; t < T; ++t) {
      int x0, x1, y0, y1;
      if (!bin_rect(screen + ((int64_t)pn * T + t) * 10, H, W, &x0, &x1, &y0, &y1))
        continue;
      for (int ty = y0; ty <= y1; ++ty)
        for (int tx = x0; tx <= x1; ++tx) {
          counts[pn * tiles + (int64_t)ty * ntx + tx] += 1;
          ++total;
        }
    }
  }
  return total;
}

/* Rasterize.swift:227-239, second half: append each triangle index to every
 * tile it touches.  Executed sequentially, each tile list is in ascending
 * triangle order.  The lists are stored compactly (offsets from an
 * exclusive scan of counts) instead of at a fixed 129-int stride; the
 * MAX_PER_TILE truncation is applied when the lists are read (orc_rast_fwd),
 * which keeps exactly the first 128 entries, as the sequential reference
 * does. */
void orc_rast_bin_fill(const float* screen, int N, int T, int H, int W,
                       const int64_t* offsets, int32_t* fill, int32_t* list) {
  int ntx = (W + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int nty = (H + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int64_t tiles = (int64_t)ntx * nty;
  memset(fill, 0, sizeof(int32_t) * (size_t)(N * tiles));
  for (int pn = 0; pn < N; ++pn) {
    for (int t = 0; t < T; ++t) {
      int x0, x1, y0, y1;
      if (!bin_rect(screen + ((int64_t)pn * T + t) * 10, H, W, &x0, &x1, &y0, &y1))
        continue;
      for (int ty = y0; ty <= y1; ++ty)
        for (int tx = x0; tx <= x1; ++tx) {
          int64_t tile = pn * tiles + (int64_t)ty * ntx + tx;
          list[offsets[tile] + fill[tile]] = t;
          fill[tile] += 1;
        }
    }
  }
}

/* Rasterize.swift:371-477 (fwd) and :487-599 (fwd_db).  rast_db may be NULL
 * (the fwd kernel); peel may be NULL (PEEL = false).  max_per_tile is the
 * reference's 128, or <= 0 for unlimited bins. */
void orc_rast_fwd(const float* screen, const int64_t* offsets,
                  const int32_t* counts, const int32_t* list,
                  const float* peel, int N, int T, int H, int W,
                  int max_per_tile, float* rast, float* rast_db) {
  int ntx = (W + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int nty = (H + ORC_TILE_SIZE - 1) / ORC_TILE_SIZE;
  int64_t tiles = (int64_t)ntx * nty;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(dynamic, 1024) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pw = (int)(pix % W);
    int ph = (int)((pix / W) % H);
    int pn = (int)(pix / ((int64_t)H * W));
    float ndc_x = 2.0f * ((float)pw + 0.5f) / (float)W - 1.0f;  /* :381 */
    float ndc_y = 1.0f - 2.0f * ((float)ph + 0.5f) / (float)H;  /* :382 */
    float peel_z = -1e30f;                                      /* :387 */
    if (peel) {
      float prev_tri = peel[pix * 4 + 3];
      if (prev_tri > 0.0f) peel_z = peel[pix * 4 + 2];
    }
    float best_z = 1e30f;
    int best_t = -1;
    float best_u = 0.0f, best_v = 0.0f;
    int64_t tile = pn * tiles + (int64_t)(ph / ORC_TILE_SIZE) * ntx + pw / ORC_TILE_SIZE;
    int tile_count = counts[tile];
    if (max_per_tile > 0 && tile_count > max_per_tile) tile_count = max_per_tile; /* :410 */
    for (int i = 0; i < tile_count; ++i) {
      int t = list[offsets[tile] + i];
      const float* r = screen + ((int64_t)pn * T + t) * 10;
      float area = r[9];
      if (area == 0.0f) continue;
      float sx0 = r[0], sy0 = r[1], sz0 = r[2];
      float sx1 = r[3], sy1 = r[4], sz1 = r[5];
      float sx2 = r[6], sy2 = r[7], sz2 = r[8];
      float minx = fminf(sx0, fminf(sx1, sx2));   /* :426-433 */
      if (ndc_x < minx) continue;
      float maxx = fmaxf(sx0, fmaxf(sx1, sx2));
      if (ndc_x > maxx) continue;
      float miny = fminf(sy0, fminf(sy1, sy2));
      if (ndc_y < miny) continue;
      float maxy = fmaxf(sy0, fmaxf(sy1, sy2));
      if (ndc_y > maxy) continue;
      float inv_area = 1.0f / area;
      float e0 = (sx1 - ndc_x) * (sy2 - ndc_y) - (sx2 - ndc_x) * (sy1 - ndc_y); /* :442 */
      float e1 = (sx2 - ndc_x) * (sy0 - ndc_y) - (sx0 - ndc_x) * (sy2 - ndc_y);
      float e2 = (sx0 - ndc_x) * (sy1 - ndc_y) - (sx1 - ndc_x) * (sy0 - ndc_y);
      if ((e0 * area) < 0.0f || (e1 * area) < 0.0f || (e2 * area) < 0.0f) continue;
      float bw = e0 * inv_area;
      float u = e1 * inv_area;
      float v = e2 * inv_area;
      float z_pix = bw * sz0 + u * sz1 + v * sz2;  /* :454 */
      if (z_pix < -1.0f || z_pix > 1.0f) continue;
      if (z_pix <= peel_z) continue;
      if (z_pix >= best_z) continue;  /* first in bin order wins a tie */
      best_z = z_pix;
      best_t = t;
      best_u = u;
      best_v = v;
    }
    float* o = rast + pix * 4;
    if (best_t < 0) {
      o[0] = o[1] = o[2] = o[3] = 0.0f;
      if (rast_db) {
        float* d = rast_db + pix * 4;
        d[0] = d[1] = d[2] = d[3] = 0.0f;
      }
      continue;
    }
    o[0] = best_u;
    o[1] = best_v;
    o[2] = best_z;
    o[3] = (float)(best_t + 1);
    if (rast_db) {  /* :586-598 */
      const float* r = screen + ((int64_t)pn * T + best_t) * 10;
      float sx0 = r[0], sy0 = r[1];
      float sx1 = r[3], sy1 = r[4];
      float sx2 = r[6], sy2 = r[7];
      float area = r[9];
      float inv_area = 1.0f / area;
      float k_x = 2.0f / (float)W;
      float k_y = -2.0f / (float)H;
      float* d = rast_db + pix * 4;
      d[0] = (sy2 - sy0) * inv_area * k_x;
      d[1] = (sx0 - sx2) * inv_area * k_y;
      d[2] = (sy0 - sy1) * inv_area * k_x;
      d[3] = (sx1 - sx0) * inv_area * k_y;
    }
  }
}

/* Rasterize.swift:637-812 (bwd): per covered pixel, chain d_rast (u,v,z)
 * and d_rast_db through the screen-space barycentrics and the perspective
 * divide; 12 scatter-adds into d_pos.  d_rast_db may be NULL (the gradDB =
 * false path passes zeros, :115). */
void orc_rast_bwd(const float* pos, int64_t pos_batch_stride,
                  const int32_t* tri, const float* rast, const float* d_rast,
                  const float* d_rast_db, int N, int V, int H, int W,
                  float* d_pos) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pw = (int)(pix % W);
    int ph = (int)((pix / W) % H);
    int pn = (int)(pix / ((int64_t)H * W));
    int64_t rb = pix * 4;
    int t = f2i(rast[rb + 3]) - 1;
    if (t < 0) continue;
    float u_val = rast[rb + 0];
    float v_val = rast[rb + 1];
    float bw_val = 1.0f - u_val - v_val;
    float d_u = d_rast[rb + 0];
    float d_v = d_rast[rb + 1];
    float d_z = d_rast[rb + 2];
    float d_db0 = d_rast_db ? d_rast_db[rb + 0] : 0.0f;
    float d_db1 = d_rast_db ? d_rast_db[rb + 1] : 0.0f;
    float d_db2 = d_rast_db ? d_rast_db[rb + 2] : 0.0f;
    float d_db3 = d_rast_db ? d_rast_db[rb + 3] : 0.0f;
    float Px = 2.0f * ((float)pw + 0.5f) / (float)W - 1.0f;
    float Py = 1.0f - 2.0f * ((float)ph + 0.5f) / (float)H;
    const float* p = pos + (int64_t)pn * pos_batch_stride;
    float* dp = d_pos + (int64_t)pn * pos_batch_stride;
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float x0 = p[(int64_t)i0 * 4 + 0], y0 = p[(int64_t)i0 * 4 + 1],
          z0 = p[(int64_t)i0 * 4 + 2], w0 = p[(int64_t)i0 * 4 + 3];
    float x1 = p[(int64_t)i1 * 4 + 0], y1 = p[(int64_t)i1 * 4 + 1],
          z1 = p[(int64_t)i1 * 4 + 2], w1 = p[(int64_t)i1 * 4 + 3];
    float x2 = p[(int64_t)i2 * 4 + 0], y2 = p[(int64_t)i2 * 4 + 1],
          z2 = p[(int64_t)i2 * 4 + 2], w2 = p[(int64_t)i2 * 4 + 3];
    float sx0 = x0 / w0, sy0 = y0 / w0, sz0 = z0 / w0;
    float sx1 = x1 / w1, sy1 = y1 / w1, sz1 = z1 / w1;
    float sx2 = x2 / w2, sy2 = y2 / w2, sz2 = z2 / w2;
    float area = (sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0);
    float inv_area = 1.0f / area;
    /* :694-699 d(area)/ds */
    float dadsx0 = sy1 - sy2, dadsx1 = sy2 - sy0, dadsx2 = sy0 - sy1;
    float dadsy0 = sx2 - sx1, dadsy1 = sx0 - sx2, dadsy2 = sx1 - sx0;
    /* :702-712 de1/ds, de2/ds */
    float de1dsx0 = Py - sy2, de1dsx2 = sy0 - Py;
    float de1dsy0 = sx2 - Px, de1dsy2 = Px - sx0;
    float de2dsx0 = sy1 - Py, de2dsx1 = Py - sy0;
    float de2dsy0 = Px - sx1, de2dsy1 = sx0 - Px;
    /* :716-728 */
    float dudsx0 = (de1dsx0 - u_val * dadsx0) * inv_area;
    float dudsx1 = (0.0f - u_val * dadsx1) * inv_area;
    float dudsx2 = (de1dsx2 - u_val * dadsx2) * inv_area;
    float dudsy0 = (de1dsy0 - u_val * dadsy0) * inv_area;
    float dudsy1 = (0.0f - u_val * dadsy1) * inv_area;
    float dudsy2 = (de1dsy2 - u_val * dadsy2) * inv_area;
    float dvdsx0 = (de2dsx0 - v_val * dadsx0) * inv_area;
    float dvdsx1 = (de2dsx1 - v_val * dadsx1) * inv_area;
    float dvdsx2 = (0.0f - v_val * dadsx2) * inv_area;
    float dvdsy0 = (de2dsy0 - v_val * dadsy0) * inv_area;
    float dvdsy1 = (de2dsy1 - v_val * dadsy1) * inv_area;
    float dvdsy2 = (0.0f - v_val * dadsy2) * inv_area;
    float dsz10 = sz1 - sz0, dsz20 = sz2 - sz0;
    /* :737-746 */
    float dsx0 = d_u * dudsx0 + d_v * dvdsx0 + d_z * (dudsx0 * dsz10 + dvdsx0 * dsz20);
    float dsx1 = d_u * dudsx1 + d_v * dvdsx1 + d_z * (dudsx1 * dsz10 + dvdsx1 * dsz20);
    float dsx2 = d_u * dudsx2 + d_v * dvdsx2 + d_z * (dudsx2 * dsz10 + dvdsx2 * dsz20);
    float dsy0 = d_u * dudsy0 + d_v * dvdsy0 + d_z * (dudsy0 * dsz10 + dvdsy0 * dsz20);
    float dsy1 = d_u * dudsy1 + d_v * dvdsy1 + d_z * (dudsy1 * dsz10 + dvdsy1 * dsz20);
    float dsy2 = d_u * dudsy2 + d_v * dvdsy2 + d_z * (dudsy2 * dsz10 + dvdsy2 * dsz20);
    float dsz0_s = d_z * bw_val, dsz1_s = d_z * u_val, dsz2_s = d_z * v_val;
    /* :755-778 rast_db chain */
    float Kx = 2.0f / (float)W;
    float Ky = -2.0f / (float)H;
    float rdb0 = (sy2 - sy0) * Kx * inv_area;
    float rdb1 = (sx0 - sx2) * Ky * inv_area;
    float rdb2 = (sy0 - sy1) * Kx * inv_area;
    float rdb3 = (sx1 - sx0) * Ky * inv_area;
    float s = d_db0 * rdb0 + d_db1 * rdb1 + d_db2 * rdb2 + d_db3 * rdb3;
    dsx0 += (-s * dadsx0) * inv_area;
    dsx1 += (-s * dadsx1) * inv_area;
    dsx2 += (-s * dadsx2) * inv_area;
    dsy0 += (-s * dadsy0) * inv_area;
    dsy1 += (-s * dadsy1) * inv_area;
    dsy2 += (-s * dadsy2) * inv_area;
    dsy0 += d_db0 * (-Kx) * inv_area;
    dsy2 += d_db0 * (Kx) * inv_area;
    dsx0 += d_db1 * (Ky) * inv_area;
    dsx2 += d_db1 * (-Ky) * inv_area;
    dsy0 += d_db2 * (Kx) * inv_area;
    dsy1 += d_db2 * (-Kx) * inv_area;
    dsx0 += d_db3 * (-Ky) * inv_area;
    dsx1 += d_db3 * (Ky) * inv_area;
    /* :781-811 perspective divide + scatter */
    float inv_w0 = 1.0f / w0, inv_w1 = 1.0f / w1, inv_w2 = 1.0f / w2;
    sadd(&dp[(int64_t)i0 * 4 + 0], dsx0 * inv_w0);
    sadd(&dp[(int64_t)i0 * 4 + 1], dsy0 * inv_w0);
    sadd(&dp[(int64_t)i0 * 4 + 2], dsz0_s * inv_w0);
    sadd(&dp[(int64_t)i0 * 4 + 3], -(sx0 * dsx0 + sy0 * dsy0 + sz0 * dsz0_s) * inv_w0);
    sadd(&dp[(int64_t)i1 * 4 + 0], dsx1 * inv_w1);
    sadd(&dp[(int64_t)i1 * 4 + 1], dsy1 * inv_w1);
    sadd(&dp[(int64_t)i1 * 4 + 2], dsz1_s * inv_w1);
    sadd(&dp[(int64_t)i1 * 4 + 3], -(sx1 * dsx1 + sy1 * dsy1 + sz1 * dsz1_s) * inv_w1);
    sadd(&dp[(int64_t)i2 * 4 + 0], dsx2 * inv_w2);
    sadd(&dp[(int64_t)i2 * 4 + 1], dsy2 * inv_w2);
    sadd(&dp[(int64_t)i2 * 4 + 2], dsz2_s * inv_w2);
    sadd(&dp[(int64_t)i2 * 4 + 3], -(sx2 * dsx2 + sy2 * dsy2 + sz2 * dsz2_s) * inv_w2);
  }
}

/* ===================================================================== */
/* interpolate                                                           */
/* ===================================================================== */

/* Interpolate.swift:137-170 (fwd). */
void orc_interp_fwd(const float* attr, int64_t attr_batch_stride,
                    const float* rast, const int32_t* tri,
                    int N, int H, int W, int V, int A, float* out) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    float u = rast[pix * 4 + 0];
    float v = rast[pix * 4 + 1];
    int t = f2i(rast[pix * 4 + 3]) - 1;
    float* o = out + pix * A;
    if (t < 0) {
      for (int a = 0; a < A; ++a) o[a] = 0.0f;
      continue;
    }
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float bw = 1.0f - u - v;
    const float* at = attr + (int64_t)n * attr_batch_stride;
    for (int a = 0; a < A; ++a) {
      float a0 = at[(int64_t)i0 * A + a];
      float a1 = at[(int64_t)i1 * A + a];
      float a2 = at[(int64_t)i2 * A + a];
      o[a] = bw * a0 + u * a1 + v * a2;
    }
  }
}

/* Interpolate.swift:175-228 (fwd_da). */
void orc_interp_fwd_da(const float* attr, int64_t attr_batch_stride,
                       const float* rast, const float* rast_db,
                       const int32_t* tri, const int32_t* diff_idx,
                       int N, int H, int W, int V, int A, int K,
                       float* out, float* out_da) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    float u = rast[pix * 4 + 0];
    float v = rast[pix * 4 + 1];
    int t = f2i(rast[pix * 4 + 3]) - 1;
    float* o = out + pix * A;
    float* od = out_da + pix * 2 * K;
    if (t < 0) {
      for (int a = 0; a < A; ++a) o[a] = 0.0f;
      for (int k = 0; k < 2 * K; ++k) od[k] = 0.0f;
      continue;
    }
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float bw = 1.0f - u - v;
    const float* at = attr + (int64_t)n * attr_batch_stride;
    for (int a = 0; a < A; ++a) {
      float a0 = at[(int64_t)i0 * A + a];
      float a1 = at[(int64_t)i1 * A + a];
      float a2 = at[(int64_t)i2 * A + a];
      o[a] = bw * a0 + u * a1 + v * a2;
    }
    float udx = rast_db[pix * 4 + 0], udy = rast_db[pix * 4 + 1];
    float vdx = rast_db[pix * 4 + 2], vdy = rast_db[pix * 4 + 3];
    for (int k = 0; k < K; ++k) {
      int a = diff_idx[k];
      float a0 = at[(int64_t)i0 * A + a];
      float a1 = at[(int64_t)i1 * A + a];
      float a2 = at[(int64_t)i2 * A + a];
      float d01 = a1 - a0, d02 = a2 - a0;
      od[2 * k + 0] = d01 * udx + d02 * vdx;
      od[2 * k + 1] = d01 * udy + d02 * vdy;
    }
  }
}

/* Interpolate.swift:231-264 (grad_attr). */
void orc_interp_grad_attr(const float* rast, const int32_t* tri,
                          const float* d_out, int N, int H, int W, int V,
                          int A, int64_t d_attr_batch_stride, float* d_attr) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    float u = rast[pix * 4 + 0];
    float v = rast[pix * 4 + 1];
    int t = f2i(rast[pix * 4 + 3]) - 1;
    if (t < 0) continue;
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float bw = 1.0f - u - v;
    float* da = d_attr + (int64_t)n * d_attr_batch_stride;
    for (int a = 0; a < A; ++a) {
      float g = d_out[pix * A + a];
      sadd(&da[(int64_t)i0 * A + a], bw * g);
      sadd(&da[(int64_t)i1 * A + a], u * g);
      sadd(&da[(int64_t)i2 * A + a], v * g);
    }
  }
}

/* Interpolate.swift:269-324 (grad_attr_da). */
void orc_interp_grad_attr_da(const float* rast, const float* rast_db,
                             const int32_t* tri, const float* d_out,
                             const float* d_out_da, const int32_t* diff_idx,
                             int N, int H, int W, int V, int A, int K,
                             int64_t d_attr_batch_stride, float* d_attr) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    float u = rast[pix * 4 + 0];
    float v = rast[pix * 4 + 1];
    int t = f2i(rast[pix * 4 + 3]) - 1;
    if (t < 0) continue;
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float bw = 1.0f - u - v;
    float* da = d_attr + (int64_t)n * d_attr_batch_stride;
    for (int a = 0; a < A; ++a) {
      float g = d_out[pix * A + a];
      sadd(&da[(int64_t)i0 * A + a], bw * g);
      sadd(&da[(int64_t)i1 * A + a], u * g);
      sadd(&da[(int64_t)i2 * A + a], v * g);
    }
    float udx = rast_db[pix * 4 + 0], udy = rast_db[pix * 4 + 1];
    float vdx = rast_db[pix * 4 + 2], vdy = rast_db[pix * 4 + 3];
    for (int k = 0; k < K; ++k) {
      int a = diff_idx[k];
      float gx = d_out_da[pix * 2 * K + 2 * k + 0];
      float gy = d_out_da[pix * 2 * K + 2 * k + 1];
      float u_term = gx * udx + gy * udy;
      float v_term = gx * vdx + gy * vdy;
      sadd(&da[(int64_t)i0 * A + a], -u_term - v_term);
      sadd(&da[(int64_t)i1 * A + a], u_term);
      sadd(&da[(int64_t)i2 * A + a], v_term);
    }
  }
}

/* Interpolate.swift:327-367 (grad_rast). */
void orc_interp_grad_rast(const float* attr, int64_t attr_batch_stride,
                          const float* rast, const int32_t* tri,
                          const float* d_out, int N, int H, int W, int V,
                          int A, float* d_rast) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    int t = f2i(rast[pix * 4 + 3]) - 1;
    float* dr = d_rast + pix * 4;
    dr[2] = 0.0f;
    dr[3] = 0.0f;
    if (t < 0) {
      dr[0] = 0.0f;
      dr[1] = 0.0f;
      continue;
    }
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    const float* at = attr + (int64_t)n * attr_batch_stride;
    float du = 0.0f, dv = 0.0f;
    for (int a = 0; a < A; ++a) {
      float a0 = at[(int64_t)i0 * A + a];
      float a1 = at[(int64_t)i1 * A + a];
      float a2 = at[(int64_t)i2 * A + a];
      float g = d_out[pix * A + a];
      du += (a1 - a0) * g;
      dv += (a2 - a0) * g;
    }
    dr[0] = du;
    dr[1] = dv;
  }
}

/* Interpolate.swift:370-417 (grad_rast_db). */
void orc_interp_grad_rast_db(const float* attr, int64_t attr_batch_stride,
                             const float* rast, const int32_t* tri,
                             const float* d_out_da, const int32_t* diff_idx,
                             int N, int H, int W, int V, int A, int K,
                             float* d_rast_db) {
  (void)V;
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int n = (int)(pix / ((int64_t)H * W));
    int t = f2i(rast[pix * 4 + 3]) - 1;
    float* dd = d_rast_db + pix * 4;
    if (t < 0) {
      dd[0] = dd[1] = dd[2] = dd[3] = 0.0f;
      continue;
    }
    int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    const float* at = attr + (int64_t)n * attr_batch_stride;
    float d_udx = 0.0f, d_udy = 0.0f, d_vdx = 0.0f, d_vdy = 0.0f;
    for (int k = 0; k < K; ++k) {
      int a = diff_idx[k];
      float a0 = at[(int64_t)i0 * A + a];
      float a1 = at[(int64_t)i1 * A + a];
      float a2 = at[(int64_t)i2 * A + a];
      float d01 = a1 - a0, d02 = a2 - a0;
      float gx = d_out_da[pix * 2 * K + 2 * k + 0];
      float gy = d_out_da[pix * 2 * K + 2 * k + 1];
      d_udx += d01 * gx;
      d_udy += d01 * gy;
      d_vdx += d02 * gx;
      d_vdy += d02 * gy;
    }
    dd[0] = d_udx;
    dd[1] = d_udy;
    dd[2] = d_vdx;
    dd[3] = d_vdy;
  }
}

/* ===================================================================== */
/* texture                                                               */
/* ===================================================================== */

/* Texture.swift:336-354 (apply_boundary). */
static inline int apply_boundary(int t, int size, int mode, float* oob) {
  if (mode == 2) {
    if (t < 0 || t >= size) {
      *oob = 1.0f;
      return 0;
    }
    *oob = 0.0f;
    return t;
  }
  if (mode == 1) {
    *oob = 0.0f;
    return t < 0 ? 0 : (t >= size ? size - 1 : t);
  }
  *oob = 0.0f;
  int r = t % size;
  if (r < 0) r += size;
  return r;
}

/* The bilinear footprint shared by every bilinear body of Texture.swift
 * (:372-391, :420-439, :485-498, :827-845). */
typedef struct {
  int ix0, ix1, iy0, iy1;
  float fx, fy;
  float ox0, ox1, oy0, oy1;
  float w00, w10, w01, w11;
} Bilin;

static inline void bilin(float u, float v, int Wk, int Hk, int boundary,
                         Bilin* b) {
  float tx = u * (float)Wk - 0.5f;
  float ty = v * (float)Hk - 0.5f;
  int tx0 = f2i(floorf(tx));
  int ty0 = f2i(floorf(ty));
  int tx1 = tx0 + 1;
  int ty1 = ty0 + 1;
  b->fx = tx - (float)tx0;
  b->fy = ty - (float)ty0;
  b->ix0 = apply_boundary(tx0, Wk, boundary, &b->ox0);
  b->ix1 = apply_boundary(tx1, Wk, boundary, &b->ox1);
  b->iy0 = apply_boundary(ty0, Hk, boundary, &b->oy0);
  b->iy1 = apply_boundary(ty1, Hk, boundary, &b->oy1);
  float fx = b->fx, fy = b->fy;
  b->w00 = (1.0f - fx) * (1.0f - fy) * (1.0f - b->ox0) * (1.0f - b->oy0);
  b->w10 = (fx) * (1.0f - fy) * (1.0f - b->ox1) * (1.0f - b->oy0);
  b->w01 = (1.0f - fx) * (fy) * (1.0f - b->ox0) * (1.0f - b->oy1);
  b->w11 = (fx) * (fy) * (1.0f - b->ox1) * (1.0f - b->oy1);
}

/* Texture.swift:359-403 (bilinear fwd). */
void orc_tex_fwd(const float* tex, int64_t tex_batch_stride, const float* uv,
                 int N, int Hi, int Wi, int Ht, int Wt, int C, int boundary,
                 float* out) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    Bilin b;
    bilin(uv[pix * 2 + 0], uv[pix * 2 + 1], Wt, Ht, boundary, &b);
    const float* tx = tex + (int64_t)pn * tex_batch_stride;
    for (int c = 0; c < C; ++c) {
      float t00 = tx[((int64_t)b.iy0 * Wt + b.ix0) * C + c];
      float t10 = tx[((int64_t)b.iy0 * Wt + b.ix1) * C + c];
      float t01 = tx[((int64_t)b.iy1 * Wt + b.ix0) * C + c];
      float t11 = tx[((int64_t)b.iy1 * Wt + b.ix1) * C + c];
      out[pix * C + c] = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
    }
  }
}

/* Texture.swift:407-459 (grad_tex). */
void orc_tex_grad_tex(const float* uv, const float* d_out, int N, int Hi,
                      int Wi, int Ht, int Wt, int C, int boundary,
                      int64_t d_tex_batch_stride, float* d_tex) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    Bilin b;
    bilin(uv[pix * 2 + 0], uv[pix * 2 + 1], Wt, Ht, boundary, &b);
    float* dt = d_tex + (int64_t)pn * d_tex_batch_stride;
    for (int c = 0; c < C; ++c) {
      float g = d_out[pix * C + c];
      sadd(&dt[((int64_t)b.iy0 * Wt + b.ix0) * C + c], b.w00 * g);
      sadd(&dt[((int64_t)b.iy0 * Wt + b.ix1) * C + c], b.w10 * g);
      sadd(&dt[((int64_t)b.iy1 * Wt + b.ix0) * C + c], b.w01 * g);
      sadd(&dt[((int64_t)b.iy1 * Wt + b.ix1) * C + c], b.w11 * g);
    }
  }
}

/* Texture.swift:472-521 (grad_uv). */
void orc_tex_grad_uv(const float* tex, int64_t tex_batch_stride,
                     const float* uv, const float* d_out, int N, int Hi,
                     int Wi, int Ht, int Wt, int C, int boundary, float* d_uv) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    Bilin b;
    bilin(uv[pix * 2 + 0], uv[pix * 2 + 1], Wt, Ht, boundary, &b);
    const float* tx = tex + (int64_t)pn * tex_batch_stride;
    float m00 = (1.0f - b.ox0) * (1.0f - b.oy0);
    float m10 = (1.0f - b.ox1) * (1.0f - b.oy0);
    float m01 = (1.0f - b.ox0) * (1.0f - b.oy1);
    float m11 = (1.0f - b.ox1) * (1.0f - b.oy1);
    float dfx_sum = 0.0f, dfy_sum = 0.0f;
    for (int c = 0; c < C; ++c) {
      float t00 = tx[((int64_t)b.iy0 * Wt + b.ix0) * C + c] * m00;
      float t10 = tx[((int64_t)b.iy0 * Wt + b.ix1) * C + c] * m10;
      float t01 = tx[((int64_t)b.iy1 * Wt + b.ix0) * C + c] * m01;
      float t11 = tx[((int64_t)b.iy1 * Wt + b.ix1) * C + c] * m11;
      float g = d_out[pix * C + c];
      dfx_sum += g * ((1.0f - b.fy) * (t10 - t00) + b.fy * (t11 - t01));
      dfy_sum += g * ((1.0f - b.fx) * (t01 - t00) + b.fx * (t11 - t10));
    }
    d_uv[pix * 2 + 0] = dfx_sum * (float)Wt;
    d_uv[pix * 2 + 1] = dfy_sum * (float)Ht;
  }
}

/* Texture.swift:545-572 (nearest fwd). */
void orc_tex_nearest_fwd(const float* tex, int64_t tex_batch_stride,
                         const float* uv, int N, int Hi, int Wi, int Ht,
                         int Wt, int C, int boundary, float* out) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    int tx = f2i(floorf(uv[pix * 2 + 0] * (float)Wt));
    int ty = f2i(floorf(uv[pix * 2 + 1] * (float)Ht));
    float ox, oy;
    int ix = apply_boundary(tx, Wt, boundary, &ox);
    int iy = apply_boundary(ty, Ht, boundary, &oy);
    float mask = (1.0f - ox) * (1.0f - oy);
    const float* t = tex + (int64_t)pn * tex_batch_stride;
    for (int c = 0; c < C; ++c)
      out[pix * C + c] = t[((int64_t)iy * Wt + ix) * C + c] * mask;
  }
}

/* Texture.swift:576-605 (nearest grad_tex). */
void orc_tex_nearest_grad_tex(const float* uv, const float* d_out, int N,
                              int Hi, int Wi, int Ht, int Wt, int C,
                              int boundary, int64_t d_tex_batch_stride,
                              float* d_tex) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    int tx = f2i(floorf(uv[pix * 2 + 0] * (float)Wt));
    int ty = f2i(floorf(uv[pix * 2 + 1] * (float)Ht));
    float ox, oy;
    int ix = apply_boundary(tx, Wt, boundary, &ox);
    int iy = apply_boundary(ty, Ht, boundary, &oy);
    float mask = (1.0f - ox) * (1.0f - oy);
    float* dt = d_tex + (int64_t)pn * d_tex_batch_stride;
    for (int c = 0; c < C; ++c)
      sadd(&dt[((int64_t)iy * Wt + ix) * C + c], d_out[pix * C + c] * mask);
  }
}

/* Texture.swift:616-636 (cube projection). */
static inline void cube_project(float x, float y, float z, int* face, float* u,
                                float* v) {
  float ax = fabsf(x), ay = fabsf(y), az = fabsf(z);
  float sc, tc, ma;
  if (ax >= ay && ax >= az) {
    ma = ax;
    if (x > 0.0f) { *face = 0; sc = -z; tc = -y; }
    else          { *face = 1; sc = z;  tc = -y; }
  } else if (ay >= az) {
    ma = ay;
    if (y > 0.0f) { *face = 2; sc = x; tc = z; }
    else          { *face = 3; sc = x; tc = -z; }
  } else {
    ma = az;
    if (z > 0.0f) { *face = 4; sc = x;  tc = -y; }
    else          { *face = 5; sc = -x; tc = -y; }
  }
  float inv_ma = 1.0f / ma;
  *u = (sc * inv_ma + 1.0f) * 0.5f;
  *v = (tc * inv_ma + 1.0f) * 0.5f;
}

typedef struct {
  int face, ix0, ix1, iy0, iy1;
  float w00, w10, w01, w11;
} CubeTap;

/* Texture.swift:656-672: clamp-within-face bilinear. */
static inline void cube_tap(const float* dir, int Ht, int Wt, CubeTap* c) {
  float u, v;
  cube_project(dir[0], dir[1], dir[2], &c->face, &u, &v);
  float tx_real = u * (float)Wt - 0.5f;
  float ty_real = v * (float)Ht - 0.5f;
  int tx0 = f2i(floorf(tx_real));
  int ty0 = f2i(floorf(ty_real));
  int tx1 = tx0 + 1, ty1 = ty0 + 1;
  float fx = tx_real - (float)tx0;
  float fy = ty_real - (float)ty0;
  c->ix0 = tx0 < 0 ? 0 : (tx0 > Wt - 1 ? Wt - 1 : tx0);
  c->ix1 = tx1 < 0 ? 0 : (tx1 > Wt - 1 ? Wt - 1 : tx1);
  c->iy0 = ty0 < 0 ? 0 : (ty0 > Ht - 1 ? Ht - 1 : ty0);
  c->iy1 = ty1 < 0 ? 0 : (ty1 > Ht - 1 ? Ht - 1 : ty1);
  c->w00 = (1.0f - fx) * (1.0f - fy);
  c->w10 = fx * (1.0f - fy);
  c->w01 = (1.0f - fx) * fy;
  c->w11 = fx * fy;
}

/* Texture.swift:638-684 (cube fwd).  tex: [N or 1, 6, Ht, Wt, C]. */
void orc_tex_cube_fwd(const float* tex, int64_t tex_batch_stride,
                      const float* dir, int N, int Hi, int Wi, int Ht, int Wt,
                      int C, float* out) {
  int64_t total = (int64_t)N * Hi * Wi;
  int64_t face_sz = (int64_t)Ht * Wt * C;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    CubeTap q;
    cube_tap(dir + pix * 3, Ht, Wt, &q);
    const float* fb = tex + (int64_t)pn * tex_batch_stride + q.face * face_sz;
    for (int c = 0; c < C; ++c) {
      float t00 = fb[((int64_t)q.iy0 * Wt + q.ix0) * C + c];
      float t10 = fb[((int64_t)q.iy0 * Wt + q.ix1) * C + c];
      float t01 = fb[((int64_t)q.iy1 * Wt + q.ix0) * C + c];
      float t11 = fb[((int64_t)q.iy1 * Wt + q.ix1) * C + c];
      out[pix * C + c] = q.w00 * t00 + q.w10 * t10 + q.w01 * t01 + q.w11 * t11;
    }
  }
}

/* Texture.swift:686-738 (cube grad_tex). */
void orc_tex_cube_grad_tex(const float* dir, const float* d_out, int N,
                           int Hi, int Wi, int Ht, int Wt, int C,
                           int64_t d_tex_batch_stride, float* d_tex) {
  int64_t total = (int64_t)N * Hi * Wi;
  int64_t face_sz = (int64_t)Ht * Wt * C;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    CubeTap q;
    cube_tap(dir + pix * 3, Ht, Wt, &q);
    float* fb = d_tex + (int64_t)pn * d_tex_batch_stride + q.face * face_sz;
    for (int c = 0; c < C; ++c) {
      float g = d_out[pix * C + c];
      sadd(&fb[((int64_t)q.iy0 * Wt + q.ix0) * C + c], q.w00 * g);
      sadd(&fb[((int64_t)q.iy0 * Wt + q.ix1) * C + c], q.w10 * g);
      sadd(&fb[((int64_t)q.iy1 * Wt + q.ix0) * C + c], q.w01 * g);
      sadd(&fb[((int64_t)q.iy1 * Wt + q.ix1) * C + c], q.w11 * g);
    }
  }
}

/* Texture.swift:144-161 (textureConstructMip): level count and shapes.
 * Downsampling continues while both dims are even and >= 2, and stops once
 * the list holds max_level + 1 entries (max_level < 0: no cap). */
int orc_mip_levels(int H, int W, int max_level, int32_t* level_h,
                   int32_t* level_w) {
  int n = 0;
  level_h[n] = H;
  level_w[n] = W;
  ++n;
  while (H >= 2 && W >= 2 && (H % 2) == 0 && (W % 2) == 0) {
    if (max_level >= 0 && n > max_level) break;
    H /= 2;
    W /= 2;
    level_h[n] = H;
    level_w[n] = W;
    ++n;
  }
  return n;
}

/* Texture.swift:156 (`reshaped([N,H2,2,W2,2,C]).mean(axes:[2,4])`) and the
 * packing of :291-304.  Level k of batch n starts at offsets[k] +
 * n*Hk*Wk*C.  The 2x2 mean is summed in row-major order of the reduced axes
 * and scaled by 1/4 (exact for a power of two). */
void orc_mip_build(const float* tex, int Nt, int H, int W, int C, int L,
                   const int64_t* offsets, float* packed) {
  memcpy(packed + offsets[0], tex, sizeof(float) * (size_t)Nt * H * W * C);
  int h = H, w = W;
  for (int k = 1; k < L; ++k) {
    int h2 = h / 2, w2 = w / 2;
    for (int n = 0; n < Nt; ++n) {
      const float* src = packed + offsets[k - 1] + (int64_t)n * h * w * C;
      float* dst = packed + offsets[k] + (int64_t)n * h2 * w2 * C;
      for (int y = 0; y < h2; ++y)
        for (int x = 0; x < w2; ++x)
          for (int c = 0; c < C; ++c) {
            float a = src[((int64_t)(2 * y) * w + 2 * x) * C + c];
            float b = src[((int64_t)(2 * y) * w + 2 * x + 1) * C + c];
            float d = src[((int64_t)(2 * y + 1) * w + 2 * x) * C + c];
            float e = src[((int64_t)(2 * y + 1) * w + 2 * x + 1) * C + c];
            dst[((int64_t)y * w2 + x) * C + c] = (((a + b) + d) + e) * 0.25f;
          }
    }
    h = h2;
    w = w2;
  }
}

/* Backward of the pyramid build + packing (MLX autodiff through
 * `concatenated` and each `mean`, Texture.swift:156,304): walking from the
 * coarsest level to the finest, the cotangent of level k is its own packed
 * slice plus one quarter of level k+1's cotangent broadcast to each 2x2
 * child.  d_tex receives level 0's total. */
void orc_mip_collapse(const float* d_packed, int Nt, int H, int W, int C,
                      int L, const int64_t* offsets, float* d_tex) {
  int32_t lh[32], lw[32];
  int h = H, w = W;
  for (int k = 0; k < L; ++k) {
    lh[k] = h;
    lw[k] = w;
    h /= 2;
    w /= 2;
  }
  /* acc holds the running cotangent of level k (largest: level 0). */
  size_t maxsz = (size_t)Nt * H * W * C;
  float* acc = (float*)malloc(sizeof(float) * maxsz);
  float* nxt = (float*)malloc(sizeof(float) * maxsz);
  int k = L - 1;
  memcpy(acc, d_packed + offsets[k], sizeof(float) * (size_t)Nt * lh[k] * lw[k] * C);
  for (k = L - 2; k >= 0; --k) {
    int hk = lh[k], wk = lw[k], hc = lh[k + 1], wc = lw[k + 1];
    for (int n = 0; n < Nt; ++n)
      for (int y = 0; y < hk; ++y)
        for (int x = 0; x < wk; ++x)
          for (int c = 0; c < C; ++c) {
            float up = acc[(((int64_t)n * hc + y / 2) * wc + x / 2) * C + c];
            float own = d_packed[offsets[k] + (((int64_t)n * hk + y) * wk + x) * C + c];
            nxt[(((int64_t)n * hk + y) * wk + x) * C + c] = own + up * 0.25f;
          }
    float* tmp = acc;
    acc = nxt;
    nxt = tmp;
  }
  memcpy(d_tex, acc, sizeof(float) * (size_t)Nt * H * W * C);
  free(acc);
  free(nxt);
}

/* Texture.swift:764-790: LOD and the two levels. */
static inline void mip_lod(const float* da, int Ht, int Wt, int L,
                           int mip_linear, int* k0, int* k1, float* frac) {
  float du_dx = da[0], du_dy = da[1], dv_dx = da[2], dv_dy = da[3];
  float sx = du_dx * (float)Wt;
  float sy = du_dy * (float)Wt;
  float tx = dv_dx * (float)Ht;
  float ty = dv_dy * (float)Ht;
  float rho_sq = fmaxf(sx * sx + tx * tx, sy * sy + ty * ty);
  float lod = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
  lod = fmaxf(0.0f, fminf((float)(L - 1), lod));
  if (mip_linear) {
    *k0 = f2i(floorf(lod));
    *k1 = *k0 + 1;
    if (*k1 >= L) *k1 = L - 1;
    *frac = lod - (float)*k0;
  } else {
    *k0 = f2i(floorf(lod + 0.5f));
    if (*k0 >= L) *k0 = L - 1;
    *k1 = *k0;
    *frac = 0.0f;
  }
}

/* Texture.swift:795-863 (trilinear / mip-nearest fwd).  level_batch_mul is 1
 * when the pyramid holds one texture per image batch and 0 when a single
 * texture serves every batch (the reference's broadcast copies are
 * identical, so the values read are the same). */
void orc_tex_mip_fwd(const float* packed, int64_t level_batch_mul,
                     const float* uv, const float* uv_da,
                     const int64_t* offsets, const int32_t* level_h,
                     const int32_t* level_w, int L, int N, int Hi, int Wi,
                     int Ht, int Wt, int C, int boundary, int mip_linear,
                     float* out) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    float u = uv[pix * 2 + 0], v = uv[pix * 2 + 1];
    int k0, k1;
    float frac;
    mip_lod(uv_da + pix * 4, Ht, Wt, L, mip_linear, &k0, &k1, &frac);
    for (int li = 0; li < 2; ++li) {
      int k = li == 0 ? k0 : k1;
      int Hk = level_h[k], Wk = level_w[k];
      const float* lv = packed + offsets[k] + (int64_t)pn * level_batch_mul * Hk * Wk * C;
      Bilin b;
      bilin(u, v, Wk, Hk, boundary, &b);
      for (int c = 0; c < C; ++c) {
        float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
        float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
        float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
        float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
        float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
        if (li == 0) out[pix * C + c] = (1.0f - frac) * sample;  /* :855 */
        else out[pix * C + c] += frac * sample;                  /* :858 */
      }
    }
  }
}

/* Texture.swift:870-932 (grad_pyramid). */
void orc_tex_mip_grad_pyramid(const float* uv, const float* uv_da,
                              const float* d_out, const int64_t* offsets,
                              const int32_t* level_h, const int32_t* level_w,
                              int L, int64_t level_batch_mul, int N, int Hi,
                              int Wi, int Ht, int Wt, int C, int boundary,
                              int mip_linear, float* d_packed) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    float u = uv[pix * 2 + 0], v = uv[pix * 2 + 1];
    int k0, k1;
    float frac;
    mip_lod(uv_da + pix * 4, Ht, Wt, L, mip_linear, &k0, &k1, &frac);
    for (int li = 0; li < 2; ++li) {
      int k = li == 0 ? k0 : k1;
      float scale = li == 0 ? (1.0f - frac) : frac;
      int Hk = level_h[k], Wk = level_w[k];
      float* lv = d_packed + offsets[k] + (int64_t)pn * level_batch_mul * Hk * Wk * C;
      Bilin b;
      bilin(u, v, Wk, Hk, boundary, &b);
      for (int c = 0; c < C; ++c) {
        float g = d_out[pix * C + c] * scale;
        sadd(&lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c], b.w00 * g);
        sadd(&lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c], b.w10 * g);
        sadd(&lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c], b.w01 * g);
        sadd(&lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c], b.w11 * g);
      }
    }
  }
}

/* Texture.swift:934-999 (grad_uv). */
void orc_tex_mip_grad_uv(const float* packed, int64_t level_batch_mul,
                         const float* uv, const float* uv_da,
                         const float* d_out, const int64_t* offsets,
                         const int32_t* level_h, const int32_t* level_w,
                         int L, int N, int Hi, int Wi, int Ht, int Wt, int C,
                         int boundary, int mip_linear, float* d_uv) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    float u = uv[pix * 2 + 0], v = uv[pix * 2 + 1];
    int k0, k1;
    float frac;
    mip_lod(uv_da + pix * 4, Ht, Wt, L, mip_linear, &k0, &k1, &frac);
    float dfx_total = 0.0f, dfy_total = 0.0f;
    for (int li = 0; li < 2; ++li) {
      int k = li == 0 ? k0 : k1;
      float scale = li == 0 ? (1.0f - frac) : frac;
      int Hk = level_h[k], Wk = level_w[k];
      const float* lv = packed + offsets[k] + (int64_t)pn * level_batch_mul * Hk * Wk * C;
      Bilin b;
      bilin(u, v, Wk, Hk, boundary, &b);
      float m00 = (1.0f - b.ox0) * (1.0f - b.oy0);
      float m10 = (1.0f - b.ox1) * (1.0f - b.oy0);
      float m01 = (1.0f - b.ox0) * (1.0f - b.oy1);
      float m11 = (1.0f - b.ox1) * (1.0f - b.oy1);
      float dfx = 0.0f, dfy = 0.0f;
      for (int c = 0; c < C; ++c) {
        float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c] * m00;
        float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c] * m10;
        float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c] * m01;
        float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c] * m11;
        float g = d_out[pix * C + c] * scale;
        dfx += g * ((1.0f - b.fy) * (t10 - t00) + b.fy * (t11 - t01));
        dfy += g * ((1.0f - b.fx) * (t01 - t00) + b.fx * (t11 - t10));
      }
      dfx_total += dfx * (float)Wk;
      dfy_total += dfy * (float)Hk;
    }
    d_uv[pix * 2 + 0] = dfx_total;
    d_uv[pix * 2 + 1] = dfy_total;
  }
}

/* Texture.swift:1011-1102 (grad_uvDA).  As in the reference, the body does
 * not consult MIP_LINEAR: mip-nearest receives the trilinear surrogate. */
void orc_tex_mip_grad_uvda(const float* packed, int64_t level_batch_mul,
                           const float* uv, const float* uv_da,
                           const float* d_out, const int64_t* offsets,
                           const int32_t* level_h, const int32_t* level_w,
                           int L, int N, int Hi, int Wi, int Ht, int Wt,
                           int C, int boundary, float* d_uv_da) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    float u = uv[pix * 2 + 0], v = uv[pix * 2 + 1];
    const float* da = uv_da + pix * 4;
    float* o = d_uv_da + pix * 4;
    float sx = da[0] * (float)Wt;
    float sy = da[1] * (float)Wt;
    float tx_ = da[2] * (float)Ht;
    float ty_ = da[3] * (float)Ht;
    float Asq = sx * sx + tx_ * tx_;
    float Bsq = sy * sy + ty_ * ty_;
    float rho_sq = fmaxf(Asq, Bsq);
    float lod_raw = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
    if (lod_raw <= 0.0f || lod_raw >= (float)(L - 1)) {
      o[0] = o[1] = o[2] = o[3] = 0.0f;
      continue;
    }
    int k0 = f2i(floorf(lod_raw));
    int k1 = k0 + 1;
    if (k1 >= L) k1 = L - 1;
    float d_lod = 0.0f;
    for (int li = 0; li < 2; ++li) {
      int k = li == 0 ? k0 : k1;
      float sign = li == 0 ? -1.0f : 1.0f;
      int Hk = level_h[k], Wk = level_w[k];
      const float* lv = packed + offsets[k] + (int64_t)pn * level_batch_mul * Hk * Wk * C;
      Bilin b;
      bilin(u, v, Wk, Hk, boundary, &b);
      for (int c = 0; c < C; ++c) {
        float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
        float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
        float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
        float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
        float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
        d_lod += sign * sample * d_out[pix * C + c];
      }
    }
    float ln2 = 0.6931471805599453f;
    float dlod_drho_sq = 1.0f / (2.0f * rho_sq * ln2);
    float A_is_max = (Asq >= Bsq) ? 1.0f : 0.0f;
    float B_is_max = 1.0f - A_is_max;
    o[0] = d_lod * dlod_drho_sq * A_is_max * 2.0f * sx * (float)Wt;
    o[1] = d_lod * dlod_drho_sq * B_is_max * 2.0f * sy * (float)Wt;
    o[2] = d_lod * dlod_drho_sq * A_is_max * 2.0f * tx_ * (float)Ht;
    o[3] = d_lod * dlod_drho_sq * B_is_max * 2.0f * ty_ * (float)Ht;
  }
}

/* ===================================================================== */
/* antialias                                                             */
/* ===================================================================== */

typedef struct {
  int32_t a, b, t, k;
} EdgeRef;

static int edge_cmp(const void* l, const void* r) {
  const EdgeRef* x = (const EdgeRef*)l;
  const EdgeRef* y = (const EdgeRef*)r;
  if (x->a != y->a) return x->a < y->a ? -1 : 1;
  if (x->b != y->b) return x->b < y->b ? -1 : 1;
  /* Tie order among equal keys does not change the result (a run of two
   * pairs its members either way; longer runs all become -2).  Fixed here
   * only to make qsort's output deterministic. */
  if (x->t != y->t) return x->t < y->t ? -1 : 1;
  return x->k < y->k ? -1 : (x->k > y->k);
}

/* Antialias.swift:19-66 (antialiasConstructTopologyHash). */
void orc_aa_topology(const int32_t* tri, int T, int32_t* topo) {
  EdgeRef* e = (EdgeRef*)malloc(sizeof(EdgeRef) * (size_t)T * 3);
  for (int t = 0; t < T; ++t) {
    int32_t v0 = tri[t * 3 + 0], v1 = tri[t * 3 + 1], v2 = tri[t * 3 + 2];
    int32_t p[3][2] = {{v1, v2}, {v2, v0}, {v0, v1}};  /* :33 */
    for (int k = 0; k < 3; ++k) {
      int32_t lo = p[k][0] < p[k][1] ? p[k][0] : p[k][1];
      int32_t hi = p[k][0] < p[k][1] ? p[k][1] : p[k][0];
      e[t * 3 + k].a = lo;
      e[t * 3 + k].b = hi;
      e[t * 3 + k].t = t;
      e[t * 3 + k].k = k;
    }
  }
  qsort(e, (size_t)T * 3, sizeof(EdgeRef), edge_cmp);
  for (int64_t i = 0; i < (int64_t)T * 3; ++i) topo[i] = -1;
  int64_t i = 0, n = (int64_t)T * 3;
  while (i < n) {
    int64_t j = i + 1;
    while (j < n && e[j].a == e[i].a && e[j].b == e[i].b) ++j;
    int64_t run = j - i;
    if (run == 2) {
      topo[e[i].t * 3 + e[i].k] = e[i + 1].t;
      topo[e[i + 1].t * 3 + e[i + 1].k] = e[i].t;
    } else if (run > 2) {
      for (int64_t q = i; q < j; ++q) topo[e[q].t * 3 + e[q].k] = -2;
    }
    i = j;
  }
  free(e);
}

/* Per-direction state of the silhouette block (Antialias.swift:168-326). */
typedef struct {
  float alpha[4];
  int64_t nbase[4];
  int active[4];
  float alpha_sum;
  int i_e0[4], i_e1[4];
  float e0x[4], e0y[4], e1x[4], e1y[4];
  float t[4], denom[4], dadxy[4];
  int horiz[4];
} Sil;

/* Antialias.swift:168-326 (silhouetteBlock), restated for pixel (pn,ph,pw). */
static void silhouette(const float* rast, const float* pos,
                       const int32_t* tri, const int32_t* topo, int pn,
                       int ph, int pw, int H, int W, int C, int V, Sil* s) {
  int64_t rast_base = (((int64_t)pn * H + ph) * W + pw) * 4;
  int tri_p = f2i(rast[rast_base + 3]) - 1;
  const float* p = pos + (int64_t)pn * V * 4;
  for (int d = 0; d < 4; ++d) {
    s->alpha[d] = 0.0f;
    s->nbase[d] = 0;
    s->active[d] = 0;
    s->i_e0[d] = s->i_e1[d] = -1;
    s->e0x[d] = s->e0y[d] = s->e1x[d] = s->e1y[d] = 0.0f;
    s->t[d] = s->denom[d] = s->dadxy[d] = 0.0f;
    s->horiz[d] = 0;
  }
  s->alpha_sum = 0.0f;
  for (int dir = 0; dir < 4; ++dir) {
    int dh = 0, dw = 0;
    if (dir == 0) dw = 1;
    else if (dir == 1) dh = 1;
    else if (dir == 2) dw = -1;
    else dh = -1;
    int nh = ph + dh, nw = pw + dw;
    if (nh < 0 || nh >= H || nw < 0 || nw >= W) continue;
    int64_t n_rast_base = (((int64_t)pn * H + nh) * W + nw) * 4;
    int tri_n = f2i(rast[n_rast_base + 3]) - 1;
    if (tri_p == tri_n) continue;
    if (tri_p < 0 && tri_n < 0) continue;
    int fg_tri, target;
    if (tri_p >= 0 && tri_n >= 0) {
      int k_at_p = -1;
      if (topo[tri_p * 3 + 0] == tri_n) k_at_p = 0;
      else if (topo[tri_p * 3 + 1] == tri_n) k_at_p = 1;
      else if (topo[tri_p * 3 + 2] == tri_n) k_at_p = 2;
      if (k_at_p < 0) continue;
      fg_tri = tri_p;
      target = tri_n;
    } else if (tri_p >= 0) {
      fg_tri = tri_p;
      target = -1;
    } else {
      fg_tri = tri_n;
      target = -1;
    }
    /* :232-264 edge selection */
    int i_e0 = -1, i_e1 = -1;
    float e0x = 0, e0y = 0, e1x = 0, e1y = 0;
    {
      float pcx = (float)pw + 0.5f, pcy = (float)ph + 0.5f;
      float ncx = (float)nw + 0.5f, ncy = (float)nh + 0.5f;
      int k_sel = -1;
      for (int kk = 0; kk < 3; ++kk) {
        if (topo[fg_tri * 3 + kk] != target) continue;
        int ie0 = tri[fg_tri * 3 + ((kk + 1) % 3)];
        int ie1 = tri[fg_tri * 3 + ((kk + 2) % 3)];
        float wc0 = p[(int64_t)ie0 * 4 + 3];
        float wc1 = p[(int64_t)ie1 * 4 + 3];
        float E0x = (p[(int64_t)ie0 * 4 + 0] / wc0 + 1.0f) * (float)W * 0.5f;
        float E0y = (1.0f - p[(int64_t)ie0 * 4 + 1] / wc0) * (float)H * 0.5f;
        float E1x = (p[(int64_t)ie1 * 4 + 0] / wc1 + 1.0f) * (float)W * 0.5f;
        float E1y = (1.0f - p[(int64_t)ie1 * 4 + 1] / wc1) * (float)H * 0.5f;
        float ex = E1x - E0x, ey = E1y - E0y;
        float side_p = ex * (pcy - E0y) - ey * (pcx - E0x);
        float side_n = ex * (ncy - E0y) - ey * (ncx - E0x);
        if (side_p * side_n < 0.0f) {
          k_sel = kk;
          i_e0 = ie0;
          i_e1 = ie1;
          e0x = E0x; e0y = E0y; e1x = E1x; e1y = E1y;
          break;
        }
      }
      if (k_sel < 0) continue;
    }
    float beta = 0.0f, t_val = 0.0f, denom = 0.0f, dbeta = 0.0f;
    int is_horiz = (dh == 0);
    float pcx = (float)pw + 0.5f, pcy = (float)ph + 0.5f;
    if (is_horiz) {  /* :274-292 */
      float dyv = e1y - e0y;
      denom = dyv;
      if (fabsf(dyv) >= 1e-7f) {
        float tval = (pcy - e0y) / dyv;
        t_val = tval;
        if (tval >= 0.0f && tval <= 1.0f) {
          float xe = e0x + tval * (e1x - e0x);
          if (xe > (float)pw && xe < (float)(pw + 1)) {
            float dd = xe - pcx;
            beta = 0.5f - fabsf(dd);
            dbeta = (dd > 0.0f) ? -1.0f : 1.0f;
          }
        }
      }
    } else {  /* :293-309 */
      float dxv = e1x - e0x;
      denom = dxv;
      if (fabsf(dxv) >= 1e-7f) {
        float tval = (pcx - e0x) / dxv;
        t_val = tval;
        if (tval >= 0.0f && tval <= 1.0f) {
          float ye = e0y + tval * (e1y - e0y);
          if (ye > (float)ph && ye < (float)(ph + 1)) {
            float dd = ye - pcy;
            beta = 0.5f - fabsf(dd);
            dbeta = (dd > 0.0f) ? -1.0f : 1.0f;
          }
        }
      }
    }
    if (beta <= 0.0f) continue;
    s->alpha[dir] = beta;
    s->nbase[dir] = (((int64_t)pn * H + nh) * W + nw) * C;
    s->active[dir] = 1;
    s->alpha_sum += beta;
    s->i_e0[dir] = i_e0;
    s->i_e1[dir] = i_e1;
    s->e0x[dir] = e0x; s->e0y[dir] = e0y;
    s->e1x[dir] = e1x; s->e1y[dir] = e1y;
    s->t[dir] = t_val;
    s->denom[dir] = denom;
    s->dadxy[dir] = dbeta;
    s->horiz[dir] = is_horiz;
  }
}

/* Antialias.swift:333-358 (fwd). */
void orc_aa_fwd(const float* color, const float* rast, const float* pos,
                const int32_t* tri, const int32_t* topo, int N, int H, int W,
                int C, int V, float* out) {
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pw = (int)(pix % W);
    int ph = (int)((pix / W) % H);
    int pn = (int)(pix / ((int64_t)H * W));
    Sil s;
    silhouette(rast, pos, tri, topo, pn, ph, pw, H, W, C, V, &s);
    for (int c = 0; c < C; ++c) {
      float cp = color[pix * C + c];
      float acc = cp;
      for (int d = 0; d < 4; ++d) {
        if (!s.active[d]) continue;
        float cn = color[s.nbase[d] + c];
        acc += s.alpha[d] * (cn - cp);
      }
      out[pix * C + c] = acc;
    }
  }
}

/* Antialias.swift:498-524 (bwd_color). */
void orc_aa_bwd_color(const float* rast, const float* pos, const int32_t* tri,
                      const int32_t* topo, const float* d_out, int N, int H,
                      int W, int C, int V, float* d_color) {
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pw = (int)(pix % W);
    int ph = (int)((pix / W) % H);
    int pn = (int)(pix / ((int64_t)H * W));
    Sil s;
    silhouette(rast, pos, tri, topo, pn, ph, pw, H, W, C, V, &s);
    for (int c = 0; c < C; ++c) {
      float g = d_out[pix * C + c];
      sadd(&d_color[pix * C + c], g * (1.0f - s.alpha_sum));
      for (int d = 0; d < 4; ++d) {
        if (!s.active[d]) continue;
        sadd(&d_color[s.nbase[d] + c], g * s.alpha[d]);
      }
    }
  }
}

/* Antialias.swift:388-496 (bwd_pos). */
void orc_aa_bwd_pos(const float* color, const float* rast, const float* pos,
                    const int32_t* tri, const int32_t* topo,
                    const float* d_out, int N, int H, int W, int C, int V,
                    float* d_pos) {
  int64_t total = (int64_t)N * H * W;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pw = (int)(pix % W);
    int ph = (int)((pix / W) % H);
    int pn = (int)(pix / ((int64_t)H * W));
    Sil s;
    silhouette(rast, pos, tri, topo, pn, ph, pw, H, W, C, V, &s);
    float halfW = (float)W * 0.5f;
    float halfH = (float)H * 0.5f;
    const float* p = pos + (int64_t)pn * V * 4;
    float* dp = d_pos + (int64_t)pn * V * 4;
    for (int d = 0; d < 4; ++d) {
      if (!s.active[d]) continue;
      float alpha = s.alpha[d];
      if (alpha <= 0.0f || alpha >= 1.0f) continue;
      float d_alpha = 0.0f;
      for (int c = 0; c < C; ++c) {
        float cp = color[pix * C + c];
        float cn = color[s.nbase[d] + c];
        float g = d_out[pix * C + c];
        d_alpha += g * (cn - cp);
      }
      if (d_alpha == 0.0f) continue;
      float e0x = s.e0x[d], e0y = s.e0y[d], e1x = s.e1x[d], e1y = s.e1y[d];
      float t = s.t[d], denom = s.denom[d], da = s.dadxy[d];
      float dade0x, dade0y, dade1x, dade1y;
      if (s.horiz[d]) {  /* :430-437 */
        float row_y = (float)ph + 0.5f;
        float ex_diff = e1x - e0x;
        float inv_denom_sq = 1.0f / (denom * denom);
        dade0x = da * (1.0f - t);
        dade1x = da * t;
        dade0y = da * ex_diff * (row_y - e1y) * inv_denom_sq;
        dade1y = da * (-ex_diff) * (row_y - e0y) * inv_denom_sq;
      } else {  /* :438-446 */
        float col_x = (float)pw + 0.5f;
        float ey_diff = e1y - e0y;
        float inv_denom_sq = 1.0f / (denom * denom);
        dade0y = da * (1.0f - t);
        dade1y = da * t;
        dade0x = da * ey_diff * (col_x - e1x) * inv_denom_sq;
        dade1x = da * (-ey_diff) * (col_x - e0x) * inv_denom_sq;
      }
      /* :450-494 */
      for (int e = 0; e < 2; ++e) {
        int iv = e == 0 ? s.i_e0[d] : s.i_e1[d];
        float dex = e == 0 ? dade0x : dade1x;
        float dey = e == 0 ? dade0y : dade1y;
        float wv = p[(int64_t)iv * 4 + 3];
        float inv_w = 1.0f / wv;
        float nd_x = p[(int64_t)iv * 4 + 0] * inv_w;
        float nd_y = p[(int64_t)iv * 4 + 1] * inv_w;
        float d_px = d_alpha * dex * halfW * inv_w;
        float d_py = d_alpha * dey * (-halfH) * inv_w;
        float d_pw = d_alpha * (dex * (-halfW * nd_x) + dey * (halfH * nd_y)) * inv_w;
        sadd(&dp[(int64_t)iv * 4 + 0], d_px);
        sadd(&dp[(int64_t)iv * 4 + 1], d_py);
        sadd(&dp[(int64_t)iv * 4 + 3], d_pw);
      }
    }
  }
}

/* ===================================================================== */
/* cube maps with mip filters, and the direction gradient                */
/* ===================================================================== */
/* An extension: the reference samples cube maps with the bilinear filter
 * only (Texture.swift:75-76) and returns a zero direction gradient
 * (:196-198).  The semantics restated here are this build's definition,
 * built from the reference's own pieces:
 *   - face selection and face (u, v) of Texture.swift:620-635;
 *   - the face (u, v) screen derivatives from the direction's derivatives
 *     dd = (dx/dX, dx/dY, dy/dX, dy/dY, dz/dX, dz/dY) by the chain rule
 *     through u = (sc/ma + 1)/2, v = (tc/ma + 1)/2 with the face fixed;
 *   - then exactly the 2D LOD, level choice, clamped bilinear sampling and
 *     two-rounding trilinear blend of :764-863 on the chosen face of each
 *     level (the pyramid is the 2x2 box pyramid of every face);
 *   - gradients: d_tex through the pyramid as in :870-932; d_dd as
 *     :1011-1102 (same lod_raw mask, A-vs-B rule and the trilinear
 *     surrogate for mip-nearest) chained through the face derivatives;
 *     d_dir through the sample position (:934-999 chained through the
 *     projection) plus, for mip filters, through the LOD's dependence on
 *     the direction.
 * Parity with the reference is unpinned by construction (it has no such
 * path); the tests pin it by reduction to the reference's 2D trilinear on
 * a face, to its cube bilinear at L = 1, and by finite differences. */

typedef struct {
  int face, as, at, am;  /* axes of sc, tc, ma */
  float ss, ts, ms;      /* their signs */
  float sc, tc, ma;
} CubeSel;

static inline CubeSel cube_select(float x, float y, float z) {
  CubeSel s;
  float ax = fabsf(x), ay = fabsf(y), az = fabsf(z);
  if (ax >= ay && ax >= az) {
    s.am = 0; s.ms = x > 0.0f ? 1.0f : -1.0f; s.ma = ax;
    s.at = 1; s.ts = -1.0f; s.tc = -y;
    if (x > 0.0f) { s.face = 0; s.as = 2; s.ss = -1.0f; s.sc = -z; }
    else          { s.face = 1; s.as = 2; s.ss = 1.0f;  s.sc = z; }
  } else if (ay >= az) {
    s.am = 1; s.ms = y > 0.0f ? 1.0f : -1.0f; s.ma = ay;
    s.as = 0; s.ss = 1.0f; s.sc = x;
    if (y > 0.0f) { s.face = 2; s.at = 2; s.ts = 1.0f;  s.tc = z; }
    else          { s.face = 3; s.at = 2; s.ts = -1.0f; s.tc = -z; }
  } else {
    s.am = 2; s.ms = z > 0.0f ? 1.0f : -1.0f; s.ma = az;
    s.at = 1; s.ts = -1.0f; s.tc = -y;
    if (z > 0.0f) { s.face = 4; s.as = 0; s.ss = 1.0f;  s.sc = x; }
    else          { s.face = 5; s.as = 0; s.ss = -1.0f; s.sc = -x; }
  }
  return s;
}

/* Face (u, v) screen derivatives (u_X, u_Y, v_X, v_Y) from dd. */
static inline void cube_face_da(const CubeSel* s, const float* dd, float* da4) {
  float inv = 0.5f / (s->ma * s->ma);
  float sX = s->ss * dd[2 * s->as], sY = s->ss * dd[2 * s->as + 1];
  float tX = s->ts * dd[2 * s->at], tY = s->ts * dd[2 * s->at + 1];
  float mX = s->ms * dd[2 * s->am], mY = s->ms * dd[2 * s->am + 1];
  da4[0] = (sX * s->ma - s->sc * mX) * inv;
  da4[1] = (sY * s->ma - s->sc * mY) * inv;
  da4[2] = (tX * s->ma - s->tc * mX) * inv;
  da4[3] = (tY * s->ma - s->tc * mY) * inv;
}

/* mode: 0 = bilinear (level 0 only), 1 = mip-nearest, 2 = trilinear.
 * packed: pyramid of the N*6 face textures (level 0 included), offsets per
 * level; level_batch_mul as in orc_tex_mip_fwd.  dd: [N,Hi,Wi,6] with any
 * bias already folded in (NULL for mode 0). */
void orc_tex_cube_mip_fwd(const float* packed, int64_t level_batch_mul, const float* dir,
                          const float* dd, const int64_t* offsets, const int32_t* level_h,
                          const int32_t* level_w, int L, int N, int Hi, int Wi, int C, int mode,
                          float* out) {
  int64_t total = (int64_t)N * Hi * Wi;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    CubeSel s = cube_select(dir[pix * 3], dir[pix * 3 + 1], dir[pix * 3 + 2]);
    float inv_ma = 1.0f / s.ma;
    float u = (s.sc * inv_ma + 1.0f) * 0.5f;
    float v = (s.tc * inv_ma + 1.0f) * 0.5f;
    int k0 = 0, k1 = 0;
    float frac = 0.0f;
    if (mode > 0) {
      float da4[4];
      cube_face_da(&s, dd + pix * 6, da4);
      mip_lod(da4, level_h[0], level_w[0], L, mode == 2, &k0, &k1, &frac);
    }
    for (int li = 0; li < 2; ++li) {
      int k = li == 0 ? k0 : k1;
      int Hk = level_h[k], Wk = level_w[k];
      const float* lv =
          packed + offsets[k] + ((int64_t)pn * level_batch_mul * 6 + s.face) * Hk * Wk * C;
      Bilin b;
      bilin(u, v, Wk, Hk, 1 /* clamp */, &b);
      for (int c = 0; c < C; ++c) {
        float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
        float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
        float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
        float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
        float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
        if (mode == 0) {
          out[pix * C + c] = sample;
        } else if (li == 0) {
          out[pix * C + c] = (1.0f - frac) * sample;
        } else {
          out[pix * C + c] += frac * sample;
        }
      }
      if (mode == 0) break;
    }
  }
}

/* Backward: d_packed (pyramid of the N*6 faces, zeroed by the caller),
 * d_dir [N,Hi,Wi,3] (NULL to skip), d_dd [N,Hi,Wi,6] (mip modes; NULL to
 * skip). */
void orc_tex_cube_mip_bwd(const float* packed, int64_t level_batch_mul, const float* dir,
                          const float* dd, const float* d_out, const int64_t* offsets,
                          const int32_t* level_h, const int32_t* level_w, int L, int N, int Hi,
                          int Wi, int C, int mode, float* d_packed, float* d_dir, float* d_dd) {
  int64_t total = (int64_t)N * Hi * Wi;
  int Ht = level_h[0], Wt = level_w[0];
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
  for (int64_t pix = 0; pix < total; ++pix) {
    int pn = (int)(pix / ((int64_t)Hi * Wi));
    const float* g = d_out + pix * C;
    CubeSel s = cube_select(dir[pix * 3], dir[pix * 3 + 1], dir[pix * 3 + 2]);
    float inv_ma = 1.0f / s.ma;
    float u = (s.sc * inv_ma + 1.0f) * 0.5f;
    float v = (s.tc * inv_ma + 1.0f) * 0.5f;
    int k0 = 0, k1 = 0;
    float frac = 0.0f;
    float da4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (mode > 0) {
      cube_face_da(&s, dd + pix * 6, da4);
      mip_lod(da4, Ht, Wt, L, mode == 2, &k0, &k1, &frac);
    }
    /* sample-position gradient (:934-999) and the pyramid scatter (:870-932) */
    float du = 0.0f, dv = 0.0f;
    for (int li = 0; li < (mode == 0 ? 1 : 2); ++li) {
      int k = li == 0 ? k0 : k1;
      float scale = mode == 0 ? 1.0f : (li == 0 ? (1.0f - frac) : frac);
      int Hk = level_h[k], Wk = level_w[k];
      int64_t base = offsets[k] + ((int64_t)pn * level_batch_mul * 6 + s.face) * Hk * Wk * C;
      const float* lv = packed + base;
      float* dl = d_packed + base;
      Bilin b;
      bilin(u, v, Wk, Hk, 1, &b);
      float dfx = 0.0f, dfy = 0.0f;
      for (int c = 0; c < C; ++c) {
        float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
        float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
        float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
        float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
        float gs = g[c] * scale;
        sadd(&dl[((int64_t)b.iy0 * Wk + b.ix0) * C + c], b.w00 * gs);
        sadd(&dl[((int64_t)b.iy0 * Wk + b.ix1) * C + c], b.w10 * gs);
        sadd(&dl[((int64_t)b.iy1 * Wk + b.ix0) * C + c], b.w01 * gs);
        sadd(&dl[((int64_t)b.iy1 * Wk + b.ix1) * C + c], b.w11 * gs);
        dfx += gs * ((1.0f - b.fy) * (t10 - t00) + b.fy * (t11 - t01));
        dfy += gs * ((1.0f - b.fx) * (t01 - t00) + b.fx * (t11 - t10));
      }
      du += dfx * (float)Wk;
      dv += dfy * (float)Hk;
    }
    float inv2 = 0.5f / (s.ma * s.ma);
    float gd[3] = {0.0f, 0.0f, 0.0f};
    /* d u / d dir = inv2 * (ss*ma e_as - sc*ms e_am), likewise v */
    gd[s.as] += du * (s.ss * s.ma * inv2);
    gd[s.at] += dv * (s.ts * s.ma * inv2);
    gd[s.am] -= (du * s.sc + dv * s.tc) * s.ms * inv2;
    float gdd[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (mode > 0) {
      float sx = da4[0] * (float)Wt, sy = da4[1] * (float)Wt;
      float tx_ = da4[2] * (float)Ht, ty_ = da4[3] * (float)Ht;
      float Asq = sx * sx + tx_ * tx_;
      float Bsq = sy * sy + ty_ * ty_;
      float rho_sq = fmaxf(Asq, Bsq);
      float lod_raw = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
      if (lod_raw > 0.0f && lod_raw < (float)(L - 1)) {
        int j0 = f2i(floorf(lod_raw));
        int j1 = j0 + 1;
        if (j1 >= L) j1 = L - 1;
        float d_lod = 0.0f;
        for (int li = 0; li < 2; ++li) {
          int k = li == 0 ? j0 : j1;
          float sign = li == 0 ? -1.0f : 1.0f;
          int Hk = level_h[k], Wk = level_w[k];
          const float* lv =
              packed + offsets[k] + ((int64_t)pn * level_batch_mul * 6 + s.face) * Hk * Wk * C;
          Bilin b;
          bilin(u, v, Wk, Hk, 1, &b);
          for (int c = 0; c < C; ++c) {
            float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
            float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
            float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
            float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
            float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
            d_lod += sign * sample * g[c];
          }
        }
        float ln2 = 0.6931471805599453f;
        float dlod_drho_sq = 1.0f / (2.0f * rho_sq * ln2);
        float A_is_max = (Asq >= Bsq) ? 1.0f : 0.0f;
        float B_is_max = 1.0f - A_is_max;
        /* gradients of the face derivatives (the 2D d_uvDA) */
        float duX = d_lod * dlod_drho_sq * A_is_max * 2.0f * sx * (float)Wt;
        float duY = d_lod * dlod_drho_sq * B_is_max * 2.0f * sy * (float)Wt;
        float dvX = d_lod * dlod_drho_sq * A_is_max * 2.0f * tx_ * (float)Ht;
        float dvY = d_lod * dlod_drho_sq * B_is_max * 2.0f * ty_ * (float)Ht;
        const float* d6 = dd + pix * 6;
        float sX = s.ss * d6[2 * s.as], sY = s.ss * d6[2 * s.as + 1];
        float tX = s.ts * d6[2 * s.at], tY = s.ts * d6[2 * s.at + 1];
        float mX = s.ms * d6[2 * s.am], mY = s.ms * d6[2 * s.am + 1];
        /* through dd: u_X = inv2 * (sX*ma - sc*mX), ... */
        gdd[2 * s.as] += duX * s.ss * s.ma * inv2;
        gdd[2 * s.as + 1] += duY * s.ss * s.ma * inv2;
        gdd[2 * s.at] += dvX * s.ts * s.ma * inv2;
        gdd[2 * s.at + 1] += dvY * s.ts * s.ma * inv2;
        gdd[2 * s.am] -= (duX * s.sc + dvX * s.tc) * s.ms * inv2;
        gdd[2 * s.am + 1] -= (duY * s.sc + dvY * s.tc) * s.ms * inv2;
        /* through the direction: d u_X / d sc = -inv2*mX,
         * d u_X / d ma = inv2*sX - 2*u_X/ma, likewise for the others */
        gd[s.as] -= (duX * mX + duY * mY) * s.ss * inv2;
        gd[s.at] -= (dvX * mX + dvY * mY) * s.ts * inv2;
        gd[s.am] += s.ms * (duX * (sX * inv2 - 2.0f * da4[0] * inv_ma) +
                            duY * (sY * inv2 - 2.0f * da4[1] * inv_ma) +
                            dvX * (tX * inv2 - 2.0f * da4[2] * inv_ma) +
                            dvY * (tY * inv2 - 2.0f * da4[3] * inv_ma));
      }
    }
    if (d_dir) {
      d_dir[pix * 3 + 0] = gd[0];
      d_dir[pix * 3 + 1] = gd[1];
      d_dir[pix * 3 + 2] = gd[2];
    }
    if (d_dd && mode > 0)
      for (int i = 0; i < 6; ++i) d_dd[pix * 6 + i] = gdd[i];
  }
}
