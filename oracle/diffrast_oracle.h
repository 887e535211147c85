/*
 * CPU restatement of the mlx-swift-diffrast hot path (rasterize, interpolate,
 * texture, antialias; forward and backward).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels and the CPU baseline timed beside them.  Nothing in the product
 * path links, loads or calls it.
 *
 * Every function restates one Metal kernel body (or one piece of host-side
 * orchestration) of the reference and cites its file:line.  The restatement
 * is executed sequentially, one "thread" after another, in thread-index
 * order.  Relaxed float atomics therefore become ordinary adds in
 * thread-index order, and the rasterizer's tile bins come out in ascending
 * triangle order (the order a sequential execution of the reference's
 * `atomic_fetch_add` append produces).
 *
 * All float arithmetic is fp32, compiled with -ffp-contract=off and no
 * fast-math, so each expression rounds exactly as written.
 *
 * Layouts are the reference's: row-major, channels last.
 */
#ifndef DIFFRAST_ORACLE_H
#define DIFFRAST_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- rasterize (Sources/MLXDiffRast/Rasterize.swift) ---------------- */

#define ORC_TILE_SIZE 16   /* Rasterize.swift:164 */
#define ORC_MAX_PER_TILE 128 /* Rasterize.swift:171 */

void orc_rast_precompute(const float* pos, int64_t pos_batch_stride,
                         const int32_t* tri, const int32_t* ranges,
                         int N, int V, int T, float* screen);

int64_t orc_rast_bin_count(const float* screen, int N, int T, int H, int W,
                           int32_t* counts);

void orc_rast_bin_fill(const float* screen, int N, int T, int H, int W,
                       const int64_t* offsets, int32_t* fill, int32_t* list);

void orc_rast_fwd(const float* screen, const int64_t* offsets,
                  const int32_t* counts, const int32_t* list,
                  const float* peel, int N, int T, int H, int W,
                  int max_per_tile, float* rast, float* rast_db);

void orc_rast_bwd(const float* pos, int64_t pos_batch_stride,
                  const int32_t* tri, const float* rast, const float* d_rast,
                  const float* d_rast_db, int N, int V, int H, int W,
                  float* d_pos);

/* ---- interpolate (Sources/MLXDiffRast/Interpolate.swift) ------------ */

void orc_interp_fwd(const float* attr, int64_t attr_batch_stride,
                    const float* rast, const int32_t* tri,
                    int N, int H, int W, int V, int A, float* out);

void orc_interp_fwd_da(const float* attr, int64_t attr_batch_stride,
                       const float* rast, const float* rast_db,
                       const int32_t* tri, const int32_t* diff_idx,
                       int N, int H, int W, int V, int A, int K,
                       float* out, float* out_da);

void orc_interp_grad_attr(const float* rast, const int32_t* tri,
                          const float* d_out, int N, int H, int W, int V,
                          int A, int64_t d_attr_batch_stride, float* d_attr);

void orc_interp_grad_attr_da(const float* rast, const float* rast_db,
                             const int32_t* tri, const float* d_out,
                             const float* d_out_da, const int32_t* diff_idx,
                             int N, int H, int W, int V, int A, int K,
                             int64_t d_attr_batch_stride, float* d_attr);

void orc_interp_grad_rast(const float* attr, int64_t attr_batch_stride,
                          const float* rast, const int32_t* tri,
                          const float* d_out, int N, int H, int W, int V,
                          int A, float* d_rast);

void orc_interp_grad_rast_db(const float* attr, int64_t attr_batch_stride,
                             const float* rast, const int32_t* tri,
                             const float* d_out_da, const int32_t* diff_idx,
                             int N, int H, int W, int V, int A, int K,
                             float* d_rast_db);

/* ---- texture (Sources/MLXDiffRast/Texture.swift) -------------------- */

enum { ORC_WRAP = 0, ORC_CLAMP = 1, ORC_ZERO = 2, ORC_CUBE = 3 };

void orc_tex_fwd(const float* tex, int64_t tex_batch_stride, const float* uv,
                 int N, int Hi, int Wi, int Ht, int Wt, int C, int boundary,
                 float* out);
void orc_tex_grad_tex(const float* uv, const float* d_out, int N, int Hi,
                      int Wi, int Ht, int Wt, int C, int boundary,
                      int64_t d_tex_batch_stride, float* d_tex);
void orc_tex_grad_uv(const float* tex, int64_t tex_batch_stride,
                     const float* uv, const float* d_out, int N, int Hi,
                     int Wi, int Ht, int Wt, int C, int boundary, float* d_uv);

void orc_tex_nearest_fwd(const float* tex, int64_t tex_batch_stride,
                         const float* uv, int N, int Hi, int Wi, int Ht,
                         int Wt, int C, int boundary, float* out);
void orc_tex_nearest_grad_tex(const float* uv, const float* d_out, int N,
                              int Hi, int Wi, int Ht, int Wt, int C,
                              int boundary, int64_t d_tex_batch_stride,
                              float* d_tex);

void orc_tex_cube_fwd(const float* tex, int64_t tex_batch_stride,
                      const float* dir, int N, int Hi, int Wi, int Ht, int Wt,
                      int C, float* out);
void orc_tex_cube_grad_tex(const float* dir, const float* d_out, int N,
                           int Hi, int Wi, int Ht, int Wt, int C,
                           int64_t d_tex_batch_stride, float* d_tex);

/* Mip pyramid: number of levels, and per-level H/W/offset (in floats of a
 * packed buffer that holds Nt batches per level). */
int orc_mip_levels(int H, int W, int max_level, int32_t* level_h,
                   int32_t* level_w);
void orc_mip_build(const float* tex, int Nt, int H, int W, int C, int L,
                   const int64_t* offsets, float* packed);
void orc_mip_collapse(const float* d_packed, int Nt, int H, int W, int C,
                      int L, const int64_t* offsets, float* d_tex);

void orc_tex_mip_fwd(const float* packed, int64_t level_batch_mul,
                     const float* uv, const float* uv_da,
                     const int64_t* offsets, const int32_t* level_h,
                     const int32_t* level_w, int L, int N, int Hi, int Wi,
                     int Ht, int Wt, int C, int boundary, int mip_linear,
                     float* out);
void orc_tex_mip_grad_pyramid(const float* uv, const float* uv_da,
                              const float* d_out, const int64_t* offsets,
                              const int32_t* level_h, const int32_t* level_w,
                              int L, int64_t level_batch_mul, int N, int Hi,
                              int Wi, int Ht, int Wt, int C, int boundary,
                              int mip_linear, float* d_packed);
void orc_tex_mip_grad_uv(const float* packed, int64_t level_batch_mul,
                         const float* uv, const float* uv_da,
                         const float* d_out, const int64_t* offsets,
                         const int32_t* level_h, const int32_t* level_w,
                         int L, int N, int Hi, int Wi, int Ht, int Wt, int C,
                         int boundary, int mip_linear, float* d_uv);
void orc_tex_mip_grad_uvda(const float* packed, int64_t level_batch_mul,
                           const float* uv, const float* uv_da,
                           const float* d_out, const int64_t* offsets,
                           const int32_t* level_h, const int32_t* level_w,
                           int L, int N, int Hi, int Wi, int Ht, int Wt,
                           int C, int boundary, float* d_uv_da);

/* Cube maps with mip filters and the direction gradient: an extension
 * (the reference has bilinear cube sampling only and a zero direction
 * gradient); mode 0 = bilinear, 1 = mip-nearest, 2 = trilinear. */
void orc_tex_cube_mip_fwd(const float* packed, int64_t level_batch_mul, const float* dir,
                          const float* dd, const int64_t* offsets, const int32_t* level_h,
                          const int32_t* level_w, int L, int N, int Hi, int Wi, int C, int mode,
                          float* out);
void orc_tex_cube_mip_bwd(const float* packed, int64_t level_batch_mul, const float* dir,
                          const float* dd, const float* d_out, const int64_t* offsets,
                          const int32_t* level_h, const int32_t* level_w, int L, int N, int Hi,
                          int Wi, int C, int mode, float* d_packed, float* d_dir, float* d_dd);

/* ---- antialias (Sources/MLXDiffRast/Antialias.swift) ---------------- */

void orc_aa_topology(const int32_t* tri, int T, int32_t* topo);

void orc_aa_fwd(const float* color, const float* rast, const float* pos,
                const int32_t* tri, const int32_t* topo, int N, int H, int W,
                int C, int V, float* out);
void orc_aa_bwd_color(const float* rast, const float* pos, const int32_t* tri,
                      const int32_t* topo, const float* d_out, int N, int H,
                      int W, int C, int V, float* d_color);
void orc_aa_bwd_pos(const float* color, const float* rast, const float* pos,
                    const int32_t* tri, const int32_t* topo,
                    const float* d_out, int N, int H, int W, int C, int V,
                    float* d_pos);

/* Threads used by the pixel loops (1 = the deterministic sequential order;
 * more threads change only the summation order of scatter-adds). */
void orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
