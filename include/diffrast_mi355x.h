/*
 * diffrast_mi355x: differentiable rasterization for AMD Instinct MI355X
 * (gfx950).  C ABI of libdiffrast_mi355x.so.
 *
 * One entry point per custom-VJP half of the reference's public ops
 * (mnmly/mlx-swift-diffrast, the Swift files under Sources/MLXDiffRast).  Each replaces
 * the Forward or VJP closure of one `CustomFunction` together with the
 * `MLXFast.metalKernel` dispatchers that closure calls:
 *
 *   dr_rasterize_fwd     Rasterize.swift:104-108, 123-128  (:823-894)
 *   dr_rasterize_bwd     Rasterize.swift:109-118, 129-139  (:850-866)
 *   dr_interpolate_fwd   Interpolate.swift:82-85, 113-119  (:475-500)
 *   dr_interpolate_bwd   Interpolate.swift:86-91, 120-127  (:502-541)
 *   dr_texture_mip_*     Texture.swift:144-161, 287-307
 *   dr_texture_fwd       Texture.swift:187-191, 222-227, 255-260, 309-315
 *   dr_texture_bwd       Texture.swift:192-199, 229-236, 261-267, 316-324
 *   dr_antialias_topology Antialias.swift:19-66
 *   dr_antialias_fwd     Antialias.swift:112-117  (:556-568)
 *   dr_antialias_bwd     Antialias.swift:118-128  (:570-600)
 *
 * and the loss and optimizer step of the reference's inverse-rendering
 * samples (Sources/{ColorFit,PoseFit,MeshFit}Example, MLXDiffRastExamples/Adam.swift):
 *
 *   dr_mse_loss          ColorFitExample/main.swift:62-66 and its gradient
 *   dr_adam_step         Adam.swift:36-43
 *
 * Conventions
 *   - All tensors are device memory (hipMalloc'd), fp32 or int32, row-major,
 *     channels last, in the reference's layouts:
 *       pos [N,V,4] clip space (x*w, y*w, z*w, w) or shared [V,4];
 *       tri [T,3]; rast / rast_db [N,H,W,4] = (u, v, z/w, tri_id+1) and
 *       (du/dx, du/dy, dv/dx, dv/dy); pixel (h=0, w=0) is the top-left.
 *   - A "batch stride" argument is the element distance between consecutive
 *     batch entries of a tensor; 0 means one tensor shared by every batch
 *     entry (the reference's N-broadcast, without materialising it).
 *   - The caller allocates every input and output.  The gradients the
 *     reference accumulates by scatter-add (d_pos of rasterize and
 *     antialias, d_attr, d_tex, d_color of antialias) are zero-filled by the
 *     library first, unless DR_ACCUMULATE is set in `flags`, in which case
 *     the library adds into what the buffer holds.  Every other output
 *     (d_rast, d_rast_db, d_uv, d_uv_da, d_bias_map) is overwritten.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL is the
 *     default stream) of the current HIP device.  Internal scratch is kept
 *     per (device, stream); calls on different streams may overlap.
 *   - Every call returns DR_OK or an error code and never throws; the message
 *     of the last error on the calling thread is dr_get_last_error().
 *   - HIP graph capture (no counterpart in the reference): a call made while
 *     its stream is being captured allocates nothing and waits for nothing,
 *     and is refused with DR_ERR_CAPTURE where it would (scratch that must
 *     grow, the first rasterize on a stream without dr_rasterize_reserve,
 *     range mode, whose ranges_host a replay would read stale).  Run each
 *     call once on the capturing stream first.  A graph uses the scratch of
 *     the stream it was captured on: replay it on that stream (or ordered
 *     with it), and not after dr_release_scratch.  Buffers a graph may use
 *     are kept when later calls grow the scratch, and one call reuses an
 *     earlier call's work (dr_rasterize_fwd_again, DR_RASTERIZE_BWD_REUSE)
 *     only within one capture once a stream has been captured.
 *   - Host-memory arguments are named *_host; everything else is device
 *     memory.
 *   - Indices are checked where they are used, so no input makes a kernel
 *     read or write out of range: a triangle with a vertex id outside
 *     [0, V) is not drawn and gets no gradient; a rast pixel whose triangle
 *     id is outside [0, T) is empty for interpolate and the backward passes;
 *     a diff_idx entry outside [0, A) gives zero derivatives.  (The
 *     reference reads out of range in these cases.)
 *   - Sizes: at most 715,827,882 triangles a call (tri is indexed as
 *     t * 3 + k in 32 bits; more returns DR_ERR_ARGUMENT) and fewer than 2^31
 *     16x16 pixel tiles; textures of any size.
 */
#ifndef DIFFRAST_MI355X_H
#define DIFFRAST_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DR_ABI_VERSION 1

typedef void* dr_stream_t; /* hipStream_t */

enum {
  DR_OK = 0,
  DR_ERR_ARGUMENT = 1, /* a shape or argument precondition failed */
  DR_ERR_HIP = 2,      /* a HIP runtime call failed */
  DR_ERR_MEMORY = 3,   /* scratch allocation failed */
  /* the call would allocate scratch memory, or wait for the device, while
   * its stream is being captured into a HIP graph (no counterpart in the
   * reference): run the same call once on that stream before capturing, or
   * size the rasterizer's scratch with dr_rasterize_reserve */
  DR_ERR_CAPTURE = 4
};

enum {
  DR_ACCUMULATE = 1u,
  /* dr_texture_bwd of a cube map: the direction gradient (an extension; the
   * reference returns zeros, Texture.swift:196-198, which is the default) */
  DR_CUBE_DIR_GRAD = 2u,
  /* dr_rasterize_bwd: the caller states that the last dr_rasterize_fwd* on
   * this stream drew this pos and tri, and that neither changed since (no
   * counterpart in the reference; an autograd wrapper knows both, e.g. for
   * every peel layer of one pos).  Per-triangle values that forward stored
   * are then reused instead of recomputed; the library still checks the
   * buffers and sizes against that forward's. */
  DR_RASTERIZE_BWD_REUSE = 4u
};

/* Texture.swift:8-17 (BoundaryMode) */
enum { DR_BOUNDARY_WRAP = 0, DR_BOUNDARY_CLAMP = 1, DR_BOUNDARY_ZERO = 2, DR_BOUNDARY_CUBE = 3 };
/* Texture.swift:35-40 (FilterMode) */
enum {
  DR_FILTER_NEAREST = 0,
  DR_FILTER_LINEAR = 1,
  DR_FILTER_LINEAR_MIPMAP_NEAREST = 2,
  DR_FILTER_LINEAR_MIPMAP_LINEAR = 3
};

int dr_abi_version(void);
const char* dr_get_last_error(void);
/* Frees the scratch memory held for the current device (all streams). */
int dr_release_scratch(void);

/* Kernel timing (no counterpart in the reference; for benchmarks).  While
 * enabled, every kernel launch is bracketed by HIP events on its stream.
 * dr_profile_report writes "name launches total_ms" lines into buf and
 * returns the full report length (it waits for the recorded events). */
int dr_profile_enable(int on);
/* Restricts timing to kernels of this name (NULL: every kernel). */
int dr_profile_select(const char* kernel);
int dr_profile_reset(void);
int dr_profile_report(char* buf, int len);

/* ---- rasterize ------------------------------------------------------- */

/* Forward of DiffRast.rasterize (Rasterize.swift:44-144).
 *   pos_batch_stride: V*4 for instanced pos [N,V,4]; 0 for range mode
 *     (shared pos [V,4]).
 *   ranges_host: NULL (every image draws triangles [0,T)), or a host array
 *     [N,2] of (first triangle, triangle count) per image (range mode).
 *   peel: NULL, or the rast [N,H,W,4] of the previous layer (depth peeling:
 *     only depths greater than that layer's are kept).
 *   rast_db: NULL for gradDB = false.
 * Unlike the reference, the per-tile triangle lists never overflow (the
 * reference drops triangles beyond 128 per 16x16 tile; see
 * dr_rasterize_fwd_ex), and equal depths resolve to the lowest triangle
 * index.
 * Host synchronisation: the first call on a stream counts every tile's
 * candidates exactly and waits for that count (it sizes the per-tile
 * lists), unless dr_rasterize_reserve sized them; later calls only read
 * back, asynchronously, the largest count of an earlier call.  A call
 * whose scratch memory must grow waits for the stream before freeing the
 * smaller buffer.  Range mode stages ranges_host through pinned memory and
 * does not wait (unless it runs four calls ahead of the device).  Calls
 * otherwise return before their work has run. */
int dr_rasterize_fwd(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                     const int32_t* ranges_host, const float* peel, int N, int V, int T,
                     int H, int W, float* rast, float* rast_db, dr_stream_t stream);

/* dr_rasterize_fwd with the reference's per-tile limit as an option
 * (MAX_PER_TILE, Rasterize.swift:164-171, 227-239, 410: a 16x16 tile keeps
 * at most 128 triangles and drops the rest in atomic append order).
 *   max_per_tile: 0 keeps every triangle (dr_rasterize_fwd); 1..1024 keeps
 *     at most that many triangles per tile: the lowest triangle indices
 *     among the tile's candidates (drawn triangles of nonzero area whose
 *     clamped pixel bounding box touches the tile), i.e. what a sequential
 *     execution of the reference's appends keeps.  max_per_tile = 128 gives
 *     the reference's result whenever its appends land in triangle order.
 * Other arguments, and the backward (dr_rasterize_bwd), as dr_rasterize_fwd. */
int dr_rasterize_fwd_ex(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                        const int32_t* ranges_host, const float* peel, int N, int V, int T,
                        int H, int W, float* rast, float* rast_db, int max_per_tile,
                        dr_stream_t stream);

/* dr_rasterize_fwd_ex for the next layer of a depth peel, or any call that
 * rasterizes the same triangles again (no counterpart call in the
 * reference, whose chained peel calls repeat their triangle setup and tile
 * binning, Rasterize.swift:36-38, 90-135).  When pos, pos_batch_stride,
 * tri, the contents of ranges_host, N, V, T, H, W and max_per_tile equal
 * those of the previous dr_rasterize_fwd / _ex / _again call on this
 * stream, that call's setup and tile lists are reused and only the
 * coverage pass runs; otherwise, or after a dr_rasterize_tile_counts call
 * on the stream, it does the full work of dr_rasterize_fwd_ex.  The caller
 * guarantees that the contents of pos and tri have not changed since that
 * call.  Results equal dr_rasterize_fwd_ex's. */
int dr_rasterize_fwd_again(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                           const int32_t* ranges_host, const float* peel, int N, int V, int T,
                           int H, int W, float* rast, float* rast_db, int max_per_tile,
                           dr_stream_t stream);

/* Binning report (no counterpart call in the reference; it exposes the
 * reference's bin counts, Rasterize.swift:227-239).  counts [N, ceil(H/16),
 * ceil(W/16)] (device int32) receives, per 16x16 tile, the number of drawn
 * triangles with nonzero area whose clamped pixel bounding box touches it:
 * the reference's bins[tile, 0].  Tiles above 128 are where the reference
 * drops triangles (MAX_PER_TILE, Rasterize.swift:164-171); this library does
 * not.  max_count_host: NULL, or receives the largest count (this waits for
 * the stream).  Arguments as dr_rasterize_fwd. */
int dr_rasterize_tile_counts(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                             const int32_t* ranges_host, int N, int V, int T, int H, int W,
                             int32_t* counts, int64_t* max_count_host, dr_stream_t stream);

/* Sizes the rasterizer's scratch on `stream` up front (no counterpart in
 * the reference, whose buffers MLX allocates per call, Rasterize.swift:
 * 256-266, 335-349): calls of up to N images of H x W drawing up to T
 * triangles each (range mode: T in all, N ranges), V vertices per image for
 * the backward's fp64 d_pos accumulator, and per-tile lists of
 * `tile_capacity` triangles.  The first forward on the stream then neither
 * counts its tiles nor waits: a tile with more candidates than the lists
 * hold takes the full scan (the same result), and the largest count, read
 * back asynchronously, raises the capacity of later calls.  For callers
 * that cannot allocate or wait inside their loop (HIP graph capture, serving
 * loops); every other call sizes the scratch itself. */
int dr_rasterize_reserve(int N, int V, int T, int H, int W, int tile_capacity,
                         dr_stream_t stream);

/* VJP of DiffRast.rasterize: d_pos (same layout and batch stride as pos;
 * range mode accumulates all images into the shared [V,4]).  d_rast_db may
 * be NULL (gradDB = false).  T = rows of tri; pixels whose triangle id is
 * outside [0, T) contribute nothing. */
int dr_rasterize_bwd(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                     const float* rast, const float* d_rast, const float* d_rast_db, int N,
                     int V, int T, int H, int W, float* d_pos, unsigned flags,
                     dr_stream_t stream);

/* ---- interpolate ----------------------------------------------------- */

/* Forward of DiffRast.interpolate (Interpolate.swift:43-132).
 *   attr [N,V,A] (attr_batch_stride = V*A) or shared [V,A] (stride 0).
 *   K = 0: basic path (rast_db, diff_idx, out_da unused).
 *   K > 0: DA path; diff_idx [K] device int32, or NULL for all attributes
 *     (then K must equal A); out_da [N,H,W,2K]. */
int dr_interpolate_fwd(const float* attr, int64_t attr_batch_stride, const float* rast,
                       const float* rast_db, const int32_t* tri, const int32_t* diff_idx,
                       int K, int N, int H, int W, int V, int T, int A, float* out,
                       float* out_da, dr_stream_t stream);

/* VJP of DiffRast.interpolate: d_attr (layout/stride d_attr_batch_stride,
 * 0 = accumulate every image into one [V,A]), d_rast [N,H,W,4] (channels 2,3
 * are zero), d_rast_db [N,H,W,4] (DA path only, may be NULL). */
int dr_interpolate_bwd(const float* attr, int64_t attr_batch_stride, const float* rast,
                       const float* rast_db, const int32_t* tri, const int32_t* diff_idx,
                       int K, const float* d_out, const float* d_out_da, int N, int H, int W,
                       int V, int T, int A, float* d_attr, int64_t d_attr_batch_stride,
                       float* d_rast, float* d_rast_db, unsigned flags, dr_stream_t stream);

/* ---- texture --------------------------------------------------------- */

/* textureConstructMip (Texture.swift:144-161): number of levels (level 0
 * included) of the 2x2 box pyramid of an [*, H, W, *] texture, capped at
 * max_level + 1 when max_level >= 0.  Writes each level's H/W (up to 32). */
int dr_texture_mip_levels(int H, int W, int max_level, int32_t* level_h_host,
                          int32_t* level_w_host);
/* Floats needed for levels 1..L-1 of Nt textures (level 0 is the texture). */
int64_t dr_texture_mip_size(int Nt, int H, int W, int C, int L);
/* Builds levels 1..L-1 of Nt textures into `pyramid`, level-major:
 * level k holds [Nt, Hk, Wk, C] starting after levels 1..k-1. */
int dr_texture_build_mip(const float* tex, int Nt, int H, int W, int C, int L, float* pyramid,
                         dr_stream_t stream);

/* Forward of DiffRast.texture (Texture.swift:62-131).
 *   tex: [Nt, Ht, Wt, C], or [Nt, 6, Ht, Wt, C] for DR_BOUNDARY_CUBE; Nt is
 *     1 (shared by every image) or N.
 *   pyramid / L: mip levels 1..L-1 from dr_texture_build_mip (mip filters;
 *     for a cube map, built for its Nt*6 faces as textures).
 *   uv: [N,Hi,Wi,2] (cube: direction [N,Hi,Wi,3]).
 *   uv_da: [N,Hi,Wi,4] (mip filters; cube: the direction's screen
 *     derivatives [N,Hi,Wi,6] = (dx/dX, dx/dY, dy/dX, dy/dY, dz/dX, dz/dY)).
 *   bias_map: NULL or [N,Hi,Wi] per-pixel mip level bias; bias: scalar
 *     bias.  Both scale uv_da by 2^bias before the LOD (Texture.swift:104-126).
 * Cube maps with the mip filters are an extension (the reference samples
 * cube maps bilinearly only, Texture.swift:75-76): the face's (u, v)
 * derivatives by the chain rule through the face projection, then the 2D
 * LOD and trilinear filter on that face. */
int dr_texture_fwd(const float* tex, const float* pyramid, int Nt, int Ht, int Wt, int C,
                   int L, const float* uv, const float* uv_da, const float* bias_map,
                   float bias, int filter, int boundary, int N, int Hi, int Wi, float* out,
                   dr_stream_t stream);

/* VJP of DiffRast.texture.  d_tex has tex's shape ([Nt,...]: a shared
 * texture receives the sum over images).  d_uv may be NULL; it is zero for
 * nearest, and for cube unless DR_CUBE_DIR_GRAD is set (then the direction
 * gradient through the sample position and, for mip filters, the LOD).
 * d_uv_da (mip filters) and d_bias_map (when bias_map is given) may be
 * NULL. */
int dr_texture_bwd(const float* tex, const float* pyramid, int Nt, int Ht, int Wt, int C,
                   int L, const float* uv, const float* uv_da, const float* bias_map,
                   float bias, int filter, int boundary, int N, int Hi, int Wi,
                   const float* d_out, float* d_tex, float* d_uv, float* d_uv_da,
                   float* d_bias_map, unsigned flags, dr_stream_t stream);

/* dr_texture_bwd that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops).  The mip filters' pyramid gradient,
 * the only memory dr_texture_bwd takes beyond its arguments, is kept in a
 * fixed device array of DR_TEXTURE_BWD_NOALLOC_FLOATS floats (32 MiB per
 * GPU, held until the process ends) instead of the library's scratch; a
 * texture whose pyramid needs more (dr_texture_mip_size of its levels, for
 * a cube map of its Nt*6 faces) is rejected with DR_ERR_ARGUMENT.  Every
 * call on one GPU shares that array, so calls that overlap on one GPU
 * (other streams, other threads) race.  Arguments and results as
 * dr_texture_bwd. */
#define DR_TEXTURE_BWD_NOALLOC_FLOATS (8 * 1024 * 1024)
int dr_texture_bwd_noalloc(const float* tex, const float* pyramid, int Nt, int Ht, int Wt,
                           int C, int L, const float* uv, const float* uv_da,
                           const float* bias_map, float bias, int filter, int boundary, int N,
                           int Hi, int Wi, const float* d_out, float* d_tex, float* d_uv,
                           float* d_uv_da, float* d_bias_map, unsigned flags,
                           dr_stream_t stream);

/* ---- antialias ------------------------------------------------------- */

/* antialiasConstructTopologyHash (Antialias.swift:19-66), on the GPU:
 * topo[t,k] = the other triangle sharing the edge opposite vertex k, -1
 * for a boundary edge, -2 for an edge of 3+ triangles.  Bit-identical to the
 * reference (the result does not depend on any ordering). */
int dr_antialias_topology(const int32_t* tri, int T, int32_t* topo, dr_stream_t stream);

/* Forward of DiffRast.antialias (Antialias.swift:90-131).  color [N,H,W,C],
 * rast [N,H,W,4], pos [N,V,4], tri [T,3], topo [T,3] -> out [N,H,W,C]. */
int dr_antialias_fwd(const float* color, const float* rast, const float* pos,
                     const int32_t* tri, const int32_t* topo, int N, int H, int W, int C,
                     int V, int T, float* out, dr_stream_t stream);

/* VJP of DiffRast.antialias: d_color [N,H,W,C], d_pos [N,V,4] (either may
 * be NULL to skip it). */
int dr_antialias_bwd(const float* color, const float* rast, const float* pos,
                     const int32_t* tri, const int32_t* topo, const float* d_out, int N, int H,
                     int W, int C, int V, int T, float* d_color, float* d_pos, unsigned flags,
                     dr_stream_t stream);

/* Size in bytes of the state dr_antialias_fwd_save keeps for the backward
 * (-1 for bad sizes). */
int64_t dr_antialias_saved_bytes(int N, int H, int W, int T);

/* dr_antialias_fwd that also fills `saved` (dr_antialias_saved_bytes bytes,
 * 16-byte aligned) for dr_antialias_bwd_saved.  Same `out` as
 * dr_antialias_fwd.  The reference recomputes the blend weights and the
 * edge geometry in its VJP (Antialias.swift:118-128); the saved state lets
 * the backward skip the pixels that do not blend and the per-triangle
 * setup.  Its first N * ceil(H/16) * ceil(W/16) * 256 bytes are the blend
 * mask, one byte per pixel: bit d set when the pixel's blend weight toward
 * direction d is nonzero (d = 0 +w, 1 +h, 2 -w, 3 -h); the byte of pixel
 * (n, h, w) is at ((n * ceil(H/16) + h/16) * ceil(W/16) + w/16) * 256 +
 * ((h%16)/8 * 2 + (w%16)/8) * 64 + (h%8) * 8 + w%8 (each 8x8 block of
 * pixels is 64 consecutive bytes).  The rest is opaque (the pixels' triangle
 * ids, which the backward reads in place of rast, then the records). */
int dr_antialias_fwd_save(const float* color, const float* rast, const float* pos,
                          const int32_t* tri, const int32_t* topo, int N, int H, int W, int C,
                          int V, int T, float* out, void* saved, dr_stream_t stream);

/* dr_antialias_bwd given the state dr_antialias_fwd_save kept for the same
 * color, rast, pos, tri and topo (other inputs give wrong gradients).  Same
 * results as dr_antialias_bwd. */
int dr_antialias_bwd_saved(const float* color, const float* rast, const float* pos,
                           const int32_t* tri, const int32_t* topo, const float* d_out,
                           const void* saved, int N, int H, int W, int C, int V, int T,
                           float* d_color, float* d_pos, unsigned flags, dr_stream_t stream);

/* ---- loss and optimizer of the inverse-rendering samples -------------- */

/* MSE loss of the samples' `lossFn`, `((out - target)^2).mean()`
 * (ColorFitExample/main.swift:62-66, PoseFitExample/main.swift:93-97,
 * MeshFitExample/main.swift:87-91), and its gradient.
 *   loss: one device float; the squares are summed in fp64 in a fixed order
 *     (the same loss on every call), then loss = (float)sum * (1/n).
 *   d_out: NULL, or [n]: d loss / d out = 2 * ((out - target) * (1/n)),
 *     overwritten. */
int dr_mse_loss(const float* out, const float* target, int64_t n, float* loss, float* d_out,
                dr_stream_t stream);

/* One step of the samples' Adam (MLXDiffRastExamples/Adam.swift:36-43):
 *   g = grad (* grad_mask if given);  m = b1*m + (1-b1)*g;
 *   v = b2*v + (1-b2)*g*g;  param_out = param - lr*(m/c1)/(sqrt(v/c2)+eps),
 * with c = 1 - beta^step (step counts from 1), each operation rounded to
 * fp32 in that order.  m and v are updated in place; param_out may be
 * param. */
int dr_adam_step(const float* param, const float* grad, const float* grad_mask, float* m,
                 float* v, float* param_out, int64_t n, int step, float lr, float beta1,
                 float beta2, float eps, dr_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
