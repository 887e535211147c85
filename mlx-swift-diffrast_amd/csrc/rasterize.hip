// rasterize: triangle setup, screen-tile binning, per-tile coverage / depth /
// barycentric forward (+ rast_db), and the d_pos backward.
//
// Semantics follow Sources/MLXDiffRast/Rasterize.swift of the reference:
//   setup    :280-328   (per-triangle perspective divide, signed area)
//   binning  :182-240   (16x16 tiles, tile range from the pixel AABB)
//   forward  :371-477 / :487-599 (inclusive edges, first-hit on equal z)
//   backward :637-812
// Differences by design: tile lists never overflow (the reference drops
// triangles beyond 128 per tile; dr_rasterize_fwd_ex with max_per_tile =
// 128 reproduces that, keeping each tile's lowest triangle indices), and
// equal depths pick the lowest triangle index (the reference picks the
// first in its atomic bin order).
//
// All float expressions are evaluated exactly as the reference writes them
// (this file is compiled with -ffp-contract=off), so the tri_id channel and
// the forward floats are bit-identical to a sequential execution of the
// reference.
#include "common.h"
#include "raster_tests.h"

namespace dr {

constexpr int kTile = 16;

// Per-triangle record, 4 x float4:
//   r0 = (sx0, sy0, sx1, sy1)  r1 = (sx2, sy2, sz0, sz1)
//   r2 = (sz2, area, 1/area, 0)
//   r3 = (X0, X1, Y0, Y1) as int bits: the image pixels whose centres lie
//        in the triangle's bounding box (the reference's box test), columns
//        X0..X1 and rows Y0..Y1; X0 > X1 or Y0 > Y1 when none does
// area == 0 marks a triangle the reference zeroes (w <= 0 or degenerate).
struct alignas(16) TriRec {
  float4 r0, r1, r2, r3;
};

// Per (image, triangle) values of the rasterize backward that do not
// depend on the pixel (Rasterize.swift:665-690, 790-797), computed once per
// triangle with the same expressions instead of once per covered pixel:
//   q0 = (sx0, sy0, sx1, sy1), q1 = (sx2, sy2, sz0, sz1),
//   q2 = (sz2, 1 / area, 1 / w0, 1 / w1), q3 = (1 / w2, i0, i1, i2)
// (the vertex ids as int bits; i0 = -1 when an id lies outside [0, V)).
struct alignas(16) RBwdRec {
  float4 q0, q1, q2, q3;
};

// The record of one triangle from its clip-space vertices (ids valid).
__device__ __forceinline__ RBwdRec rbwd_rec_of(float4 P0, float4 P1, float4 P2, int i0, int i1,
                                               int i2) {
  const float sx0 = P0.x / P0.w, sy0 = P0.y / P0.w, sz0 = P0.z / P0.w;
  const float sx1 = P1.x / P1.w, sy1 = P1.y / P1.w, sz1 = P1.z / P1.w;
  const float sx2 = P2.x / P2.w, sy2 = P2.y / P2.w, sz2 = P2.z / P2.w;
  const float area = (sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0);
  RBwdRec r;
  r.q0 = make_float4(sx0, sy0, sx1, sy1);
  r.q1 = make_float4(sx2, sy2, sz0, sz1);
  r.q2 = make_float4(sz2, 1.0f / area, 1.0f / P0.w, 1.0f / P1.w);
  r.q3 = make_float4(1.0f / P2.w, __int_as_float(i0), __int_as_float(i1), __int_as_float(i2));
  return r;
}

// Smallest i in [0, n) with p(i) for p false then true (n if none), and
// largest i in [0, n) with p(i) for p true then false (-1 if none), from a
// guess i0 (a few steps when the guess is close; at most n).
template <typename P>
__device__ __forceinline__ int first_true(int i0, int n, P p) {
  int i = min(max(i0, 0), n);
  while (i > 0 && p(i - 1)) --i;
  while (i < n && !p(i)) ++i;
  return i;
}
template <typename P>
__device__ __forceinline__ int last_true(int i0, int n, P p) {
  int i = min(max(i0, -1), n - 1);
  while (i < n - 1 && p(i + 1)) ++i;
  while (i >= 0 && !p(i)) --i;
  return i;
}

// Pixel coordinate of a bounding-box edge, clamped to a range where the
// float -> int conversion is exact (only a guess for first/last_true).
__device__ __forceinline__ int px_guess(float v) {
  return f2i(fminf(fmaxf(v, -4.0e6f), 4.0e6f));
}

// Rasterize.swift:280-328 (+ the AABB and tile range of :191-223).  The
// first nzero threads also clear zero[0, nzero) (the fill pass's counters,
// which nothing reads before the binning), sparing a fill launch.
__global__ void __launch_bounds__(256) k_setup(const float* __restrict__ pos, int64_t pos_stride,
                                               const int32_t* __restrict__ tri, int Npos, int V,
                                               int T, int H, int W, TriRec* __restrict__ rec,
                                               int4* __restrict__ rect, int* __restrict__ zero,
                                               int64_t nzero, RBwdRec* __restrict__ brec) {
  // the workgroup's records are assembled in LDS and written out as
  // consecutive 16-byte stores (a thread's own 64-byte record would take
  // four strided stores)
  __shared__ float4 s_rec[256 * 4];
  __shared__ float4 s_brec[256 * 4];
  const int64_t base = (int64_t)blockIdx.x * 256;
  const int64_t i = base + threadIdx.x;
  const int64_t n_rec = (int64_t)Npos * T;
  if (i < nzero) zero[i] = 0;
  if (base >= n_rec) return;  // uniform: a workgroup past the records only clears
  if (i < n_rec) {
    int64_t n;
    int t;
    divmod64(i, T, n, t);
    const float* p = pos + n * pos_stride;
    const int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    const bool ok = verts_ok(i0, i1, i2, V);  // else not drawn
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0, v2 = v0;
    if (ok) {
      v0 = *reinterpret_cast<const float4*>(p + (int64_t)i0 * 4);
      v1 = *reinterpret_cast<const float4*>(p + (int64_t)i1 * 4);
      v2 = *reinterpret_cast<const float4*>(p + (int64_t)i2 * 4);
    }
    TriRec r;
    int4 rc = make_int4(-1, -1, -1, -1);
    if (!ok || v0.w <= 0.0f || v1.w <= 0.0f || v2.w <= 0.0f) {
      r.r0 = r.r1 = r.r2 = make_float4(0.f, 0.f, 0.f, 0.f);
      r.r3 = make_float4(__int_as_float(1), __int_as_float(0), __int_as_float(1),
                         __int_as_float(0));  // no pixel
    } else {
      const float sx0 = v0.x / v0.w, sy0 = v0.y / v0.w, sz0 = v0.z / v0.w;
      const float sx1 = v1.x / v1.w, sy1 = v1.y / v1.w, sz1 = v1.z / v1.w;
      const float sx2 = v2.x / v2.w, sy2 = v2.y / v2.w, sz2 = v2.z / v2.w;
      const float area = (sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0);
      const float minx = fminf(sx0, fminf(sx1, sx2));
      const float maxx = fmaxf(sx0, fmaxf(sx1, sx2));
      const float miny = fminf(sy0, fminf(sy1, sy2));
      const float maxy = fmaxf(sy0, fmaxf(sy1, sy2));
      r.r0 = make_float4(sx0, sy0, sx1, sy1);
      r.r1 = make_float4(sx2, sy2, sz0, sz1);
      r.r2 = make_float4(sz2, area, 1.0f / area, 0.0f);
      // pixel centres as every kernel computes them (monotonic in the index)
      const float fW = (float)W * 0.5f, fH = (float)H * 0.5f;
      auto cx = [&](int X) { return 2.0f * ((float)X + 0.5f) / (float)W - 1.0f; };
      auto cy = [&](int Y) { return 1.0f - 2.0f * ((float)Y + 0.5f) / (float)H; };
      const int X0 = first_true(px_guess(ceilf((minx + 1.0f) * fW - 0.5f)), W,
                                [&](int i) { return !(cx(i) < minx); });
      const int X1 = last_true(px_guess(floorf((maxx + 1.0f) * fW - 0.5f)), W,
                               [&](int i) { return !(cx(i) > maxx); });
      const int Y0 = first_true(px_guess(ceilf((1.0f - maxy) * fH - 0.5f)), H,
                                [&](int i) { return !(cy(i) > maxy); });
      const int Y1 = last_true(px_guess(floorf((1.0f - miny) * fH - 0.5f)), H,
                               [&](int i) { return !(cy(i) < miny); });
      r.r3 = make_float4(__int_as_float(X0), __int_as_float(X1), __int_as_float(Y0),
                         __int_as_float(Y1));
      if (area != 0.0f) {
        const float px_min = (minx + 1.0f) * (float)W * 0.5f - 0.5f;
        const float px_max = (maxx + 1.0f) * (float)W * 0.5f - 0.5f;
        const float py_min = (1.0f - maxy) * (float)H * 0.5f - 0.5f;
        const float py_max = (1.0f - miny) * (float)H * 0.5f - 0.5f;
        int x0 = f2i(floorf(px_min)), x1 = f2i(floorf(px_max));
        int y0 = f2i(floorf(py_min)), y1 = f2i(floorf(py_max));
        if (x0 < 0) x0 = 0;
        if (x1 >= W) x1 = W - 1;
        if (y0 < 0) y0 = 0;
        if (y1 >= H) y1 = H - 1;
        if (x0 <= x1 && y0 <= y1) rc = make_int4(x0 / kTile, x1 / kTile, y0 / kTile, y1 / kTile);
      }
    }
    float4* sr = s_rec + threadIdx.x * 4;
    sr[0] = r.r0; sr[1] = r.r1; sr[2] = r.r2; sr[3] = r.r3;
    rect[i] = rc;
    if (brec) {  // the backward's record of the triangle, as k_rbwd_rec writes it
      RBwdRec z;
      if (ok) {
        z = rbwd_rec_of(v0, v1, v2, i0, i1, i2);
      } else {
        z.q0 = z.q1 = z.q2 = make_float4(0.f, 0.f, 0.f, 0.f);
        z.q3 = make_float4(0.f, __int_as_float(-1), 0.f, 0.f);
      }
      float4* sb = s_brec + threadIdx.x * 4;
      sb[0] = z.q0; sb[1] = z.q1; sb[2] = z.q2; sb[3] = z.q3;
    }
  }
  __syncthreads();
  const int nr = (int)min((int64_t)256, n_rec - base) * 4;
  float4* dr = reinterpret_cast<float4*>(rec + base);
  for (int j = threadIdx.x; j < nr; j += 256) dr[j] = s_rec[j];
  if (brec) {
    float4* db = reinterpret_cast<float4*>(brec + base);
    for (int j = threadIdx.x; j < nr; j += 256) db[j] = s_brec[j];
  }
}

// Work item -> (image n, triangle t, record index).  Instanced mode: every
// image draws [0,T) from its own records.  Range mode: image n draws
// [start_n, start_n + count_n) from the shared records.
struct Items {
  const int64_t* prefix;  // [N+1] range mode, else nullptr
  const int64_t* start;   // [N]
  int T;
};

__device__ __forceinline__ void item_of(const Items& it, int64_t i, int N, int& n, int& t,
                                        int64_t& r) {
  if (it.prefix == nullptr) {
    n = (int)(i / it.T);
    t = (int)(i - (int64_t)n * it.T);
    r = i;
  } else {
    int lo = 0, hi = N;  // largest n with prefix[n] <= i
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (it.prefix[mid] <= i) lo = mid; else hi = mid;
    }
    n = lo;
    t = (int)(it.start[n] + (i - it.prefix[n]));
    r = t;
  }
}

// Binning atomics.  Consecutive triangles are neighbours in the mesh and
// mostly land in the same tile, and lanes of one atomic instruction on one
// address are serialised; so each triangle's first kHeld tiles are taken one
// at a time across the wave, runs of one tile along each 16-lane row are
// counted with DPP, and only the run's last lane issues the atomic.
constexpr int kHeld = 4;

// Tile k of a triangle's tile rectangle (row-major), or -1.
__device__ __forceinline__ int rect_tile(int4 rc, int ntx, int base, int k) {
  if (rc.x < 0) return -1;
  const int w = rc.y - rc.x + 1, h = rc.w - rc.z + 1;
  if (k >= w * h) return -1;
  return base + (rc.z + k / w) * ntx + rc.x + k % w;
}

__device__ __forceinline__ int rect_tiles(int4 rc) {
  return rc.x < 0 ? 0 : (rc.y - rc.x + 1) * (rc.w - rc.z + 1);
}

// Key of tile j for a run search: lanes without a tile get keys of their own.
__device__ __forceinline__ uint64_t tile_key(int j, int lane) {
  return j >= 0 ? (uint64_t)(uint32_t)j : (0xFFFFFFFF00000000ull | (uint64_t)lane);
}

// Rasterize.swift:227-233, first half: per-tile counts.
__global__ void __launch_bounds__(256) k_bin_count(Items it, int64_t n_items, int N,
                                                   const int4* __restrict__ rect, int ntx,
                                                   int tiles, int* __restrict__ cnt) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = lane_id();
  int4 rc = make_int4(-1, -1, -1, -1);
  int base = 0;
  if (i < n_items) {
    int n, t;
    int64_t r;
    item_of(it, i, N, n, t, r);
    rc = rect[r];
    base = n * tiles;
  }
#pragma unroll
  for (int k = 0; k < kHeld; ++k) {  // every lane takes part (row shifts)
    const int j = rect_tile(rc, ntx, base, k);
    const RowRun run = row_run(tile_key(j, lane));
    if (j >= 0 && run.tail) atomicAdd(&cnt[j], run.li - run.s + 1);
  }
  const int nt = rect_tiles(rc);
  for (int k = kHeld; k < nt; ++k) atomicAdd(&cnt[rect_tile(rc, ntx, base, k)], 1);
}

// Largest per-tile count (sizes the next call's per-tile list capacity)
// and, when out_sum is given, the sum of the counts (the list entries,
// which tell how many tiles a triangle spans on average).  By one
// workgroup: the outputs are the pinned host cells of the capacity
// protocol, written directly (no device atomics, no copy).
__global__ void __launch_bounds__(256) k_tile_max(const int* __restrict__ c, int64_t n,
                                                  int64_t* __restrict__ out,
                                                  int64_t* __restrict__ out_sum) {
  __shared__ int s_m[4];
  __shared__ long long s_s[4];
  int m0 = 0, m1 = 0, m2 = 0, m3 = 0;
  long long sum = 0;
  int64_t j = threadIdx.x;
  for (; j + 768 < n; j += 1024) {
    const int a = c[j], b = c[j + 256], d = c[j + 512], e = c[j + 768];
    m0 = max(m0, a);
    m1 = max(m1, b);
    m2 = max(m2, d);
    m3 = max(m3, e);
    sum += (long long)a + b + d + e;
  }
  for (; j < n; j += 256) {
    m0 = max(m0, c[j]);
    sum += c[j];
  }
  const int m = wave_max(max(max(m0, m1), max(m2, m3)));
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, kWave);
  if (lane_id() == 0) {
    s_m[threadIdx.x >> 6] = m;
    s_s[threadIdx.x >> 6] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    *out = max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3]));
    if (out_sum) *out_sum = s_s[0] + s_s[1] + s_s[2] + s_s[3];
  }
}

// Rasterize.swift:227-239, second half: append t to each touched tile's
// list of `cap` slots (tile j's list starts at j * cap; a tile whose count
// ends above cap is rasterized by a full scan instead).  The last lane of a
// run reserves the run's slots; the others take theirs from it by rank.
__global__ void __launch_bounds__(256) k_bin_fill(Items it, int64_t n_items, int N,
                                                  const int4* __restrict__ rect, int ntx,
                                                  int tiles, int* __restrict__ fill,
                                                  int* __restrict__ list, int cap) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = lane_id();
  int4 rc = make_int4(-1, -1, -1, -1);
  int base = 0, t = 0;
  if (i < n_items) {
    int n;
    int64_t r;
    item_of(it, i, N, n, t, r);
    rc = rect[r];
    base = n * tiles;
  }
#pragma unroll
  for (int k = 0; k < kHeld; ++k) {  // every lane takes part (row shifts, shuffle)
    const int j = rect_tile(rc, ntx, base, k);
    const RowRun run = row_run(tile_key(j, lane));
    // position of the run's last lane: the first tail at or after this lane
    int tp = run.tail ? run.li : 16;
    {
      int a = dpp_shift<0x101>(tp);
      if (run.li + 1 <= 15) tp = min(tp, a);
      a = dpp_shift<0x102>(tp);
      if (run.li + 2 <= 15) tp = min(tp, a);
      a = dpp_shift<0x104>(tp);
      if (run.li + 4 <= 15) tp = min(tp, a);
      a = dpp_shift<0x108>(tp);
      if (run.li + 8 <= 15) tp = min(tp, a);
    }
    int slot0 = 0;
    if (j >= 0 && run.tail) slot0 = atomicAdd(&fill[j], run.li - run.s + 1);
    slot0 = __shfl(slot0, (lane & ~15) + min(tp, 15), kWave);
    if (j >= 0) {
      const int p = slot0 + (run.li - run.s);
      if (p < cap) list[(int64_t)j * cap + p] = t;
    }
  }
  const int nt = rect_tiles(rc);
  for (int k = kHeld; k < nt; ++k) {
    const int j = rect_tile(rc, ntx, base, k);
    const int p = atomicAdd(&fill[j], 1);
    if (p < cap) list[(int64_t)j * cap + p] = t;
  }
}

// Binning through LDS (used while an image has at most kBinLdsTiles tiles):
// one workgroup per (image, chunk of kBinChunk items of that image).  The
// chunk's per-tile counts are taken with LDS atomics; one global atomic per
// touched tile then adds them to the tile's count (consecutive lanes on
// consecutive tiles, so a wave's atomics share few cache lines) and, when
// filling, returns where the chunk's slots start; a second LDS pass hands
// the slots out.  Raster results do not depend on list order (ties go to
// the lower triangle id).
constexpr int kBinChunk = 1024;
constexpr int kBinLdsTiles = 16384;
// Threads per workgroup: one item each.  Few chunks per image leave most of
// the chip idle, so a chunk's LDS counter passes and its items are spread
// as wide as a workgroup goes (0.030 -> 0.027 ms at 8 x 1024^2; 1.34 ->
// 0.64 ms per step at 16 x 2048^2, 1.3M triangles).
constexpr int kBinThreads = 1024;
// The balanced fill (k_bin_lds<true, true>): from this many tiles per
// triangle on, for images of at most kBinBalTiles tiles (its LDS holds the
// chunk's rectangles and offsets beside the tile counters) and at most 256
// triangles (one triangle over 169 tiles: 18 -> 8 us, six triangles per
// 512^2 image: 17 -> 8 us; 512 per 256^2 image: 0.65 -> 0.75 ms per
// 4,096 images, so those keep one triangle per thread).
constexpr double kBinBalTilesPerItem = 4.0;
constexpr int kBinBalTiles = 8192;

// With `wstats` (the fill pass, when the caller wants this call's tile
// statistics): each wave writes its largest final tile count (the returned
// count plus its own, for the chunk that adds last) and its list entries to
// wstats[2 * (kBinThreads / 64 * workgroup + wave) + {0, 1}], pinned host
// memory that the host reduces after the kernel has run.  Waves of an empty
// chunk write 0s.
// A thread's walk over its run of the chunk's (item, tile) pairs: item k
// and its tile (x, y), starting at pair u of item k (the item whose pairs
// hold u); next() steps along the rectangle's rows and on to the next item
// with pairs.  Called only while a pair follows in the thread's run, so an
// item with pairs lies ahead (a step past the chunk's last pair would scan
// every empty item after it).
struct BalWalk {
  const int4* rect;
  const int* off;
  int k, x, y;
  int4 rc;
  __device__ __forceinline__ BalWalk(const int4* r, const int* o, int k0, int u)
      : rect(r), off(o), k(k0) {
    rc = rect[k];
    const int rw = rc.y - rc.x + 1, l = u - off[k];
    y = rc.z + l / rw;
    x = rc.x + (l - (l / rw) * rw);
  }
  __device__ __forceinline__ void next() {
    if (++x <= rc.y) return;
    x = rc.x;
    if (++y <= rc.w) return;
    do {
      ++k;
    } while (k < kBinThreads && off[k + 1] == off[k]);  // items without pairs
    if (k < kBinThreads) {
      rc = rect[k];
      x = rc.x;
      y = rc.z;
    }
  }
};

// BAL (large triangles, many tiles each): the workgroup's (item, tile)
// pairs are dealt out evenly, each thread a contiguous run of them, instead
// of one item per thread walking its whole tile rectangle (one triangle
// over 169 tiles took 18 us in one thread).
template <bool FILL, bool BAL>
__global__ void __launch_bounds__(kBinThreads) k_bin_lds(Items it, int chunks,
                                                 const int4* __restrict__ rect, int ntx,
                                                 int tiles, int* __restrict__ cnt,
                                                 int* __restrict__ list, int cap,
                                                 int64_t* __restrict__ wstats) {
  extern __shared__ int s_tile[];
  __shared__ int4 s_rect[BAL ? kBinThreads : 1];  // the chunk's tile rectangles
  __shared__ int s_off[BAL ? kBinThreads + 1 : 1];  // pairs before each item
  __shared__ int s_wsum[BAL ? kBinThreads / 64 : 1];
  const int n = (int)blockIdx.x / chunks;
  const int c = (int)blockIdx.x - n * chunks;
  int64_t i0, i1, r0;  // items [i0, i1) of image n; item i uses record r0 + (i - i0)
  if (it.prefix) {
    i0 = it.prefix[n];
    i1 = it.prefix[n + 1];
    r0 = it.start[n];
  } else {
    i0 = (int64_t)n * it.T;
    i1 = i0 + it.T;
    r0 = i0;
  }
  const int64_t b0 = i0 + (int64_t)c * kBinChunk;
  const int64_t b1 = min(i1, b0 + kBinChunk);
  const int tid = threadIdx.x;
  int m = 0;        // largest final count this thread saw
  long long e = 0;  // list entries this thread added
  if (b0 < b1) {    // uniform over the workgroup
    for (int k = tid; k < tiles; k += kBinThreads) s_tile[k] = 0;
    int npairs = 0, ulo = 0, uhi = 0, k0 = 0;
    if (BAL) {
      // each item's pair count, and their exclusive prefix over the chunk
      int4 rc = make_int4(-1, -1, -1, -1);
      int a = 0;
      if (b0 + tid < b1) {
        rc = rect[r0 + (b0 + tid - i0)];
        if (rc.x >= 0) a = (rc.y - rc.x + 1) * (rc.w - rc.z + 1);
      }
      s_rect[tid] = rc;
      int inc = a;  // inclusive scan within the wave
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(inc, d, kWave);
        if ((tid & 63) >= d) inc += o;
      }
      if ((tid & 63) == 63) s_wsum[tid >> 6] = inc;
      __syncthreads();
      int before = 0;
      for (int w = 0; w < (tid >> 6); ++w) before += s_wsum[w];
      npairs = 0;
      for (int w = 0; w < kBinThreads / 64; ++w) npairs += s_wsum[w];
      s_off[tid] = before + inc - a;
      if (tid == kBinThreads - 1) s_off[kBinThreads] = npairs;
      // this thread's pairs [ulo, uhi) and the item of the first
      ulo = (int)((int64_t)npairs * tid / kBinThreads);
      uhi = (int)((int64_t)npairs * (tid + 1) / kBinThreads);
    }
    __syncthreads();
    if (BAL) {
      if (ulo < uhi) {  // last item with s_off <= ulo (items of no pairs are skipped over)
        int lo = 0, hi = kBinThreads - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_off[mid] <= ulo) lo = mid;
          else hi = mid - 1;
        }
        k0 = lo;
      }
      BalWalk wk(s_rect, s_off, k0, ulo);
      for (int u = ulo; u < uhi; ++u) {
        atomicAdd(&s_tile[wk.y * ntx + wk.x], 1);
        if (u + 1 < uhi) wk.next();
      }
    } else {
      for (int64_t i = b0 + tid; i < b1; i += kBinThreads) {
        const int4 rc = rect[r0 + (i - i0)];
        if (rc.x < 0) continue;
        for (int y = rc.z; y <= rc.w; ++y)
          for (int x = rc.x; x <= rc.y; ++x) atomicAdd(&s_tile[y * ntx + x], 1);
      }
    }
    __syncthreads();
    int* cimg = cnt + (int64_t)n * tiles;
    for (int k = tid; k < tiles; k += kBinThreads) {
      const int v = s_tile[k];
      if (v > 0) {
        const int at = atomicAdd(&cimg[k], v);
        if (FILL) s_tile[k] = at;
        m = max(m, at + v);
        e += v;
      }
    }
    if (FILL) {
      __syncthreads();
      int* limg = list + (int64_t)n * tiles * cap;
      if (BAL) {
        BalWalk wk(s_rect, s_off, k0, ulo);
        for (int u = ulo; u < uhi; ++u) {
          const int64_t r = r0 + (b0 + wk.k - i0);
          const int t = (int)(it.prefix ? r : b0 + wk.k - i0);
          const int j = wk.y * ntx + wk.x;
          const int p = atomicAdd(&s_tile[j], 1);
          if (p < cap) limg[(int64_t)j * cap + p] = t;
          if (u + 1 < uhi) wk.next();
        }
      } else {
        for (int64_t i = b0 + tid; i < b1; i += kBinThreads) {
          const int64_t r = r0 + (i - i0);
          const int4 rc = rect[r];
          if (rc.x < 0) continue;
          const int t = (int)(it.prefix ? r : i - i0);
          for (int y = rc.z; y <= rc.w; ++y)
            for (int x = rc.x; x <= rc.y; ++x) {
              const int j = y * ntx + x;
              const int p = atomicAdd(&s_tile[j], 1);
              if (p < cap) limg[(int64_t)j * cap + p] = t;
            }
        }
      }
    }
  }
  if (wstats == nullptr) return;  // uniform
  m = wave_max(m);
  for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o, kWave);
  if ((tid & 63) == 0)
    *reinterpret_cast<longlong2*>(wstats + 2 * ((int64_t)blockIdx.x * (kBinThreads / 64) + (tid >> 6))) =
        make_longlong2((long long)m, e);
}

__device__ __forceinline__ TriRec load_rec(const TriRec* __restrict__ rec, int64_t r) {
  const float4* q = reinterpret_cast<const float4*>(rec + r);
  TriRec R;
  R.r0 = q[0];
  R.r1 = q[1];
  R.r2 = q[2];
  R.r3 = q[3];
  return R;
}

// Largest per-tile cap of the reference-compatible mode, and the largest
// list that mode ranks in LDS (longer lists take the ordered full scan).
constexpr int kMaxPerTileCap = 1024;
constexpr int kRankMax = 4096;
// The triangle-parallel kernel's bound: its ranking buffer (4 KiB of LDS,
// in the capped variant only) also holds the kept ids, so the workgroup
// stays small enough for full occupancy (a 16 KiB buffer and a separate
// kept list held 29 KiB: 8 x 1024^2 with the limit 128, rasterize 0.197 ms
// against 0.106 uncapped).  Longer lists take the ordered full scan.
constexpr int kRankMaxTri = 1024;

// The `keep` lowest of a tile's `count` distinct candidate ids (keep <
// count, count at most the buffer's size, a power of two) into s_keep,
// ascending (s_keep may be s_all): a bitonic sort of the list, padded with
// INT_MAX to a power of two, in s_all by the whole workgroup;
// log2(n)(log2(n)+1)/2 compare-exchange stages instead of count^2
// comparisons.
__device__ __forceinline__ void keep_lowest(const int* ids, int count, int keep, int* s_all,
                                            int* s_keep) {
  int n2 = 2;
  while (n2 < count) n2 <<= 1;
  for (int i = (int)threadIdx.x; i < n2; i += (int)blockDim.x)
    s_all[i] = i < count ? ids[i] : 0x7fffffff;
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = (int)threadIdx.x; i < n2; i += (int)blockDim.x) {
        const int l = i ^ j;
        if (l > i) {
          const int a = s_all[i], b = s_all[l];
          if ((a > b) == ((i & k) == 0)) {
            s_all[i] = b;
            s_all[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = (int)threadIdx.x; i < keep; i += (int)blockDim.x) s_keep[i] = s_all[i];
  __syncthreads();
}

// Forward kernel choice: k_raster_px when triangles span at least this many
// tiles each on average.
constexpr double kPxTilesPerItem = 8.0;

// Triangle-parallel coverage: threads per workgroup (each with kRPix of the
// tile's 256 pixels), candidates staged per round, pixels per work item,
// work items per pass.
constexpr int kRThreads = 128;
constexpr int kRPix = 256 / kRThreads;
constexpr int kRChunk = 64;
constexpr int kRSub = 4;
constexpr int kRItems = 1024;

// Depth-then-index key of a covering triangle: the float depth mapped to an
// unsigned order (-0 taken as +0, as the reference's == compares it) above
// `id` (the triangle index, or index << 7 | LDS slot while indices fit in
// 25 bits), so the smallest key is the reference's winner (the lower index
// on equal depth).
__device__ __forceinline__ unsigned long long zkey(float z, uint32_t id) {
  uint32_t b = z == 0.0f ? 0u : __float_as_uint(z);
  b ^= (uint32_t)((int32_t)b >> 31) | 0x80000000u;
  return ((unsigned long long)b << 32) | id;
}

// Rasterize.swift:371-599.  One workgroup per (image, 16x16 tile); the
// tile's candidates are taken triangle-parallel.  Each candidate gets the
// exact set of tile pixels the reference's bounding-box test keeps (its
// record's pixel box clipped to the tile), its pixels
// are cut into work items of kRSub and the items are dealt out evenly over
// the workgroup; each covering pixel folds (depth, triangle) into a 64-bit
// LDS z-buffer by atomic min.  A last pass gives each thread its pixel and
// recomputes the winner's barycentrics with the same expressions, so every
// output equals a sequential scan's.
//
// CAPPED (max_per_tile > 0): the reference's per-tile limit
// (Rasterize.swift:164-171, 227-239, 410) with its appends in triangle
// order, i.e. a tile keeps its max_per_tile lowest triangle indices.  A
// complete list above the limit is ranked in LDS and only the kept ids are
// rasterized; a list that overflowed its capacity takes the full scan in
// triangle order and stops at the limit.
template <bool DB, bool PEEL, bool CAPPED>
__global__ void __launch_bounds__(kRThreads) k_raster(
    const TriRec* __restrict__ rec, const int4* __restrict__ rect, Items it, int64_t rec_stride,
    const int* __restrict__ cnt, const int* __restrict__ list, int cap,
    const float* __restrict__ peel, int N, int H, int W, int ntx, int nty, int max_per_tile,
    int slot_keys, float* __restrict__ rast, float* __restrict__ rast_db) {
  // the candidates' records, one array per 16-byte row (a record's rows
  // 64 bytes apart would put the work items' reads of different
  // candidates on the same few banks)
  __shared__ float4 s_r0[kRChunk], s_r1[kRChunk], s_r2[kRChunk], s_r3[kRChunk];
  __shared__ int s_t[kRChunk];
  __shared__ int s_box[kRChunk];             // x0 | y0 << 4 | (w - 1) << 8 | (h - 1) << 12
  __shared__ uint16_t s_item[kRItems];       // candidate << 6 | piece
  __shared__ unsigned long long s_zb[256];   // per tile pixel: smallest zkey, ~0 = none
  __shared__ float s_x[16], s_y[16];         // pixel-centre x of tile columns, y of rows
  __shared__ float s_pz[PEEL ? 256 : 1];     // depth of the peeled layer (-1e30 = none)
  __shared__ int s_all[CAPPED ? kRankMaxTri : 1];  // ranking buffer, then the kept ids
  __shared__ int s_total[2];                 // work items of the round, by round parity
  const int tiles = ntx * nty;
  const int B = tiles * N;
  const int b = xcd_remap((int)blockIdx.x, B);
  const int n = b / tiles;
  const int tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int tid = threadIdx.x;
  const int64_t j = (int64_t)n * tiles + tile;
  const int* ids = list + j * (int64_t)cap;
  // the first round's ids are read together with the count (slots past the
  // count hold stale ids and are not used)
  const int t_first = tid < kRChunk && tid < cap ? ids[tid] : 0;
  int count = cnt[j];
  bool ranked = false;
  int scan_limit = 0x7fffffff;  // full scan: stop after this many tile candidates
  if (CAPPED && count > max_per_tile) {  // uniform over the workgroup
    if (count <= cap && count <= kRankMaxTri) {
      // the max_per_tile lowest ids of the complete list, ascending, in
      // place at the front of s_all
      keep_lowest(ids, count, max_per_tile, s_all, s_all);
      ids = s_all;
      count = max_per_tile;
      ranked = true;
    } else {
      count = cap + 1;  // take the ordered full scan
      scan_limit = max_per_tile;
    }
  }
  const int x0t = tx * kTile, y0t = ty * kTile;
  const int nx = min(kTile, W - x0t), ny = min(kTile, H - y0t);  // tile pixels inside the image
  const int64_t rbase = (int64_t)n * rec_stride;
  // thread tid has tile pixels tid + q * kRThreads (q < kRPix): column
  // tid & 15, rows (tid >> 4) + q * kRThreads / 16
  auto pix_of = [&](int q, int& lx, int& ly, bool& valid) -> int64_t {
    const int p = tid + q * kRThreads;
    lx = p & 15;
    ly = p >> 4;
    valid = lx < nx && ly < ny;
    return ((int64_t)n * H + min(y0t + ly, H - 1)) * W + min(x0t + lx, W - 1);
  };
  // R: the winner's record when the caller has it (else it is loaded)
  auto write_px = [&](int64_t pix, const Best& best, const TriRec* Rw) {
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f), d4 = o4;
    if (best.t >= 0) {
      o4 = make_float4(best.u, best.v, best.z, (float)(best.t + 1));
      if (DB) {  // Rasterize.swift:586-598
        const TriRec R = Rw ? *Rw : load_rec(rec, rbase + best.t);
        const float k_x = 2.0f / (float)W, k_y = -2.0f / (float)H;
        d4 = make_float4((R.r1.y - R.r0.y) * R.r2.z * k_x, (R.r0.x - R.r1.x) * R.r2.z * k_y,
                         (R.r0.y - R.r0.w) * R.r2.z * k_x, (R.r0.z - R.r0.x) * R.r2.z * k_y);
      }
    }
    st_nt4(rast + pix * 4, o4);
    if (DB) st_nt4(rast_db + pix * 4, d4);
  };
  // the peeled layer's depth at both pixels, loaded together (the pixel
  // index is clamped into the image)
  float peel_z[kRPix];
  float4 pl[kRPix];
#pragma unroll
  for (int q = 0; q < kRPix; ++q) {
    int lx, ly;
    bool valid;
    const int64_t pix = pix_of(q, lx, ly, valid);
    if (PEEL) pl[q] = *reinterpret_cast<const float4*>(peel + pix * 4);
  }
#pragma unroll
  for (int q = 0; q < kRPix; ++q) {
    int lx, ly;
    bool valid;
    pix_of(q, lx, ly, valid);
    peel_z[q] = PEEL && valid && pl[q].w > 0.0f ? pl[q].z : -1e30f;
  }

  if (count > cap) {
    // The tile's list overflowed its capacity (sized from an earlier
    // call): each thread scans the image's whole triangle range for its
    // pixels with the same tile test the binning uses (same candidate set,
    // so the same result), uniform up to the tile's pixel-centre box.
    int t0 = 0, t1 = it.T;
    if (it.prefix != nullptr) {
      t0 = (int)it.start[n];
      t1 = t0 + (int)(it.prefix[n + 1] - it.prefix[n]);
    }
    Best best[kRPix];
    float px[kRPix], py[kRPix];
#pragma unroll
    for (int q = 0; q < kRPix; ++q) {
      int lx, ly;
      bool valid;
      pix_of(q, lx, ly, valid);
      best[q] = {1e30f, 0.0f, 0.0f, -1};
      px[q] = 2.0f * ((float)(x0t + lx) + 0.5f) / (float)W - 1.0f;
      py[q] = 1.0f - 2.0f * ((float)(y0t + ly) + 0.5f) / (float)H;
    }
    int taken = 0;  // tile candidates so far, in triangle order
    for (int t = t0; t < t1; ++t) {
      const int4 rc = rect[rbase + t];
      if (rc.x < 0 || tx < rc.x || tx > rc.y || ty < rc.z || ty > rc.w) continue;
      if (CAPPED && ++taken > scan_limit) break;  // uniform: the same tile test everywhere
      const TriRec R = load_rec(rec, rbase + t);
      if (__float_as_int(R.r3.y) < x0t || __float_as_int(R.r3.x) > x0t + nx - 1 ||
          __float_as_int(R.r3.w) < y0t || __float_as_int(R.r3.z) > y0t + ny - 1)
        continue;  // no pixel centre of the tile in its box
#pragma unroll
      for (int q = 0; q < kRPix; ++q) {
        const int p = tid + q * kRThreads;
        test_tri(R, t, px[q], py[q], x0t + (p & 15), y0t + (p >> 4), peel_z[q], best[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < kRPix; ++q) {
      int lx, ly;
      bool valid;
      const int64_t pix = pix_of(q, lx, ly, valid);
      if (valid) write_px(pix, best[q], nullptr);
    }
    return;
  }

#pragma unroll
  for (int q = 0; q < kRPix; ++q) {
    s_zb[tid + q * kRThreads] = ~0ull;
    if (PEEL) s_pz[tid + q * kRThreads] = peel_z[q];
  }
  if (tid < 16) s_x[tid] = 2.0f * ((float)(x0t + tid) + 0.5f) / (float)W - 1.0f;
  else if (tid < 32) s_y[tid - 16] = 1.0f - 2.0f * ((float)(y0t + tid - 16) + 0.5f) / (float)H;
  if (tid == 0) s_total[0] = s_total[1] = 0;
  // one round: every candidate's record stays in LDS, and the keys carry
  // its slot (slot_keys: all record indices below 2^25)
  const bool slots = slot_keys && count <= kRChunk;
  // a round's ids were loaded with the previous round's records (one round
  // trip a round instead of two); threads past the count take the list's
  // last id, whose record they do not read
  int t_cur = ranked ? ids[min(tid, count - 1)] : t_first;
  for (int c0 = 0, round = 0; c0 < count; c0 += kRChunk, ++round) {
    const int nb = min(kRChunk, count - c0);
    __syncthreads();  // s_x / s_y / s_zb set; the previous round's items done
    // the next round's counter: its last reader (two rounds back) is done
    if (tid == 0) s_total[(round + 1) & 1] = 0;
    // 1) one candidate per thread: record, exact pixel box, work items
    int base = 0, pieces = 0;
    const int t = t_cur;
    t_cur = ids[min(c0 + kRChunk + tid, count - 1)];
    if (tid < nb) {
      const TriRec R = load_rec(rec, rbase + t);
      // the record's pixel box, clipped to the tile
      const int bx0 = max(__float_as_int(R.r3.x) - x0t, 0);
      const int bx1 = min(__float_as_int(R.r3.y) - x0t, nx - 1);
      const int by0 = max(__float_as_int(R.r3.z) - y0t, 0);
      const int by1 = min(__float_as_int(R.r3.w) - y0t, ny - 1);
      // stored whatever the box (a slot without work items is not read), so
      // the record's four rows load together rather than its box row first
      s_r0[tid] = R.r0;
      s_r1[tid] = R.r1;
      s_r2[tid] = R.r2;
      s_r3[tid] = R.r3;
      s_t[tid] = t;
      if (bx0 <= bx1 && by0 <= by1) {
        const int bw = bx1 - bx0 + 1, bh = by1 - by0 + 1;
        s_box[tid] = bx0 | (by0 << 4) | ((bw - 1) << 8) | ((bh - 1) << 12);
        pieces = (bw * bh + kRSub - 1) / kRSub;
        base = atomicAdd(&s_total[round & 1], pieces);
        for (int q = 0; q < pieces && base + q < kRItems; ++q)
          s_item[base + q] = (uint16_t)((tid << 6) | q);
      }
    }
    __syncthreads();
    const int total = s_total[round & 1];
    // 2) the work items, kRItems per pass
    for (int p0 = 0; p0 < total; p0 += kRItems) {
      if (p0 > 0) {  // later passes (more than kRItems items this round)
        __syncthreads();
        for (int q = max(p0 - base, 0); q < pieces && base + q < p0 + kRItems; ++q)
          s_item[base + q - p0] = (uint16_t)((tid << 6) | q);
        __syncthreads();
      }
      const int np = min(kRItems, total - p0);
      for (int e = tid; e < np; e += blockDim.x) {
        const int ie = s_item[e];
        const int k = ie >> 6, q = ie & 63;
        const float4 R0 = s_r0[k], R1 = s_r1[k], R2 = s_r2[k];  // r3 (the box) is not needed
        const int t = s_t[k], bx = s_box[k];
        const int bx0 = bx & 15, by0 = (bx >> 4) & 15, bw = ((bx >> 8) & 15) + 1;
        const int bh = ((bx >> 12) & 15) + 1;
        const int o0 = q * kRSub, o1 = min(o0 + kRSub, bw * bh);
        // row of o0 (o0 < 256, bw <= 16: the product with the reciprocal
        // stays well clear of an integer)
        int ry = f2i(((float)o0 + 0.5f) * __builtin_amdgcn_rcpf((float)bw));
        int rx = o0 - ry * bw;
        const float sx0 = R0.x, sy0 = R0.y, sx1 = R0.z, sy1 = R0.w;
        const float sx2 = R1.x, sy2 = R1.y, sz0 = R1.z, sz1 = R1.w;
        const float sz2 = R2.x, area = R2.y, inv_area = R2.z;
        for (int o = o0; o < o1; ++o) {
          const int cx = bx0 + rx, cy = by0 + ry;
          const float px = s_x[cx], py = s_y[cy];
          // Rasterize.swift:417-462 (the box test holds by construction)
          const float e0 = (sx1 - px) * (sy2 - py) - (sx2 - px) * (sy1 - py);
          const float e1 = (sx2 - px) * (sy0 - py) - (sx0 - px) * (sy2 - py);
          const float e2 = (sx0 - px) * (sy1 - py) - (sx1 - px) * (sy0 - py);
          if (!((e0 * area) < 0.0f || (e1 * area) < 0.0f || (e2 * area) < 0.0f)) {
            const float u = e1 * inv_area, v = e2 * inv_area;
            const float z = e0 * inv_area * sz0 + u * sz1 + v * sz2;
            const int pi = cy * 16 + cx;
            if (z >= -1.0f && z <= 1.0f && !(PEEL && z <= s_pz[pi]))
              atomicMin(&s_zb[pi], zkey(z, slots ? ((uint32_t)t << 7) | (uint32_t)k : (uint32_t)t));
          }
          if (++rx == bw) {
            rx = 0;
            ++ry;
          }
        }
      }
    }
  }
  __syncthreads();
  // 3) each thread its pixels: the winner's outputs, recomputed
#pragma unroll
  for (int q = 0; q < kRPix; ++q) {
    int lx, ly;
    bool valid;
    const int64_t pix = pix_of(q, lx, ly, valid);
    if (!valid) continue;
    const unsigned long long key = s_zb[tid + q * kRThreads];
    Best best = {1e30f, 0.0f, 0.0f, -1};
    TriRec R;
    if (key != ~0ull) {
      const uint32_t id = (uint32_t)key;
      const int t = slots ? (int)(id >> 7) : (int)id;
      if (slots) {
        const int sl = id & 127;
        R.r0 = s_r0[sl];
        R.r1 = s_r1[sl];
        R.r2 = s_r2[sl];
        R.r3 = s_r3[sl];
      } else {
        R = load_rec(rec, rbase + t);
      }
      test_tri(R, t, s_x[lx], s_y[ly], x0t + lx, y0t + ly, -1e30f, best);  // as the scan
    }
    write_px(pix, best, &R);  // R is read only when best.t >= 0, i.e. it was set
  }
}

// The same forward, pixel-parallel, for large triangles (a candidate's box
// then holds most of the tile, and the work items of k_raster cost more
// than one test per pixel): Rasterize.swift:371-599.  One workgroup per
// (image, 16x16 tile); wave w owns the 8x8 quadrant (w&1, w>>1).  Each triangle of the tile's list is
// first tested against the quadrant's pixel-centre box by its bounding box
// (exact: the pixel -> NDC map is monotonic), 64 triangles at a time, one
// per lane, then by a conservative edge-function test of the quadrant's
// pixel-centre box (edge_excludes: a large triangle's bounding box overlaps
// many quadrants the triangle itself misses) and, once every pixel of the
// quadrant holds a triangle, a conservative depth test (depth_excludes);
// only the survivors are tested against the quadrant's 64 pixels.  Both
// culls are fp32 corner evaluations with margins over the rounding
// (raster_tests.h; in fp64 they took 11.6 ms of the 4096 x 256^2 batch's
// 72 ms per step, in fp32 8.5: fp64 issues at half the fp32 rate).
//
// CAPPED (max_per_tile > 0): the reference's per-tile limit
// (Rasterize.swift:164-171, 227-239, 410) with its appends in triangle
// order, i.e. a tile keeps its max_per_tile lowest triangle indices.  A
// complete list above the limit is ranked in LDS and only the kept ids are
// rasterized; a list that overflowed its capacity takes the full scan in
// triangle order and stops at the limit.
template <bool DB, bool PEEL, bool CAPPED>
__global__ void __launch_bounds__(256) k_raster_px(
    const TriRec* __restrict__ rec, const int4* __restrict__ rect, Items it, int64_t rec_stride,
    const int* __restrict__ cnt, const int* __restrict__ list, int cap,
    const float* __restrict__ peel, int N, int H, int W, int ntx, int nty, int max_per_tile,
    float* __restrict__ rast, float* __restrict__ rast_db) {
  __shared__ TriRec s_rec[4][kWave];
  __shared__ int s_t[4][kWave];
  __shared__ int s_keep[CAPPED ? kMaxPerTileCap : 1];
  static_assert(sizeof(s_rec) >= kRankMax * sizeof(int), "the ranking's buffer");
  const int tiles = ntx * nty;
  const int B = tiles * N;
  const int b = xcd_remap((int)blockIdx.x, B);
  const int n = b / tiles;
  const int tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t j = (int64_t)n * tiles + tile;
  int count = cnt[j];
  const int* ids = list + j * (int64_t)cap;
  int scan_limit = 0x7fffffff;  // full scan: stop after this many tile candidates
  if (CAPPED && count > max_per_tile) {  // uniform over the workgroup
    if (count <= cap && count <= kRankMax) {
      // the max_per_tile lowest ids of the complete list, ascending (the
      // record slots serve as the sort's buffer, free again after it)
      keep_lowest(ids, count, max_per_tile, reinterpret_cast<int*>(&s_rec[0][0]), s_keep);
      ids = s_keep;
      count = max_per_tile;
    } else {
      count = cap + 1;  // take the ordered full scan
      scan_limit = max_per_tile;
    }
  }
  const int qx0 = tx * kTile + (wave & 1) * 8;
  const int qy0 = ty * kTile + (wave >> 1) * 8;
  if (qx0 >= W || qy0 >= H) return;  // whole quadrant outside the image
  const int pw = qx0 + (lane & 7);
  const int ph = qy0 + (lane >> 3);
  const bool valid = pw < W && ph < H;
  const int qx1 = min(qx0 + 7, W - 1), qy1 = min(qy0 + 7, H - 1);

  const float x = 2.0f * ((float)pw + 0.5f) / (float)W - 1.0f;
  const float y = 1.0f - 2.0f * ((float)ph + 0.5f) / (float)H;
  // the quadrant's pixel-centre box, with the per-pixel expressions
  const float cxa = 2.0f * ((float)qx0 + 0.5f) / (float)W - 1.0f;
  const float cxb = 2.0f * ((float)qx1 + 0.5f) / (float)W - 1.0f;
  const float cya = 1.0f - 2.0f * ((float)qy1 + 0.5f) / (float)H;
  const float cyb = 1.0f - 2.0f * ((float)qy0 + 0.5f) / (float)H;

  const int64_t pix = ((int64_t)n * H + ph) * W + pw;
  float peel_z = -1e30f;
  if (PEEL && valid) {
    const float4 pl = *reinterpret_cast<const float4*>(peel + pix * 4);
    if (pl.w > 0.0f) peel_z = pl.z;
  }
  Best best = {1e30f, 0.0f, 0.0f, -1};
  const int64_t rbase = (int64_t)n * rec_stride;
  if (count <= cap) {
    // 64 candidates at a time: each lane loads one candidate's record
    // (vector gathers, one round trip for all 64) and tests it against the
    // quadrant's box; the survivors are then taken one by one, their
    // records read back from the wave's LDS slots at a uniform address (a
    // broadcast read; cheaper than 17 readlanes and their SGPR hazards).
    // The next chunk's ids are loaded with this chunk's records: one round
    // trip a chunk instead of two (4096 x 256^2: 8.55 -> 8.37 ms a step).
    // Lanes past the count take the list's last id, so every record read
    // is a candidate's; a lane past nb ignores its record.
    int next_t = count > 0 ? ids[min(lane, count - 1)] : 0;
    for (int c0 = 0; c0 < count; c0 += kWave) {
      const int nb = min(kWave, count - c0);
      // the quadrant's farthest best depth so far; while a pixel of the
      // image is still uncovered (depth 1e30) no candidate is culled by it
      const float zq = __int_as_float(wave_reduce_i(
          __float_as_int(valid ? best.z : -1e30f),
          [](int a, int b) { return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b))); }));
      const int myt = next_t;
      TriRec Rl;
      bool hit = false;
      next_t = ids[min(c0 + kWave + lane, count - 1)];  // in the list: count <= cap
      Rl = load_rec(rec, rbase + myt);
      if (lane < nb) {
        hit = !(__float_as_int(Rl.r3.y) < qx0 || __float_as_int(Rl.r3.x) > qx1 ||
                __float_as_int(Rl.r3.w) < qy0 || __float_as_int(Rl.r3.z) > qy1);
        if (hit && fabsf(Rl.r2.y) > 1e-30f) {
          hit = !edge_excludes(Rl, cxa, cxb, cya, cyb);
          if (hit && zq <= 1.0f) hit = !depth_excludes(Rl, cxa, cxb, cya, cyb, zq);
        }
      }
      uint64_t m = __ballot(hit);
      if (hit) {
        s_rec[wave][lane] = Rl;
        s_t[wave][lane] = myt;
      }
      // LDS is ordered within a wave; the barrier keeps the compiler from
      // moving the reads above the writes
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      while (m) {
        const int j = __ffsll((long long)m) - 1;
        m &= m - 1;
        const int t = s_t[wave][j];
        const TriRec R = s_rec[wave][j];
        if (valid) test_tri(R, t, x, y, pw, ph, peel_z, best);
      }
      __builtin_amdgcn_wave_barrier();  // reads done before the next chunk writes
    }
  } else {
    // The tile's list overflowed its capacity (sized from an earlier
    // call): scan the image's whole triangle range with the same tile test
    // the binning uses (same candidate set, so the same result).
    int t0 = 0, t1 = it.T;
    if (it.prefix != nullptr) {
      t0 = (int)it.start[n];
      t1 = t0 + (int)(it.prefix[n + 1] - it.prefix[n]);
    }
    int taken = 0;  // tile candidates so far, in triangle order
    for (int t = t0; t < t1; ++t) {
      const int4 rc = rect[rbase + t];
      if (rc.x < 0 || tx < rc.x || tx > rc.y || ty < rc.z || ty > rc.w) continue;
      if (CAPPED && ++taken > scan_limit) break;  // uniform: the same tile test everywhere
      const TriRec R = load_rec(rec, rbase + t);
      if (__float_as_int(R.r3.y) < qx0 || __float_as_int(R.r3.x) > qx1 ||
          __float_as_int(R.r3.w) < qy0 || __float_as_int(R.r3.z) > qy1)
        continue;
      if (valid) test_tri(R, t, x, y, pw, ph, peel_z, best);
    }
  }
  if (!valid) return;
  float4 o4, d4 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (best.t < 0) {
    o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    o4 = make_float4(best.u, best.v, best.z, (float)(best.t + 1));
    if (DB) {  // Rasterize.swift:586-598
      const TriRec R = load_rec(rec, rbase + best.t);
      const float sx0 = R.r0.x, sy0 = R.r0.y, sx1 = R.r0.z, sy1 = R.r0.w;
      const float sx2 = R.r1.x, sy2 = R.r1.y;
      const float inv_area = R.r2.z;
      const float k_x = 2.0f / (float)W;
      const float k_y = -2.0f / (float)H;
      d4 = make_float4((sy2 - sy0) * inv_area * k_x, (sx0 - sx2) * inv_area * k_y,
                       (sy0 - sy1) * inv_area * k_x, (sx1 - sx0) * inv_area * k_y);
    }
  }
  *reinterpret_cast<float4*>(rast + pix * 4) = o4;
  if (DB) *reinterpret_cast<float4*>(rast_db + pix * 4) = d4;
}

__global__ void __launch_bounds__(256) k_rbwd_rec(const float* __restrict__ pos, int64_t pos_stride,
                                                  const int32_t* __restrict__ tri, int64_t NT,
                                                  int V, int T, RBwdRec* __restrict__ out) {
  __shared__ float4 s_r[256 * 4];
  const int64_t base = (int64_t)blockIdx.x * 256;
  const int64_t i = base + threadIdx.x;
  if (i < NT) {
    int64_t n;
    int t;
    divmod64(i, T, n, t);
    const int i0 = tri[t * 3 + 0], i1 = tri[t * 3 + 1], i2 = tri[t * 3 + 2];
    float4* r = s_r + threadIdx.x * 4;
    if (!verts_ok(i0, i1, i2, V)) {
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      r[0] = z; r[1] = z; r[2] = z;
      r[3] = make_float4(0.f, __int_as_float(-1), 0.f, 0.f);
    } else {
      const float* p = pos + n * pos_stride;
      const RBwdRec q = rbwd_rec_of(*reinterpret_cast<const float4*>(p + (int64_t)i0 * 4),
                                    *reinterpret_cast<const float4*>(p + (int64_t)i1 * 4),
                                    *reinterpret_cast<const float4*>(p + (int64_t)i2 * 4), i0, i1,
                                    i2);
      r[0] = q.q0; r[1] = q.q1; r[2] = q.q2; r[3] = q.q3;
    }
  }
  __syncthreads();
  const int nrec = (int)min((int64_t)256, NT - base);
  float4* d = reinterpret_cast<float4*>(out + base);
  for (int j = threadIdx.x; j < nrec * 4; j += 256) d[j] = s_r[j];
}

// Rasterize.swift:637-812.  16x16 tiles, a 16x4 strip per wave; runs of
// same-triangle lanes along a pixel row are summed before the LDS table
// adds the 12 d_pos terms; the table is written out into an fp64
// accumulator laid out as pos.  REC: a covered pixel loads its triangle's
// record (k_rbwd_rec) together with its cotangents, one round trip after
// its rast value; else it gathers tri -> pos and builds the same record
// itself (cheaper when triangles cover few pixels each: the records of
// every (image, triangle) then cost more to write than they save).
template <bool REC>
__global__ void __launch_bounds__(256) k_raster_bwd(
    const RBwdRec* __restrict__ trec, int64_t rec_stride, const float* __restrict__ pos,
    int64_t pos_stride, const int32_t* __restrict__ tri, int V, const float* __restrict__ rast,
    const float* __restrict__ d_rast, const float* __restrict__ d_rast_db, int N, int T, int H,
    int W, int ntx, int nty, double* __restrict__ d_pos) {
  __shared__ LdsTableU<4, 256> tab;  // d_pos rows touched by this tile
  __shared__ int s_any[4];           // per wave: a covered pixel
  const int tiles = ntx * nty;
  const int b = xcd_remap((int)blockIdx.x, tiles * N);
  const int n = b / tiles;
  const int tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // 16x4 strip per wave: each 16-lane row holds one pixel row, so runs of
  // one triangle along a row are summed with DPP row shifts.
  const int pw = tx * kTile + (lane & 15);
  const int ph = ty * kTile + wave * 4 + (lane >> 4);
  bool valid = pw < W && ph < H;
  const int64_t pix = ((int64_t)n * H + min(ph, H - 1)) * W + min(pw, W - 1);
  const float4 r = *reinterpret_cast<const float4*>(rast + pix * 4);
  const int t = f2i(r.w) - 1;
  valid = valid && t >= 0 && t < T;
  RBwdRec R;
  float4 dr = make_float4(0.f, 0.f, 0.f, 0.f), ddb = dr;
  if (valid) {
    if (REC) R = trec[(int64_t)n * rec_stride + t];
    dr = *reinterpret_cast<const float4*>(d_rast + pix * 4);
    if (d_rast_db) ddb = *reinterpret_cast<const float4*>(d_rast_db + pix * 4);
  }
  {
    const uint64_t any = __ballot(valid);
    if (lane == 0) s_any[wave] = any != 0ull;
  }
  __syncthreads();
  if (!(s_any[0] | s_any[1] | s_any[2] | s_any[3])) return;  // uniform: nothing to add
  lds_table_clear(tab);
  __syncthreads();
  float val[12];
  int i0 = 0, i1 = 0, i2 = 0;
#pragma unroll
  for (int q = 0; q < 12; ++q) val[q] = 0.0f;
  double* dp = d_pos + (int64_t)n * pos_stride;
  if (valid && !REC) {
    const int j0 = tri[t * 3 + 0], j1 = tri[t * 3 + 1], j2 = tri[t * 3 + 2];
    if (verts_ok(j0, j1, j2, V)) {
      const float* p = pos + (int64_t)n * pos_stride;
      R = rbwd_rec_of(*reinterpret_cast<const float4*>(p + (int64_t)j0 * 4),
                      *reinterpret_cast<const float4*>(p + (int64_t)j1 * 4),
                      *reinterpret_cast<const float4*>(p + (int64_t)j2 * 4), j0, j1, j2);
    } else {
      R.q3.y = __int_as_float(-1);
    }
  }
  if (valid) {
    i0 = __float_as_int(R.q3.y);
    i1 = __float_as_int(R.q3.z);
    i2 = __float_as_int(R.q3.w);
    valid = i0 >= 0;  // the triangle's vertex ids lie in [0, V)
  }
  if (valid) {
    // Rasterize.swift:694-798, regrouped (equal up to rounding).  With
    // e1 = area * u and e2 = area * v, u and v depend on a screen vertex
    // coordinate q through (de1/dq - u * darea/dq) / area, likewise for v,
    // and z = bw * sz0 + u * sz1 + v * sz2, so the pixel's d_u, d_v, d_z
    // reach q as (de1/dq * A + de2/dq * B - darea/dq * (u A + v B)) / area
    // with A = d_u + d_z (sz1 - sz0), B = d_v + d_z (sz2 - sz0).  rast_db
    // = (dx / area) * (-2/W or 2/H factors) adds -darea/dq * s / area, s its
    // cotangent's product with rast_db, plus the terms of the edge vectors
    // themselves.
    const float u_val = r.x, v_val = r.y;
    const float bw_val = 1.0f - u_val - v_val;
    const float d_u = dr.x, d_v = dr.y, d_z = dr.z;
    const float d_db0 = ddb.x, d_db1 = ddb.y, d_db2 = ddb.z, d_db3 = ddb.w;
    const float Px = 2.0f * ((float)pw + 0.5f) / (float)W - 1.0f;
    const float Py = 1.0f - 2.0f * ((float)ph + 0.5f) / (float)H;
    const float sx0 = R.q0.x, sy0 = R.q0.y, sx1 = R.q0.z, sy1 = R.q0.w;
    const float sx2 = R.q1.x, sy2 = R.q1.y, sz0 = R.q1.z, sz1 = R.q1.w;
    const float sz2 = R.q2.x, ia = R.q2.y;  // 1 / area
    const float kx = (2.0f / (float)W) * ia, ky = (-2.0f / (float)H) * ia;
    const float A = fmaf(d_z, sz1 - sz0, d_u), B = fmaf(d_z, sz2 - sz0, d_v);
    // s: the rast_db cotangent against rast_db's dependence on area
    const float s_db = kx * fmaf(d_db0, sy2 - sy0, d_db2 * (sy0 - sy1)) +
                       ky * fmaf(d_db1, sx0 - sx2, d_db3 * (sx1 - sx0));
    const float Q = fmaf(u_val, A, fmaf(v_val, B, s_db));
    const float ex0 = Py - sy2, ex2 = sy0 - Py, fx0 = sy1 - Py, fx1 = Py - sy0;  // de1/dsx, de2/dsx
    const float ey0 = sx2 - Px, ey2 = Px - sx0, fy0 = Px - sx1, fy1 = sx0 - Px;  // de1/dsy, de2/dsy
    float dsx0 = ia * fmaf(ex0, A, fmaf(fx0, B, -(sy1 - sy2) * Q));
    float dsx1 = ia * fmaf(fx1, B, -(sy2 - sy0) * Q);
    float dsx2 = ia * fmaf(ex2, A, -(sy0 - sy1) * Q);
    float dsy0 = ia * fmaf(ey0, A, fmaf(fy0, B, -(sx2 - sx1) * Q));
    float dsy1 = ia * fmaf(fy1, B, -(sx0 - sx2) * Q);
    float dsy2 = ia * fmaf(ey2, A, -(sx1 - sx0) * Q);
    // rast_db's own dependence on the edge vectors
    dsy0 = fmaf(d_db2 - d_db0, kx, dsy0);
    dsy1 = fmaf(-d_db2, kx, dsy1);
    dsy2 = fmaf(d_db0, kx, dsy2);
    dsx0 = fmaf(d_db1 - d_db3, ky, dsx0);
    dsx1 = fmaf(d_db3, ky, dsx1);
    dsx2 = fmaf(-d_db1, ky, dsx2);
    const float dsz0_s = d_z * bw_val, dsz1_s = d_z * u_val, dsz2_s = d_z * v_val;
    const float inv_w0 = R.q2.z, inv_w1 = R.q2.w, inv_w2 = R.q3.x;
    val[0] = dsx0 * inv_w0;
    val[1] = dsy0 * inv_w0;
    val[2] = dsz0_s * inv_w0;
    val[3] = -fmaf(sx0, dsx0, fmaf(sy0, dsy0, sz0 * dsz0_s)) * inv_w0;
    val[4] = dsx1 * inv_w1;
    val[5] = dsy1 * inv_w1;
    val[6] = dsz1_s * inv_w1;
    val[7] = -fmaf(sx1, dsx1, fmaf(sy1, dsy1, sz1 * dsz1_s)) * inv_w1;
    val[8] = dsx2 * inv_w2;
    val[9] = dsy2 * inv_w2;
    val[10] = dsz2_s * inv_w2;
    val[11] = -fmaf(sx2, dsx2, fmaf(sy2, dsy2, sz2 * dsz2_s)) * inv_w2;
  }
  // Lanes of a row on the same triangle add into the same three rows: sum
  // each run first, its last lane adds the total.
  const bool tail = row_run_sum(valid ? (uint64_t)t : (1ull << 63) | (uint64_t)lane, val);
  if (valid && tail) {
    lds_table_add(tab, dp + (int64_t)i0 * 4, &val[0]);
    lds_table_add(tab, dp + (int64_t)i1 * 4, &val[4]);
    lds_table_add(tab, dp + (int64_t)i2 * 4, &val[8]);
  }
  __syncthreads();
  lds_table_flush_last<4, 256, double>(tab);  // the taken rows only
}

// The one rounding of the fp64 sums; the accumulator is left zero for the
// next call.
__global__ void __launch_bounds__(256) k_acc_to_f32(double* __restrict__ acc,
                                                    float* __restrict__ dst, int64_t n,
                                                    int accumulate) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double a = acc[i];
  // only elements that received an addition are written back: the rows of
  // vertices no pixel reached (most of them, for a peeled layer) stay
  // untouched in memory
  if (__double_as_longlong(a) != 0) acc[i] = 0.0;
  const float v = (float)a;
  dst[i] = accumulate ? dst[i] + v : v;
}

double* acc64_begin(hipStream_t stream, int64_t n) {
  Scratch* sc = scratch_for(stream);
  if (!sc) return nullptr;
  double* a = (double*)scratch_get(sc, stream, SLOT_DPOS64, (size_t)std::max<int64_t>(n, 1) * 8);
  if (!a) return nullptr;
  if (sc->acc64_buf != a) {  // a new buffer: its contents are unknown
    sc->acc64_buf = a;
    sc->acc64_zero = 0;
  }
  if (sc->acc64_zero < n && fill_async(a, 0.0, n, stream) != hipSuccess) {
    set_error("fp64 accumulator: fill launch failed");
    return nullptr;
  }
  sc->acc64_zero = 0;  // in use until acc64_end has queued its conversion
  return a;
}

int acc64_end(double* acc, float* dst, int64_t n, bool accumulate, hipStream_t stream) {
  if (n <= 0) return DR_OK;
  {
    DR_TIMED("k_acc_to_f32", stream);
    hipLaunchKernelGGL(k_acc_to_f32, dim3(grid_for(n, 256)), dim3(256), 0, stream, acc, dst, n,
                       accumulate ? 1 : 0);
  }
  DR_CHECK_LAUNCH();
  Scratch* sc = scratch_for(stream);
  if (sc && sc->acc64_buf == acc) sc->acc64_zero = n;
  return DR_OK;
}

}  // namespace dr

using namespace dr;

// The (image, triangle) items a call draws: every (n, t) in instanced mode;
// in range mode, each image's clamped range, listed through a prefix sum
// that is written into a pinned staging buffer and copied to the device
// asynchronously (no wait for the stream).
static int plan_items(Scratch* sc, hipStream_t stream, const int32_t* ranges_host, int N, int T,
                      Items& it, int64_t& n_items, int64_t& max_items) {
  it = Items{nullptr, nullptr, T};
  n_items = (int64_t)N * T;
  max_items = T;
  if (!ranges_host) return DR_OK;
  const size_t nh = 2 * (size_t)N + 1;
  int slot = 0;
  int64_t* h = stage_acquire(sc, nh, slot);
  if (!h) return scratch_fail();
  h[0] = 0;
  max_items = 0;
  for (int n = 0; n < N; ++n) {
    int64_t s = ranges_host[2 * n], c = ranges_host[2 * n + 1];
    int64_t lo = s < 0 ? 0 : s, hi = s + c > T ? T : s + c;
    if (hi < lo) hi = lo;
    h[n + 1] = h[n] + (hi - lo);
    h[N + 1 + n] = lo;
    max_items = std::max<int64_t>(max_items, hi - lo);
  }
  n_items = h[N];
  int64_t* d = (int64_t*)scratch_get(sc, stream, SLOT_RAST_ITEMS, nh * sizeof(int64_t));
  if (!d) return scratch_fail();
  DR_CHECK_HIP(hipMemcpyAsync(d, h, nh * sizeof(int64_t), hipMemcpyHostToDevice, stream));
  const int st = stage_release(sc, slot, stream);
  if (st) return st;
  it.prefix = d;
  it.start = d + N + 1;
  return DR_OK;
}

static int check_raster_args(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                             const int32_t* ranges_host, int N, int V, int T, int H, int W) {
  DR_CHECK_ARG(N >= 1 && V >= 0 && T >= 0 && H >= 1 && W >= 1, "rasterize: bad sizes");
  DR_CHECK_ARG(pos && tri, "rasterize: null tensor");
  DR_CHECK_ARG(ranges_host != nullptr || pos_batch_stride == (int64_t)V * 4,
               "rasterize: instanced pos needs pos_batch_stride = V*4");
  DR_CHECK_ARG(ranges_host == nullptr || pos_batch_stride == 0,
               "rasterize: range mode needs a shared pos (pos_batch_stride = 0)");
  DR_CHECK_ARG((int64_t)N * T < (int64_t)1 << 40, "rasterize: too many triangles");
  DR_CHECK_ARG(T <= INT32_MAX / 3, "rasterize: at most 715827882 triangles (tri is indexed in 32 bits)");
  const int64_t n_tiles =
      (int64_t)N * ((W + kTile - 1) / kTile) * (int64_t)((H + kTile - 1) / kTile);
  DR_CHECK_ARG(n_tiles < (int64_t)1 << 31, "rasterize: too many tiles");
  return DR_OK;
}

// Workgroups per image of k_bin_lds, or 0 when the LDS path does not apply.
static int bin_lds_chunks(int N, int tiles, int64_t max_items) {
  const int64_t chunks = (max_items + kBinChunk - 1) / kBinChunk;
  if (tiles > kBinLdsTiles || chunks == 0 || (int64_t)N * chunks > ((int64_t)1 << 23)) return 0;
  return (int)chunks;
}

// Per-tile counts (FILL false) or counts and lists (FILL true) of the items.
// With `wstats` (room for `wcap` waves), the LDS fill pass also writes the
// per-wave tile statistics; returns the number of waves that did (0: none,
// k_tile_max must compute them).
// bal: deal the (item, tile) pairs out evenly (large triangles, from the
// tile statistics of an earlier call)
static int64_t launch_binning(bool fill, const Items& it, int64_t n_items, int64_t max_items,
                              int N, const int4* rect, int ntx, int tiles, int* cnt, int* list,
                              int cap, hipStream_t stream, int64_t* wstats = nullptr,
                              int64_t wcap = 0, bool bal = false) {
  if (n_items == 0) return 0;
  const int chunks = bin_lds_chunks(N, tiles, max_items);
  if (chunks > 0) {
    const dim3 grid((unsigned)((int64_t)N * chunks));
    const size_t lds = (size_t)tiles * sizeof(int);
    if (fill) {
      const int64_t waves = (int64_t)N * chunks * (kBinThreads / 64);
      if (waves > wcap) wstats = nullptr;
      DR_TIMED(bal ? "k_bin_fill_bal" : "k_bin_fill", stream);
      if (bal)
        hipLaunchKernelGGL((k_bin_lds<true, true>), grid, dim3(kBinThreads), lds, stream, it,
                           chunks, rect, ntx, tiles, cnt, list, cap, wstats);
      else
        hipLaunchKernelGGL((k_bin_lds<true, false>), grid, dim3(kBinThreads), lds, stream, it,
                           chunks, rect, ntx, tiles, cnt, list, cap, wstats);
      return wstats ? waves : 0;
    }
    DR_TIMED("k_bin_count", stream);
    hipLaunchKernelGGL((k_bin_lds<false, false>), grid, dim3(kBinThreads), lds, stream, it, chunks,
                       rect, ntx, tiles, cnt, list, cap, (int64_t*)nullptr);
  } else if (fill) {
    DR_TIMED("k_bin_fill", stream);
    hipLaunchKernelGGL(k_bin_fill, dim3(grid_for(n_items, 256)), dim3(256), 0, stream, it,
                       n_items, N, rect, ntx, tiles, cnt, list, cap);
  } else {
    DR_TIMED("k_bin_count", stream);
    hipLaunchKernelGGL(k_bin_count, dim3(grid_for(n_items, 256)), dim3(256), 0, stream, it,
                       n_items, N, rect, ntx, tiles, cnt);
  }
  return 0;
}

extern "C" int dr_rasterize_tile_counts(const float* pos, int64_t pos_batch_stride,
                                        const int32_t* tri, const int32_t* ranges_host, int N,
                                        int V, int T, int H, int W, int32_t* counts,
                                        int64_t* max_count_host, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  int st = check_raster_args(pos, pos_batch_stride, tri, ranges_host, N, V, T, H, W);
  if (st) return st;
  DR_CHECK_ARG(counts, "rasterize_tile_counts: null counts");
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  if (max_count_host && sc->cur_capture) {
    set_error("rasterize_tile_counts: the largest count is waited for, which a stream being "
              "captured into a HIP graph cannot do");
    return DR_ERR_CAPTURE;
  }
  sc->last_raster.valid = false;  // its setup and item buffers are rewritten here
  const int ntx = (W + kTile - 1) / kTile, nty = (H + kTile - 1) / kTile;
  const int tiles = ntx * nty;
  const int64_t n_tiles = (int64_t)N * tiles;
  Items it;
  int64_t n_items = 0, max_items = 0;
  st = plan_items(sc, stream, ranges_host, N, T, it, n_items, max_items);
  if (st) return st;
  const int Npos = ranges_host ? 1 : N;
  const int64_t n_rec = (int64_t)Npos * T;
  TriRec* rec = (TriRec*)scratch_get(sc, stream, SLOT_RAST_REC, (size_t)n_rec * sizeof(TriRec));
  int4* rect = (int4*)scratch_get(sc, stream, SLOT_RAST_RECT, (size_t)n_rec * sizeof(int4));
  int* small = (int*)scratch_get(sc, stream, SLOT_SMALL, 64);
  if (!rec || !rect || !small) return scratch_fail();
  if (n_rec > 0) {
    DR_TIMED("k_setup", stream);
    hipLaunchKernelGGL(k_setup, dim3(grid_for(n_rec, 256)), dim3(256), 0, stream, pos,
                       ranges_host ? (int64_t)0 : pos_batch_stride, tri, Npos, V, T, H, W, rec,
                       rect, (int*)nullptr, (int64_t)0, (RBwdRec*)nullptr);
    DR_CHECK_LAUNCH();
  }
  DR_CHECK_HIP(fill_async(counts, 0, n_tiles, stream));
  launch_binning(false, it, n_items, max_items, N, rect, ntx, tiles, (int*)counts, nullptr, 0,
                 stream);
  DR_CHECK_LAUNCH();
  if (max_count_host) {
    int64_t* tmax = reinterpret_cast<int64_t*>(small + 8);
    hipLaunchKernelGGL(k_tile_max, dim3(1), dim3(256), 0, stream, (const int*)counts, n_tiles,
                       tmax, (int64_t*)nullptr);
    DR_CHECK_LAUNCH();
    int64_t mx = 0;
    DR_CHECK_HIP(hipMemcpyAsync(&mx, tmax, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    DR_CHECK_HIP(hipStreamSynchronize(stream));
    *max_count_host = (int)mx;
  }
  return DR_OK;
}

extern "C" int dr_rasterize_fwd(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                                const int32_t* ranges_host, const float* peel, int N, int V,
                                int T, int H, int W, float* rast, float* rast_db,
                                dr_stream_t stream_) {
  return dr_rasterize_fwd_ex(pos, pos_batch_stride, tri, ranges_host, peel, N, V, T, H, W, rast,
                             rast_db, 0, stream_);
}

// The forward; `again`: reuse the previous call's triangle setup and tile
// lists when its arguments match (dr_rasterize_fwd_again).
static int raster_fwd(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                      const int32_t* ranges_host, const float* peel, int N, int V, int T, int H,
                      int W, float* rast, float* rast_db, int max_per_tile, bool again,
                      hipStream_t stream) {
  int st = check_raster_args(pos, pos_batch_stride, tri, ranges_host, N, V, T, H, W);
  if (st) return st;
  DR_CHECK_ARG(rast, "rasterize: null tensor");
  DR_CHECK_ARG(max_per_tile >= 0 && max_per_tile <= kMaxPerTileCap,
               "rasterize: max_per_tile must be in [0, 1024] (0: no limit)");
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();

  const int ntx = (W + kTile - 1) / kTile, nty = (H + kTile - 1) / kTile;
  const int tiles = ntx * nty;
  const int64_t n_tiles = (int64_t)N * tiles;

  const int Npos = ranges_host ? 1 : N;
  const int64_t n_rec = (int64_t)Npos * T;
  const int64_t rec_stride = ranges_host ? 0 : T;
  auto& L = sc->last_raster;
  const bool reuse =
      again && sc->last_raster_reusable() && L.pos == pos && L.tri == tri &&
      L.pos_stride == pos_batch_stride &&
      L.N == N && L.V == V && L.T == T && L.H == H && L.W == W &&
      L.max_per_tile == max_per_tile && L.range == (ranges_host != nullptr) &&
      (!ranges_host || std::equal(L.ranges.begin(), L.ranges.end(), ranges_host));

  // Items: which (image, triangle) pairs are drawn.
  Items it{nullptr, nullptr, T};
  int64_t n_items = 0, max_items = 0;
  TriRec* rec;
  int4* rect;
  int* fillc;
  int* list;
  int C;
  bool want_stats = false;
  int64_t stat_waves = 0;
  RBwdRec* brec = nullptr;
  if (reuse) {  // the previous call's setup and lists, untouched since
    if (ranges_host) {
      int64_t* d = (int64_t*)sc->ptr[SLOT_RAST_ITEMS];
      it.prefix = d;
      it.start = d + N + 1;
    }
    n_items = L.n_items;
    max_items = L.max_items;
    C = L.C;
    rec = (TriRec*)sc->ptr[SLOT_RAST_REC];
    rect = (int4*)sc->ptr[SLOT_RAST_RECT];
    fillc = (int*)sc->ptr[SLOT_RAST_CNT] + n_tiles;
    list = (int*)sc->ptr[SLOT_RAST_LIST];
  } else {
  L.valid = false;
  st = plan_items(sc, stream, ranges_host, N, T, it, n_items, max_items);
  if (st) return st;
  rec = (TriRec*)scratch_get(sc, stream, SLOT_RAST_REC, (size_t)n_rec * sizeof(TriRec));
  rect = (int4*)scratch_get(sc, stream, SLOT_RAST_RECT, (size_t)n_rec * sizeof(int4));
  char* cbuf = (char*)scratch_get(sc, stream, SLOT_RAST_CNT, (size_t)n_tiles * 16);
  if (!rec || !rect || !cbuf) return scratch_fail();
  int* cnt = (int*)cbuf;
  fillc = cnt + n_tiles;

  // A backward ran on this stream: write this call's records with the
  // setup (a backward of this call then skips k_rbwd_rec, or the per-pixel
  // record building; same record layout as the backward reads when pos is
  // per image or ranged)
  if (sc->rbwd_want && n_rec > 0 && (ranges_host != nullptr || pos_batch_stride != 0)) {
    brec = (RBwdRec*)scratch_get(sc, stream, SLOT_RBWD_REC, (size_t)n_rec * sizeof(RBwdRec));
    if (!brec) return scratch_fail();
  }
  if (n_rec > 0) {  // also clears the fill pass's counters
    DR_TIMED("k_setup", stream);
    hipLaunchKernelGGL(k_setup, dim3(grid_for(std::max(n_rec, n_tiles), 256)), dim3(256), 0,
                       stream, pos, ranges_host ? (int64_t)0 : pos_batch_stride, tri, Npos, V, T,
                       H, W, rec, rect, fillc, n_tiles, brec);
    DR_CHECK_LAUNCH();
  } else {
    DR_CHECK_HIP(fill_async(fillc, 0, n_tiles, stream));
  }

  // Per-tile list capacity: the largest tile count seen so far plus a
  // quarter.  The first call counts exactly (one host sync); afterwards the
  // previous call's largest count, read back asynchronously through pinned
  // memory, only ever raises it, and a tile that overflows is rasterized by
  // a full scan, so results never depend on the capacity.
  auto grow = [](int64_t m) { return (int)std::min<int64_t>(((m + m / 4) + 31) / 32 * 32 + 32, 1 << 30); };
  C = sc->bin_cap;
  auto take_stats = [&](int64_t items) {
    sc->tiles_per_item = (double)sc->pinned_total[1] / (double)std::max<int64_t>(items, 1);
  };
  // Under graph capture nothing is read back or recorded for later calls
  // (the host must not query the device), and the first call's count,
  // which waits, is refused.
  const bool capturing = sc->cur_capture != 0;
  if (!capturing && sc->total_pending && hipEventQuery(sc->total_event) == hipSuccess) {
    if (sc->stat_waves > 0) {  // the binning's per-wave figures
      int64_t mx = 0, sum = 0;
      for (int64_t w = 0; w < sc->stat_waves; ++w) {
        mx = std::max(mx, sc->wave_stats[2 * w]);
        sum += sc->wave_stats[2 * w + 1];
      }
      sc->pinned_total[0] = mx;
      sc->pinned_total[1] = sum;
    }
    const int64_t mx = sc->pinned_total[0];
    take_stats(sc->stat_items);
    sc->total_pending = false;
    if (mx > C) C = grow(mx);
  }
  if (C == 0 && capturing) {
    set_error("rasterize: the first call on a stream counts its tiles and waits for the count; "
              "run it once on this stream before capturing into a HIP graph, or size the lists "
              "with dr_rasterize_reserve");
    return DR_ERR_CAPTURE;
  }
  if (C == 0) {
    DR_CHECK_HIP(fill_async(cnt, 0, n_tiles, stream));
    launch_binning(false, it, n_items, max_items, N, rect, ntx, tiles, cnt, nullptr, 0, stream);
    DR_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_tile_max, dim3(1), dim3(256), 0, stream, cnt, n_tiles,
                       sc->pinned_total_dev, sc->pinned_total_dev + 1);
    DR_CHECK_LAUNCH();
    DR_CHECK_HIP(hipStreamSynchronize(stream));
    C = grow(sc->pinned_total[0]);
    take_stats(n_items);
  }
  // at most 4 GiB of lists (a 16 x 2048^2 batch of a 1.3M-triangle mesh
  // needs ~1,500 slots per tile); a tile above the capacity takes the full
  // scan
  const int64_t c_budget = std::max<int64_t>(32, ((int64_t)1 << 30) / std::max<int64_t>(n_tiles, 1));
  C = (int)std::min<int64_t>(C, c_budget);
  if (C > sc->bin_cap) sc->bin_cap = C;
  list = (int*)scratch_get(sc, stream, SLOT_RAST_LIST, (size_t)n_tiles * C * 4);
  if (!list) return scratch_fail();

  // (fillc was cleared with the setup) this call's largest count and list
  // entries, for the next call (when the previous ones have been read)
  want_stats = !sc->total_pending && !capturing;
  // a few large triangles per image (4 tiles each or more on average, in
  // the last counted call, and at most a quarter of a workgroup's threads):
  // the fill pass deals their (triangle, tile) pairs out evenly
  const bool bal = sc->tiles_per_item >= kBinBalTilesPerItem && tiles <= kBinBalTiles &&
                   max_items <= kBinThreads / 4;
  stat_waves = launch_binning(true, it, n_items, max_items, N, rect, ntx, tiles, fillc, list, C,
                              stream, want_stats ? sc->wave_stats_dev : nullptr,
                              Scratch::kWaveStatsMax, bal);
  DR_CHECK_LAUNCH();
  }
  const dim3 grid((unsigned)n_tiles), block(256);
  const int slot_keys = n_rec <= ((int64_t)1 << 25) ? 1 : 0;  // record indices fit in 25 bits
  // Triangles spanning kPxTilesPerItem tiles or more on average (the last
  // counted call's list entries per item) are large: pixel-parallel.
  const bool px = reuse ? L.px : sc->tiles_per_item >= kPxTilesPerItem;
#define DR_RASTER(DBV, PV, CV)                                                                     \
  do {                                                                                            \
    if (px)                                                                                       \
      hipLaunchKernelGGL((k_raster_px<DBV, PV, CV>), grid, block, 0, stream, rec, rect, it,       \
                         rec_stride, fillc, list, C, peel, N, H, W, ntx, nty, max_per_tile, rast, \
                         rast_db);                                                                \
    else                                                                                          \
      hipLaunchKernelGGL((k_raster<DBV, PV, CV>), grid, dim3(kRThreads), 0, stream, rec, rect,   \
                         it, rec_stride, fillc, list, C, peel, N, H, W, ntx, nty, max_per_tile,   \
                         slot_keys, rast, rast_db);                                               \
  } while (0)
#define DR_RASTER_C(DBV, PV)                                 \
  do {                                                       \
    if (max_per_tile > 0) DR_RASTER(DBV, PV, true);          \
    else DR_RASTER(DBV, PV, false);                          \
  } while (0)
  {
    DR_TIMED(px ? "k_raster_px" : "k_raster", stream);
    if (rast_db) {
      if (peel) DR_RASTER_C(true, true); else DR_RASTER_C(true, false);
    } else {
      if (peel) DR_RASTER_C(false, true); else DR_RASTER_C(false, false);
    }
  }
#undef DR_RASTER_C
#undef DR_RASTER
  DR_CHECK_LAUNCH();
  if (reuse) return DR_OK;
  if (want_stats) {  // largest count and list entries of this call, for the next one
    if (stat_waves == 0) {
      hipLaunchKernelGGL(k_tile_max, dim3(1), dim3(256), 0, stream, fillc, n_tiles,
                         sc->pinned_total_dev, sc->pinned_total_dev + 1);
      DR_CHECK_LAUNCH();
    }
    sc->stat_items = n_items;
    sc->stat_waves = stat_waves;
    DR_CHECK_HIP(hipEventRecord(sc->total_event, stream));
    sc->total_pending = true;
  }
  L.pos = pos;
  L.tri = tri;
  L.pos_stride = pos_batch_stride;
  L.N = N; L.V = V; L.T = T; L.H = H; L.W = W;
  L.max_per_tile = max_per_tile;
  L.range = ranges_host != nullptr;
  L.ranges.assign(ranges_host ? ranges_host : nullptr, ranges_host ? ranges_host + 2 * N : nullptr);
  L.n_items = n_items;
  L.max_items = max_items;
  L.C = C;
  L.px = px;
  L.brec = brec != nullptr;
  L.capture_id = sc->cur_capture;
  L.valid = true;
  return DR_OK;
}

extern "C" int dr_rasterize_fwd_ex(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                                   const int32_t* ranges_host, const float* peel, int N, int V,
                                   int T, int H, int W, float* rast, float* rast_db,
                                   int max_per_tile, dr_stream_t stream) {
  return raster_fwd(pos, pos_batch_stride, tri, ranges_host, peel, N, V, T, H, W, rast, rast_db,
                    max_per_tile, false, (hipStream_t)stream);
}

extern "C" int dr_rasterize_fwd_again(const float* pos, int64_t pos_batch_stride,
                                      const int32_t* tri, const int32_t* ranges_host,
                                      const float* peel, int N, int V, int T, int H, int W,
                                      float* rast, float* rast_db, int max_per_tile,
                                      dr_stream_t stream) {
  return raster_fwd(pos, pos_batch_stride, tri, ranges_host, peel, N, V, T, H, W, rast, rast_db,
                    max_per_tile, true, (hipStream_t)stream);
}


extern "C" int dr_rasterize_reserve(int N, int V, int T, int H, int W, int tile_capacity,
                                    dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  DR_CHECK_ARG(N >= 1 && V >= 0 && T >= 0 && H >= 1 && W >= 1 && tile_capacity >= 1,
               "rasterize_reserve: bad sizes");
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  const int ntx = (W + kTile - 1) / kTile, nty = (H + kTile - 1) / kTile;
  const int64_t n_tiles = (int64_t)N * ntx * nty;
  const int64_t n_rec = (int64_t)N * std::max(T, 1);
  // the same list budget as the forward's
  const int64_t c_budget = std::max<int64_t>(32, ((int64_t)1 << 30) / std::max<int64_t>(n_tiles, 1));
  const int C = (int)std::min<int64_t>(tile_capacity, c_budget);
  const bool ok =
      scratch_get(sc, stream, SLOT_RAST_REC, (size_t)n_rec * sizeof(TriRec)) &&
      scratch_get(sc, stream, SLOT_RAST_RECT, (size_t)n_rec * sizeof(int4)) &&
      scratch_get(sc, stream, SLOT_RAST_CNT, (size_t)n_tiles * 16) &&
      scratch_get(sc, stream, SLOT_RAST_LIST, (size_t)n_tiles * C * 4) &&
      scratch_get(sc, stream, SLOT_SMALL, 64) &&
      scratch_get(sc, stream, SLOT_RBWD_REC, (size_t)n_rec * sizeof(RBwdRec)) &&
      scratch_get(sc, stream, SLOT_DPOS64, (size_t)std::max<int64_t>((int64_t)N * V * 4, 1) * 8);
  if (!ok) return scratch_fail();
  if (C > sc->bin_cap) sc->bin_cap = C;
  return DR_OK;
}

extern "C" int dr_rasterize_bwd(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                                const float* rast, const float* d_rast, const float* d_rast_db,
                                int N, int V, int T, int H, int W, float* d_pos, unsigned flags,
                                dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  DR_CHECK_ARG(N >= 1 && V >= 0 && T >= 0 && H >= 1 && W >= 1, "rasterize_bwd: bad sizes");
  DR_CHECK_ARG(pos && tri && rast && d_rast && d_pos, "rasterize_bwd: null tensor");
  DR_CHECK_ARG(pos_batch_stride == 0 || pos_batch_stride == (int64_t)V * 4,
               "rasterize_bwd: pos_batch_stride must be 0 or V*4");
  const int64_t npos = (pos_batch_stride ? (int64_t)N : 1) * V * 4;
  // d_pos is summed in fp64 across workgroups and rounded once, so it does
  // not depend on the order in which their additions land
  double* acc = acc64_begin(stream, npos);
  if (!acc) return scratch_fail();
  const int ntx = (W + kTile - 1) / kTile, nty = (H + kTile - 1) / kTile;
  const int64_t blocks = (int64_t)N * ntx * nty;
  // per (image, triangle) records (one set for all images when pos is
  // shared): those the forward stored, else built here when the triangles
  // average at least 8 pixels of the images (below that, each pixel builds
  // its triangle's record itself)
  const int64_t nrec = (pos_batch_stride ? (int64_t)N : 1) * T;
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  // DR_RASTERIZE_BWD_REUSE: the caller states that the last forward on this
  // stream drew this pos and tri, unchanged since; if that forward wrote the
  // records, they are used as they are
  const auto& L = sc->last_raster;
  const bool reuse = nrec > 0 && (flags & DR_RASTERIZE_BWD_REUSE) && sc->last_raster_reusable() &&
                     L.brec &&
                     L.pos == pos && L.tri == tri && L.N == N && L.V == V && L.T == T &&
                     (L.range ? pos_batch_stride == 0
                              : pos_batch_stride != 0 && L.pos_stride == pos_batch_stride) &&
                     sc->ptr[SLOT_RBWD_REC] &&
                     sc->cap[SLOT_RBWD_REC] >= (size_t)nrec * sizeof(RBwdRec);
  const bool use_rec = reuse || (nrec > 0 && nrec * 8 <= (int64_t)N * H * W);
  RBwdRec* trec = nullptr;
  if (use_rec) {
    if (reuse) {
      trec = (RBwdRec*)sc->ptr[SLOT_RBWD_REC];
    } else {
      trec = (RBwdRec*)scratch_get(sc, stream, SLOT_RBWD_REC, (size_t)nrec * sizeof(RBwdRec));
      if (!trec) return scratch_fail();
      sc->last_raster.brec = false;  // the slot now holds this call's records
      DR_TIMED("k_rbwd_rec", stream);
      hipLaunchKernelGGL(k_rbwd_rec, dim3((unsigned)((nrec + 255) / 256)), dim3(256), 0, stream,
                         pos, pos_batch_stride, tri, nrec, V, T, trec);
    }
  }
  sc->rbwd_want = true;
  DR_CHECK_LAUNCH();
  {
    DR_TIMED("k_raster_bwd", stream);
    const int64_t rs = pos_batch_stride ? (int64_t)T : (int64_t)0;
    if (use_rec)
      hipLaunchKernelGGL(k_raster_bwd<true>, dim3((unsigned)blocks), dim3(256), 0, stream, trec,
                         rs, pos, pos_batch_stride, tri, V, rast, d_rast, d_rast_db, N, T, H, W,
                         ntx, nty, acc);
    else
      hipLaunchKernelGGL(k_raster_bwd<false>, dim3((unsigned)blocks), dim3(256), 0, stream, trec,
                         rs, pos, pos_batch_stride, tri, V, rast, d_rast, d_rast_db, N, T, H, W,
                         ntx, nty, acc);
  }
  DR_CHECK_LAUNCH();
  return acc64_end(acc, d_pos, npos, (flags & DR_ACCUMULATE) != 0, stream);
}
