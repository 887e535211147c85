// antialias: topology hash, silhouette-edge blend forward, and a fused
// backward (d_color gathered through an LDS exchange of the blend weights,
// d_pos scattered with wave-grouped atomics).
//
// Semantics follow Sources/MLXDiffRast/Antialias.swift of the reference:
//   topology hash      :19-66   (here: a GPU edge hash table; the result does
//                                not depend on any ordering, so it is
//                                bit-identical to the reference's sort)
//   silhouette block   :168-326
//   forward            :333-358
//   d_color            :498-524 (atomic scatter in the reference; here each
//                                pixel gathers what its neighbours would
//                                have scattered into it)
//   d_pos              :388-496
#include "common.h"

namespace dr {

// ---------------------------------------------------------------------------
// topology hash
// ---------------------------------------------------------------------------

constexpr unsigned long long kEmpty = ~0ull;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Edge k of triangle t is the edge opposite vertex k (Antialias.swift:33),
// keyed by (min, max) of its vertex ids.
__device__ __forceinline__ uint64_t edge_key(const int32_t* __restrict__ tri, int64_t e) {
  const int64_t t = e / 3;
  const int k = (int)(e - t * 3);
  const int32_t v0 = tri[t * 3 + 0], v1 = tri[t * 3 + 1], v2 = tri[t * 3 + 2];
  int32_t p = k == 0 ? v1 : (k == 1 ? v2 : v0);
  int32_t q = k == 0 ? v2 : (k == 1 ? v0 : v1);
  const int32_t lo = p < q ? p : q, hi = p < q ? q : p;
  return ((uint64_t)(uint32_t)lo << 32) | (uint64_t)(uint32_t)hi;
}

__global__ void __launch_bounds__(256) k_topo_insert(const int32_t* __restrict__ tri, int64_t E,
                                                     unsigned long long* __restrict__ keys,
                                                     int* __restrict__ cnt, int* __restrict__ slot,
                                                     uint64_t mask) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const uint64_t key = edge_key(tri, e);
  uint64_t h = mix64(key) & mask;
  for (;;) {
    const unsigned long long prev = atomicCAS(&keys[h], kEmpty, (unsigned long long)key);
    if (prev == kEmpty || prev == key) break;
    h = (h + 1) & mask;
  }
  const int c = atomicAdd(&cnt[h], 1);
  if (c < 2) slot[2 * h + c] = (int)e;
}

__global__ void __launch_bounds__(256) k_topo_resolve(const int32_t* __restrict__ tri, int64_t E,
                                                      const unsigned long long* __restrict__ keys,
                                                      const int* __restrict__ cnt,
                                                      const int* __restrict__ slot, uint64_t mask,
                                                      int32_t* __restrict__ topo) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const uint64_t key = edge_key(tri, e);
  uint64_t h = mix64(key) & mask;
  while (keys[h] != key) h = (h + 1) & mask;
  const int c = cnt[h];
  int32_t r;
  if (c == 1) r = -1;                 // boundary
  else if (c == 2) {                  // manifold: the other triangle
    const int other = slot[2 * h] == (int)e ? slot[2 * h + 1] : slot[2 * h];
    r = other / 3;
  } else r = -2;                      // non-manifold (3+ triangles)
  topo[e] = r;
}

// ---------------------------------------------------------------------------
// silhouette (Antialias.swift:168-326)
// ---------------------------------------------------------------------------

// Per (image, triangle) record gathered once per call, so a pixel next to a
// triangle edge needs one 48-byte load instead of the chain topology ->
// vertex ids -> vertex positions:
//   s01 = (x0, y0, x1, y1), s2 = (x2, y2, topo[0] bits, topo[1] bits),
//   tv = (topo[2], v0, v1, v2)
// with pixel-space vertices from the expressions of Antialias.swift:247-250:
// x = (x/w + 1) * W/2, y = (1 - y/w) * H/2.
struct alignas(16) AARec {
  float4 s01, s2;
  int4 tv;
};

// The d_pos factors of a triangle's three corners (Antialias.swift:462-465):
// c[k] = (inv_w, x * inv_w, y * inv_w, 0) of corner k's clip position, with
// inv_w = 1 / w, so the backward loads them beside the record instead of
// gathering the vertices after it.
struct alignas(16) AAPersp {
  float4 c[3];
};

__device__ __forceinline__ float4 persp_of(float4 P) {
  const float inv_w = 1.0f / P.w;
  return make_float4(inv_w, P.x * inv_w, P.y * inv_w, 0.0f);
}

// One thread per record; the records of a workgroup (and their corner
// factors) are assembled in LDS and written out as contiguous 16-byte
// stores.
__global__ void __launch_bounds__(256) k_aa_rec(const float* __restrict__ pos,
                                                const int32_t* __restrict__ tri,
                                                const int32_t* __restrict__ topo, int64_t NT,
                                                int T, int V, int H, int W,
                                                AARec* __restrict__ rec,
                                                AAPersp* __restrict__ persp) {
  __shared__ float4 s_rec[256 * 3];
  __shared__ float4 s_persp[256 * 3];
  const int64_t base = (int64_t)blockIdx.x * 256;
  const int64_t i = base + threadIdx.x;
  if (i < NT) {
    int64_t n;
    int t;
    divmod64(i, T, n, t);
    const float* p = pos + n * V * 4;
    const int v0 = tri[(int64_t)t * 3 + 0], v1 = tri[(int64_t)t * 3 + 1],
              v2 = tri[(int64_t)t * 3 + 2];
    const int k0 = topo[(int64_t)t * 3 + 0], k1 = topo[(int64_t)t * 3 + 1],
              k2 = topo[(int64_t)t * 3 + 2];
    float4* r = s_rec + threadIdx.x * 3;
    float4* q = s_persp + threadIdx.x * 3;
    if (!verts_ok(v0, v1, v2, V)) {
      // a vertex id outside [0, V): NaN corners, so no edge of this triangle
      // separates two pixel centres (it never blends, nothing reads its
      // vertices)
      const float nan = __int_as_float(0x7fc00000);
      r[0] = make_float4(nan, nan, nan, nan);
      r[1] = make_float4(nan, nan, __int_as_float(k0), __int_as_float(k1));
      r[2] = make_float4(__int_as_float(k2), __int_as_float(-1), __int_as_float(-1),
                         __int_as_float(-1));
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      q[0] = z; q[1] = z; q[2] = z;
    } else {
      const float4 P0 = *reinterpret_cast<const float4*>(p + (int64_t)v0 * 4);
      const float4 P1 = *reinterpret_cast<const float4*>(p + (int64_t)v1 * 4);
      const float4 P2 = *reinterpret_cast<const float4*>(p + (int64_t)v2 * 4);
      const float hw = (float)W, hh = (float)H;
      r[0] = make_float4((P0.x / P0.w + 1.0f) * hw * 0.5f, (1.0f - P0.y / P0.w) * hh * 0.5f,
                         (P1.x / P1.w + 1.0f) * hw * 0.5f, (1.0f - P1.y / P1.w) * hh * 0.5f);
      r[1] = make_float4((P2.x / P2.w + 1.0f) * hw * 0.5f, (1.0f - P2.y / P2.w) * hh * 0.5f,
                         __int_as_float(k0), __int_as_float(k1));
      r[2] = make_float4(__int_as_float(k2), __int_as_float(v0), __int_as_float(v1),
                         __int_as_float(v2));
      q[0] = persp_of(P0);
      q[1] = persp_of(P1);
      q[2] = persp_of(P2);
    }
  }
  __syncthreads();
  const int nrec = (int)min((int64_t)256, NT - base);
  float4* dr = reinterpret_cast<float4*>(rec + base);
  for (int j = threadIdx.x; j < nrec * 3; j += 256) dr[j] = s_rec[j];
  if (persp) {
    float4* dq = reinterpret_cast<float4*>(persp + base);
    for (int j = threadIdx.x; j < nrec * 3; j += 256) dq[j] = s_persp[j];
  }
}

struct SilDir {
  float alpha;  // > 0 when active
  int ie0, ie1;
  float e0x, e0y, e1x, e1y, t, denom, dbeta;
};

// Pair (pixel (ph, pw), its neighbour in direction dir): the edge of the
// foreground triangle R whose adjacency entry is `target` and whose line
// separates the two pixel centres (:227-262), then the blend weight of the
// pixel (:264-310). Returns false when the pair contributes nothing.
__device__ __forceinline__ bool sil_geom(const AARec& R, int target, int ph, int pw, int dir,
                                         SilDir& s) {
  const int dw = dir == 0 ? 1 : (dir == 2 ? -1 : 0);
  const int dh = dir == 1 ? 1 : (dir == 3 ? -1 : 0);
  const float pcx = (float)pw + 0.5f, pcy = (float)ph + 0.5f;
  const float ncx = (float)(pw + dw) + 0.5f, ncy = (float)(ph + dh) + 0.5f;
  const int tk[3] = {__float_as_int(R.s2.z), __float_as_int(R.s2.w), R.tv.x};
  const float X[3] = {R.s01.x, R.s01.z, R.s2.x};
  const float Y[3] = {R.s01.y, R.s01.w, R.s2.y};
  const int VI[3] = {R.tv.y, R.tv.z, R.tv.w};
  bool found = false;
  float e0x = 0.f, e0y = 0.f, e1x = 0.f, e1y = 0.f;
  int ie0 = -1, ie1 = -1;
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    const int k1 = (kk + 1) % 3, k2 = (kk + 2) % 3;
    if (!found && tk[kk] == target) {
      const float E0x = X[k1], E0y = Y[k1], E1x = X[k2], E1y = Y[k2];
      const float ex = E1x - E0x, ey = E1y - E0y;
      const float side_p = ex * (pcy - E0y) - ey * (pcx - E0x);
      const float side_n = ex * (ncy - E0y) - ey * (ncx - E0x);
      if (side_p * side_n < 0.0f) {
        found = true;
        ie0 = VI[k1]; ie1 = VI[k2];
        e0x = E0x; e0y = E0y; e1x = E1x; e1y = E1y;
      }
    }
  }
  if (!found) return false;
  float beta = 0.0f, t_val = 0.0f, denom, dbeta = 0.0f;
  if (dh == 0) {  // :274-292
    const float dyv = e1y - e0y;
    denom = dyv;
    if (fabsf(dyv) >= 1e-7f) {
      const float tval = (pcy - e0y) / dyv;
      t_val = tval;
      if (tval >= 0.0f && tval <= 1.0f) {
        const float xe = e0x + tval * (e1x - e0x);
        if (xe > (float)pw && xe < (float)(pw + 1)) {
          const float d = xe - pcx;
          beta = 0.5f - fabsf(d);
          dbeta = (d > 0.0f) ? -1.0f : 1.0f;
        }
      }
    }
  } else {  // :293-309
    const float dxv = e1x - e0x;
    denom = dxv;
    if (fabsf(dxv) >= 1e-7f) {
      const float tval = (pcx - e0x) / dxv;
      t_val = tval;
      if (tval >= 0.0f && tval <= 1.0f) {
        const float ye = e0y + tval * (e1y - e0y);
        if (ye > (float)ph && ye < (float)(ph + 1)) {
          const float d = ye - pcy;
          beta = 0.5f - fabsf(d);
          dbeta = (d > 0.0f) ? -1.0f : 1.0f;
        }
      }
    }
  }
  if (beta <= 0.0f) return false;
  s.alpha = beta;
  s.ie0 = ie0;
  s.ie1 = ie1;
  s.e0x = e0x; s.e0y = e0y; s.e1x = e1x; s.e1y = e1y;
  s.t = t_val;
  s.denom = denom;
  s.dbeta = dbeta;
  return true;
}

// LDS row strides of the tile arrays: a wave's 8x8 quadrant reaches LDS 32
// lanes (four rows of eight) at a time, and a row stride of 8 mod 32 words
// puts those four rows on disjoint banks.
constexpr int kTriRow = 40;    // s_tri[18][kTriRow]: 18 used
constexpr int kAlphaRow = 24;  // s_alpha[4][16][kAlphaRow]: 16 used

// Triangle ids of a 16x16 tile and its 1-pixel border (corners unused).
// kOut marks a neighbour outside the image; ids outside [0, T) read as empty.
constexpr int kOut = -2;

struct AATile {
  int n, x0, y0, lx, ly, pw, ph;
  bool inside;
};

// Triangle id of a rast pixel from its fourth channel; ids outside [0, T)
// read as empty.
__device__ __forceinline__ int aa_id(float w, int T) {
  const int id = f2i(w) - 1;
  return (unsigned)id < (unsigned)T ? id : -1;
}

// The workgroup's tile and this thread's pixel (no memory access).
__device__ __forceinline__ AATile aa_tile(int H, int W, int ntx, int nty) {
  AATile g;
  const int tiles = ntx * nty;
  const int b = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  g.n = b / tiles;
  const int tile = b - g.n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  g.x0 = tx * 16;
  g.y0 = ty * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  g.lx = (wave & 1) * 8 + (lane & 7);
  g.ly = (wave >> 1) * 8 + (lane >> 3);
  g.pw = g.x0 + g.lx;
  g.ph = g.y0 + g.ly;
  g.inside = g.pw < W && g.ph < H;
  return g;
}

// The border pixel of lanes 0..15 of each wave (wave 0: left column,
// 1: right, 2: top row, 3: bottom): its cell in the 18x18 tile array, the
// direction from it into the tile, and whether it lies in the image.
struct AABorder {
  bool lane, in;
  int qh, qw, r, c, d;
  int64_t q;  // pixel index (when in)
};

__device__ __forceinline__ AABorder aa_border(const AATile& g, int H, int W) {
  AABorder b;
  const int side = threadIdx.x >> 6, i = threadIdx.x & 15;
  b.lane = (threadIdx.x & 63) < 16;
  if (side == 0) { b.qw = g.x0 - 1;  b.qh = g.y0 + i;  b.r = i + 1; b.c = 0;     b.d = 0; }
  else if (side == 1) { b.qw = g.x0 + 16; b.qh = g.y0 + i;  b.r = i + 1; b.c = 17;    b.d = 2; }
  else if (side == 2) { b.qw = g.x0 + i;  b.qh = g.y0 - 1;  b.r = 0;     b.c = i + 1; b.d = 1; }
  else { b.qw = g.x0 + i;  b.qh = g.y0 + 16; b.r = 17;    b.c = i + 1; b.d = 3; }
  b.in = b.lane && b.qh >= 0 && b.qh < H && b.qw >= 0 && b.qw < W;
  b.q = ((int64_t)g.n * H + b.qh) * W + b.qw;
  return b;
}

// Triangle ids of the tile and its border into s_tri (corners unused): the
// kernels issue these rast loads together with their other per-pixel loads
// and store afterwards, so the loads share one round trip.
__device__ __forceinline__ void aa_store_ids(const AATile& g, const AABorder& bd, float own_w,
                                             float border_w, int T, int (*s_tri)[kTriRow]) {
  s_tri[g.ly + 1][g.lx + 1] = g.inside ? aa_id(own_w, T) : kOut;
  if (bd.lane) s_tri[bd.r][bd.c] = bd.in ? aa_id(border_w, T) : kOut;
}

// Blend-mask byte of pixel (n, h, w): 16x16 tiles in row-major order, 256
// bytes each, a tile's 8x8 quadrants in the order of the waves that own
// them and pixels row-major within a quadrant, so each wave writes and
// reads 64 consecutive bytes.
__device__ __forceinline__ int64_t mask_index(int n, int h, int w, int ntx, int nty) {
  const int ly = h & 15, lx = w & 15;
  return (((int64_t)n * nty + (h >> 4)) * ntx + (w >> 4)) * 256 +
         ((ly >> 3) * 2 + (lx >> 3)) * 64 + (ly & 7) * 8 + (lx & 7);
}

// Neighbour of tile cell (r, c) (1-based, border included) in direction d:
// 0 = +w, 1 = +h, 2 = -w, 3 = -h.
__device__ __forceinline__ int aa_nb(int (*s_tri)[kTriRow], int r, int c, int d) {
  return d == 0 ? s_tri[r][c + 1] : d == 1 ? s_tri[r + 1][c] : d == 2 ? s_tri[r][c - 1]
                                                                      : s_tri[r - 1][c];
}

// Whether the pair (own triangle tp, neighbour tn) is a silhouette
// candidate (:203-204): inside the image, different, not both empty.
__device__ __forceinline__ bool aa_cand(int tp, int tn) {
  return tn != kOut && tn != tp && (tp >= 0 || tn >= 0);
}

// Full per-direction state of one candidate pair: the foreground is the
// pixel's own triangle when it has one (record rp), else the neighbour's
// (:206-222).
__device__ __forceinline__ bool aa_pair(const AARec* __restrict__ recn, const AARec& rp, int tp,
                                        int tn, int ph, int pw, int d, SilDir& s) {
  if (tp >= 0) return sil_geom(rp, tn, ph, pw, d, s);
  const AARec rn = recn[tn];
  return sil_geom(rn, -1, ph, pw, d, s);
}

template <int CT>
__device__ __forceinline__ void ld_px(const float* __restrict__ p, int C, float* v) {
  if constexpr (CT == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
#pragma unroll
    for (int c = 0; c < (CT > 0 ? CT : 1); ++c) v[c] = p[c];
  }
}

template <int CT>
__device__ __forceinline__ void st_px(float* __restrict__ p, const float* v) {
  if constexpr (CT == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int c = 0; c < CT; ++c) p[c] = v[c];
  }
}

// Antialias.swift:333-358 on 16x16 tiles: triangle ids of the tile and its
// border are staged in LDS once; only pixels next to a different triangle
// load a record. CT = channel count when 1..4 (registers), 0 = any C.
template <int CT>
__global__ void __launch_bounds__(256) k_aa_fwd(const float* __restrict__ rast,
                                                const AARec* __restrict__ rec,
                                                const float* __restrict__ color, int H, int W,
                                                int T, int C, int ntx, int nty,
                                                float* __restrict__ out,
                                                uint8_t* __restrict__ blend_mask,
                                                int* __restrict__ saved_ids) {
  __shared__ int s_tri[18][kTriRow];
  // colours of the tile and its border (CT > 0), so a blend reads its
  // neighbour from LDS rather than in a third global round trip
  __shared__ __align__(16) float s_col[18][18][CT > 0 ? CT : 1];
  const AATile g = aa_tile(H, W, ntx, nty);
  const AABorder bd = aa_border(g, H, W);
  const int64_t pix = ((int64_t)g.n * H + min(g.ph, H - 1)) * W + min(g.pw, W - 1);
  // every load before the barrier is issued first: own and border ids and colours
  const float own_w = rast[pix * 4 + 3];
  float border_w = 0.0f;
  if (bd.in) border_w = rast[bd.q * 4 + 3];
  float cp[CT > 0 ? CT : 1];
  float cb[CT > 0 ? CT : 1];
  if constexpr (CT > 0) {
    if (g.inside) ld_px<CT>(color + pix * CT, CT, cp);
    if (bd.in) ld_px<CT>(color + bd.q * CT, CT, cb);
  }
  aa_store_ids(g, bd, own_w, border_w, T, s_tri);
  if constexpr (CT > 0) {
    if (g.inside) st_px<CT>(&s_col[g.ly + 1][g.lx + 1][0], cp);
    if (bd.in) st_px<CT>(&s_col[bd.r][bd.c][0], cb);
  }
  __syncthreads();
  if (!g.inside) return;
  const int r = g.ly + 1, c = g.lx + 1;
  const int tp = s_tri[r][c];
  int tn[4];
  bool any = false;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    tn[d] = aa_nb(s_tri, r, c, d);
    any = any || aa_cand(tp, tn[d]);
  }
  float alpha[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool blend = false;
  int bits = 0;
  if (any) {
    const AARec* recn = rec + (int64_t)g.n * T;
    AARec rp;
    if (tp >= 0) rp = recn[tp];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      if (!aa_cand(tp, tn[d])) continue;
      SilDir s;
      if (aa_pair(recn, rp, tp, tn[d], g.ph, g.pw, d, s)) {
        alpha[d] = s.alpha;
        blend = true;
        bits |= 1 << d;
      }
    }
  }
  if (blend_mask) {
    const int64_t mi = mask_index(g.n, g.ph, g.pw, ntx, nty);
    blend_mask[mi] = (uint8_t)bits;
    saved_ids[mi] = tp;
  }
  if constexpr (CT > 0) {
    if (blend) {
      float acc[CT];
#pragma unroll
      for (int k = 0; k < CT; ++k) acc[k] = cp[k];
      // a blending neighbour is a candidate, so it lies in the image and
      // its colour is in s_col
      const int nr[4] = {r, r + 1, r, r - 1}, nc[4] = {c + 1, c, c - 1, c};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        if (alpha[d] > 0.0f) {
          float cn[CT];
          ld_px<CT>(&s_col[nr[d]][nc[d]][0], CT, cn);
#pragma unroll
          for (int k = 0; k < CT; ++k) acc[k] += alpha[d] * (cn[k] - cp[k]);
        }
      }
      st_px<CT>(out + pix * CT, acc);
    } else {
      st_px<CT>(out + pix * CT, cp);
    }
  } else {
    const float* cp = color + pix * C;
    float* o = out + pix * C;
    const int64_t nb[4] = {pix + 1, pix + W, pix - 1, pix - W};
    for (int k = 0; k < C; ++k) {
      const float cpc = cp[k];
      float acc = cpc;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        if (alpha[d] > 0.0f) acc += alpha[d] * (color[nb[d] * C + k] - cpc);
      o[k] = acc;
    }
  }
}

// d_pos terms of one partial blend (Antialias.swift:405-495): the blend
// weight's gradient d_alpha = sum_c g * (c_neighbour - c_own) through the
// crossing point into the edge's two clip-space vertices P0, P1.
// Q0, Q1: the edge vertices' (inv_w, x * inv_w, y * inv_w) (persp_of).
__device__ __forceinline__ void aa_dpos_add(const SilDir& s, int d, int ph, int pw, float d_alpha,
                                            float4 Q0, float4 Q1, double* __restrict__ dp,
                                            float halfW, float halfH, LdsTableU<4, 128>& tab) {
  float dade0x, dade0y, dade1x, dade1y;
  const float inv_denom_sq = 1.0f / (s.denom * s.denom);
  if (d == 0 || d == 2) {
    const float row_y = (float)ph + 0.5f;
    const float ex_diff = s.e1x - s.e0x;
    dade0x = s.dbeta * (1.0f - s.t);
    dade1x = s.dbeta * s.t;
    dade0y = s.dbeta * ex_diff * (row_y - s.e1y) * inv_denom_sq;
    dade1y = s.dbeta * (-ex_diff) * (row_y - s.e0y) * inv_denom_sq;
  } else {
    const float col_x = (float)pw + 0.5f;
    const float ey_diff = s.e1y - s.e0y;
    dade0y = s.dbeta * (1.0f - s.t);
    dade1y = s.dbeta * s.t;
    dade0x = s.dbeta * ey_diff * (col_x - s.e1x) * inv_denom_sq;
    dade1x = s.dbeta * (-ey_diff) * (col_x - s.e0x) * inv_denom_sq;
  }
  const int iv[2] = {s.ie0, s.ie1};
  const float dex[2] = {dade0x, dade1x}, dey[2] = {dade0y, dade1y};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float4 Q = e == 0 ? Q0 : Q1;
    const float inv_w = Q.x, nd_x = Q.y, nd_y = Q.z;
    const float dv[4] = {
        d_alpha * dex[e] * halfW * inv_w, d_alpha * dey[e] * (-halfH) * inv_w, 0.0f,
        d_alpha * (dex[e] * (-halfW * nd_x) + dey[e] * (halfH * nd_y)) * inv_w};
    lds_table_add(tab, dp + (int64_t)iv[e] * 4, dv);
  }
}

// The same with d_alpha and the vertices loaded from global memory.
__device__ __forceinline__ bool aa_dpos_terms(const SilDir& s, int d, int ph, int pw, int Cn,
                                              const float* __restrict__ gp,
                                              const float* __restrict__ cpp,
                                              const float* __restrict__ cnp,
                                              const float* __restrict__ p, double* __restrict__ dp,
                                              float halfW, float halfH, LdsTableU<4, 128>& tab) {
  float d_alpha = 0.0f;
  for (int k = 0; k < Cn; ++k) d_alpha += gp[k] * (cnp[k] - cpp[k]);
  if (d_alpha == 0.0f) return false;
  const float4 P0 = *reinterpret_cast<const float4*>(p + (int64_t)s.ie0 * 4);
  const float4 P1 = *reinterpret_cast<const float4*>(p + (int64_t)s.ie1 * 4);
  aa_dpos_add(s, d, ph, pw, d_alpha, persp_of(P0), persp_of(P1), dp, halfW, halfH, tab);
  return true;
}

// A partial blend queued for its d_pos terms: the edge state and where.
struct PosItem {
  float e0x, e0y, e1x, e1y, t, denom, dbeta;
  int ie0, ie1;
  int where;  // local pixel (ly * 16 + lx) * 4 + direction
};
constexpr int kPosQueue = 256;

// Fused backward on 16x16 tiles (one 8x8 quadrant per wave): each pixel's
// blend weights come first, its partial blends are queued in LDS; d_color
// (Antialias.swift:498-524) is gathered through an LDS exchange of the
// blend weights; then every thread takes one queued blend and adds its
// d_pos terms (summed per vertex in LDS), so the few lanes with partial
// blends do not each walk the whole chain of loads while the rest idle.
template <int CT>
__global__ void __launch_bounds__(256) k_aa_bwd(const float* __restrict__ rast,
                                                const AARec* __restrict__ rec,
                                                const float* __restrict__ pos,
                                                const float* __restrict__ color,
                                                const float* __restrict__ d_out, int H, int W,
                                                int V, int T, int C, int ntx, int nty,
                                                float* __restrict__ d_color,
                                                double* __restrict__ d_pos, int accumulate) {
  __shared__ int s_tri[18][kTriRow];
  __shared__ float s_alpha[4][16][kAlphaRow];
  __shared__ float s_halo[4][16];
  __shared__ LdsTableU<4, 128> tab;  // d_pos rows touched by this tile
  __shared__ PosItem s_q[kPosQueue];
  __shared__ int s_nq;              // queued partial blends
  __shared__ int s_need;            // the table holds terms
  if (d_pos) lds_table_clear(tab);
  if (threadIdx.x == 0) { s_need = 0; s_nq = 0; }
  const AATile g = aa_tile(H, W, ntx, nty);
  const AABorder bd = aa_border(g, H, W);
  const int64_t pix = ((int64_t)g.n * H + min(g.ph, H - 1)) * W + min(g.pw, W - 1);
  // every load before the barrier is issued first: own and border ids, own cotangent
  const float own_w = rast[pix * 4 + 3];
  float border_w = 0.0f;
  if (bd.in) border_w = rast[bd.q * 4 + 3];
  float gv[CT > 0 ? CT : 1], old[CT > 0 ? CT : 1];
  if constexpr (CT > 0) {
    if (d_color && g.inside) {
      ld_px<CT>(d_out + pix * CT, CT, gv);
      if (accumulate) ld_px<CT>(d_color + pix * CT, CT, old);
    }
  }
  aa_store_ids(g, bd, own_w, border_w, T, s_tri);
  __syncthreads();
  const AARec* recn = rec + (int64_t)g.n * T;
  const int r = g.ly + 1, c = g.lx + 1;
  const int tp = s_tri[r][c];
  const int Cn = CT > 0 ? CT : C;

  // 1) own blend weights; the partial ones are queued for their d_pos terms.
  float alpha[4];
  float asum = 0.0f;
  int ovf = 0;
  {
    int tn[4];
    bool any = false;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      tn[d] = aa_nb(s_tri, r, c, d);
      any = any || (g.inside && aa_cand(tp, tn[d]));
    }
    AARec rp;
    if (any && tp >= 0) rp = recn[tp];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      SilDir s;
      const bool on = any && aa_cand(tp, tn[d]) && aa_pair(recn, rp, tp, tn[d], g.ph, g.pw, d, s);
      alpha[d] = on ? s.alpha : 0.0f;
      s_alpha[d][g.ly][g.lx] = alpha[d];
      asum += alpha[d];
      if (d_pos && on && s.alpha < 1.0f) {
        const int slot = atomicAdd(&s_nq, 1);
        if (slot < kPosQueue) {
          PosItem it;
          it.e0x = s.e0x; it.e0y = s.e0y; it.e1x = s.e1x; it.e1y = s.e1y;
          it.t = s.t; it.denom = s.denom; it.dbeta = s.dbeta;
          it.ie0 = s.ie0; it.ie1 = s.ie1;
          it.where = ((g.ly * 16 + g.lx) << 2) | d;
          s_q[slot] = it;
        } else {
          ovf |= 1 << d;  // queue full: this lane adds these terms itself, below
        }
      }
    }
  }
  if (ovf) s_need = 1;
  // 2) border: the one direction of each outside neighbour that points into
  //    the tile; lanes 0..15 of each wave take one side.
  if (bd.lane) {
    float al = 0.0f;
    const int tq = s_tri[bd.r][bd.c];
    if (tq != kOut) {
      const int tn = aa_nb(s_tri, bd.r, bd.c, bd.d);
      if (aa_cand(tq, tn)) {
        AARec rq;
        if (tq >= 0) rq = recn[tq];
        SilDir s;
        if (aa_pair(recn, rq, tq, tn, bd.qh, bd.qw, bd.d, s)) al = s.alpha;
      }
    }
    s_halo[threadIdx.x >> 6][threadIdx.x & 15] = al;
  }
  __syncthreads();

  const int lx = g.lx, ly = g.ly;
  // 3) d_color: own term + what each neighbour's blend sends here.
  if (d_color && g.inside) {
    float wn[4];
    wn[0] = lx < 15 ? s_alpha[2][ly][lx + 1] : s_halo[1][ly];  // right neighbour, its dir 2
    wn[1] = ly < 15 ? s_alpha[3][ly + 1][lx] : s_halo[3][lx];  // lower neighbour, its dir 3
    wn[2] = lx > 0 ? s_alpha[0][ly][lx - 1] : s_halo[0][ly];   // left neighbour, its dir 0
    wn[3] = ly > 0 ? s_alpha[1][ly - 1][lx] : s_halo[2][lx];   // upper neighbour, its dir 1
    const int64_t qn[4] = {pix + 1, pix + W, pix - 1, pix - W};
    if constexpr (CT > 0) {
      float acc[CT];
#pragma unroll
      for (int k = 0; k < CT; ++k) acc[k] = gv[k] * (1.0f - asum);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        if (wn[d] > 0.0f) {
          float gq[CT];
          ld_px<CT>(d_out + qn[d] * CT, CT, gq);
#pragma unroll
          for (int k = 0; k < CT; ++k) acc[k] += gq[k] * wn[d];
        }
      }
      if (accumulate) {
#pragma unroll
        for (int k = 0; k < CT; ++k) acc[k] = old[k] + acc[k];
      }
      st_px<CT>(d_color + pix * CT, acc);
    } else {
      const float* gp = d_out + pix * C;
      float* dc = d_color + pix * C;
      for (int k = 0; k < C; ++k) {
        float acc = gp[k] * (1.0f - asum);
#pragma unroll
        for (int d = 0; d < 4; ++d)
          if (wn[d] > 0.0f) acc += d_out[qn[d] * C + k] * wn[d];
        dc[k] = accumulate ? dc[k] + acc : acc;
      }
    }
  }
  // 4) d_pos terms of the queued partial blends, one per thread, then the
  //    per-vertex sums are written out.
  if (!d_pos) return;  // uniform
  const int nq = min(s_nq, kPosQueue);
  if (nq == 0 && !s_need) return;  // uniform: both read after the barrier
  for (int i = threadIdx.x; i < nq; i += blockDim.x) {
    const PosItem it = s_q[i];
    SilDir s;
    s.e0x = it.e0x; s.e0y = it.e0y; s.e1x = it.e1x; s.e1y = it.e1y;
    s.t = it.t; s.denom = it.denom; s.dbeta = it.dbeta;
    s.ie0 = it.ie0; s.ie1 = it.ie1;
    const int d = it.where & 3, lp = it.where >> 2;
    const int qlx = lp & 15, qly = lp >> 4;
    const int qph = g.y0 + qly, qpw = g.x0 + qlx;
    const int64_t qp = ((int64_t)g.n * H + qph) * W + qpw;
    const int64_t qn = d == 0 ? qp + 1 : d == 1 ? qp + W : d == 2 ? qp - 1 : qp - W;
    aa_dpos_terms(s, d, qph, qpw, Cn, d_out + qp * Cn, color + qp * Cn, color + qn * Cn,
                  pos + (int64_t)g.n * V * 4, d_pos + (int64_t)g.n * V * 4, (float)W * 0.5f,
                  (float)H * 0.5f, tab);
  }
  if (ovf) {  // blends that did not fit the queue: recompute the edge state
    AARec rp;
    if (tp >= 0) rp = recn[tp];
    for (int d = 0; d < 4; ++d) {
      if (!((ovf >> d) & 1)) continue;
      SilDir s;
      if (!aa_pair(recn, rp, tp, aa_nb(s_tri, r, c, d), g.ph, g.pw, d, s)) continue;
      const int64_t qn = d == 0 ? pix + 1 : d == 1 ? pix + W : d == 2 ? pix - 1 : pix - W;
      aa_dpos_terms(s, d, g.ph, g.pw, Cn, d_out + pix * Cn, color + pix * Cn, color + qn * Cn,
                    pos + (int64_t)g.n * V * 4, d_pos + (int64_t)g.n * V * 4, (float)W * 0.5f,
                    (float)H * 0.5f, tab);
    }
  }
  __syncthreads();
  lds_table_flush_last<4, 128, double>(tab);  // the taken rows only
}

constexpr int kMaskQueue = 256 * 4 + 64;

// A queued pair with its loads in flight: cell and direction, the
// foreground record, and (d_pos, inside the tile) its corners' d_pos
// factors and the two pixels' colours (CT > 0), all issued together.
template <int CT>
struct AAPairIn {
  int cell, d, tq, tn;
  bool ok, border;
  AARec R;
  float4 Q[3];
  float cp[CT > 0 ? CT : 1], cn[CT > 0 ? CT : 1];
};

template <int CT>
__device__ __forceinline__ void aa_pair_load(int e, int (*s_tri)[kTriRow], const AATile& g, int H,
                                             int W, const AARec* __restrict__ recn,
                                             const AAPersp* __restrict__ perspn,
                                             const float* __restrict__ color, bool want_pos,
                                             AAPairIn<CT>& P) {
  P.d = e & 3;
  P.cell = e >> 2;
  const int rr = P.cell / 18, cc = P.cell - rr * 18;
  P.tq = s_tri[rr][cc];
  P.tn = aa_nb(s_tri, rr, cc, P.d);
  // a mask the forward wrote only marks candidate pairs; anything else is
  // skipped, so no mask content can make the record index go out of range
  P.ok = aa_cand(P.tq, P.tn);
  if (!P.ok) return;
  P.border = rr == 0 || rr == 17 || cc == 0 || cc == 17;
  // the foreground record (:206-222): the pixel's own, else the neighbour's
  const int fg = P.tq >= 0 ? P.tq : P.tn;
  P.R = recn[fg];
  if (want_pos && !P.border) {
    P.Q[0] = perspn[fg].c[0];
    P.Q[1] = perspn[fg].c[1];
    P.Q[2] = perspn[fg].c[2];
    if constexpr (CT > 0) {
      // a masked pair of the tile blends (alpha in (0, 0.5]), so with d_pos
      // its colours are needed: load them now rather than after the record
      const int qph = g.y0 + rr - 1, qpw = g.x0 + cc - 1;
      const int64_t qp = ((int64_t)g.n * H + qph) * W + qpw;
      const int64_t qn = P.d == 0 ? qp + 1 : P.d == 1 ? qp + W : P.d == 2 ? qp - 1 : qp - W;
      ld_px<CT>(color + qp * CT, CT, P.cp);
      ld_px<CT>(color + qn * CT, CT, P.cn);
    }
  }
}

// The pair's blend weight (into s_alpha, or s_halo for a border pixel) and,
// for the tile's own pixels, its d_pos terms.
template <int CT>
__device__ __forceinline__ void aa_pair_eval(const AAPairIn<CT>& P, const AATile& g, int H, int W,
                                             int C, float (*s_alpha)[16][kAlphaRow],
                                             float (*s_halo)[16],
                                             const float (*s_g)[CT > 0 ? CT : 1],
                                             const float* __restrict__ color,
                                             const float* __restrict__ d_out,
                                             double* __restrict__ dpn, LdsTableU<4, 128>& tab) {
  if (!P.ok) return;
  const int rr = P.cell / 18, cc = P.cell - rr * 18, d = P.d;
  const int qph = g.y0 + rr - 1, qpw = g.x0 + cc - 1;
  SilDir s;
  const bool on = sil_geom(P.R, P.tq >= 0 ? P.tn : -1, qph, qpw, d, s);
  const float al = on ? s.alpha : 0.0f;
  if (P.border) {
    const int side = cc == 0 ? 0 : cc == 17 ? 1 : rr == 0 ? 2 : 3;
    s_halo[side][side < 2 ? rr - 1 : cc - 1] = al;
    return;
  }
  s_alpha[d][rr - 1][cc - 1] = al;
  if (!dpn || !on || !(s.alpha < 1.0f)) return;
  float d_alpha = 0.0f;
  if constexpr (CT > 0) {
#pragma unroll
    for (int k = 0; k < CT; ++k) d_alpha += s_g[P.cell][k] * (P.cn[k] - P.cp[k]);
  } else {
    const int64_t qp = ((int64_t)g.n * H + qph) * W + qpw;
    const int64_t qn = d == 0 ? qp + 1 : d == 1 ? qp + W : d == 2 ? qp - 1 : qp - W;
    for (int k = 0; k < C; ++k)
      d_alpha += d_out[qp * C + k] * (color[qn * C + k] - color[qp * C + k]);
  }
  if (d_alpha == 0.0f) return;
  const int4 tv = P.R.tv;
  const float4 Q0 = s.ie0 == tv.y ? P.Q[0] : s.ie0 == tv.z ? P.Q[1] : P.Q[2];
  const float4 Q1 = s.ie1 == tv.y ? P.Q[0] : s.ie1 == tv.z ? P.Q[1] : P.Q[2];
  aa_dpos_add(s, d, qph, qpw, d_alpha, Q0, Q1, dpn, (float)W * 0.5f, (float)H * 0.5f, tab);
}

// Backward with the forward's blend mask (bit d of a pixel set when its
// blend weight toward direction d is nonzero).  Only the masked pairs are
// evaluated: the tile's own pairs and the border pairs that point into the
// tile are compacted into an LDS queue (it holds every pair of the tile, so
// it cannot overflow); each thread takes one, recomputes its edge state
// with the forward's expressions, leaves the blend weight for the d_color
// exchange and, for the tile's own pixels, adds the d_pos terms.  Pixels
// without blends load no record.  A tile costs two memory round trips:
// its ids, mask bytes and cotangents (with CT > 0 those of the border too,
// staged in LDS), then each pair's record, corner factors and colours.
template <int CT>
__global__ void __launch_bounds__(256) k_aa_bwd_masked(
    const int* __restrict__ saved_ids, const AARec* __restrict__ rec,
    const AAPersp* __restrict__ persp, const float* __restrict__ color,
    const float* __restrict__ d_out, const uint8_t* __restrict__ blend_mask, int H, int W, int V,
    int T, int C, int ntx, int nty, float* __restrict__ d_color, double* __restrict__ d_pos,
    int accumulate) {
  constexpr int CS = CT > 0 ? CT : 1;
  constexpr int kCells = CT > 0 ? 18 * 18 : 1;
  __shared__ int s_tri[18][kTriRow];
  __shared__ float s_alpha[4][16][kAlphaRow];
  __shared__ float s_halo[4][16];
  __shared__ LdsTableU<4, 128> tab;      // d_pos rows touched by this tile
  __shared__ uint16_t s_q[kMaskQueue];   // (cell r * 18 + c) << 2 | direction
  __shared__ int s_nq;
  __shared__ float s_g[kCells][CS];  // d_out of the tile and its border (CT > 0)
  if (d_pos) lds_table_clear(tab);
  if (threadIdx.x == 0) s_nq = 0;
  const AATile g = aa_tile(H, W, ntx, nty);
  const AABorder bd = aa_border(g, H, W);
  const int64_t pix = ((int64_t)g.n * H + min(g.ph, H - 1)) * W + min(g.pw, W - 1);
  const int lx = g.lx, ly = g.ly;
  const int own = (ly + 1) * 18 + (lx + 1);
  // every load before the barriers is issued first: the own pixel's id, mask
  // byte and cotangent, and (lanes 0..15 of each wave) one border pixel's
  // id, mask byte and cotangent.  The ids are the forward's (the triangle
  // ids of rast, 4 bytes a pixel beside the mask instead of rast's 16).
  const int64_t mi = mask_index(g.n, min(g.ph, H - 1), min(g.pw, W - 1), ntx, nty);
  const int own_id = saved_ids[mi];
  const int own_m = blend_mask[mi];
  int border_id = -1, border_m = 0;
  float gown[CS], gbd[CS];
  if constexpr (CT > 0) ld_px<CT>(d_out + pix * CT, CT, gown);
  if (bd.in) {
    const int64_t bi = mask_index(g.n, bd.qh, bd.qw, ntx, nty);
    border_id = saved_ids[bi];
    border_m = blend_mask[bi];
    if constexpr (CT > 0) ld_px<CT>(d_out + bd.q * CT, CT, gbd);
  }
  // s_nq = 0 is seen by every wave before its first queue slot is taken
  // (the loads above are in flight meanwhile)
  __syncthreads();
  // a saved id outside [0, T) reads as empty, as a rast id does, so no
  // state content can make a record index go out of range
  s_tri[ly + 1][lx + 1] = g.inside ? ((unsigned)own_id < (unsigned)T ? own_id : -1) : kOut;
  if (bd.lane) s_tri[bd.r][bd.c] = bd.in ? ((unsigned)border_id < (unsigned)T ? border_id : -1) : kOut;
  if constexpr (CT > 0) {
#pragma unroll
    for (int k = 0; k < CT; ++k) s_g[own][k] = gown[k];
    if (bd.in) {
#pragma unroll
      for (int k = 0; k < CT; ++k) s_g[bd.r * 18 + bd.c][k] = gbd[k];
    }
  }
  // 1) queue the masked pairs: own pixel (all four directions), and the
  //    border pixel's direction into the tile.
  {
    const int m = g.inside ? own_m & 15 : 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) s_alpha[d][ly][lx] = 0.0f;
    if (bd.lane) s_halo[threadIdx.x >> 6][threadIdx.x & 15] = 0.0f;
    const int hm = bd.in && ((border_m >> bd.d) & 1);
    const int cnt = __popc(m) + hm;
    if (cnt) {
      int slot = atomicAdd(&s_nq, cnt);
#pragma unroll
      for (int d = 0; d < 4; ++d)
        if ((m >> d) & 1) s_q[slot++] = (uint16_t)((own << 2) | d);
      if (hm) s_q[slot] = (uint16_t)(((bd.r * 18 + bd.c) << 2) | bd.d);
    }
  }
  __syncthreads();
  // 2) one queued pair per thread: blend weight and the d_pos terms.
  const AARec* recn = rec + (int64_t)g.n * T;
  const AAPersp* perspn = persp + (int64_t)g.n * T;
  double* dpn = d_pos ? d_pos + (int64_t)g.n * V * 4 : nullptr;
  const int nq = s_nq;
  for (int i = threadIdx.x; i < nq; i += blockDim.x) {
    AAPairIn<CT> P;
    aa_pair_load<CT>(s_q[i], s_tri, g, H, W, recn, perspn, color, dpn != nullptr, P);
    aa_pair_eval<CT>(P, g, H, W, C, s_alpha, s_halo, s_g, color, d_out, dpn, tab);
  }
  __syncthreads();
  // 3) d_color: own term + what each neighbour's blend sends here.
  if (d_color && g.inside) {
    float asum = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) asum += s_alpha[d][ly][lx];
    float wn[4];
    wn[0] = lx < 15 ? s_alpha[2][ly][lx + 1] : s_halo[1][ly];  // right neighbour, its dir 2
    wn[1] = ly < 15 ? s_alpha[3][ly + 1][lx] : s_halo[3][lx];  // lower neighbour, its dir 3
    wn[2] = lx > 0 ? s_alpha[0][ly][lx - 1] : s_halo[0][ly];   // left neighbour, its dir 0
    wn[3] = ly > 0 ? s_alpha[1][ly - 1][lx] : s_halo[2][lx];   // upper neighbour, its dir 1
    if constexpr (CT > 0) {
      // a neighbour with a nonzero weight lies in the image, so its
      // cotangent is in s_g (a border cell when outside the tile)
      const int nc[4] = {own + 1, own + 18, own - 1, own - 18};
      float acc[CT];
#pragma unroll
      for (int k = 0; k < CT; ++k) acc[k] = s_g[own][k] * (1.0f - asum);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        if (wn[d] > 0.0f) {
#pragma unroll
          for (int k = 0; k < CT; ++k) acc[k] += s_g[nc[d]][k] * wn[d];
        }
      }
      if (accumulate) {
        float old[CT];
        ld_px<CT>(d_color + pix * CT, CT, old);
#pragma unroll
        for (int k = 0; k < CT; ++k) acc[k] = old[k] + acc[k];
      }
      st_px<CT>(d_color + pix * CT, acc);
    } else {
      const int64_t qn[4] = {pix + 1, pix + W, pix - 1, pix - W};
      const float* gp = d_out + pix * C;
      float* dc = d_color + pix * C;
      for (int k = 0; k < C; ++k) {
        float acc = gp[k] * (1.0f - asum);
#pragma unroll
        for (int d = 0; d < 4; ++d)
          if (wn[d] > 0.0f) acc += d_out[qn[d] * C + k] * wn[d];
        dc[k] = accumulate ? dc[k] + acc : acc;
      }
    }
  }
  if (!d_pos || nq == 0) return;  // uniform: nq was read after the barrier
  __syncthreads();
  lds_table_flush_last<4, 128, double>(tab);  // the taken rows only
}

}  // namespace dr

using namespace dr;

extern "C" int dr_antialias_topology(const int32_t* tri, int T, int32_t* topo,
                                     dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  DR_CHECK_ARG(tri && topo && T >= 0, "antialias_topology: bad arguments");
  DR_CHECK_ARG(T <= INT32_MAX / 3, "antialias_topology: at most 715827882 triangles (edges are indexed in 32 bits)");
  if (T == 0) return DR_OK;
  const int64_t E = (int64_t)T * 3;
  uint64_t S = 64;
  while (S < (uint64_t)E * 2) S <<= 1;
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  char* buf = (char*)scratch_get(sc, stream, SLOT_TOPO, (size_t)S * 16);
  if (!buf) return scratch_fail();
  unsigned long long* keys = (unsigned long long*)buf;
  int* cnt = (int*)(buf + S * 8);
  int* slot = cnt + S;
  DR_CHECK_HIP(fill_async(keys, kEmpty, (int64_t)S, stream));
  DR_CHECK_HIP(fill_async(cnt, 0, (int64_t)S, stream));
  {
  DR_TIMED("k_topo_insert", stream);
  hipLaunchKernelGGL(k_topo_insert, dim3(grid_for(E, 256)), dim3(256), 0, stream, tri, E, keys,
                     cnt, slot, S - 1);
  }
  DR_CHECK_LAUNCH();
  DR_TIMED("k_topo_resolve", stream);
  hipLaunchKernelGGL(k_topo_resolve, dim3(grid_for(E, 256)), dim3(256), 0, stream, tri, E, keys,
                     cnt, slot, S - 1, topo);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

// Per-(image, triangle) records into rec (scratch when rec is null), and
// their corners' d_pos factors into persp when it is not null.
static int aa_records(const float* pos, const int32_t* tri, const int32_t* topo, int N, int V,
                      int T, int H, int W, hipStream_t stream, AARec* rec, AAPersp* persp,
                      AARec** out) {
  const int64_t nt = (int64_t)N * T;
  if (!rec) {
    Scratch* sc = scratch_for(stream);
    if (!sc) return scratch_fail();
    rec = (AARec*)scratch_get(sc, stream, SLOT_AA_REC, (size_t)(nt > 0 ? nt : 1) * sizeof(AARec));
    if (!rec) return scratch_fail();
  }
  if (nt > 0) {
    DR_TIMED("k_aa_rec", stream);
    hipLaunchKernelGGL(k_aa_rec, dim3(grid_for(nt, 256)), dim3(256), 0, stream, pos, tri, topo,
                       nt, T, V, H, W, rec, persp);
  }
  DR_CHECK_LAUNCH();
  *out = rec;
  return DR_OK;
}

// Saved state of dr_antialias_fwd_save: the blend mask (one byte per pixel
// of the image padded to 16x16 tiles, a multiple of 256 bytes), then the
// per-(image, triangle) records, then their corners' d_pos factors.
// Saved state of dr_antialias_fwd_save: the blend mask (one byte a pixel,
// mask_index order), the pixels' triangle ids (int32, same order), then the
// records and their corner factors.
static int64_t aa_mask_bytes(int N, int H, int W) {
  return (int64_t)N * ((H + 15) / 16) * ((W + 15) / 16) * 256;
}

static int check_aa(const float* color, const float* rast, const float* pos, const int32_t* tri,
                    const int32_t* topo, int N, int H, int W, int C, int V, int T) {
  DR_CHECK_ARG(color && rast && pos && tri && topo, "antialias: null tensor");
  DR_CHECK_ARG(N >= 1 && H >= 1 && W >= 1 && C >= 1 && V >= 0 && T >= 0, "antialias: bad sizes");
  DR_CHECK_ARG(T <= INT32_MAX / 3, "antialias: at most 715827882 triangles (edges are indexed in 32 bits)");
  return DR_OK;
}

// Channel count as a template argument when it fits in registers (float4
// accesses need 16-byte aligned rows).
static int aa_ct(int C, const void* a, const void* b, const void* c) {
  const bool al = (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) == 0;
  if (C == 4) return al ? 4 : 0;
  return C <= 3 ? C : 0;
}

#define DR_AA_DISPATCH(KER, CT, ...)                                               \
  switch (CT) {                                                                   \
    case 1: hipLaunchKernelGGL((KER<1>), __VA_ARGS__); break;                     \
    case 2: hipLaunchKernelGGL((KER<2>), __VA_ARGS__); break;                     \
    case 3: hipLaunchKernelGGL((KER<3>), __VA_ARGS__); break;                     \
    case 4: hipLaunchKernelGGL((KER<4>), __VA_ARGS__); break;                     \
    default: hipLaunchKernelGGL((KER<0>), __VA_ARGS__); break;                    \
  }

static int aa_fwd(const float* color, const float* rast, const float* pos, const int32_t* tri,
                  const int32_t* topo, int N, int H, int W, int C, int V, int T, float* out,
                  uint8_t* saved, hipStream_t stream) {
  (void)hipGetLastError();
  int st = check_aa(color, rast, pos, tri, topo, N, H, W, C, V, T);
  if (st) return st;
  DR_CHECK_ARG(out != nullptr, "antialias: null output");
  DR_CHECK_ARG(((uintptr_t)saved & 15) == 0, "antialias_fwd_save: saved must be 16-byte aligned");
  uint8_t* mask = saved;
  int* saved_ids = saved ? (int*)(saved + aa_mask_bytes(N, H, W)) : nullptr;
  AARec* rec = nullptr;
  AARec* saved_rec = saved ? (AARec*)(saved + 5 * aa_mask_bytes(N, H, W)) : nullptr;
  AAPersp* saved_persp = saved ? (AAPersp*)(saved_rec + (int64_t)N * T) : nullptr;
  int st2 = aa_records(pos, tri, topo, N, V, T, H, W, stream, saved_rec, saved_persp, &rec);
  if (st2) return st2;
  const int ntx = (W + 15) / 16, nty = (H + 15) / 16;
  const int64_t total = (int64_t)N * ntx * nty;
  DR_CHECK_ARG(total <= INT32_MAX - 4096, "antialias: too many tiles");
  const int ct = aa_ct(C, color, out, color);
  const dim3 grid((unsigned)total), block(256);
  DR_TIMED("k_aa_fwd", stream);
  DR_AA_DISPATCH(k_aa_fwd, ct, grid, block, 0, stream, rast, rec, color, H, W, T, C, ntx, nty,
                 out, mask, saved_ids);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

static int aa_bwd(const float* color, const float* rast, const float* pos, const int32_t* tri,
                  const int32_t* topo, const float* d_out, const uint8_t* saved, int N, int H,
                  int W, int C, int V, int T, float* d_color, float* d_pos, unsigned flags,
                  hipStream_t stream) {
  (void)hipGetLastError();
  int st = check_aa(color, rast, pos, tri, topo, N, H, W, C, V, T);
  if (st) return st;
  DR_CHECK_ARG(d_out != nullptr, "antialias_bwd: null d_out");
  DR_CHECK_ARG(((uintptr_t)saved & 15) == 0, "antialias_bwd_saved: saved must be 16-byte aligned");
  if (!d_color && !d_pos) return DR_OK;
  const bool acc = (flags & DR_ACCUMULATE) != 0;
  // d_pos is summed in fp64 across workgroups and rounded once, so it does
  // not depend on the order in which their additions land
  double* dpos64 = nullptr;
  if (d_pos) {
    dpos64 = acc64_begin(stream, (int64_t)N * V * 4);
    if (!dpos64) return scratch_fail();
  }
  const AARec* rec = nullptr;
  const AAPersp* persp = nullptr;
  if (saved) {  // the forward's records
    rec = (const AARec*)(saved + 5 * aa_mask_bytes(N, H, W));
    persp = (const AAPersp*)(rec + (int64_t)N * T);
  } else {
    AARec* r = nullptr;
    int st2 = aa_records(pos, tri, topo, N, V, T, H, W, stream, nullptr, nullptr, &r);
    if (st2) return st2;
    rec = r;
  }
  const int ntx = (W + 15) / 16, nty = (H + 15) / 16;
  const int64_t total = (int64_t)N * ntx * nty;
  DR_CHECK_ARG(total <= INT32_MAX - 4096, "antialias: too many tiles");
  const dim3 grid((unsigned)total), block(256);
  const int ct = aa_ct(C, color, d_out, d_color);
  {
    DR_TIMED("k_aa_bwd", stream);
    if (saved) {
      DR_AA_DISPATCH(k_aa_bwd_masked, ct, grid, block, 0, stream,
                     (const int*)(saved + aa_mask_bytes(N, H, W)), rec, persp, color, d_out, saved,
                     H, W, V, T, C, ntx, nty, d_color, dpos64, acc ? 1 : 0);
    } else {
      DR_AA_DISPATCH(k_aa_bwd, ct, grid, block, 0, stream, rast, rec, pos, color, d_out, H, W,
                     V, T, C, ntx, nty, d_color, dpos64, acc ? 1 : 0);
    }
  }
  DR_CHECK_LAUNCH();
  if (d_pos) return acc64_end(dpos64, d_pos, (int64_t)N * V * 4, acc, stream);
  return DR_OK;
}

extern "C" int dr_antialias_fwd(const float* color, const float* rast, const float* pos,
                                const int32_t* tri, const int32_t* topo, int N, int H, int W,
                                int C, int V, int T, float* out, dr_stream_t stream) {
  return aa_fwd(color, rast, pos, tri, topo, N, H, W, C, V, T, out, nullptr,
                (hipStream_t)stream);
}

extern "C" int dr_antialias_bwd(const float* color, const float* rast, const float* pos,
                                const int32_t* tri, const int32_t* topo, const float* d_out,
                                int N, int H, int W, int C, int V, int T, float* d_color,
                                float* d_pos, unsigned flags, dr_stream_t stream) {
  return aa_bwd(color, rast, pos, tri, topo, d_out, nullptr, N, H, W, C, V, T, d_color, d_pos,
                flags, (hipStream_t)stream);
}

extern "C" int64_t dr_antialias_saved_bytes(int N, int H, int W, int T) {
  if (N < 1 || H < 1 || W < 1 || T < 0) return -1;
  return 5 * aa_mask_bytes(N, H, W) + (int64_t)N * T * (int64_t)(sizeof(AARec) + sizeof(AAPersp));
}

extern "C" int dr_antialias_fwd_save(const float* color, const float* rast, const float* pos,
                                     const int32_t* tri, const int32_t* topo, int N, int H,
                                     int W, int C, int V, int T, float* out, void* saved,
                                     dr_stream_t stream) {
  DR_CHECK_ARG(saved != nullptr, "antialias_fwd_save: null saved");
  return aa_fwd(color, rast, pos, tri, topo, N, H, W, C, V, T, out, (uint8_t*)saved,
                (hipStream_t)stream);
}

extern "C" int dr_antialias_bwd_saved(const float* color, const float* rast, const float* pos,
                                      const int32_t* tri, const int32_t* topo,
                                      const float* d_out, const void* saved, int N, int H,
                                      int W, int C, int V, int T, float* d_color, float* d_pos,
                                      unsigned flags, dr_stream_t stream) {
  DR_CHECK_ARG(saved != nullptr, "antialias_bwd_saved: null saved");
  return aa_bwd(color, rast, pos, tri, topo, d_out, (const uint8_t*)saved, N, H, W, C, V, T,
                d_color, d_pos, flags, (hipStream_t)stream);
}
