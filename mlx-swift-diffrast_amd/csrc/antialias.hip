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
// silhouette (Antialias.swift:168-326), one direction at a time
// ---------------------------------------------------------------------------

struct SilDir {
  bool active;
  float alpha;  // beta > 0 when active
  int ie0, ie1;
  float e0x, e0y, e1x, e1y, t, denom, dbeta;
};

struct AAIn {
  const float* rast;
  const float* pos;
  const int32_t* tri;
  const int32_t* topo;
  const float2* scr;  // [N, V] pixel-space vertex positions
  int H, W, V;
};

// Pixel-space position of every vertex, with the expressions of
// Antialias.swift:247-250: x = (x/w + 1) * W/2, y = (1 - y/w) * H/2.
__global__ void __launch_bounds__(256) k_aa_screen(const float* __restrict__ pos, int64_t NV,
                                                   int H, int W, float2* __restrict__ scr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= NV) return;
  const float4 P = *reinterpret_cast<const float4*>(pos + i * 4);
  scr[i] = make_float2((P.x / P.w + 1.0f) * (float)W * 0.5f,
                       (1.0f - P.y / P.w) * (float)H * 0.5f);
}

__device__ __forceinline__ int tri_at(const AAIn& a, int n, int h, int w) {
  return f2i(a.rast[((((int64_t)n * a.H + h) * a.W + w) << 2) + 3]) - 1;
}

// Direction dir of pixel (n, ph, pw) whose own triangle is tri_p;
// s.active is false when the pair contributes nothing.
__device__ __forceinline__ bool sil_dir_impl(const AAIn& a, int n, int ph, int pw, int tri_p,
                                             int dir, SilDir& s) {
  const int dw = dir == 0 ? 1 : (dir == 2 ? -1 : 0);
  const int dh = dir == 1 ? 1 : (dir == 3 ? -1 : 0);
  const int nh = ph + dh, nw = pw + dw;
  if (nh < 0 || nh >= a.H || nw < 0 || nw >= a.W) return false;
  const int tri_n = tri_at(a, n, nh, nw);
  if (tri_p == tri_n) return false;
  if (tri_p < 0 && tri_n < 0) return false;
  int fg, target;
  if (tri_p >= 0 && tri_n >= 0) {
    const int32_t* tp = a.topo + (int64_t)tri_p * 3;
    if (!(tp[0] == tri_n || tp[1] == tri_n || tp[2] == tri_n)) return false;
    fg = tri_p;
    target = tri_n;
  } else if (tri_p >= 0) {
    fg = tri_p;
    target = -1;
  } else {
    fg = tri_n;
    target = -1;
  }
  const float2* sp = a.scr + (int64_t)n * a.V;
  const float pcx = (float)pw + 0.5f, pcy = (float)ph + 0.5f;
  const float ncx = (float)nw + 0.5f, ncy = (float)nh + 0.5f;
  int ie0 = -1, ie1 = -1;
  float e0x = 0.f, e0y = 0.f, e1x = 0.f, e1y = 0.f;
  bool found = false;
  for (int kk = 0; kk < 3; ++kk) {  // :240-262
    if (a.topo[(int64_t)fg * 3 + kk] != target) continue;
    const int c0 = a.tri[(int64_t)fg * 3 + ((kk + 1) % 3)];
    const int c1 = a.tri[(int64_t)fg * 3 + ((kk + 2) % 3)];
    const float2 Q0 = sp[c0], Q1 = sp[c1];
    const float E0x = Q0.x, E0y = Q0.y, E1x = Q1.x, E1y = Q1.y;
    const float ex = E1x - E0x, ey = E1y - E0y;
    const float side_p = ex * (pcy - E0y) - ey * (pcx - E0x);
    const float side_n = ex * (ncy - E0y) - ey * (ncx - E0x);
    if (side_p * side_n < 0.0f) {
      ie0 = c0; ie1 = c1;
      e0x = E0x; e0y = E0y; e1x = E1x; e1y = E1y;
      found = true;
      break;
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

__device__ __forceinline__ SilDir sil_dir(const AAIn& a, int n, int ph, int pw, int tri_p,
                                          int dir) {
  SilDir s;
  s.alpha = 0.0f;
  s.ie0 = s.ie1 = 0;
  s.e0x = s.e0y = s.e1x = s.e1y = s.t = s.denom = s.dbeta = 0.0f;
  s.active = sil_dir_impl(a, n, ph, pw, tri_p, dir, s);
  return s;
}

// Antialias.swift:333-358.
__global__ void __launch_bounds__(256) k_aa_fwd(AAIn a, const float* __restrict__ color, int N,
                                                int C, float* __restrict__ out) {
  const int64_t pix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t P = (int64_t)N * a.H * a.W;
  if (pix >= P) return;
  const int pw = (int)(pix % a.W);
  const int ph = (int)((pix / a.W) % a.H);
  const int n = (int)(pix / ((int64_t)a.H * a.W));
  const int tri_p = tri_at(a, n, ph, pw);
  float alpha[4];
  int64_t nb[4];
  int any = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const SilDir s = sil_dir(a, n, ph, pw, tri_p, d);
    alpha[d] = s.active ? s.alpha : 0.0f;
    const int nh = ph + (d == 1 ? 1 : (d == 3 ? -1 : 0));
    const int nw = pw + (d == 0 ? 1 : (d == 2 ? -1 : 0));
    nb[d] = (((int64_t)n * a.H + nh) * a.W + nw) * C;
    any |= s.active;
  }
  const float* cp = color + pix * C;
  float* o = out + pix * C;
  if (!any) {
    for (int c = 0; c < C; ++c) o[c] = cp[c];
    return;
  }
  for (int c = 0; c < C; ++c) {
    const float cpc = cp[c];
    float acc = cpc;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      if (alpha[d] > 0.0f) acc += alpha[d] * (color[nb[d] + c] - cpc);
    o[c] = acc;
  }
}

// Fused backward on 16x16 tiles (one 8x8 quadrant per wave).
__global__ void __launch_bounds__(256) k_aa_bwd(AAIn a, const float* __restrict__ color,
                                                const float* __restrict__ d_out, int N, int C,
                                                int ntx, int nty, float* __restrict__ d_color,
                                                float* __restrict__ d_pos, int accumulate) {
  __shared__ float s_alpha[4][16][17];
  __shared__ float s_halo[4][16];
  __shared__ LdsTable<4, 128> tab;  // d_pos rows touched by this tile
  lds_table_clear(tab);
  const int tiles = ntx * nty;
  const int b = (int)blockIdx.x;
  const int n = b / tiles;
  const int tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int x0 = tx * 16, y0 = ty * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lx = (wave & 1) * 8 + (lane & 7), ly = (wave >> 1) * 8 + (lane >> 3);
  const int pw = x0 + lx, ph = y0 + ly;
  const bool inside = pw < a.W && ph < a.H;
  const int tri_p = inside ? tri_at(a, n, ph, pw) : -1;

  // 1) own blend weights.
  SilDir sd[4];
  float asum = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    sd[d] = sil_dir(a, n, ph, pw, tri_p, d);
    sd[d].active = sd[d].active && inside;
    const float al = sd[d].active ? sd[d].alpha : 0.0f;
    s_alpha[d][ly][lx] = al;
    asum += al;
  }
  // 2) halo: the one direction of each outside neighbour that points into
  //    the tile.
  if (threadIdx.x < 64) {
    const int side = threadIdx.x >> 4, i = threadIdx.x & 15;
    int qh, qw, qd;
    if (side == 0) { qw = x0 - 1;  qh = y0 + i; qd = 0; }       // left column, looks +w
    else if (side == 1) { qw = x0 + 16; qh = y0 + i; qd = 2; }  // right column, looks -w
    else if (side == 2) { qw = x0 + i; qh = y0 - 1;  qd = 1; }  // top row, looks +h
    else { qw = x0 + i; qh = y0 + 16; qd = 3; }                 // bottom row, looks -h
    float al = 0.0f;
    if (qh >= 0 && qh < a.H && qw >= 0 && qw < a.W) {
      const SilDir s = sil_dir(a, n, qh, qw, tri_at(a, n, qh, qw), qd);
      if (s.active) al = s.alpha;
    }
    s_halo[side][i] = al;
  }
  __syncthreads();

  const int64_t pix = ((int64_t)n * a.H + min(ph, a.H - 1)) * a.W + min(pw, a.W - 1);
  const float* g = d_out + pix * C;
  // 3) d_color: own term + what each neighbour's blend sends here.
  if (d_color && inside) {
    float wn[4];
    int64_t qn[4];
    wn[0] = lx < 15 ? s_alpha[2][ly][lx + 1] : s_halo[1][ly];  // right neighbour, its dir 2
    wn[1] = ly < 15 ? s_alpha[3][ly + 1][lx] : s_halo[3][lx];  // lower neighbour, its dir 3
    wn[2] = lx > 0 ? s_alpha[0][ly][lx - 1] : s_halo[0][ly];   // left neighbour, its dir 0
    wn[3] = ly > 0 ? s_alpha[1][ly - 1][lx] : s_halo[2][lx];   // upper neighbour, its dir 1
    qn[0] = pix + 1;
    qn[1] = pix + a.W;
    qn[2] = pix - 1;
    qn[3] = pix - a.W;
    float* dc = d_color + pix * C;
    for (int c = 0; c < C; ++c) {
      float acc = g[c] * (1.0f - asum);
#pragma unroll
      for (int d = 0; d < 4; ++d)
        if (wn[d] > 0.0f) acc += d_out[qn[d] * C + c] * wn[d];
      dc[c] = accumulate ? dc[c] + acc : acc;
    }
  }
  // 4) d_pos (Antialias.swift:405-495), summed per vertex in LDS.
  if (!d_pos) return;  // uniform: no barrier follows
  const float halfW = (float)a.W * 0.5f, halfH = (float)a.H * 0.5f;
  const float* p = a.pos + (int64_t)n * a.V * 4;
  float* dp = d_pos + (int64_t)n * a.V * 4;
  const float* cpp = color + pix * C;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    bool on = sd[d].active && sd[d].alpha > 0.0f && sd[d].alpha < 1.0f;
    if (on) {
      const int nh = ph + (d == 1 ? 1 : (d == 3 ? -1 : 0));
      const int nw = pw + (d == 0 ? 1 : (d == 2 ? -1 : 0));
      const float* cnp = color + (((int64_t)n * a.H + nh) * a.W + nw) * C;
      float d_alpha = 0.0f;
      for (int c = 0; c < C; ++c) d_alpha += g[c] * (cnp[c] - cpp[c]);
      on = d_alpha != 0.0f;
      if (on) {
        const SilDir& s = sd[d];
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
          const float4 P = *reinterpret_cast<const float4*>(p + (int64_t)iv[e] * 4);
          const float inv_w = 1.0f / P.w;
          const float nd_x = P.x * inv_w, nd_y = P.y * inv_w;
          const float dv[4] = {
              d_alpha * dex[e] * halfW * inv_w, d_alpha * dey[e] * (-halfH) * inv_w, 0.0f,
              d_alpha * (dex[e] * (-halfW * nd_x) + dey[e] * (halfH * nd_y)) * inv_w};
          lds_table_add(tab, dp + (int64_t)iv[e] * 4, dv);
        }
      }
    }
  }
  __syncthreads();
  lds_table_flush(tab);
}

}  // namespace dr

using namespace dr;

extern "C" int dr_antialias_topology(const int32_t* tri, int T, int32_t* topo,
                                     dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  DR_CHECK_ARG(tri && topo && T >= 0, "antialias_topology: bad arguments");
  if (T == 0) return DR_OK;
  const int64_t E = (int64_t)T * 3;
  uint64_t S = 64;
  while (S < (uint64_t)E * 2) S <<= 1;
  Scratch* sc = scratch_for(stream);
  if (!sc) return DR_ERR_HIP;
  char* buf = (char*)scratch_get(sc, stream, SLOT_TOPO, (size_t)S * 16);
  if (!buf) return DR_ERR_MEMORY;
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

static int aa_screen(const float* pos, int N, int V, int H, int W, hipStream_t stream,
                     float2** out) {
  Scratch* sc = scratch_for(stream);
  if (!sc) return DR_ERR_HIP;
  const int64_t nv = (int64_t)N * V;
  float2* scr = (float2*)scratch_get(sc, stream, SLOT_AA_SCREEN, (size_t)(nv > 0 ? nv : 1) * 8);
  if (!scr) return DR_ERR_MEMORY;
  if (nv > 0) {
    DR_TIMED("k_aa_screen", stream);
    hipLaunchKernelGGL(k_aa_screen, dim3(grid_for(nv, 256)), dim3(256), 0, stream, pos, nv, H, W,
                       scr);
  }
  DR_CHECK_LAUNCH();
  *out = scr;
  return DR_OK;
}

static int check_aa(const float* color, const float* rast, const float* pos, const int32_t* tri,
                    const int32_t* topo, int N, int H, int W, int C, int V, int T) {
  DR_CHECK_ARG(color && rast && pos && tri && topo, "antialias: null tensor");
  DR_CHECK_ARG(N >= 1 && H >= 1 && W >= 1 && C >= 1 && V >= 0 && T >= 0, "antialias: bad sizes");
  return DR_OK;
}

extern "C" int dr_antialias_fwd(const float* color, const float* rast, const float* pos,
                                const int32_t* tri, const int32_t* topo, int N, int H, int W,
                                int C, int V, int T, float* out, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  int st = check_aa(color, rast, pos, tri, topo, N, H, W, C, V, T);
  if (st) return st;
  DR_CHECK_ARG(out != nullptr, "antialias: null output");
  float2* scr = nullptr;
  int st2 = aa_screen(pos, N, V, H, W, stream, &scr);
  if (st2) return st2;
  AAIn a{rast, pos, tri, topo, scr, H, W, V};
  const int64_t P = (int64_t)N * H * W;
  DR_TIMED("k_aa_fwd", stream);
  hipLaunchKernelGGL(k_aa_fwd, dim3(grid_for(P, 256)), dim3(256), 0, stream, a, color, N, C, out);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

extern "C" int dr_antialias_bwd(const float* color, const float* rast, const float* pos,
                                const int32_t* tri, const int32_t* topo, const float* d_out,
                                int N, int H, int W, int C, int V, int T, float* d_color,
                                float* d_pos, unsigned flags, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  int st = check_aa(color, rast, pos, tri, topo, N, H, W, C, V, T);
  if (st) return st;
  DR_CHECK_ARG(d_out != nullptr, "antialias_bwd: null d_out");
  if (!d_color && !d_pos) return DR_OK;
  const bool acc = (flags & DR_ACCUMULATE) != 0;
  if (d_pos && !acc) DR_CHECK_HIP(fill_async(d_pos, 0.0f, (int64_t)N * V * 4, stream));
  float2* scr = nullptr;
  int st2 = aa_screen(pos, N, V, H, W, stream, &scr);
  if (st2) return st2;
  AAIn a{rast, pos, tri, topo, scr, H, W, V};
  const int ntx = (W + 15) / 16, nty = (H + 15) / 16;
  DR_TIMED("k_aa_bwd", stream);
  hipLaunchKernelGGL(k_aa_bwd, dim3((unsigned)((int64_t)N * ntx * nty)), dim3(256), 0, stream, a,
                     color, d_out, N, C, ntx, nty, d_color, d_pos, acc ? 1 : 0);
  DR_CHECK_LAUNCH();
  return DR_OK;
}
