// interpolate: barycentric gather of per-vertex attributes (+ screen-space
// derivatives), and the fused backward (d_attr scatter, d_rast, d_rast_db in
// one pass over the pixels instead of three).
//
// Semantics follow Sources/MLXDiffRast/Interpolate.swift of the reference:
//   forward    :137-170 (basic), :175-228 (DA)
//   backward   :231-264 / :269-324 (d_attr), :327-367 (d_rast),
//              :370-417 (d_rast_db)
// u weights vertex 1, v weights vertex 2, bw = 1 - u - v weights vertex 0
// (CONVENTIONS.md of the reference).
#include "common.h"

namespace dr {
// Tile order.  Workgroups are dealt round-robin to the 8 XCDs, each with
// its own 4 MiB L2.  A vertex table (one image's V x A attributes) that
// fits one L2 is cached whole by every XCD, and round-robin tiles then
// stream best (8 x 1024^2, 41K x 2 floats: interpolate forward 0.081 ms
// against 0.089 with contiguous runs, backward 0.114 against 0.123).  A
// larger one is shared only by neighbouring tiles, so each XCD takes a
// contiguous run of tiles (xcd_remap) and keeps the vertex rows and the
// d_attr atomics its tiles share: 16 x 2048^2 with 655K x 6 floats,
// backward 3.51 -> 3.37 ms per step of four layers; 4096 x 256^2 with
// 6.3M x 3, backward 5.50 -> 4.79 ms.
constexpr int64_t kXcdL2Bytes = 4 << 20;

// Compile-time attribute / derivative counts for the common shapes; 0 means
// "given at run time".
template <int AT>
__device__ __forceinline__ int dimA(int A) { return AT > 0 ? AT : A; }

// Stores n consecutive floats; two or four at a time when the count and the
// (16-byte aligned) buffers allow.
template <int NC>
__device__ __forceinline__ void st_run(float* __restrict__ p, const float* v, int n) {
  if constexpr (NC == 2) {
    st_nt2(p, make_float2(v[0], v[1]));
  } else if constexpr (NC == 4) {
    st_nt4(p, make_float4(v[0], v[1], v[2], v[3]));
  } else {
    for (int i = 0; i < n; ++i) p[i] = v[i];
  }
}

// Pixels per thread of the forward: two, each round of their loads issued
// together (16 x 2048^2 at ~2.5 pixels per triangle, six attributes: 2.46
// -> 2.39 ms per step of four layers against four pixels a thread; 4096 x
// 256^2, three attributes and their derivatives: 3.54 -> 3.43 ms).
template <int AT>
constexpr int interp_pix() {
  return 2;
}

// Width of the forward's pixel strips: a wave takes a 16x4 strip when a
// 16-pixel row of its outputs fills whole 128-byte lines (an even attribute
// count), since the strip's triangles share more vertex rows than a 64-pixel
// row's and its attribute gathers touch fewer cache lines (16 x 2048^2 at
// ~2.5 pixels per triangle, six attributes: 3.09 -> 2.78 ms per step of four
// layers); otherwise a 64-pixel row, whose output rows stay whole lines
// (three attributes and their derivatives on 16-pixel rows: 3.6 -> 4.6 ms at
// 4096 x 256^2).
template <int AT>
constexpr int interp_strip() {
  return (AT == 2 || AT == 4 || AT == 6) ? 16 : 64;
}

// A workgroup covers SW x (256 / SW * PX) pixels of one image: each wave a
// strip SW wide and 64 / SW rows tall per pixel slot.
template <int AT, int KT>
__global__ void __launch_bounds__(256) k_interp_fwd(
    const float* __restrict__ attr, int64_t attr_stride, const float* __restrict__ rast,
    const float* __restrict__ rast_db, const int32_t* __restrict__ tri,
    const int32_t* __restrict__ diff_idx, int K_, int H, int W, int ntx, int nty, int V, int T,
    int A_, float* __restrict__ out, float* __restrict__ out_da, int xcd) {
  constexpr int PX = interp_pix<AT>();
  constexpr int NA = AT > 0 ? AT : 8;       // register slots for attributes
  constexpr int NK = KT > 0 ? 2 * KT : 8;   // and for derivative outputs
  const int A = dimA<AT>(A_);
  const int K = KT > 0 ? KT : K_;
  const int tiles = ntx * nty;
  const int b = xcd ? xcd_remap((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int img = b / tiles;
  const int tile = b - img * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  constexpr int SW = interp_strip<AT>(), SH = 256 / SW;  // a slot's tile: SW x SH
  const int pw = tx * SW + ((int)threadIdx.x & (SW - 1));
  const int ph0 = ty * SH * PX + (int)threadIdx.x / SW;
  const float* at = attr + (int64_t)img * attr_stride;
  float4 r[PX];
  int t[PX];
  int64_t pixq[PX];
  bool in[PX];
  // Every slot's loads of one round (rast, triangle ids, vertex rows) are
  // issued before any of them is used: a select, check or store between the
  // slots' loads makes the wave wait for each slot's round trip in turn.  So
  // the loads are not predicated per lane: a lane outside the image reads
  // its clamped pixel, and in a wave where some lane has a triangle, lanes
  // without one read triangle 0 and vertex row 0 (the values are dropped).
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    const int ph = ph0 + q * SH;
    in[q] = pw < W && ph < H;
    pixq[q] = ((int64_t)img * H + min(ph, H - 1)) * W + min(pw, W - 1);
  }
  // (addresses first: a register of a pending load that the code does not
  // read, such as rast's depth, is not reused for them, which would wait)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < PX; ++q) r[q] = ld_nt4(rast + pixq[q] * 4);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    t[q] = in[q] ? f2i(r[q].w) - 1 : -1;
    if (t[q] >= T) t[q] = -1;  // not a triangle of this mesh: empty
  }
  bool any = false;
#pragma unroll
  for (int q = 0; q < PX; ++q) any = any || t[q] >= 0;
  const bool wave_any = __ballot(any) != 0ull;  // uniform: then T > 0
  int iv[PX][3];
#pragma unroll
  for (int q = 0; q < PX; ++q) iv[q][0] = iv[q][1] = iv[q][2] = 0;
  if (wave_any) {
#pragma unroll
    for (int q = 0; q < PX; ++q) {
      const int tt = t[q] >= 0 ? t[q] : 0;
      iv[q][0] = tri[tt * 3 + 0];
      iv[q][1] = tri[tt * 3 + 1];
      iv[q][2] = tri[tt * 3 + 2];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    if (!(t[q] >= 0 && verts_ok(iv[q][0], iv[q][1], iv[q][2], V))) {
      t[q] = -1;
      iv[q][0] = iv[q][1] = iv[q][2] = 0;
    }
  }
  if (AT == 0 || KT == 0 && K > 0) {  // any shape: element by element
#pragma unroll
    for (int q = 0; q < PX; ++q) {
      const int64_t pix = pixq[q];
      if (!in[q]) continue;
      float* o = out + pix * A;
      float* od = K > 0 ? out_da + pix * 2 * K : nullptr;
      if (t[q] < 0) {
        for (int a = 0; a < A; ++a) o[a] = 0.0f;
        for (int k = 0; k < 2 * K; ++k) od[k] = 0.0f;
        continue;
      }
      const float* a0p = at + (int64_t)iv[q][0] * A;
      const float* a1p = at + (int64_t)iv[q][1] * A;
      const float* a2p = at + (int64_t)iv[q][2] * A;
      const float u = r[q].x, v = r[q].y;
      const float bw = 1.0f - u - v;
      for (int a = 0; a < A; ++a) o[a] = bw * a0p[a] + u * a1p[a] + v * a2p[a];
      if (K > 0) {
        const float4 db = *reinterpret_cast<const float4*>(rast_db + pix * 4);
        for (int k = 0; k < K; ++k) {
          const int a = diff_idx ? diff_idx[k] : k;
          if ((unsigned)a >= (unsigned)A) {  // not an attribute: zero derivatives
            od[2 * k + 0] = od[2 * k + 1] = 0.0f;
            continue;
          }
          const float d01 = a1p[a] - a0p[a];
          const float d02 = a2p[a] - a0p[a];
          od[2 * k + 0] = d01 * db.x + d02 * db.z;
          od[2 * k + 1] = d01 * db.y + d02 * db.w;
        }
      }
    }
    return;
  }
  // compile-time shape (identity diff_idx when KT > 0)
  bool rows = false;
#pragma unroll
  for (int q = 0; q < PX; ++q) rows = rows || t[q] >= 0;
  const bool wave_rows = __ballot(rows) != 0ull;  // uniform: then V > 0
  float a0[PX][NA], a1[PX][NA], a2[PX][NA];
  float4 db[PX];
#pragma unroll
  for (int q = 0; q < PX; ++q) {
#pragma unroll
    for (int a = 0; a < NA; ++a) a0[q][a] = a1[q][a] = a2[q][a] = 0.0f;
    db[q] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (wave_rows) {
#pragma unroll
    for (int q = 0; q < PX; ++q) {
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        a0[q][a] = at[(int64_t)iv[q][0] * NA + a];
        a1[q][a] = at[(int64_t)iv[q][1] * NA + a];
        a2[q][a] = at[(int64_t)iv[q][2] * NA + a];
      }
      if (KT > 0) db[q] = *reinterpret_cast<const float4*>(rast_db + pixq[q] * 4);
    }
  }
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    if (!in[q]) continue;
    const int64_t pix = pixq[q];
    float ov[NA], odv[NK];
#pragma unroll
    for (int a = 0; a < NA; ++a) ov[a] = 0.0f;
#pragma unroll
    for (int k = 0; k < NK; ++k) odv[k] = 0.0f;
    if (t[q] >= 0) {
      const float u = r[q].x, v = r[q].y;
      const float bw = 1.0f - u - v;
#pragma unroll
      for (int a = 0; a < NA; ++a) ov[a] = bw * a0[q][a] + u * a1[q][a] + v * a2[q][a];
#pragma unroll
      for (int k = 0; k < (KT > 0 ? KT : 0); ++k) {
        const float d01 = a1[q][k] - a0[q][k];
        const float d02 = a2[q][k] - a0[q][k];
        odv[2 * k + 0] = d01 * db[q].x + d02 * db[q].z;
        odv[2 * k + 1] = d01 * db[q].y + d02 * db[q].w;
      }
    }
    st_run<NA>(out + pix * NA, ov, NA);
    if (KT > 0) st_run<NK>(out_da + pix * NK, odv, NK);
  }
}

// Fused backward.  Pixels are walked in 16x16 tiles, a 16x4 strip per wave;
// runs of one triangle along a pixel row are summed before their d_attr
// terms meet the LDS table.
template <int AT, int KT>
__global__ void __launch_bounds__(256) k_interp_bwd(
    const float* __restrict__ attr, int64_t attr_stride, const float* __restrict__ rast,
    const float* __restrict__ rast_db, const int32_t* __restrict__ tri,
    const int32_t* __restrict__ diff_idx, int K_, const float* __restrict__ d_out,
    const float* __restrict__ d_out_da, int N, int H, int W, int ntx, int nty, int V, int T,
    int A_, float* __restrict__ d_attr, int64_t d_attr_stride, int ncopy, int64_t copy_stride,
    float* __restrict__ d_rast, float* __restrict__ d_rast_db, int xcd) {
  __shared__ LdsTableU<(AT > 0 ? AT : 1), 256> tab;  // d_attr rows (or elements) touched by this tile
  __shared__ int s_any[4];  // per wave: a covered pixel
  const int tiles = ntx * nty;
  const int b = xcd ? xcd_remap((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int n = b / tiles;
  const int tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // 16x4 strip per wave: each 16-lane row holds one pixel row
  const int pw = tx * 16 + (lane & 15), ph = ty * 16 + wave * 4 + (lane >> 4);
  const bool inside = pw < W && ph < H;
  const int64_t pix = ((int64_t)n * H + min(ph, H - 1)) * W + min(pw, W - 1);

  const float4 r = *reinterpret_cast<const float4*>(rast + pix * 4);
  const int t = f2i(r.w) - 1;
  bool valid = inside && t >= 0 && t < T;
  {
    const uint64_t any = __ballot(valid);
    if (lane == 0) s_any[wave] = any != 0ull;
  }
  __syncthreads();
  if (!(s_any[0] | s_any[1] | s_any[2] | s_any[3])) {  // uniform: an empty tile
    if (inside) {
      *reinterpret_cast<float4*>(d_rast + pix * 4) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (K_ > 0 && d_rast_db)
        *reinterpret_cast<float4*>(d_rast_db + pix * 4) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  lds_table_clear(tab);
  __syncthreads();
  const float u = r.x, v = r.y;
  const float bw = 1.0f - u - v;
  const float* at = attr + (int64_t)n * attr_stride;
  // ncopy > 0: d_attr is copy (workgroup mod ncopy) of ncopy copies
  float* da = d_attr + (ncopy ? (int64_t)(b % ncopy) * copy_stride : 0) + (int64_t)n * d_attr_stride;
  int i0 = 0, i1 = 0, i2 = 0;

  if constexpr (AT > 0) {
    // Compile-time shape (identity diff_idx when KT > 0): every input of the
    // pixel is loaded once, the cotangents and rast_db together with the
    // triangle's vertex ids, then the three attribute rows.
    constexpr int NK = KT > 0 ? KT : 1;
    float gv[AT], gdv[2 * NK], a0[AT], a1[AT], a2[AT];
    float4 db = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int a = 0; a < AT; ++a) gv[a] = a0[a] = a1[a] = a2[a] = 0.0f;
#pragma unroll
    for (int k = 0; k < 2 * NK; ++k) gdv[k] = 0.0f;
    if (valid) {
      i0 = tri[t * 3 + 0];
      i1 = tri[t * 3 + 1];
      i2 = tri[t * 3 + 2];
#pragma unroll
      for (int a = 0; a < AT; ++a) gv[a] = d_out[pix * AT + a];
      if constexpr (KT > 0) {
#pragma unroll
        for (int k = 0; k < 2 * KT; ++k) gdv[k] = d_out_da[pix * 2 * KT + k];
        db = *reinterpret_cast<const float4*>(rast_db + pix * 4);
      }
      valid = verts_ok(i0, i1, i2, V);  // pixels of foreign ids are empty
    }
    if (valid) {
#pragma unroll
      for (int a = 0; a < AT; ++a) {
        a0[a] = at[(int64_t)i0 * AT + a];
        a1[a] = at[(int64_t)i1 * AT + a];
        a2[a] = at[(int64_t)i2 * AT + a];
      }
    }
    // d_rast (Interpolate.swift:327-367) and d_rast_db (:370-417).
    float du = 0.0f, dv = 0.0f;
    float d_udx = 0.0f, d_udy = 0.0f, d_vdx = 0.0f, d_vdy = 0.0f;
    if (valid) {
#pragma unroll
      for (int a = 0; a < AT; ++a) {
        du += (a1[a] - a0[a]) * gv[a];
        dv += (a2[a] - a0[a]) * gv[a];
      }
#pragma unroll
      for (int k = 0; k < (KT > 0 ? KT : 0); ++k) {
        const float d01 = a1[k] - a0[k], d02 = a2[k] - a0[k];
        const float gx = gdv[2 * k + 0], gy = gdv[2 * k + 1];
        d_udx += d01 * gx;
        d_udy += d01 * gy;
        d_vdx += d02 * gx;
        d_vdy += d02 * gy;
      }
    }
    if (inside) {
      *reinterpret_cast<float4*>(d_rast + pix * 4) = make_float4(du, dv, 0.0f, 0.0f);
      if (KT > 0 && d_rast_db)
        *reinterpret_cast<float4*>(d_rast_db + pix * 4) = make_float4(d_udx, d_udy, d_vdx, d_vdy);
    }
    // d_attr (Interpolate.swift:231-264, :269-324), summed per vertex row in
    // LDS before the global atomics.
    float rv[3 * AT];  // rows of i0, i1, i2
#pragma unroll
    for (int q = 0; q < 3 * AT; ++q) rv[q] = 0.0f;
    if (valid) {
#pragma unroll
      for (int a = 0; a < AT; ++a) {
        rv[a] = bw * gv[a];
        rv[AT + a] = u * gv[a];
        rv[2 * AT + a] = v * gv[a];
      }
#pragma unroll
      for (int k = 0; k < (KT > 0 ? KT : 0); ++k) {
        const float gx = gdv[2 * k + 0], gy = gdv[2 * k + 1];
        const float u_term = gx * db.x + gy * db.y;
        const float v_term = gx * db.z + gy * db.w;
        rv[k] += -u_term - v_term;
        rv[AT + k] += u_term;
        rv[2 * AT + k] += v_term;
      }
    }
    // Runs of same-triangle lanes along a pixel row add into the same rows:
    // sum each run first, its last lane adds the total.
    const bool tail = row_run_sum(valid ? (uint64_t)t : (1ull << 63) | (uint64_t)lane, rv);
    if (valid && tail) {
      lds_table_add(tab, da + (int64_t)i0 * AT, &rv[0]);
      lds_table_add(tab, da + (int64_t)i1 * AT, &rv[AT]);
      lds_table_add(tab, da + (int64_t)i2 * AT, &rv[2 * AT]);
    }
  } else {
    // Any shape: element by element.
    const int A = A_;
    const int K = K_;
    if (valid) {
      i0 = tri[t * 3 + 0];
      i1 = tri[t * 3 + 1];
      i2 = tri[t * 3 + 2];
      valid = verts_ok(i0, i1, i2, V);  // pixels of foreign ids are empty
    }
    const float* g = d_out + pix * A;
    float4 db = make_float4(0.f, 0.f, 0.f, 0.f);
    if (K > 0 && valid) db = *reinterpret_cast<const float4*>(rast_db + pix * 4);
    float du = 0.0f, dv = 0.0f;
    if (valid) {
      for (int a = 0; a < A; ++a) {
        const float a0 = at[(int64_t)i0 * A + a], a1 = at[(int64_t)i1 * A + a],
                    a2 = at[(int64_t)i2 * A + a];
        du += (a1 - a0) * g[a];
        dv += (a2 - a0) * g[a];
      }
    }
    float d_udx = 0.0f, d_udy = 0.0f, d_vdx = 0.0f, d_vdy = 0.0f;
    if (K > 0 && valid) {
      const float* gd = d_out_da + pix * 2 * K;
      for (int k = 0; k < K; ++k) {
        const int a = diff_idx ? diff_idx[k] : k;
        if ((unsigned)a >= (unsigned)A) continue;  // not an attribute
        const float a0 = at[(int64_t)i0 * A + a], a1 = at[(int64_t)i1 * A + a],
                    a2 = at[(int64_t)i2 * A + a];
        const float d01 = a1 - a0, d02 = a2 - a0;
        const float gx = gd[2 * k + 0], gy = gd[2 * k + 1];
        d_udx += d01 * gx;
        d_udy += d01 * gy;
        d_vdx += d02 * gx;
        d_vdy += d02 * gy;
      }
    }
    if (inside) {
      *reinterpret_cast<float4*>(d_rast + pix * 4) = make_float4(du, dv, 0.0f, 0.0f);
      if (K > 0 && d_rast_db)
        *reinterpret_cast<float4*>(d_rast_db + pix * 4) = make_float4(d_udx, d_udy, d_vdx, d_vdy);
    }
    if (valid) {
      for (int a = 0; a < A; ++a) {
        const float ga = g[a];
        const float v0[1] = {bw * ga}, v1[1] = {u * ga}, v2[1] = {v * ga};
        lds_table_add(tab, da + (int64_t)i0 * A + a, v0);
        lds_table_add(tab, da + (int64_t)i1 * A + a, v1);
        lds_table_add(tab, da + (int64_t)i2 * A + a, v2);
      }
      if (K > 0) {
        const float* gd = d_out_da + pix * 2 * K;
        for (int k = 0; k < K; ++k) {
          const int a = diff_idx ? diff_idx[k] : k;
          if ((unsigned)a >= (unsigned)A) continue;  // not an attribute
          const float gx = gd[2 * k + 0], gy = gd[2 * k + 1];
          const float u_term = gx * db.x + gy * db.y;
          const float v_term = gx * db.z + gy * db.w;
          const float v0[1] = {-u_term - v_term}, v1[1] = {u_term}, v2[1] = {v_term};
          lds_table_add(tab, da + (int64_t)i0 * A + a, v0);
          lds_table_add(tab, da + (int64_t)i1 * A + a, v1);
          lds_table_add(tab, da + (int64_t)i2 * A + a, v2);
        }
      }
    }
  }
  __syncthreads();
  lds_table_flush_last(tab);  // the taken rows only
}

// d_attr[i] = (accumulate ? d_attr[i] : 0) + the sum of the 256 copies'
// element i, one workgroup per element (thread c reads copy c; the loads
// are independent, the sum a fixed tree); the copies are left zero.
__global__ void __launch_bounds__(256) k_sum_copies(float* __restrict__ copies, int64_t n,
                                                    float* __restrict__ d_attr, int accumulate) {
  __shared__ float s_w[4];
  const int64_t i = blockIdx.x;
  float* p = copies + (int64_t)threadIdx.x * n + i;
  float v = *p;
  *p = 0.0f;
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float s = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
    d_attr[i] = accumulate ? d_attr[i] + s : s;
  }
}

}  // namespace dr

using namespace dr;

#define DR_INTERP_DISPATCH(KERNEL, GRID, ...)                                              \
  do {                                                                                     \
    if (A == 2 && K == 0) hipLaunchKernelGGL((KERNEL<2, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else if (A == 2 && K == 2 && !diff_idx) hipLaunchKernelGGL((KERNEL<2, 2>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else if (A == 3 && K == 0) hipLaunchKernelGGL((KERNEL<3, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else if (A == 3 && K == 3 && !diff_idx) hipLaunchKernelGGL((KERNEL<3, 3>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else if (A == 4 && K == 0) hipLaunchKernelGGL((KERNEL<4, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else if (A == 6 && K == 0) hipLaunchKernelGGL((KERNEL<6, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__); \
    else hipLaunchKernelGGL((KERNEL<0, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__);      \
  } while (0)

static int check_interp(const float* attr, const float* rast, const int32_t* tri,
                        const float* rast_db, int K, int N, int H, int W, int V, int T, int A,
                        int64_t attr_stride, const int32_t* diff_idx) {
  DR_CHECK_ARG(N >= 1 && H >= 1 && W >= 1 && V >= 0 && T >= 0 && A >= 1 && K >= 0,
               "interpolate: bad sizes");
  DR_CHECK_ARG(attr && rast && tri, "interpolate: null tensor");
  DR_CHECK_ARG(T <= INT32_MAX / 3, "interpolate: at most 715827882 triangles (tri is indexed in 32 bits)");
  DR_CHECK_ARG(attr_stride == 0 || attr_stride == (int64_t)V * A,
               "interpolate: attr_batch_stride must be 0 or V*A");
  DR_CHECK_ARG(K == 0 || rast_db, "interpolate: rastDB is required when diffAttrs is set");
  DR_CHECK_ARG(K == 0 || diff_idx || K == A, "interpolate: diff_idx NULL needs K == A");
  return DR_OK;
}

extern "C" int dr_interpolate_fwd(const float* attr, int64_t attr_batch_stride,
                                  const float* rast, const float* rast_db, const int32_t* tri,
                                  const int32_t* diff_idx, int K, int N, int H, int W, int V,
                                  int T, int A, float* out, float* out_da, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  int st = check_interp(attr, rast, tri, rast_db, K, N, H, W, V, T, A, attr_batch_stride, diff_idx);
  if (st) return st;
  DR_CHECK_ARG(out && (K == 0 || out_da), "interpolate: null output");
  DR_TIMED("k_interp_fwd", stream);
  // the compile-time shapes store with 8/16-byte vector writes
  const bool aligned = (((uintptr_t)out | (uintptr_t)(out_da ? out_da : out)) & 15) == 0;
  // the dispatched kernel's pixels per thread (DR_INTERP_DISPATCH's choice)
  const int px = aligned && A == 6 && K == 0 ? interp_pix<6>() : interp_pix<0>();
  // and its strip width: the shapes of DR_INTERP_DISPATCH with an even A
  const bool even = aligned && (A == 2 || A == 4 || A == 6) &&
                    ((A == 2 && (K == 0 || (K == 2 && !diff_idx))) || (A != 2 && K == 0));
  const int sw = even ? interp_strip<2>() : interp_strip<0>(), sh = 256 / sw;
  const int ntx = (W + sw - 1) / sw, nty = (H + sh * px - 1) / (sh * px);
  const int64_t nblk = (int64_t)N * ntx * nty;
  DR_CHECK_ARG(nblk < ((int64_t)1 << 31), "interpolate: too many pixels");
  const dim3 grid((unsigned)nblk);
  const int xcd = (int64_t)V * A * (int64_t)sizeof(float) > kXcdL2Bytes;
  if (!aligned)
    hipLaunchKernelGGL((k_interp_fwd<0, 0>), grid, dim3(256), 0, stream, attr, attr_batch_stride,
                       rast, rast_db, tri, diff_idx, K, H, W, ntx, nty, V, T, A, out, out_da, xcd);
  else
    DR_INTERP_DISPATCH(k_interp_fwd, grid, attr, attr_batch_stride, rast, rast_db, tri, diff_idx,
                       K, H, W, ntx, nty, V, T, A, out, out_da, xcd);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

extern "C" int dr_interpolate_bwd(const float* attr, int64_t attr_batch_stride,
                                  const float* rast, const float* rast_db, const int32_t* tri,
                                  const int32_t* diff_idx, int K, const float* d_out,
                                  const float* d_out_da, int N, int H, int W, int V, int T,
                                  int A, float* d_attr, int64_t d_attr_batch_stride,
                                  float* d_rast, float* d_rast_db, unsigned flags,
                                  dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  int st = check_interp(attr, rast, tri, rast_db, K, N, H, W, V, T, A, attr_batch_stride, diff_idx);
  if (st) return st;
  DR_CHECK_ARG(d_out && d_attr && d_rast && (K == 0 || d_out_da), "interpolate_bwd: null tensor");
  DR_CHECK_ARG(d_attr_batch_stride == 0 || d_attr_batch_stride == (int64_t)V * A,
               "interpolate_bwd: d_attr_batch_stride must be 0 or V*A");
  const int64_t nattr = (d_attr_batch_stride ? (int64_t)N : 1) * V * A;
  const int ntx = (W + 15) / 16, nty = (H + 15) / 16;
  const int64_t tiles = (int64_t)N * ntx * nty;
  const dim3 grid((unsigned)tiles);
  // A small d_attr (a few shared vertices: every tile adds into the same
  // few rows, and device atomics on one address are serialised) is summed
  // into kCopies copies, workgroup b into copy b % kCopies, then added up.
  constexpr int kCopies = 256;
  const bool copy = nattr > 0 && nattr <= 4096 && tiles >= 4 * kCopies;
  float* target = d_attr;
  if (copy) {
    Scratch* sc = scratch_for(stream);
    if (!sc) return scratch_fail();
    const int64_t nc = nattr * kCopies;
    float* c = (float*)scratch_get(sc, stream, SLOT_DATTR_COPY, (size_t)nc * sizeof(float));
    if (!c) return scratch_fail();
    if (sc->copy_buf != c) {  // a new buffer: its contents are unknown
      sc->copy_buf = c;
      sc->copy_zero = 0;
    }
    if (sc->copy_zero < nc) DR_CHECK_HIP(fill_async(c, 0.0f, nc, stream));
    sc->copy_zero = 0;  // in use until k_sum_copies is queued
    target = c;
  } else if (!(flags & DR_ACCUMULATE)) {
    DR_CHECK_HIP(fill_async(d_attr, 0.0f, nattr, stream));
  }
  const int xcd = (int64_t)V * A * (int64_t)sizeof(float) > kXcdL2Bytes;
  {
    DR_TIMED("k_interp_bwd", stream);
    DR_INTERP_DISPATCH(k_interp_bwd, grid, attr, attr_batch_stride, rast, rast_db, tri, diff_idx,
                       K, d_out, d_out_da, N, H, W, ntx, nty, V, T, A, target,
                       d_attr_batch_stride, copy ? kCopies : 0, nattr, d_rast, d_rast_db, xcd);
  }
  DR_CHECK_LAUNCH();
  if (copy) {
    {
      DR_TIMED("k_sum_copies", stream);
      static_assert(kCopies == 256, "k_sum_copies: one thread per copy");
      hipLaunchKernelGGL(k_sum_copies, dim3((unsigned)nattr), dim3(kCopies), 0, stream, target,
                         nattr, d_attr, (flags & DR_ACCUMULATE) ? 1 : 0);
    }
    DR_CHECK_LAUNCH();
    Scratch* sc = scratch_for(stream);
    if (sc && sc->copy_buf == target) sc->copy_zero = nattr * kCopies;
  }
  return DR_OK;
}
