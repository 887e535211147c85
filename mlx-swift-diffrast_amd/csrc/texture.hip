// texture: mip pyramid, nearest / bilinear / mip-nearest / trilinear / cube
// sampling, and one fused backward per filter (d_tex or d_pyramid scatter,
// d_uv, d_uvDA and the mip-bias gradient in a single pass).
//
// Semantics follow Sources/MLXDiffRast/Texture.swift of the reference:
//   boundary modes     :336-354       bilinear   :359-403, :407-521
//   nearest            :545-605       cube       :616-738
//   LOD + levels       :764-790       mip fwd    :795-863
//   mip backward       :870-1102      pyramid    :144-161 (2x2 mean)
//   mip bias fold      :104-126 (uvDA * 2^map * 2^bias, folded in-kernel)
// The pyramid is built once per distinct texture (Nt = 1 serves every
// image), not once per broadcast copy; d_tex of a shared texture is the sum
// over images, as MLX's broadcast backward gives.
#include <mutex>
#include <string>

#include "common.h"

namespace dr {

constexpr int kMaxLevels = 16;

// Pyramid geometry.  Level 0 is the texture itself; levels 1..L-1 live in
// one buffer, level-major, each [Nt, Hk, Wk, C].
struct MipDesc {
  int L;
  int h[kMaxLevels];
  int w[kMaxLevels];
  int64_t off[kMaxLevels];  // float offset of level k (k >= 1) in the pyramid buffer
  int64_t nc;               // Nt * C
};

// Level k's size and pyramid offset computed from level 0 (every level
// halves both sizes exactly), so a per-lane level never indexes the
// descriptor arrays in kernel-argument memory.  Valid for 0 <= k < L.
__device__ __forceinline__ int mip_h(const MipDesc& m, int k) { return m.h[0] >> k; }
__device__ __forceinline__ int mip_w(const MipDesc& m, int k) { return m.w[0] >> k; }
__device__ __forceinline__ int64_t mip_off(const MipDesc& m, int k) {
  // sum_{j=1}^{k-1} Nt*C*(H*W / 4^j) = Nt*C*(H*W - H_{k-1}*W_{k-1}) / 3
  const int j = k > 0 ? k - 1 : 0;
  const uint64_t a = (uint64_t)(uint32_t)m.h[0] * (uint32_t)m.w[0];
  if (a < (1ull << 32)) {  // 32-bit arithmetic (uniform branch)
    const uint32_t b = ((uint32_t)m.h[0] >> j) * ((uint32_t)m.w[0] >> j);
    return m.nc * (int64_t)(((uint32_t)a - b) / 3u);
  }
  const uint64_t b = (uint64_t)(m.h[0] >> j) * (uint64_t)(m.w[0] >> j);
  return m.nc * (int64_t)((a - b) / 3);
}

// Texture.swift:336-354.
__device__ __forceinline__ int apply_boundary(int t, int size, int mode, float& oob) {
  if (mode == DR_BOUNDARY_ZERO) {
    if (t < 0 || t >= size) {
      oob = 1.0f;
      return 0;
    }
    oob = 0.0f;
    return t;
  }
  if (mode == DR_BOUNDARY_CLAMP) {
    oob = 0.0f;
    return t < 0 ? 0 : (t >= size ? size - 1 : t);
  }
  oob = 0.0f;
  int r = t % size;
  if (r < 0) r += size;
  return r;
}

struct Bilin {
  int ix0, ix1, iy0, iy1;
  float fx, fy, m00, m10, m01, m11, w00, w10, w01, w11;
};

// The bilinear footprint of Texture.swift:372-391 (and its copies).
__device__ __forceinline__ Bilin bilin(float u, float v, int Wk, int Hk, int mode) {
  Bilin b;
  const float tx = u * (float)Wk - 0.5f;
  const float ty = v * (float)Hk - 0.5f;
  const int tx0 = f2i(floorf(tx)), ty0 = f2i(floorf(ty));
  const int tx1 = tx0 + 1, ty1 = ty0 + 1;
  b.fx = tx - (float)tx0;
  b.fy = ty - (float)ty0;
  float ox0, ox1, oy0, oy1;
  b.ix0 = apply_boundary(tx0, Wk, mode, ox0);
  b.ix1 = apply_boundary(tx1, Wk, mode, ox1);
  b.iy0 = apply_boundary(ty0, Hk, mode, oy0);
  b.iy1 = apply_boundary(ty1, Hk, mode, oy1);
  b.m00 = (1.0f - ox0) * (1.0f - oy0);
  b.m10 = (1.0f - ox1) * (1.0f - oy0);
  b.m01 = (1.0f - ox0) * (1.0f - oy1);
  b.m11 = (1.0f - ox1) * (1.0f - oy1);
  const float fx = b.fx, fy = b.fy;
  b.w00 = (1.0f - fx) * (1.0f - fy) * (1.0f - ox0) * (1.0f - oy0);
  b.w10 = (fx) * (1.0f - fy) * (1.0f - ox1) * (1.0f - oy0);
  b.w01 = (1.0f - fx) * (fy) * (1.0f - ox0) * (1.0f - oy1);
  b.w11 = (fx) * (fy) * (1.0f - ox1) * (1.0f - oy1);
  return b;
}

// Texture.swift:616-672: cube face + clamped bilinear footprint.
__device__ __forceinline__ int cube_bilin(float x, float y, float z, int Wt, int Ht, Bilin& b) {
  const float ax = fabsf(x), ay = fabsf(y), az = fabsf(z);
  int face;
  float sc, tc, ma;
  if (ax >= ay && ax >= az) {
    ma = ax;
    if (x > 0.0f) { face = 0; sc = -z; tc = -y; }
    else          { face = 1; sc = z;  tc = -y; }
  } else if (ay >= az) {
    ma = ay;
    if (y > 0.0f) { face = 2; sc = x; tc = z; }
    else          { face = 3; sc = x; tc = -z; }
  } else {
    ma = az;
    if (z > 0.0f) { face = 4; sc = x;  tc = -y; }
    else          { face = 5; sc = -x; tc = -y; }
  }
  const float inv_ma = 1.0f / ma;
  const float u = (sc * inv_ma + 1.0f) * 0.5f;
  const float v = (tc * inv_ma + 1.0f) * 0.5f;
  const float txr = u * (float)Wt - 0.5f;
  const float tyr = v * (float)Ht - 0.5f;
  const int tx0 = f2i(floorf(txr)), ty0 = f2i(floorf(tyr));
  const int tx1 = tx0 + 1, ty1 = ty0 + 1;
  const float fx = txr - (float)tx0, fy = tyr - (float)ty0;
  b.fx = fx;
  b.fy = fy;
  b.ix0 = max(0, min(Wt - 1, tx0));
  b.ix1 = max(0, min(Wt - 1, tx1));
  b.iy0 = max(0, min(Ht - 1, ty0));
  b.iy1 = max(0, min(Ht - 1, ty1));
  b.m00 = b.m10 = b.m01 = b.m11 = 1.0f;
  b.w00 = (1.0f - fx) * (1.0f - fy);
  b.w10 = fx * (1.0f - fy);
  b.w01 = (1.0f - fx) * fy;
  b.w11 = fx * fy;
  return face;
}

// Texture.swift:764-790 on the bias-folded derivatives.
struct Lod {
  int k0, k1;
  float frac;
};

__device__ __forceinline__ Lod mip_lod(float4 da, int Ht, int Wt, int L, bool linear) {
  const float sx = da.x * (float)Wt, sy = da.y * (float)Wt;
  const float tx = da.z * (float)Ht, ty = da.w * (float)Ht;
  const float rho_sq = fmaxf(sx * sx + tx * tx, sy * sy + ty * ty);
  float lod = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
  lod = fmaxf(0.0f, fminf((float)(L - 1), lod));
  Lod r;
  if (linear) {
    r.k0 = f2i(floorf(lod));
    r.k1 = min(r.k0 + 1, L - 1);
    r.frac = lod - (float)r.k0;
  } else {
    r.k0 = min(f2i(floorf(lod + 0.5f)), L - 1);
    r.k1 = r.k0;
    r.frac = 0.0f;
  }
  return r;
}

// uvDA * (2^map * 2^bias) (Texture.swift:109-126).  scale_bias = 2^bias.
__device__ __forceinline__ float bias_scale(const float* __restrict__ bias_map, int64_t pix,
                                            float scale_bias, bool has_bias) {
  if (bias_map) {
    const float s = exp2f(bias_map[pix]);
    return has_bias ? s * scale_bias : s;
  }
  return scale_bias;
}

template <int CT>
__device__ __forceinline__ int dimC(int C) { return CT > 0 ? CT : C; }

// Loads channels [0,C) of one texel.
template <int CT>
__device__ __forceinline__ void load_texel(const float* __restrict__ p, int C, float* out) {
  if (CT == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    out[0] = q.x; out[1] = q.y; out[2] = q.z; out[3] = q.w;
  } else {
#pragma unroll
    for (int c = 0; c < dimC<CT>(C); ++c) out[c] = p[c];
  }
}

constexpr int kMaxC = 4;  // register arrays for compile-time C; larger C uses CT = 0

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------

template <int FILTER, bool CUBE, int CT>
__device__ __forceinline__ void tex_fwd_px(
    const float* __restrict__ tex, const float* __restrict__ pyr, const MipDesc& md,
    int64_t tex_stride, int Ht, int Wt, int C_, const float* __restrict__ uv,
    const float* __restrict__ uv_da, const float* __restrict__ bias_map, float scale_bias,
    int has_bias, int boundary, int64_t P, int n, float* __restrict__ out, int64_t pix) {
  if (pix >= P) return;
  const int C = dimC<CT>(C_);
  float* o = out + pix * C;
  if (CUBE) {  // Texture.swift:638-684
    const float x = uv[pix * 3 + 0], y = uv[pix * 3 + 1], z = uv[pix * 3 + 2];
    Bilin b;
    const int face = cube_bilin(x, y, z, Wt, Ht, b);
    const float* fb = tex + n * tex_stride + (int64_t)face * Ht * Wt * C;
    for (int c = 0; c < C; ++c) {
      const float t00 = fb[((int64_t)b.iy0 * Wt + b.ix0) * C + c];
      const float t10 = fb[((int64_t)b.iy0 * Wt + b.ix1) * C + c];
      const float t01 = fb[((int64_t)b.iy1 * Wt + b.ix0) * C + c];
      const float t11 = fb[((int64_t)b.iy1 * Wt + b.ix1) * C + c];
      o[c] = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
    }
    return;
  }
  const float2 uvp = ld_nt2(uv + pix * 2);
  if (FILTER == DR_FILTER_NEAREST) {  // Texture.swift:545-572
    const int tx = f2i(floorf(uvp.x * (float)Wt));
    const int ty = f2i(floorf(uvp.y * (float)Ht));
    float ox, oy;
    const int ix = apply_boundary(tx, Wt, boundary, ox);
    const int iy = apply_boundary(ty, Ht, boundary, oy);
    const float mask = (1.0f - ox) * (1.0f - oy);
    const float* tp = tex + n * tex_stride + ((int64_t)iy * Wt + ix) * C;
    for (int c = 0; c < C; ++c) o[c] = tp[c] * mask;
    return;
  }
  if (FILTER == DR_FILTER_LINEAR) {  // Texture.swift:359-403
    const Bilin b = bilin(uvp.x, uvp.y, Wt, Ht, boundary);
    const float* tb = tex + n * tex_stride;
    if (CT > 0) {
      float t00[kMaxC], t10[kMaxC], t01[kMaxC], t11[kMaxC];
      load_texel<CT>(tb + ((int64_t)b.iy0 * Wt + b.ix0) * C, C, t00);
      load_texel<CT>(tb + ((int64_t)b.iy0 * Wt + b.ix1) * C, C, t10);
      load_texel<CT>(tb + ((int64_t)b.iy1 * Wt + b.ix0) * C, C, t01);
      load_texel<CT>(tb + ((int64_t)b.iy1 * Wt + b.ix1) * C, C, t11);
#pragma unroll
      for (int c = 0; c < (CT > 0 ? CT : 1); ++c)
        o[c] = b.w00 * t00[c] + b.w10 * t10[c] + b.w01 * t01[c] + b.w11 * t11[c];
    } else {
      for (int c = 0; c < C; ++c) {
        const float t00 = tb[((int64_t)b.iy0 * Wt + b.ix0) * C + c];
        const float t10 = tb[((int64_t)b.iy0 * Wt + b.ix1) * C + c];
        const float t01 = tb[((int64_t)b.iy1 * Wt + b.ix0) * C + c];
        const float t11 = tb[((int64_t)b.iy1 * Wt + b.ix1) * C + c];
        o[c] = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
      }
    }
    return;
  }
  // Mip filters (Texture.swift:795-863).
  float4 da = ld_nt4(uv_da + pix * 4);
  const float s = bias_scale(bias_map, pix, scale_bias, has_bias != 0);
  if (bias_map || has_bias) da = make_float4(da.x * s, da.y * s, da.z * s, da.w * s);
  const Lod ld = mip_lod(da, Ht, Wt, md.L, FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR);
  const bool shared = tex_stride == 0;
  if constexpr (CT > 0) {  // texels as vectors, the sum in registers
    float acc[CT];
#pragma unroll
    for (int li = 0; li < 2; ++li) {
      // a zero weight adds +0 to every channel: the second level is not read
      // (the result differs only for non-finite texels, where 0 * inf is NaN)
      if (li == 1 && ld.frac == 0.0f) break;
      const int k = li == 0 ? ld.k0 : ld.k1;
      const int Hk = mip_h(md, k), Wk = mip_w(md, k);
      const float* lv = k == 0 ? tex + n * tex_stride
                               : pyr + mip_off(md, k) + (shared ? 0 : (int64_t)n * Hk * Wk * C);
      const Bilin b = bilin(uvp.x, uvp.y, Wk, Hk, boundary);
      const float wgt = li == 0 ? (1.0f - ld.frac) : ld.frac;
      float t00[kMaxC], t10[kMaxC], t01[kMaxC], t11[kMaxC];
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix0) * C, C, t00);
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix1) * C, C, t10);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix0) * C, C, t01);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix1) * C, C, t11);
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const float sample = b.w00 * t00[c] + b.w10 * t10[c] + b.w01 * t01[c] + b.w11 * t11[c];
        acc[c] = li == 0 ? wgt * sample : acc[c] + wgt * sample;  // two roundings, as :855 / :858
      }
    }
    if constexpr (CT == 4) {
      *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else {
#pragma unroll
      for (int c = 0; c < CT; ++c) o[c] = acc[c];
    }
    return;
  }
  for (int li = 0; li < 2; ++li) {
    const int k = li == 0 ? ld.k0 : ld.k1;
    const int Hk = mip_h(md, k), Wk = mip_w(md, k);
    const float* lv = k == 0 ? tex + n * tex_stride
                             : pyr + mip_off(md, k) + (shared ? 0 : (int64_t)n * Hk * Wk * C);
    const Bilin b = bilin(uvp.x, uvp.y, Wk, Hk, boundary);
    const float wgt = li == 0 ? (1.0f - ld.frac) : ld.frac;
    for (int c = 0; c < C; ++c) {
      const float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
      const float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
      const float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
      const float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
      const float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
      if (li == 0) o[c] = wgt * sample;  // two roundings, as :855 / :858
      else o[c] = o[c] + wgt * sample;
    }
  }
}

// BND: the boundary mode as a compile-time constant (DR_BOUNDARY_CUBE for
// cube maps), so the clamp and wrap footprints carry no out-of-range masks.
// One workgroup per 16x16 pixel tile, a 16x4 strip per wave: neighbouring
// pixels sample neighbouring texels, so a wave's gathers share cache lines
// (measured 0.105 -> 0.089 ms at 8 x 1024^2 against whole pixel rows).
template <int FILTER, int BND, int CT>
__global__ void __launch_bounds__(256) k_tex_fwd(
    const float* __restrict__ tex, const float* __restrict__ pyr, MipDesc md, int64_t tex_stride,
    int Ht, int Wt, int C_, const float* __restrict__ uv, const float* __restrict__ uv_da,
    const float* __restrict__ bias_map, float scale_bias, int has_bias, int64_t P, int Hi,
    int Wi, float* __restrict__ out) {
  const int ntx = (Wi + 15) >> 4, tiles = ntx * ((Hi + 15) >> 4);
  const int b = (int)blockIdx.x, n = b / tiles, tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int ph = ty * 16 + ((int)threadIdx.x >> 4), pw = tx * 16 + ((int)threadIdx.x & 15);
  // pixels past the image's right or bottom edge get index P: no work
  const int64_t pix = ph < Hi && pw < Wi ? ((int64_t)n * Hi + ph) * Wi + pw : P;
  tex_fwd_px<FILTER, BND == DR_BOUNDARY_CUBE, CT>(tex, pyr, md, tex_stride, Ht, Wt, C_, uv, uv_da,
                                                  bias_map, scale_bias, has_bias, BND, P, n, out,
                                                  pix);
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

// Per-wave accumulator of one bilinear footprint's gradient.  A large group
// of lanes on one footprint (in practice: every background pixel samples the
// same clamped texel) adds its wave-summed values here instead of issuing
// atomics; the accumulator is written out when a different footprint takes
// its place and when the wave has finished all its tiles.  Wave-uniform.
template <int CT>
struct FootAcc {
  float* p[4];  // the footprint's four texels (wave-uniform)
  float v;      // lane j < 4*CT: running sum of value j = 4 * channel + tap
  bool on;
};

template <int CT>
__device__ __forceinline__ void acc_init(FootAcc<CT>& a) {
  a.on = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) a.p[i] = nullptr;
  a.v = 0.0f;
}

template <int CT>
__device__ __forceinline__ void acc_flush(FootAcc<CT>& a) {
  if (!a.on) return;
  const int l = lane_id();
  if (l < 4 * CT && a.v != 0.0f) {
    const int tap = l & 3;
    float* q = tap == 0 ? a.p[0] : tap == 1 ? a.p[1] : tap == 2 ? a.p[2] : a.p[3];
    unsafeAtomicAdd(q + (l >> 2), a.v);
  }
  a.on = false;
}

// Adds the wave sums of val[0..M) (M <= 16) to the accumulator.
template <int CT, int M>
__device__ __forceinline__ void acc_add(FootAcc<CT>& a, const float (&val)[M], bool member) {
  static_assert(M <= 16, "at most 16 values");
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = (i < M && member) ? val[i < M ? i : 0] : 0.0f;
  a.v += wave_sum16(x);
}

// Scatter of one bilinear footprint's gradient (w * g * scale) into one
// level.  Taps that land on the same texel (clamped borders) are merged
// first; lanes sharing the footprint are summed across the wave.
constexpr int kTexTable = 512;  // LDS aggregation entries per tile (texels)

template <int CT, int CAP = kTexTable>
using TexTable = LdsTable<(CT > 0 ? CT : 1), CAP>;

// The cube backward's table: a cube map's footprints spread over more
// texels per tile (a per-pixel LOD bias splits them over two or three
// levels), and a full table sends the rest of the tile's taps straight to
// device atomics (4096 x 256^2, 6 x 512^2 x 3 with a random bias map:
// 91 -> 47 ms with 1,024 entries, 43 ms with 2,048).
constexpr int kCubeTable = 2048;
template <int CT>
using CubeTable = LdsTableU<(CT > 0 ? CT : 1), kCubeTable>;

template <int CT, bool USE_ACC = true, typename Tab = TexTable<CT>>
__device__ __forceinline__ void scatter_footprint(bool valid, float* __restrict__ base, int Wk,
                                                  int C, const Bilin& b, const float* g,
                                                  float scale,
                                                  FootAcc<(CT > 0 ? CT : 1)>& acc,
                                                  Tab& tab) {
  float w00 = b.w00, w10 = b.w10, w01 = b.w01, w11 = b.w11;
  if (b.ix1 == b.ix0) {
    w00 += w10;
    w01 += w11;
    w10 = 0.0f;
    w11 = 0.0f;
  }
  if (b.iy1 == b.iy0) {
    w00 += w01;
    w10 += w11;
    w01 = 0.0f;
    w11 = 0.0f;
  }
  float* const p[4] = {base + ((int64_t)b.iy0 * Wk + b.ix0) * C, base + ((int64_t)b.iy0 * Wk + b.ix1) * C,
                       base + ((int64_t)b.iy1 * Wk + b.ix0) * C, base + ((int64_t)b.iy1 * Wk + b.ix1) * C};
  if (CT > 0) {
    constexpr int M = 4 * (CT > 0 ? CT : 1);
    float val[M];
#pragma unroll
    for (int c = 0; c < (CT > 0 ? CT : 1); ++c) {
      const float gc = valid ? g[c] * scale : 0.0f;
      val[4 * c + 0] = w00 * gc;
      val[4 * c + 1] = w10 * gc;
      val[4 * c + 2] = w01 * gc;
      val[4 * c + 3] = w11 * gc;
    }
    // The probes pay where many lanes share a footprint: a magnified
    // texture (a texel cell three or more pixels wide repeats its taps over
    // runs of three lanes or more along the pixel rows) or one texel under
    // a whole wave.  Unless at least two lanes share their first tap with
    // the lane two before them they are skipped: footprints shared in pairs
    // only, as under a per-pixel LOD bias, never form a group worth them
    // (cube backward at 4096 x 256^2: 39.0 -> 36.9 ms).  Every lane executes
    // the shifts (callers keep the wave convergent).
    const uint64_t a0 = (uint64_t)p[0];
    const uint32_t l_lo = (uint32_t)dpp_shift<0x112>((int)(uint32_t)a0);
    const uint32_t l_hi = (uint32_t)dpp_shift<0x112>((int)(uint32_t)(a0 >> 32));
    const bool run3 = valid && (lane_id() & 15) >= 2 && (((uint64_t)l_hi << 32) | l_lo) == a0;
    uint64_t pending = __popcll(__ballot(run3)) >= 2 ? __ballot(valid) : 0ull;
    bool mine = valid;
    const int lane = lane_id();
#pragma unroll 1
    for (int probe = 0; probe < kProbes && pending; ++probe) {
      const int leader = probe_leader(pending, probe);
      float* lp[4];
      bool same = mine;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        lp[t] = (float*)lane_value((uint64_t)p[t], leader);
        same = same && p[t] == lp[t];
      }
      const uint64_t members = __ballot(same);
      pending &= ~members;
      if (__popcll(members) >= kGroupMin && !USE_ACC) {
#pragma unroll
        for (int i = 0; i < M; ++i) {
          const float sm = wave_sum(same ? val[i] : 0.0f);
          if (lane == leader && sm != 0.0f) unsafeAtomicAdd(lp[i & 3] + (i >> 2), sm);
        }
        if (same) mine = false;
      } else if (__popcll(members) >= kGroupMin) {
        const bool hit = acc.on && acc.p[0] == lp[0] && acc.p[1] == lp[1] && acc.p[2] == lp[2] &&
                         acc.p[3] == lp[3];
        if (!hit) {
          acc_flush(acc);
#pragma unroll
          for (int t = 0; t < 4; ++t) acc.p[t] = (float*)uni((uint64_t)lp[t]);
          acc.v = 0.0f;
          acc.on = true;
        }
        acc_add(acc, val, same);
        if (same) mine = false;
      }
    }
    if (mine) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float v[CT > 0 ? CT : 1];
#pragma unroll
        for (int c = 0; c < (CT > 0 ? CT : 1); ++c) v[c] = val[4 * c + t];
        lds_table_add(tab, p[t], v);
      }
    }
  } else {
    const uint32_t key2 = ((uint32_t)b.ix1 << 16) ^ (uint32_t)b.iy1;
    for (int c = 0; c < C; ++c) {
      const float gc = valid ? g[c] * scale : 0.0f;
      float val[4] = {w00 * gc, w10 * gc, w01 * gc, w11 * gc};
      float* addr[4] = {p[0] + c, p[1] + c, p[2] + c, p[3] + c};
      group_atomic_add<4>(valid, (uint64_t)p[0], addr, val, key2);
    }
  }
}

// d_uv terms of one level (Texture.swift:500-520 / :979-995), summed over C.
// IDX: the element offsets' type, int64_t for any level, or uint32_t where
// the caller guarantees a level below 2^32 elements (sides at most 32767,
// C at most 4).
template <typename IDX = int64_t>
__device__ __forceinline__ void duv_level(const float* __restrict__ lv, int Wk, int C,
                                          const Bilin& b, const float* g, float scale,
                                          float& dfx, float& dfy, float& dlod_sample) {
  dfx = 0.0f;
  dfy = 0.0f;
  dlod_sample = 0.0f;
  const IDX r0 = (IDX)b.iy0 * (IDX)Wk, r1 = (IDX)b.iy1 * (IDX)Wk;
  const float* p00 = lv + (r0 + (IDX)b.ix0) * (IDX)C;
  const float* p10 = lv + (r0 + (IDX)b.ix1) * (IDX)C;
  const float* p01 = lv + (r1 + (IDX)b.ix0) * (IDX)C;
  const float* p11 = lv + (r1 + (IDX)b.ix1) * (IDX)C;
  for (int c = 0; c < C; ++c) {
    const float r00 = p00[c], r10 = p10[c], r01 = p01[c], r11 = p11[c];
    const float t00 = r00 * b.m00, t10 = r10 * b.m10, t01 = r01 * b.m01, t11 = r11 * b.m11;
    const float gc = g[c] * scale;
    dfx += gc * ((1.0f - b.fy) * (t10 - t00) + b.fy * (t11 - t01));
    dfy += gc * ((1.0f - b.fx) * (t01 - t00) + b.fx * (t11 - t10));
    const float sample = b.w00 * r00 + b.w10 * r10 + b.w01 * r01 + b.w11 * r11;
    dlod_sample += sample * g[c];
  }
}

struct TexBwdArgs {
  const float* tex;
  const float* pyr;
  MipDesc md;
  int64_t tex_stride;
  int Ht, Wt, C, boundary, has_bias;
  const float* uv;
  const float* uv_da;
  const float* bias_map;
  float scale_bias;
  int N, Hi, Wi, ntx, nty;
  const float* d_out;
  float* d_tex;
  float* d_pyr;
  float* d_uv;
  float* d_uv_da;
  float* d_bias;
};

// One 16x16 pixel tile of the fused backward (one 8x8 quadrant per wave).
template <int FILTER, bool CUBE, int CT>
__device__ __forceinline__ void tex_bwd_tile(const TexBwdArgs& A, int bidx,
                                             FootAcc<(CT > 0 ? CT : 1)>& acc0,
                                             TexTable<CT>& tab) {
  const float* __restrict__ tex = A.tex;
  const float* __restrict__ pyr = A.pyr;
  const MipDesc& md = A.md;
  const int64_t tex_stride = A.tex_stride;
  const int Ht = A.Ht, Wt = A.Wt, C_ = A.C, boundary = A.boundary, has_bias = A.has_bias;
  const float* __restrict__ uv = A.uv;
  const float* __restrict__ uv_da = A.uv_da;
  const float* __restrict__ bias_map = A.bias_map;
  const float scale_bias = A.scale_bias;
  const int Hi = A.Hi, Wi = A.Wi, ntx = A.ntx, nty = A.nty;
  const float* __restrict__ d_out = A.d_out;
  float* __restrict__ d_tex = A.d_tex;
  float* __restrict__ d_pyr = A.d_pyr;
  float* __restrict__ d_uv = A.d_uv;
  float* __restrict__ d_uv_da = A.d_uv_da;
  float* __restrict__ d_bias = A.d_bias;
  const int tiles = ntx * nty;
  const int n = bidx / tiles;
  const int tile = bidx - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qx0 = tx * 16 + (wave & 1) * 8, qy0 = ty * 16 + (wave >> 1) * 8;
  if (qx0 >= Wi || qy0 >= Hi) return;
  const int pw = qx0 + (lane & 7), ph = qy0 + (lane >> 3);
  const bool valid = pw < Wi && ph < Hi;
  const int64_t pix = ((int64_t)n * Hi + min(ph, Hi - 1)) * Wi + min(pw, Wi - 1);
  const int C = dimC<CT>(C_);
  float g[CT > 0 ? CT : kMaxC];
  const float* gp = d_out + pix * C;
  float* dt = d_tex + n * tex_stride;  // tex_stride 0: shared texture

  if (CUBE) {  // Texture.swift:686-738 (d_dir is zero: :196-198)
    const float x = uv[pix * 3 + 0], y = uv[pix * 3 + 1], z = uv[pix * 3 + 2];
    Bilin b;
    const int face = cube_bilin(x, y, z, Wt, Ht, b);
    float* fb = dt + (int64_t)face * Ht * Wt * C;
    if (CT > 0) {
#pragma unroll
      for (int c = 0; c < (CT > 0 ? CT : 1); ++c) g[c] = gp[c];
      scatter_footprint<CT>(valid, fb, Wt, C, b, g, 1.0f, acc0, tab);
    } else {
      for (int c = 0; c < C; ++c) {
        const float gc = valid ? gp[c] : 0.0f;
        float val[4] = {b.w00 * gc, b.w10 * gc, b.w01 * gc, b.w11 * gc};
        float* addr[4] = {fb + ((int64_t)b.iy0 * Wt + b.ix0) * C + c,
                          fb + ((int64_t)b.iy0 * Wt + b.ix1) * C + c,
                          fb + ((int64_t)b.iy1 * Wt + b.ix0) * C + c,
                          fb + ((int64_t)b.iy1 * Wt + b.ix1) * C + c};
        group_atomic_add<4>(valid, (uint64_t)addr[0], addr, val,
                            ((uint32_t)b.ix1 << 16) ^ (uint32_t)b.iy1);
      }
    }
    if (d_uv && valid) {
      d_uv[pix * 3 + 0] = 0.0f;
      d_uv[pix * 3 + 1] = 0.0f;
      d_uv[pix * 3 + 2] = 0.0f;
    }
    return;
  }

  const float2 uvp = ld_nt2(uv + pix * 2);
  if (FILTER == DR_FILTER_NEAREST) {  // Texture.swift:576-605; d_uv = 0 (:234)
    const int txi = f2i(floorf(uvp.x * (float)Wt));
    const int tyi = f2i(floorf(uvp.y * (float)Ht));
    float ox, oy;
    const int ix = apply_boundary(txi, Wt, boundary, ox);
    const int iy = apply_boundary(tyi, Ht, boundary, oy);
    const float mask = (1.0f - ox) * (1.0f - oy);
    float* tp = dt + ((int64_t)iy * Wt + ix) * C;
    if (CT > 0) {
      if (valid) {
        float v[CT > 0 ? CT : 1];
#pragma unroll
        for (int c = 0; c < (CT > 0 ? CT : 1); ++c) v[c] = gp[c] * mask;
        lds_table_add(tab, tp, v);
      }
    } else {
      for (int c = 0; c < C; ++c) {
        float val[1] = {valid ? gp[c] * mask : 0.0f};
        float* addr[1] = {tp + c};
        group_atomic_add<1>(valid, (uint64_t)tp, addr, val);
      }
    }
    if (d_uv && valid) *reinterpret_cast<float2*>(d_uv + pix * 2) = make_float2(0.0f, 0.0f);
    return;
  }

  for (int c = 0; c < C && c < (CT > 0 ? CT : kMaxC); ++c) g[c] = valid ? gp[c] : 0.0f;
  const float* gsrc = CT > 0 ? g : gp;  // run-time C reads d_out directly

  if (FILTER == DR_FILTER_LINEAR) {  // Texture.swift:407-521
    const Bilin b = bilin(uvp.x, uvp.y, Wt, Ht, boundary);
    const float* tb = tex + n * tex_stride;
    scatter_footprint<CT>(valid, dt, Wt, C, b, gsrc, 1.0f, acc0, tab);
    if (d_uv && valid) {
      float dfx, dfy, unused;
      duv_level(tb, Wt, C, b, gsrc, 1.0f, dfx, dfy, unused);
      *reinterpret_cast<float2*>(d_uv + pix * 2) = make_float2(dfx * (float)Wt, dfy * (float)Ht);
    }
    return;
  }

  // Mip filters: Texture.swift:870-1102 fused.
  const float4 da_in = *reinterpret_cast<const float4*>(uv_da + pix * 4);
  const float s = bias_scale(bias_map, pix, scale_bias, has_bias != 0);
  const bool scaled = bias_map || has_bias;
  const float4 da = scaled ? make_float4(da_in.x * s, da_in.y * s, da_in.z * s, da_in.w * s) : da_in;
  const bool linear = FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR;
  const Lod ld = mip_lod(da, Ht, Wt, md.L, linear);
  const bool shared = tex_stride == 0;
  auto level_ptr = [&](int k) -> const float* {
    return k == 0 ? tex + n * tex_stride
                  : pyr + mip_off(md, k) + (shared ? 0 : (int64_t)n * mip_h(md, k) * mip_w(md, k) * C);
  };
  auto dlevel_ptr = [&](int k) -> float* {
    return k == 0 ? dt : d_pyr + mip_off(md, k) + (shared ? 0 : (int64_t)n * mip_h(md, k) * mip_w(md, k) * C);
  };
  float dfx_total = 0.0f, dfy_total = 0.0f;
  float samp[2] = {0.0f, 0.0f};  // sum_c g_c * sample_c per level (for d_lod)
  for (int li = 0; li < 2; ++li) {
    const int k = li == 0 ? ld.k0 : ld.k1;
    const float scale = li == 0 ? (1.0f - ld.frac) : ld.frac;
    const int Hk = mip_h(md, k), Wk = mip_w(md, k);
    const Bilin b = bilin(uvp.x, uvp.y, Wk, Hk, boundary);
    // A zero weight adds nothing; skip the level's atomics (but keep the
    // wave convergent for the grouping).
    if (li == 0)
      scatter_footprint<CT, true>(valid && scale != 0.0f, dlevel_ptr(k), Wk, C, b, gsrc, scale, acc0,
                                  tab);
    else
      scatter_footprint<CT, false>(valid && scale != 0.0f, dlevel_ptr(k), Wk, C, b, gsrc, scale, acc0,
                                   tab);
    if (valid) {
      float dfx, dfy;
      duv_level(level_ptr(k), Wk, C, b, gsrc, scale, dfx, dfy, samp[li]);
      dfx_total += dfx * (float)Wk;
      dfy_total += dfy * (float)Hk;
    }
  }
  if (!valid) return;
  if (d_uv) *reinterpret_cast<float2*>(d_uv + pix * 2) = make_float2(dfx_total, dfy_total);
  if (!d_uv_da && !d_bias) return;
  // Texture.swift:1011-1102 (mip-nearest also takes this trilinear surrogate).
  const float sx = da.x * (float)Wt, sy = da.y * (float)Wt;
  const float tx_ = da.z * (float)Ht, ty_ = da.w * (float)Ht;
  const float Asq = sx * sx + tx_ * tx_;
  const float Bsq = sy * sy + ty_ * ty_;
  const float rho_sq = fmaxf(Asq, Bsq);
  const float lod_raw = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
  float4 d_eff = make_float4(0.f, 0.f, 0.f, 0.f);
  if (!(lod_raw <= 0.0f || lod_raw >= (float)(md.L - 1))) {
    float d_lod;
    const int k0 = f2i(floorf(lod_raw));
    if (linear) {
      d_lod = -samp[0] + samp[1];
    } else {
      const int k1 = min(k0 + 1, md.L - 1);
      float s0 = 0.0f, s1 = 0.0f, u0, u1;
      const Bilin b0 = bilin(uvp.x, uvp.y, mip_w(md, k0), mip_h(md, k0), boundary);
      duv_level(level_ptr(k0), mip_w(md, k0), C, b0, gsrc, 0.0f, u0, u1, s0);
      const Bilin b1 = bilin(uvp.x, uvp.y, mip_w(md, k1), mip_h(md, k1), boundary);
      duv_level(level_ptr(k1), mip_w(md, k1), C, b1, gsrc, 0.0f, u0, u1, s1);
      d_lod = -s0 + s1;
    }
    const float ln2 = 0.6931471805599453f;
    const float dlod_drho_sq = 1.0f / (2.0f * rho_sq * ln2);
    const float A_is_max = (Asq >= Bsq) ? 1.0f : 0.0f;
    const float B_is_max = 1.0f - A_is_max;
    d_eff = make_float4(d_lod * dlod_drho_sq * A_is_max * 2.0f * sx * (float)Wt,
                        d_lod * dlod_drho_sq * B_is_max * 2.0f * sy * (float)Wt,
                        d_lod * dlod_drho_sq * A_is_max * 2.0f * tx_ * (float)Ht,
                        d_lod * dlod_drho_sq * B_is_max * 2.0f * ty_ * (float)Ht);
  }
  // Backward of the bias fold: d_uvDA = d_eff * scale,
  // d_map = sum_c(d_eff_c * uvDA_c) * scale * ln 2.
  if (d_uv_da) {
    const float4 o = scaled ? make_float4(d_eff.x * s, d_eff.y * s, d_eff.z * s, d_eff.w * s) : d_eff;
    *reinterpret_cast<float4*>(d_uv_da + pix * 4) = o;
  }
  if (d_bias && bias_map) {
    const float gm = d_eff.x * da_in.x + d_eff.y * da_in.y + d_eff.z * da_in.z + d_eff.w * da_in.w;
    d_bias[pix] = gm * s * 0.6931471805599453f;
  }
}

template <int FILTER, bool CUBE, int CT>
__global__ void __launch_bounds__(256) k_tex_bwd(TexBwdArgs A, int total_tiles) {
  __shared__ TexTable<CT> tab;
  FootAcc<(CT > 0 ? CT : 1)> acc0;
  acc_init(acc0);
  lds_table_clear(tab);
  __syncthreads();
  for (int t = (int)blockIdx.x; t < total_tiles; t += (int)gridDim.x) {
    tex_bwd_tile<FILTER, CUBE, CT>(A, t, acc0, tab);
    __syncthreads();
    lds_table_flush(tab);
    __syncthreads();
  }
  acc_flush(acc0);
}

// ---------------------------------------------------------------------------
// Windowed backward for the sampled filters (linear, linear-mipmap-*), C in
// 1..4.  Per 16x16 pixel tile the texel bounding box of the footprints on
// the two lowest levels in use is taken, and contributions are summed into
// dense fp64 LDS windows over those boxes (direct indexing, no hashing; the
// two windows share one pool).  The windows are written out row by row, so
// consecutive lanes issue atomics to consecutive addresses.  Big groups of lanes on one footprint (the
// background texel) go to the per-wave accumulator; taps on other levels,
// or boxes too large for a window, go to the LDS hash table.
// ---------------------------------------------------------------------------

constexpr int kWinWaves = 4;                  // waves per workgroup; a tile is 16 x (4 * kWinWaves) pixels
constexpr int kWinTexels = 192 * kWinWaves;  // texels of the two windows together
constexpr int kWinFallback = 32 * kWinWaves;  // LDS hash table entries
constexpr int kWinThreads = 64 * kWinWaves;

struct TapSlot {
  int k;         // level
  float scale;   // (1 - frac) or frac; 0 = unused
  int ix0, ix1, iy0, iy1;
  float w00, w10, w01, w11;
};

__device__ __forceinline__ void slot_box(const TapSlot& q, int& x0, int& x1, int& y0, int& y1) {
  const bool c0 = q.w00 != 0.0f || q.w01 != 0.0f, c1 = q.w10 != 0.0f || q.w11 != 0.0f;
  const bool r0 = q.w00 != 0.0f || q.w10 != 0.0f, r1 = q.w01 != 0.0f || q.w11 != 0.0f;
  x0 = 0x7fffffff; x1 = -1; y0 = 0x7fffffff; y1 = -1;
  if (c0) { x0 = min(x0, q.ix0); x1 = max(x1, q.ix0); }
  if (c1) { x0 = min(x0, q.ix1); x1 = max(x1, q.ix1); }
  if (r0) { y0 = min(y0, q.iy0); y1 = max(y1, q.iy0); }
  if (r1) { y0 = min(y0, q.iy1); y1 = max(y1, q.iy1); }
}


template <int FILTER, int CT, int BND, bool BIAS>
// Five waves per SIMD (the register budget this asks for costs a few
// spilled values; measured cheaper than four or six).
__global__ void __launch_bounds__(kWinThreads, 5) k_tex_bwd_win(TexBwdArgs A, int total_tiles) {
  // channel-major (win[c * kWinTexels + texel]): a wave's run tails on
  // neighbouring texels then add 8 bytes apart, spread over the banks,
  // rather than 8 * CT bytes apart on a few of them
  __shared__ double win[kWinTexels * CT];
  __shared__ __align__(16) int s_lmask[kWinWaves];  // per wave: the levels in use (bit mask)
  __shared__ int2 s_lbox[kWinWaves][kMaxLevels];     // per wave and level: packed box
  __shared__ int s_tab_used[2];    // per tile parity: the table took entries
  __shared__ LdsTable<CT, kWinFallback> tab;
  FootAcc<CT> acc;
  acc_init(acc);
  const int tid = threadIdx.x;
  for (int i = tid; i < kWinTexels * CT; i += kWinThreads) win[i] = 0.0;
  lds_table_clear(tab);
  if (tid < 2) s_tab_used[tid] = 0;
  __syncthreads();

  const MipDesc& md = A.md;
  const bool mip = FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR || FILTER == DR_FILTER_LINEAR_MIPMAP_NEAREST;
  const bool shared_tex = A.tex_stride == 0;
  const int wave = tid >> 6, lane = tid & 63;
  const int tiles = A.ntx * A.nty;

  int it = 0;
  // the tile's (n, ty, tx), advanced by the grid stride each step (scalar
  // adds; a division only when the stride crosses an image)
  const int G = (int)gridDim.x;
  const int Gy = G / A.ntx, Gx = G - Gy * A.ntx;
  int n = (int)blockIdx.x / tiles;
  int ty = ((int)blockIdx.x - n * tiles) / A.ntx;
  int tx = (int)blockIdx.x - n * tiles - ty * A.ntx;
  for (int bt = (int)blockIdx.x; bt < total_tiles; bt += G, ++it) {
    if (it > 0) {
      tx += Gx;
      ty += Gy;
      if (tx >= A.ntx) {
        tx -= A.ntx;
        ++ty;
      }
      if (ty >= A.nty) {
        const int q = ty / A.nty;
        n += q;
        ty -= q * A.nty;
      }
    }
    const int pw = tx * 16 + (lane & 15);  // 16x4 strip per wave, one pixel row per 16 lanes
    const int ph = ty * (4 * kWinWaves) + wave * 4 + (lane >> 4);
    const bool valid = pw < A.Wi && ph < A.Hi;
    const int64_t pix = ((int64_t)n * A.Hi + min(ph, A.Hi - 1)) * A.Wi + min(pw, A.Wi - 1);
    auto level_ptr = [&](int k) -> const float* {
      return k == 0 ? A.tex + n * A.tex_stride
                    : A.pyr + mip_off(md, k) + (shared_tex ? 0 : (int64_t)n * mip_h(md, k) * mip_w(md, k) * CT);
    };
    auto dlevel_ptr = [&](int k) -> float* {
      return k == 0 ? A.d_tex + n * A.tex_stride
                    : A.d_pyr + mip_off(md, k) + (shared_tex ? 0 : (int64_t)n * mip_h(md, k) * mip_w(md, k) * CT);
    };

    // -- per pixel: footprints, gradients of uv / uvDA ------------------------
    float g[CT];
    if constexpr (CT == 4) {  // one vector load
      const float4 q4 = ld_nt4(A.d_out + pix * 4);
      g[0] = q4.x; g[1 % CT] = q4.y; g[2 % CT] = q4.z; g[3 % CT] = q4.w;
    } else {
      load_texel<CT>(A.d_out + pix * CT, CT, g);
    }
#pragma unroll
    for (int c = 0; c < CT; ++c) g[c] = valid ? g[c] : 0.0f;
    const float2 uvp = ld_nt2(A.uv + pix * 2);
    TapSlot q[2];
    float4 da_in = make_float4(0.f, 0.f, 0.f, 0.f), da = da_in;
    float s = 1.0f;
    bool scaled = false;
    // The second level's texels are read only when they count: a nonzero
    // weight, or (trilinear) a LOD inside (0, L-1) at an integer, where
    // d_lod needs its sample.  Magnified and background pixels (LOD clamped
    // to 0) skip them.
    bool need1 = false;
    bool lod0 = true;  // LOD clamped to 0: no d_lod sample is needed
    if (mip) {
      da_in = ld_nt4(A.uv_da + pix * 4);
      if (BIAS) {
        s = bias_scale(A.bias_map, pix, A.scale_bias, A.has_bias != 0);
        scaled = true;
      }
      da = scaled ? make_float4(da_in.x * s, da_in.y * s, da_in.z * s, da_in.w * s) : da_in;
      const Lod ld = mip_lod(da, A.Ht, A.Wt, md.L, FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR);
      q[0].k = ld.k0;
      q[0].scale = 1.0f - ld.frac;
      q[1].k = ld.k1;
      q[1].scale = ld.frac;
      need1 = ld.frac != 0.0f || (FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR && ld.k0 != 0);
      lod0 = FILTER != DR_FILTER_LINEAR_MIPMAP_LINEAR || (ld.k0 == 0 && ld.frac == 0.0f);
    } else {
      q[0].k = 0;
      q[0].scale = 1.0f;
      q[1].k = 0;
      q[1].scale = 0.0f;
    }
    float dfx_total = 0.0f, dfy_total = 0.0f, samp[2] = {0.0f, 0.0f};
#pragma unroll
    for (int li = 0; li < 2; ++li) {
      if (li == 1 && !__ballot(valid && (q[1].scale != 0.0f || need1))) {
        // no lane weights or samples the second level (magnified and
        // background waves): its footprint would only be discarded
        q[1].ix0 = q[1].ix1 = q[1].iy0 = q[1].iy1 = 0;
        q[1].w00 = q[1].w10 = q[1].w01 = q[1].w11 = 0.0f;
        continue;
      }
      const int k = q[li].k, Hk = mip_h(md, k), Wk = mip_w(md, k);
      const Bilin b = bilin(uvp.x, uvp.y, Wk, Hk, BND);
      float w00 = b.w00, w10 = b.w10, w01 = b.w01, w11 = b.w11;
      if (b.ix1 == b.ix0) { w00 += w10; w01 += w11; w10 = 0.0f; w11 = 0.0f; }
      if (b.iy1 == b.iy0) { w00 += w01; w10 += w11; w01 = 0.0f; w11 = 0.0f; }
      q[li].ix0 = b.ix0; q[li].ix1 = b.ix1; q[li].iy0 = b.iy0; q[li].iy1 = b.iy1;
      const bool on = valid && q[li].scale != 0.0f;
      q[li].w00 = on ? w00 : 0.0f; q[li].w10 = on ? w10 : 0.0f;
      q[li].w01 = on ? w01 : 0.0f; q[li].w11 = on ? w11 : 0.0f;
      // A footprint collapsed onto one texel (clamped at a corner; every
      // background pixel) has zero texel differences: its uv gradient is
      // zero and, at LOD 0, its sample is not needed.
      const bool flat = BND != DR_BOUNDARY_ZERO && b.ix0 == b.ix1 && b.iy0 == b.iy1 && lod0;
      if (valid && (li == 0 || need1) && !flat) {
        float dfx, dfy;
        duv_level<uint32_t>(level_ptr(k), Wk, CT, b, g, mip ? q[li].scale : 1.0f, dfx, dfy, samp[li]);
        dfx_total += dfx * (float)Wk;
        dfy_total += dfy * (float)Hk;
      }
    }
    if (valid && A.d_uv)
      st_nt2(A.d_uv + pix * 2, make_float2(dfx_total, dfy_total));
    if (mip && valid && (A.d_uv_da || A.d_bias)) {  // Texture.swift:1011-1102
      const float sx = da.x * (float)A.Wt, sy = da.y * (float)A.Wt;
      const float tx_ = da.z * (float)A.Ht, ty_ = da.w * (float)A.Ht;
      const float Asq = sx * sx + tx_ * tx_;
      const float Bsq = sy * sy + ty_ * ty_;
      const float rho_sq = fmaxf(Asq, Bsq);
      const float lod_raw = 0.5f * log2f(fmaxf(rho_sq, 1e-20f));
      float4 d_eff = make_float4(0.f, 0.f, 0.f, 0.f);
      if (!(lod_raw <= 0.0f || lod_raw >= (float)(md.L - 1))) {
        float d_lod;
        if (FILTER == DR_FILTER_LINEAR_MIPMAP_LINEAR) {
          d_lod = -samp[0] + samp[1];
        } else {
          const int k0 = f2i(floorf(lod_raw));
          const int k1 = min(k0 + 1, md.L - 1);
          float s0 = 0.0f, s1 = 0.0f, u0, u1;
          const Bilin b0 = bilin(uvp.x, uvp.y, mip_w(md, k0), mip_h(md, k0), BND);
          duv_level<uint32_t>(level_ptr(k0), mip_w(md, k0), CT, b0, g, 0.0f, u0, u1, s0);
          const Bilin b1 = bilin(uvp.x, uvp.y, mip_w(md, k1), mip_h(md, k1), BND);
          duv_level<uint32_t>(level_ptr(k1), mip_w(md, k1), CT, b1, g, 0.0f, u0, u1, s1);
          d_lod = -s0 + s1;
        }
        const float ln2 = 0.6931471805599453f;
        // A gradient: the hardware reciprocal (1 ulp) is well inside tolerance.
        const float dlod_drho_sq = __builtin_amdgcn_rcpf(2.0f * rho_sq * ln2);
        const float A_is_max = (Asq >= Bsq) ? 1.0f : 0.0f;
        const float B_is_max = 1.0f - A_is_max;
        d_eff = make_float4(d_lod * dlod_drho_sq * A_is_max * 2.0f * sx * (float)A.Wt,
                            d_lod * dlod_drho_sq * B_is_max * 2.0f * sy * (float)A.Wt,
                            d_lod * dlod_drho_sq * A_is_max * 2.0f * tx_ * (float)A.Ht,
                            d_lod * dlod_drho_sq * B_is_max * 2.0f * ty_ * (float)A.Ht);
      }
      if (A.d_uv_da) {
        const float4 o = scaled ? make_float4(d_eff.x * s, d_eff.y * s, d_eff.z * s, d_eff.w * s) : d_eff;
        st_nt4(A.d_uv_da + pix * 4, o);
      }
      if (BIAS && A.d_bias && A.bias_map) {
        const float gm = d_eff.x * da_in.x + d_eff.y * da_in.y + d_eff.z * da_in.z + d_eff.w * da_in.w;
        A.d_bias[pix] = gm * s * 0.6931471805599453f;
      }
    }

    // -- hot footprint of slot 0: groups on one texel go to the accumulator
    bool hot = false;
    {
      const bool on0 = q[0].w00 != 0.0f || q[0].w10 != 0.0f || q[0].w01 != 0.0f || q[0].w11 != 0.0f;
      const int Wk = mip_w(md, q[0].k);
      const uint64_t key = ((uint64_t)q[0].k << 48) | (uint64_t)((int64_t)q[0].iy0 * Wk + q[0].ix0);
      const uint32_t key2 = ((uint32_t)(q[0].ix1 - q[0].ix0) << 16) ^ (uint32_t)(q[0].iy1 - q[0].iy0);
      // flat footprints only (all the weight on one texel: every background
      // pixel), in groups of any size: a few background pixels kept out of
      // the windows keep a tile that mixes them with the object from boxes
      // spanning both, which the windows cannot hold (their taps then went to
      // the hash table: 0.299 -> 0.294 ms at 8 x 1024^2); other footprints,
      // however many lanes share them, take the windows' run sums
      const bool flat = on0 && q[0].ix0 == q[0].ix1 && q[0].iy0 == q[0].iy1;
      uint64_t pending = __ballot(flat);
#pragma unroll 1
      for (int probe = 0; probe < 2 && pending; ++probe) {
        const int leader = probe_leader(pending, probe);  // wave-uniform: readlane
        const uint64_t lkey = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key >> 32), leader) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, leader);
        const uint32_t lkey2 = (uint32_t)__builtin_amdgcn_readlane((int)key2, leader);
        const bool same = flat && !hot && key == lkey && key2 == lkey2;
        const uint64_t members = __ballot(same);
        pending &= ~members;
        const int lk = __builtin_amdgcn_readlane(q[0].k, leader);
        float* base = dlevel_ptr(lk);
        const int lW = mip_w(md, lk);
        float* lp[4];
        const int lix0 = __builtin_amdgcn_readlane(q[0].ix0, leader);
        const int lix1 = __builtin_amdgcn_readlane(q[0].ix1, leader);
        const int liy0 = __builtin_amdgcn_readlane(q[0].iy0, leader);
        const int liy1 = __builtin_amdgcn_readlane(q[0].iy1, leader);
        lp[0] = base + ((int64_t)liy0 * lW + lix0) * CT;
        lp[1] = base + ((int64_t)liy0 * lW + lix1) * CT;
        lp[2] = base + ((int64_t)liy1 * lW + lix0) * CT;
        lp[3] = base + ((int64_t)liy1 * lW + lix1) * CT;
        const bool hit = acc.on && acc.p[0] == lp[0] && acc.p[1] == lp[1] && acc.p[2] == lp[2] &&
                         acc.p[3] == lp[3];
        if (!hit) {
          acc_flush(acc);
#pragma unroll
          for (int t = 0; t < 4; ++t) acc.p[t] = (float*)uni((uint64_t)lp[t]);
          acc.v = 0.0f;
          acc.on = true;
        }
        // all the weight is on tap 0 (one texel): four sums, one per channel
        float x[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          x[c] = (c < CT && same) ? q[0].w00 * (g[c < CT ? c : 0] * q[0].scale) : 0.0f;
        const float z = wave_sum4(x);  // lane l: total of value l & 3
        const float zc = __shfl(z, (lane >> 2) & 3, kWave);
        if (lane < 4 * CT && (lane & 3) == 0) acc.v += zc;  // lane 4c: channel c, tap 0
        if (same) hot = true;
      }
    }

    // -- per wave: the levels in use and the box on each; the block's windows
    //    cover every level any wave uses ------------------------------------
    const bool use0 = !hot && (q[0].w00 != 0.0f || q[0].w10 != 0.0f || q[0].w01 != 0.0f || q[0].w11 != 0.0f);
    const bool use1 = q[1].w00 != 0.0f || q[1].w10 != 0.0f || q[1].w01 != 0.0f || q[1].w11 != 0.0f;
    const int par = it & 1;
    {
      const int lm = wave_or((use0 ? 1 << q[0].k : 0) | (use1 ? 1 << q[1].k : 0));
#pragma unroll 1
      for (int rem = lm; rem != 0; rem &= rem - 1) {  // uniform: one level at a time
        const int L = __builtin_ctz(rem);
        // texel coordinates fit in 16 bits (window path needs sizes <= 32767):
        // (x0, -x1) and (y0, -y1) are reduced as packed 16-bit minima
        int x0 = 32767, x1 = -32767, y0 = 32767, y1 = -32767;
#pragma unroll
        for (int li = 0; li < 2; ++li) {
          const bool u = li == 0 ? use0 : use1;
          if (!u || q[li].k != L) continue;
          int a0, a1, b0, b1;
          slot_box(q[li], a0, a1, b0, b1);
          x0 = min(x0, a0); x1 = max(x1, a1); y0 = min(y0, b0); y1 = max(y1, b1);
        }
        const int px = wave_min_pk16(pack16(x0, -x1));
        const int py = wave_min_pk16(pack16(y0, -y1));
        if (lane == 0) s_lbox[wave][L] = make_int2(px, py);
      }
      if (lane == 0) s_lmask[wave] = lm;
    }
    __syncthreads();
    if (tid == 0) s_tab_used[par ^ 1] = 0;  // read by every thread before the last barrier
    // Level L's window, in lane L of each 16-lane row: the union of the
    // waves' boxes on L and its place in the pool (levels in ascending
    // order; a box larger than the pool is left out).  A lane then takes
    // its slots' windows from the lanes of their levels.
    const int4 wm = *reinterpret_cast<const int4*>(s_lmask);
    const int lmask = __builtin_amdgcn_readfirstlane(wm.x | wm.y | wm.z | wm.w);
    // (x0 | y0 << 16) and (width | height << 10 | (pool offset + 1) << 20),
    // offset + 1 = 0 for no window (a box in the pool has at most 768 texels,
    // so each of its sides and its offset fit in 10 bits)
    int wxy, wsz;
    {
      const int L = lane & 15;
      int px = pack16(32767, 32767), py = px;
#pragma unroll
      for (int v = 0; v < kWinWaves; ++v) {
        const int mv = v == 0 ? wm.x : v == 1 ? wm.y : v == 2 ? wm.z : wm.w;
        if ((mv >> L) & 1) {
          const int2 b = s_lbox[v][L];
          px = pk16_min(px, b.x);
          py = pk16_min(py, b.y);
        }
      }
      const int x0 = unpack16_lo(px), x1 = -unpack16_hi(px);
      const int y0 = unpack16_lo(py), y1 = -unpack16_hi(py);
      const bool present = L < kMaxLevels && ((lmask >> L) & 1) && x1 >= x0 && y1 >= y0;
      const int area = present ? (x1 - x0 + 1) * (y1 - y0 + 1) : 0;
      const int fit = area <= kWinTexels ? area : 0;
      // inclusive prefix sum of the fitting areas along the row
      int incl = fit;
      int t = dpp_shift<0x111>(incl);
      incl += t;
      t = dpp_shift<0x112>(incl);
      incl += t;
      t = dpp_shift<0x114>(incl);
      incl += t;
      t = dpp_shift<0x118>(incl);
      incl += t;
      const bool usable = present && area == fit && incl <= kWinTexels;
      static_assert(kWinTexels < 1024, "window sides and offsets are 10-bit fields");
      wxy = x0 | (y0 << 16);
      wsz = usable ? (x1 - x0 + 1) | ((y1 - y0 + 1) << 10) | ((incl - fit + 1) << 20) : 0;
    }

    // -- accumulate: runs of one footprint along a pixel row are summed
    //    first (lanes of one LDS atomic on one address are serialised), the
    //    run's last lane adds the totals ----------------------------------------
#pragma unroll
    for (int li = 0; li < 2; ++li) {
      const bool u = li == 0 ? use0 : use1;
      if (__ballot(u) == 0) continue;  // no lane uses this slot (uniform)
      const int k = q[li].k;
      // the window of level k (every lane executes the permutes)
      const int sxy = __builtin_amdgcn_ds_bpermute(k << 2, wxy);
      const int ssz = __builtin_amdgcn_ds_bpermute(k << 2, wsz);
      const float sc = mip ? q[li].scale : 1.0f;
      // level and the four texel coordinates (each < 32767 on the window
      // path) fix the taps; an unused slot gets a key no footprint has
      const uint64_t key =
          !u ? (0x7FFFull << 45) | (uint64_t)lane
             : ((uint64_t)k << 60) | ((uint64_t)q[li].ix0 << 45) | ((uint64_t)q[li].ix1 << 30) |
                   ((uint64_t)q[li].iy0 << 15) | (uint64_t)q[li].iy1;
      const RowRun run = row_run(key);
      const int maxlen = wave_max(run.li - run.s + 1);  // longest run in the wave
      const bool adds = u && run.tail;
      const bool in_win = ssz != 0;
      // the 16 values (tap-major) of the footprint, then one segmented scan
      // over all of them
      const float wt[4] = {q[li].w00, q[li].w10, q[li].w01, q[li].w11};
      float gs[CT];
#pragma unroll
      for (int c = 0; c < CT; ++c) gs[c] = !u ? 0.0f : g[c] * sc;
      float v[4 * CT];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < CT; ++c) v[t * CT + c] = wt[t] * gs[c];
      row_run_scan_n(run, v, maxlen);
      if (adds && in_win) {
        // window indices of the four taps.  The box holds every tap with a
        // nonzero weight in some lane of the run; a tap whose weight is zero
        // in all of them (a texel column or row with zero weight, outside
        // the image for the zero boundary) may lie outside it, and its
        // coordinates are clamped into the box, where it adds 0.
        const int wx = sxy & 0xffff, wy = sxy >> 16;
        const int ww = ssz & 0x3ff, wh = (ssz >> 10) & 0x3ff, sbase = (ssz >> 20) - 1;
        const int cx0 = min(max(q[li].ix0 - wx, 0), ww - 1);
        const int cx1 = min(max(q[li].ix1 - wx, 0), ww - 1);
        const int r0 = sbase + min(max(q[li].iy0 - wy, 0), wh - 1) * ww;
        const int r1 = sbase + min(max(q[li].iy1 - wy, 0), wh - 1) * ww;
        const int o[4] = {r0 + cx0, r0 + cx1, r1 + cx0, r1 + cx1};  // < sbase + area
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int c = 0; c < CT; ++c)
            atomicAdd(win + c * kWinTexels + o[t], (double)v[t * CT + c]);
      }
      if (adds && !in_win) {  // boxes that the pool could not hold
        s_tab_used[par] = 1;
        float* base = dlevel_ptr(k);
        const int Wk = mip_w(md, k);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int tx_ = (t & 1) ? q[li].ix1 : q[li].ix0;
          const int ty_ = (t & 2) ? q[li].iy1 : q[li].iy0;
          lds_table_add(tab, base + ((int64_t)ty_ * Wk + tx_) * CT, &v[t * CT]);
        }
      }
    }
    __syncthreads();

    // -- write the windows out, row by row -----------------------------------
#pragma unroll 1
    for (int rem = lmask; rem != 0; rem &= rem - 1) {  // uniform
      const int k = __builtin_ctz(rem);
      const int sz = __builtin_amdgcn_readlane(wsz, k);
      if (sz == 0) continue;
      const int xy = __builtin_amdgcn_readlane(wxy, k);
      const int bx0 = xy & 0xffff, by0 = xy >> 16, bw = sz & 0x3ff, bh = (sz >> 10) & 0x3ff;
      const int base_k = (sz >> 20) - 1;
      float* base = dlevel_ptr(k);
      const int Wk = mip_w(md, k);
      const int row = bw * CT;
      const int total = row * bh;
      double* wb = win + base_k;
      // consecutive lanes take consecutive channels of a texel, so the
      // device atomics of a row share cache lines; (r, cpos) of element i
      // advance by a uniform step instead of a division per element
      const int dr = kWinThreads / row, dc = kWinThreads - dr * row;
      int r = tid / row, cpos = tid - r * row;
      for (int i = tid; i < total; i += kWinThreads) {
        const int tx = cpos / CT, c = cpos - tx * CT;
        double* e = wb + c * kWinTexels + r * bw + tx;
        const double v = *e;
        if (v != 0.0) {
          unsafeAtomicAdd(base + ((int64_t)(by0 + r) * Wk + bx0) * CT + cpos, (float)v);
          *e = 0.0;
        }
        r += dr;
        cpos += dc;
        if (cpos >= row) {
          cpos -= row;
          ++r;
        }
      }
    }
    if (s_tab_used[par]) lds_table_flush(tab);  // uniform; contains a barrier
  }
  acc_flush(acc);
}

// Texture.swift:156: level k = 2x2 mean of level k-1.
__global__ void __launch_bounds__(256) k_mip_down(const float* __restrict__ src,
                                                  float* __restrict__ dst, int Nt, int h, int w,
                                                  int C) {
  const int h2 = h / 2, w2 = w / 2;
  const int64_t total = (int64_t)Nt * h2 * w2 * C;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i % C);
  int64_t r = i / C;
  const int x = (int)(r % w2);
  r /= w2;
  const int y = (int)(r % h2);
  const int n = (int)(r / h2);
  const float* s = src + (int64_t)n * h * w * C;
  const float a = s[((int64_t)(2 * y) * w + 2 * x) * C + c];
  const float b = s[((int64_t)(2 * y) * w + 2 * x + 1) * C + c];
  const float d = s[((int64_t)(2 * y + 1) * w + 2 * x) * C + c];
  const float e = s[((int64_t)(2 * y + 1) * w + 2 * x + 1) * C + c];
  dst[i] = (((a + b) + d) + e) * 0.25f;
}

// Builds up to five levels at once: each workgroup reduces a 2^m x 2^m
// block of level s through levels s+1..s+m in LDS (m <= 5; the sizes of
// levels s..s+m-1 are even, so the blocks tile level s exactly).  Same 2x2
// sums as k_mip_down, in the same order.
constexpr int kMipMaxC = 4;

__global__ void __launch_bounds__(256) k_mip_block(const float* __restrict__ src,
                                                   float* __restrict__ pyr, MipDesc md, int s,
                                                   int m, int Nt, int C) {
  __shared__ float buf[2][256 * kMipMaxC];
  const int bs = 1 << m;  // source block edge
  const int Ws = md.w[s];
  const int nbx = Ws / bs;
  const int bx = (int)blockIdx.x % nbx, by = (int)blockIdx.x / nbx;
  const int n = (int)blockIdx.y;
  const float* lvl = src + (int64_t)n * md.h[s] * Ws * C;
  int cur = 0;
  for (int j = 1; j <= m; ++j) {
    const int e = bs >> j;  // output edge at this step
    const int k = s + j;
    const int Wk = md.w[k];
    float* dst = pyr + md.off[k] + (int64_t)n * md.h[k] * Wk * C;
    for (int t = threadIdx.x; t < e * e * C; t += blockDim.x) {
      const int c = t % C, q = t / C;
      const int x = q % e, y = q / e;
      float a, b, d, f;
      if (j == 1) {
        const int sx = bx * bs + 2 * x, sy = by * bs + 2 * y;
        a = lvl[((int64_t)sy * Ws + sx) * C + c];
        b = lvl[((int64_t)sy * Ws + sx + 1) * C + c];
        d = lvl[((int64_t)(sy + 1) * Ws + sx) * C + c];
        f = lvl[((int64_t)(sy + 1) * Ws + sx + 1) * C + c];
      } else {
        const int pe = 2 * e;
        const float* pb = buf[cur ^ 1];
        a = pb[((2 * y) * pe + 2 * x) * C + c];
        b = pb[((2 * y) * pe + 2 * x + 1) * C + c];
        d = pb[((2 * y + 1) * pe + 2 * x) * C + c];
        f = pb[((2 * y + 1) * pe + 2 * x + 1) * C + c];
      }
      const float v = (((a + b) + d) + f) * 0.25f;
      buf[cur][(y * e + x) * C + c] = v;
      const int ox = bx * e + x, oy = by * e + y;
      dst[((int64_t)oy * Wk + ox) * C + c] = v;
    }
    __syncthreads();
    cur ^= 1;
  }
}

// k_mip_block for four channels: one output texel per thread, 16-byte
// loads and stores, the same sums in the same order.
__global__ void __launch_bounds__(256) k_mip_block_c4(const float* __restrict__ src,
                                                      float* __restrict__ pyr, MipDesc md, int s,
                                                      int m) {
  __shared__ float4 buf[2][256];
  const int bs = 1 << m;  // source block edge
  const int Ws = md.w[s];
  const int nbx = Ws / bs;
  const int bx = (int)blockIdx.x % nbx, by = (int)blockIdx.x / nbx;
  const int n = (int)blockIdx.y;
  const float4* lvl = reinterpret_cast<const float4*>(src) + (int64_t)n * md.h[s] * Ws;
  auto mean4 = [](float4 a, float4 b, float4 d, float4 f) {
    return make_float4((((a.x + b.x) + d.x) + f.x) * 0.25f, (((a.y + b.y) + d.y) + f.y) * 0.25f,
                       (((a.z + b.z) + d.z) + f.z) * 0.25f, (((a.w + b.w) + d.w) + f.w) * 0.25f);
  };
  int cur = 0;
  for (int j = 1; j <= m; ++j) {
    const int e = bs >> j;  // output edge at this step
    const int k = s + j;
    const int Wk = md.w[k];
    float4* dst = reinterpret_cast<float4*>(pyr + md.off[k]) + (int64_t)n * md.h[k] * Wk;
    for (int t = threadIdx.x; t < e * e; t += blockDim.x) {
      const int x = t % e, y = t / e;
      float4 v;
      if (j == 1) {
        const int sx = bx * bs + 2 * x, sy = by * bs + 2 * y;
        v = mean4(lvl[(int64_t)sy * Ws + sx], lvl[(int64_t)sy * Ws + sx + 1],
                  lvl[(int64_t)(sy + 1) * Ws + sx], lvl[(int64_t)(sy + 1) * Ws + sx + 1]);
      } else {
        const int pe = 2 * e;
        const float4* pb = buf[cur ^ 1];
        v = mean4(pb[(2 * y) * pe + 2 * x], pb[(2 * y) * pe + 2 * x + 1],
                  pb[(2 * y + 1) * pe + 2 * x], pb[(2 * y + 1) * pe + 2 * x + 1]);
      }
      buf[cur][y * e + x] = v;
      dst[(int64_t)(by * e + y) * Wk + bx * e + x] = v;
    }
    __syncthreads();
    cur ^= 1;
  }
}

// Backward of the pyramid (MLX autodiff of concatenate + mean): level k's
// total cotangent is its own gradient plus 1/4 of level k+1's total,
// accumulated from the coarsest level down; level 0's total is added to
// d_tex (which already holds level 0's own gradient).
__global__ void __launch_bounds__(256) k_mip_collapse(const float* __restrict__ d_pyr, MipDesc md,
                                                      int C, int bpr, float* __restrict__ d_tex) {
  // one thread per texel of level 0: block = 256 texels of one row
  const int64_t row = (int64_t)blockIdx.x / bpr;  // n * H + y
  const int x = (int)((int64_t)blockIdx.x - row * bpr) * 256 + (int)threadIdx.x;
  if (x >= md.w[0] || md.L < 2) return;
  const int y = (int)(row % md.h[0]);
  const int n = (int)(row / md.h[0]);
  const int kL = md.L - 1;
  float* dt = d_tex + (row * md.w[0] + x) * C;
  for (int c = 0; c < C; ++c) {
    auto at = [&](int k) {
      return d_pyr[md.off[k] + (((int64_t)n * md.h[k] + (y >> k)) * md.w[k] + (x >> k)) * C + c];
    };
    float acc = at(kL);
    for (int k = kL - 1; k >= 1; --k) acc = at(k) + acc * 0.25f;
    dt[c] = dt[c] + acc * 0.25f;
  }
}

// The same collapse for C = 4 in two passes with texel vectors: level 1's
// totals first, in place (one thread per level-1 texel walks its chain of
// ancestors, the same sums in the same order), then level 0 adds a quarter
// of its parent's total.
__global__ void __launch_bounds__(256) k_mip_collapse1_c4(float* __restrict__ d_pyr, MipDesc md,
                                                          int64_t n1) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n1) return;
  const int W1 = md.w[1], H1 = md.h[1];
  const int64_t r = i % ((int64_t)H1 * W1);
  const int n = (int)(i / ((int64_t)H1 * W1));
  const int y = (int)(r / W1), x = (int)(r - (int64_t)(r / W1) * W1);
  const int kL = md.L - 1;
  auto at = [&](int k) {
    const int sh = k - 1;
    return *reinterpret_cast<const float4*>(
        d_pyr + md.off[k] + (((int64_t)n * md.h[k] + (y >> sh)) * md.w[k] + (x >> sh)) * 4);
  };
  float4 acc = at(kL);
  for (int k = kL - 1; k >= 1; --k) {
    const float4 o = at(k);
    acc = make_float4(o.x + acc.x * 0.25f, o.y + acc.y * 0.25f, o.z + acc.z * 0.25f,
                      o.w + acc.w * 0.25f);
  }
  *reinterpret_cast<float4*>(d_pyr + md.off[1] + i * 4) = acc;
}

__global__ void __launch_bounds__(256) k_mip_collapse0_c4(const float* __restrict__ d_pyr,
                                                          MipDesc md, int64_t n0,
                                                          float* __restrict__ d_tex) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n0) return;
  const int W = md.w[0], H = md.h[0];
  const int64_t r = i % ((int64_t)H * W);
  const int n = (int)(i / ((int64_t)H * W));
  const int y = (int)(r / W), x = (int)(r - (int64_t)(r / W) * W);
  const float4 t = *reinterpret_cast<const float4*>(
      d_pyr + md.off[1] + (((int64_t)n * md.h[1] + (y >> 1)) * md.w[1] + (x >> 1)) * 4);
  float4* dp = reinterpret_cast<float4*>(d_tex + i * 4);
  const float4 d = *dp;
  *dp = make_float4(d.x + t.x * 0.25f, d.y + t.y * 0.25f, d.z + t.z * 0.25f, d.w + t.w * 0.25f);
}

template <int FILTER, int CT, int BND, bool BIAS>
hipError_t launch_tex_bwd_win_bb(const TexBwdArgs& args, int total_tiles, hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_tex_bwd_win<FILTER, CT, BND, BIAS>,
                                                     kWinThreads, 0) != hipSuccess ||
        b <= 0)
      b = 2;
    per_cu = b;
  }
  const int64_t resident = (int64_t)device_cu_count() * per_cu;
  const unsigned grid = (unsigned)(total_tiles < resident ? total_tiles : resident);
  hipLaunchKernelGGL((k_tex_bwd_win<FILTER, CT, BND, BIAS>), dim3(grid), dim3(kWinThreads), 0,
                     stream, args, total_tiles);
  return hipGetLastError();
}

template <int FILTER, int CT, int BND>
hipError_t launch_tex_bwd_win_b(const TexBwdArgs& args, int total_tiles, hipStream_t stream) {
  if (args.bias_map || args.has_bias)
    return launch_tex_bwd_win_bb<FILTER, CT, BND, true>(args, total_tiles, stream);
  return launch_tex_bwd_win_bb<FILTER, CT, BND, false>(args, total_tiles, stream);
}

// The boundary mode is a compile-time constant of the windowed kernel (the
// clamp and wrap footprints need no out-of-range masks).
template <int FILTER, int CT>
hipError_t launch_tex_bwd_win(const TexBwdArgs& args, int total_tiles, hipStream_t stream) {
  if (args.boundary == DR_BOUNDARY_CLAMP)
    return launch_tex_bwd_win_b<FILTER, CT, DR_BOUNDARY_CLAMP>(args, total_tiles, stream);
  if (args.boundary == DR_BOUNDARY_WRAP)
    return launch_tex_bwd_win_b<FILTER, CT, DR_BOUNDARY_WRAP>(args, total_tiles, stream);
  return launch_tex_bwd_win_b<FILTER, CT, DR_BOUNDARY_ZERO>(args, total_tiles, stream);
}

// Launches the persistent backward with as many workgroups as fit on the
// device at once.
template <int FILTER, bool CUBE, int CT>
hipError_t launch_tex_bwd(const TexBwdArgs& args, int total_tiles, hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_tex_bwd<FILTER, CUBE, CT>, 256, 0) !=
            hipSuccess ||
        b <= 0)
      b = 2;
    per_cu = b;
  }
  const int64_t resident = (int64_t)device_cu_count() * per_cu;
  const unsigned grid = (unsigned)(total_tiles < resident ? total_tiles : resident);
  hipLaunchKernelGGL((k_tex_bwd<FILTER, CUBE, CT>), dim3(grid), dim3(256), 0, stream, args,
                     total_tiles);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// cube maps with mip filters, and the direction gradient
// ---------------------------------------------------------------------------
// An extension of the reference, which samples cube maps bilinearly only
// (Texture.swift:75-76) and returns a zero direction gradient (:196-198).
// Faces and face (u, v) as :620-635; the face (u, v) screen derivatives
// from the direction's (dx/dX, dx/dY, dy/dX, dy/dY, dz/dX, dz/dY) by the
// chain rule through u = (sc/ma + 1)/2, v = (tc/ma + 1)/2 with the face
// fixed; then the 2D LOD, clamped bilinear taps and two-rounding trilinear
// blend of :764-863 on the chosen face of each level.  The backward adds
// the direction gradient through the sample position and, for mip
// filters, through the LOD; the pyramid is every face's 2x2 box pyramid.

struct CubeSel {
  int face, as, at, am;  // axes of sc, tc, ma
  float ss, ts, ms;      // their signs
  float sc, tc, ma;
};

__device__ __forceinline__ CubeSel cube_select(float x, float y, float z) {
  CubeSel s;
  const float ax = fabsf(x), ay = fabsf(y), az = fabsf(z);
  if (ax >= ay && ax >= az) {
    s.am = 0; s.ms = x > 0.0f ? 1.0f : -1.0f; s.ma = ax;
    s.at = 1; s.ts = -1.0f; s.tc = -y;
    s.as = 2;
    if (x > 0.0f) { s.face = 0; s.ss = -1.0f; s.sc = -z; }
    else          { s.face = 1; s.ss = 1.0f;  s.sc = z; }
  } else if (ay >= az) {
    s.am = 1; s.ms = y > 0.0f ? 1.0f : -1.0f; s.ma = ay;
    s.as = 0; s.ss = 1.0f; s.sc = x;
    s.at = 2;
    if (y > 0.0f) { s.face = 2; s.ts = 1.0f;  s.tc = z; }
    else          { s.face = 3; s.ts = -1.0f; s.tc = -z; }
  } else {
    s.am = 2; s.ms = z > 0.0f ? 1.0f : -1.0f; s.ma = az;
    s.at = 1; s.ts = -1.0f; s.tc = -y;
    s.as = 0;
    if (z > 0.0f) { s.face = 4; s.ss = 1.0f;  s.sc = x; }
    else          { s.face = 5; s.ss = -1.0f; s.sc = -x; }
  }
  return s;
}

__device__ __forceinline__ float pick3(int a, float v0, float v1, float v2) {
  return a == 0 ? v0 : (a == 1 ? v1 : v2);
}

// The direction's screen derivatives as (d/dX, d/dY) per axis.
struct DirDA {
  float x[3], y[3];
};

// Face (u_X, u_Y, v_X, v_Y) from the direction's derivatives.
__device__ __forceinline__ float4 cube_face_da(const CubeSel& s, const DirDA& d) {
  const float inv = 0.5f / (s.ma * s.ma);
  const float sX = s.ss * pick3(s.as, d.x[0], d.x[1], d.x[2]);
  const float sY = s.ss * pick3(s.as, d.y[0], d.y[1], d.y[2]);
  const float tX = s.ts * pick3(s.at, d.x[0], d.x[1], d.x[2]);
  const float tY = s.ts * pick3(s.at, d.y[0], d.y[1], d.y[2]);
  const float mX = s.ms * pick3(s.am, d.x[0], d.x[1], d.x[2]);
  const float mY = s.ms * pick3(s.am, d.y[0], d.y[1], d.y[2]);
  return make_float4((sX * s.ma - s.sc * mX) * inv, (sY * s.ma - s.sc * mY) * inv,
                     (tX * s.ma - s.tc * mX) * inv, (tY * s.ma - s.tc * mY) * inv);
}

struct CubeArgs {
  const float* tex;  // [Nt, 6, Ht, Wt, C]
  const float* pyr;  // levels 1..L-1 of the Nt*6 faces
  MipDesc md;        // built for Nt*6 textures
  int64_t tex_stride;  // 6*Ht*Wt*C, or 0 for one shared cube map
  int Ht, Wt, C;
  const float* dir;      // [N, Hi, Wi, 3]
  const float* dir_da;   // [N, Hi, Wi, 6] (mip modes)
  const float* bias_map;
  float scale_bias;
  int has_bias;
  int64_t P;
  int HWi;
  int Wi;      // image width (the forward's 16x16 tiles)
  float* out;  // forward
  // backward
  const float* d_out;
  float* d_tex;
  float* d_pyr;
  float* d_dir;     // NULL: not requested
  int dir_grad;     // 0: d_dir is written as zeros (the reference's value)
  float* d_dir_da;
  float* d_bias;
};

__device__ __forceinline__ const float* cube_level(const CubeArgs& A, int n, int face, int k,
                                                   int Hk, int Wk) {
  if (k == 0) return A.tex + n * A.tex_stride + (int64_t)face * A.Ht * A.Wt * A.C;
  const int64_t nt = A.tex_stride ? n : 0;
  return A.pyr + mip_off(A.md, k) + (nt * 6 + face) * (int64_t)Hk * Wk * A.C;
}

__device__ __forceinline__ float* cube_dlevel(const CubeArgs& A, int n, int face, int k, int Hk,
                                              int Wk) {
  if (k == 0) return A.d_tex + n * A.tex_stride + (int64_t)face * A.Ht * A.Wt * A.C;
  const int64_t nt = A.tex_stride ? n : 0;
  return A.d_pyr + mip_off(A.md, k) + (nt * 6 + face) * (int64_t)Hk * Wk * A.C;
}

// Per-pixel set-up shared by both passes.
struct CubePx {
  CubeSel s;
  float u, v, inv_ma, bscale;
  bool scaled;
  DirDA dd, dd_in;  // folded (dd) and as given (dd_in)
  float4 da;        // face derivatives
  Lod ld;
};

template <int MODE>
__device__ __forceinline__ CubePx cube_px(const CubeArgs& A, int64_t pix) {
  CubePx p;
  // the direction, its derivatives and the bias are loaded together, ahead
  // of the face selection's branches (one round trip instead of two)
  const float* dp = A.dir + pix * 3;
  const float x = dp[0], y = dp[1], z = dp[2];
  float2 a = make_float2(0.f, 0.f), b = a, c = a;
  float bm = 0.0f;
  if (MODE > 0) {
    const float2* q = reinterpret_cast<const float2*>(A.dir_da + pix * 6);
    a = q[0];
    b = q[1];
    c = q[2];
    if (A.bias_map) bm = A.bias_map[pix];
  }
  p.s = cube_select(x, y, z);
  p.inv_ma = 1.0f / p.s.ma;
  p.u = (p.s.sc * p.inv_ma + 1.0f) * 0.5f;
  p.v = (p.s.tc * p.inv_ma + 1.0f) * 0.5f;
  p.ld.k0 = p.ld.k1 = 0;
  p.ld.frac = 0.0f;
  p.scaled = false;
  p.bscale = 1.0f;
  if (MODE > 0) {
    p.dd_in.x[0] = a.x; p.dd_in.y[0] = a.y;
    p.dd_in.x[1] = b.x; p.dd_in.y[1] = b.y;
    p.dd_in.x[2] = c.x; p.dd_in.y[2] = c.y;
    p.dd = p.dd_in;
    p.scaled = A.bias_map != nullptr || A.has_bias;
    if (p.scaled) {
      p.bscale = A.bias_map ? (A.has_bias ? exp2f(bm) * A.scale_bias : exp2f(bm)) : A.scale_bias;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        p.dd.x[i] = p.dd_in.x[i] * p.bscale;
        p.dd.y[i] = p.dd_in.y[i] * p.bscale;
      }
    }
    p.da = cube_face_da(p.s, p.dd);
    p.ld = mip_lod(p.da, A.Ht, A.Wt, A.md.L, MODE == 2);
  }
  return p;
}

// MODE: 1 = mip-nearest, 2 = trilinear (bilinear cube sampling is k_tex_fwd).
// One 16x16 pixel tile per workgroup (a 16x4 strip per wave), so a wave's
// texel gathers share cache lines along both image axes.
template <int MODE, int CT>
__global__ void __launch_bounds__(256) k_cube_fwd(CubeArgs A) {
  const int Wi = A.Wi, Hi = A.HWi / Wi;
  const int ntx = (Wi + 15) >> 4, tiles = ntx * ((Hi + 15) >> 4);
  const int b = (int)blockIdx.x, n = b / tiles, tile = b - n * tiles;
  const int ty = tile / ntx, tx = tile - ty * ntx;
  const int ph = ty * 16 + ((int)threadIdx.x >> 4), pw = tx * 16 + ((int)threadIdx.x & 15);
  if (ph >= Hi || pw >= Wi) return;
  const int64_t pix = ((int64_t)n * Hi + ph) * Wi + pw;
  const int C = dimC<CT>(A.C);
  const CubePx p = cube_px<MODE>(A, pix);
  float* op = A.out + pix * C;
  float acc[kMaxC];
  for (int li = 0; li < 2; ++li) {
    const int k = li == 0 ? p.ld.k0 : p.ld.k1;
    const int Hk = mip_h(A.md, k), Wk = mip_w(A.md, k);
    const float* lv = cube_level(A, n, p.s.face, k, Hk, Wk);
    const Bilin b = bilin(p.u, p.v, Wk, Hk, DR_BOUNDARY_CLAMP);
    const float wgt = li == 0 ? (1.0f - p.ld.frac) : p.ld.frac;
    if constexpr (CT > 0) {
      float t00[kMaxC], t10[kMaxC], t01[kMaxC], t11[kMaxC];
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix0) * C, C, t00);
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix1) * C, C, t10);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix0) * C, C, t01);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix1) * C, C, t11);
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const float sample = b.w00 * t00[c] + b.w10 * t10[c] + b.w01 * t01[c] + b.w11 * t11[c];
        acc[c] = li == 0 ? wgt * sample : acc[c] + wgt * sample;
      }
    } else {
      for (int c = 0; c < C; ++c) {
        const float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
        const float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
        const float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
        const float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
        const float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
        op[c] = li == 0 ? wgt * sample : op[c] + wgt * sample;
      }
    }
  }
  if constexpr (CT > 0) {
#pragma unroll
    for (int c = 0; c < CT; ++c) op[c] = acc[c];
  }
}

// MODE: 0 = bilinear (only with the direction gradient), 1 / 2 as above.
// One pixel of the backward; every lane of the wave calls it (the scatter
// groups lanes across the wave), `valid` marks the lanes with a pixel.
template <int MODE, int CT>
__device__ __forceinline__ void cube_bwd_px(const CubeArgs& A, int64_t pix, bool valid, int n,
                                            FootAcc<(CT > 0 ? CT : 1)>& acc0,
                                            CubeTable<CT>& tab) {
  const int C = dimC<CT>(A.C);
  const float* gp = A.d_out + pix * C;
  float g[CT > 0 ? CT : 1];
  if constexpr (CT > 0) load_texel<CT>(gp, C, g);  // pix is clamped into the image
  const CubePx p = cube_px<MODE>(A, pix);
  if constexpr (CT > 0) {
#pragma unroll
    for (int c = 0; c < CT; ++c) g[c] = valid ? g[c] : 0.0f;
  }
  const float* gsrc = CT > 0 ? g : gp;  // run-time C reads d_out directly
  const CubeSel& s = p.s;
  // Trilinear with the LOD inside (0, L-1): the LOD gradient needs both
  // levels' samples (:1011-1102), and those levels are the two the filter
  // blends (the same LOD expression), so the texels read here serve it too.
  float lod_raw = 0.0f, Asq = 0.0f, Bsq = 0.0f;
  bool lod_in = false;
  if (MODE > 0) {
    const float sx = p.da.x * (float)A.Wt, sy = p.da.y * (float)A.Wt;
    const float tx_ = p.da.z * (float)A.Ht, ty_ = p.da.w * (float)A.Ht;
    Asq = sx * sx + tx_ * tx_;
    Bsq = sy * sy + ty_ * ty_;
    lod_raw = 0.5f * log2f(fmaxf(fmaxf(Asq, Bsq), 1e-20f));
    lod_in = lod_raw > 0.0f && lod_raw < (float)(A.md.L - 1);
  }
  const bool lod_here = MODE == 2 && valid && lod_in;
  // sample position gradient (:934-999) and the pyramid scatter (:870-932);
  // a level of zero weight adds nothing and is skipped (uniformly per wave)
  float du = 0.0f, dv = 0.0f, d_lod = 0.0f;
  for (int li = 0; li < (MODE == 0 ? 1 : 2); ++li) {
    const int k = li == 0 ? p.ld.k0 : p.ld.k1;
    const float scale = MODE == 0 ? 1.0f : (li == 0 ? (1.0f - p.ld.frac) : p.ld.frac);
    const bool on = valid && scale != 0.0f;
    const bool rd = on || lod_here;  // the texels are read
    if (__ballot(rd) == 0ull) continue;
    const int Hk = mip_h(A.md, k), Wk = mip_w(A.md, k);
    const float* lv = cube_level(A, n, s.face, k, Hk, Wk);
    float* dl = cube_dlevel(A, n, s.face, k, Hk, Wk);
    const Bilin b = bilin(p.u, p.v, Wk, Hk, DR_BOUNDARY_CLAMP);
    if (__ballot(on)) {
      if (li == 0)
        scatter_footprint<CT, true, CubeTable<CT>>(on, dl, Wk, C, b, gsrc, scale, acc0, tab);
      else
        scatter_footprint<CT, false, CubeTable<CT>>(on, dl, Wk, C, b, gsrc, scale, acc0, tab);
    }
    if (!rd) continue;
    const float sign = li == 0 ? -1.0f : 1.0f;
    float dfx = 0.0f, dfy = 0.0f;
    // a texel's channels in one load (CT > 0) rather than one per channel
    // (4096 x 256^2, 6 x 512^2 x 3: 37.7 -> 36.1 ms)
    float q00[kMaxC], q10[kMaxC], q01[kMaxC], q11[kMaxC];
    if constexpr (CT > 0) {
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix0) * C, C, q00);
      load_texel<CT>(lv + ((int64_t)b.iy0 * Wk + b.ix1) * C, C, q10);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix0) * C, C, q01);
      load_texel<CT>(lv + ((int64_t)b.iy1 * Wk + b.ix1) * C, C, q11);
    }
    for (int c = 0; c < C; ++c) {
      const float t00 = CT > 0 ? q00[c] : lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
      const float t10 = CT > 0 ? q10[c] : lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
      const float t01 = CT > 0 ? q01[c] : lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
      const float t11 = CT > 0 ? q11[c] : lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
      const float gs = gsrc[c] * scale;
      dfx += gs * ((1.0f - b.fy) * (t10 - t00) + b.fy * (t11 - t01));
      dfy += gs * ((1.0f - b.fx) * (t01 - t00) + b.fx * (t11 - t10));
      if (lod_here) {
        const float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
        d_lod += sign * sample * gsrc[c];
      }
    }
    du += dfx * (float)Wk;
    dv += dfy * (float)Hk;
  }
  if (!valid) return;
  const float* g_ = gsrc;
  const float inv2 = 0.5f / (s.ma * s.ma);
  // d u / d dir = inv2 * (ss*ma e_as - sc*ms e_am), likewise v; the axes
  // are distinct, so each sum below lands in its own component
  const float g_as = du * (s.ss * s.ma * inv2);
  const float g_at = dv * (s.ts * s.ma * inv2);
  const float g_am = -((du * s.sc + dv * s.tc) * s.ms * inv2);
  float gdd_x[3] = {0.0f, 0.0f, 0.0f}, gdd_y[3] = {0.0f, 0.0f, 0.0f};
  float l_as = 0.0f, l_at = 0.0f, l_am = 0.0f;
  if (MODE > 0) {
    const float sx = p.da.x * (float)A.Wt, sy = p.da.y * (float)A.Wt;
    const float tx_ = p.da.z * (float)A.Ht, ty_ = p.da.w * (float)A.Ht;
    const float rho_sq = fmaxf(Asq, Bsq);
    if (lod_in) {
      if (MODE == 1) {  // mip-nearest: the LOD's two levels are not the one sampled
        const int j0 = f2i(floorf(lod_raw));
        const int j1 = min(j0 + 1, A.md.L - 1);
        for (int li = 0; li < 2; ++li) {
          const int k = li == 0 ? j0 : j1;
          const float sign = li == 0 ? -1.0f : 1.0f;
          const int Hk = mip_h(A.md, k), Wk = mip_w(A.md, k);
          const float* lv = cube_level(A, n, s.face, k, Hk, Wk);
          const Bilin b = bilin(p.u, p.v, Wk, Hk, DR_BOUNDARY_CLAMP);
          for (int c = 0; c < C; ++c) {
            const float t00 = lv[((int64_t)b.iy0 * Wk + b.ix0) * C + c];
            const float t10 = lv[((int64_t)b.iy0 * Wk + b.ix1) * C + c];
            const float t01 = lv[((int64_t)b.iy1 * Wk + b.ix0) * C + c];
            const float t11 = lv[((int64_t)b.iy1 * Wk + b.ix1) * C + c];
            const float sample = b.w00 * t00 + b.w10 * t10 + b.w01 * t01 + b.w11 * t11;
            d_lod += sign * sample * g_[c];
          }
        }
      }
      const float ln2 = 0.6931471805599453f;
      const float dlod_drho_sq = 1.0f / (2.0f * rho_sq * ln2);
      const float A_is_max = (Asq >= Bsq) ? 1.0f : 0.0f;
      const float B_is_max = 1.0f - A_is_max;
      const float duX = d_lod * dlod_drho_sq * A_is_max * 2.0f * sx * (float)A.Wt;
      const float duY = d_lod * dlod_drho_sq * B_is_max * 2.0f * sy * (float)A.Wt;
      const float dvX = d_lod * dlod_drho_sq * A_is_max * 2.0f * tx_ * (float)A.Ht;
      const float dvY = d_lod * dlod_drho_sq * B_is_max * 2.0f * ty_ * (float)A.Ht;
      const DirDA& d6 = p.dd;
      const float sX = s.ss * pick3(s.as, d6.x[0], d6.x[1], d6.x[2]);
      const float sY = s.ss * pick3(s.as, d6.y[0], d6.y[1], d6.y[2]);
      const float tX = s.ts * pick3(s.at, d6.x[0], d6.x[1], d6.x[2]);
      const float tY = s.ts * pick3(s.at, d6.y[0], d6.y[1], d6.y[2]);
      const float mX = s.ms * pick3(s.am, d6.x[0], d6.x[1], d6.x[2]);
      const float mY = s.ms * pick3(s.am, d6.y[0], d6.y[1], d6.y[2]);
      // through the direction derivatives: u_X = inv2 * (sX*ma - sc*mX), ...
      const float ex_as = duX * s.ss * s.ma * inv2, ey_as = duY * s.ss * s.ma * inv2;
      const float ex_at = dvX * s.ts * s.ma * inv2, ey_at = dvY * s.ts * s.ma * inv2;
      const float ex_am = -((duX * s.sc + dvX * s.tc) * s.ms * inv2);
      const float ey_am = -((duY * s.sc + dvY * s.tc) * s.ms * inv2);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        gdd_x[i] = i == s.as ? ex_as : (i == s.at ? ex_at : ex_am);
        gdd_y[i] = i == s.as ? ey_as : (i == s.at ? ey_at : ey_am);
      }
      // through the direction: d u_X / d sc = -inv2*mX,
      // d u_X / d ma = inv2*sX - 2*u_X/ma, likewise for the others
      l_as = -((duX * mX + duY * mY) * s.ss * inv2);
      l_at = -((dvX * mX + dvY * mY) * s.ts * inv2);
      l_am = s.ms * (duX * (sX * inv2 - 2.0f * p.da.x * p.inv_ma) +
                     duY * (sY * inv2 - 2.0f * p.da.y * p.inv_ma) +
                     dvX * (tX * inv2 - 2.0f * p.da.z * p.inv_ma) +
                     dvY * (tY * inv2 - 2.0f * p.da.w * p.inv_ma));
    }
  }
  if (A.d_dir) {
    float o[3] = {0.0f, 0.0f, 0.0f};
    if (A.dir_grad) {
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const float a = i == s.as ? g_as : (i == s.at ? g_at : g_am);
        const float l = i == s.as ? l_as : (i == s.at ? l_at : l_am);
        o[i] = a + l;
      }
    }
    float* dd_o = A.d_dir + pix * 3;
    dd_o[0] = o[0];
    dd_o[1] = o[1];
    dd_o[2] = o[2];
  }
  if (MODE > 0 && A.d_dir_da) {
    float2* q = reinterpret_cast<float2*>(A.d_dir_da + pix * 6);
    const float sc_ = p.scaled ? p.bscale : 1.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i) q[i] = make_float2(gdd_x[i] * sc_, gdd_y[i] * sc_);
  }
  if (MODE > 0 && A.d_bias && A.bias_map) {
    float gm = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i) gm = gm + gdd_x[i] * p.dd_in.x[i] + gdd_y[i] * p.dd_in.y[i];
    A.d_bias[pix] = gm * p.bscale * 0.6931471805599453f;
  }
}

// Persistent 16x16 pixel tiles, one pixel per thread: each tile's d_tex /
// d_pyramid contributions are summed in the LDS table (large groups of
// lanes on one footprint across the wave first, the most frequent one in a
// per-wave accumulator kept across tiles), then written out.
template <int MODE, int CT>
__global__ void __launch_bounds__(256) k_cube_bwd(CubeArgs A, int Hi, int Wi, int ntx,
                                                  int total_tiles) {
  __shared__ CubeTable<CT> tab;
  FootAcc<(CT > 0 ? CT : 1)> acc0;
  acc_init(acc0);
  lds_table_clear(tab);
  __syncthreads();
  const int tiles = ntx * ((Hi + 15) >> 4);
  for (int t = (int)blockIdx.x; t < total_tiles; t += (int)gridDim.x) {
    const int n = t / tiles, tile = t - n * tiles;
    const int ty = tile / ntx, tx = tile - ty * ntx;
    const int ph = ty * 16 + ((int)threadIdx.x >> 4), pw = tx * 16 + ((int)threadIdx.x & 15);
    const bool valid = ph < Hi && pw < Wi;
    const int64_t pix = ((int64_t)n * Hi + min(ph, Hi - 1)) * Wi + min(pw, Wi - 1);
    cube_bwd_px<MODE, CT>(A, pix, valid, n, acc0, tab);
    __syncthreads();
    lds_table_flush(tab);
    __syncthreads();
  }
  acc_flush(acc0);
}

}  // namespace dr

using namespace dr;

static int build_desc(int Ht, int Wt, int C, int Nt, int L, MipDesc& md) {
  DR_CHECK_ARG(L >= 1 && L <= kMaxLevels, "texture: mip level count out of range");
  md.L = L;
  md.nc = (int64_t)Nt * C;
  int h = Ht, w = Wt;
  int64_t off = 0;
  for (int k = 0; k < L; ++k) {
    md.h[k] = h;
    md.w[k] = w;
    md.off[k] = k == 0 ? 0 : off;
    if (k > 0) off += (int64_t)Nt * h * w * C;
    if (k + 1 < L) {
      DR_CHECK_ARG(h >= 2 && w >= 2 && h % 2 == 0 && w % 2 == 0,
                   "texture: mip levels need even sizes down to the last level");
      h /= 2;
      w /= 2;
    }
  }
  for (int k = L; k < kMaxLevels; ++k) {
    md.h[k] = md.w[k] = 1;
    md.off[k] = 0;
  }
  return DR_OK;
}

extern "C" int dr_texture_mip_levels(int H, int W, int max_level, int32_t* level_h,
                                     int32_t* level_w) {
  int n = 0;
  if (level_h) level_h[n] = H;
  if (level_w) level_w[n] = W;
  ++n;
  while (H >= 2 && W >= 2 && H % 2 == 0 && W % 2 == 0 && n < 32) {
    if (max_level >= 0 && n > max_level) break;
    H /= 2;
    W /= 2;
    if (level_h) level_h[n] = H;
    if (level_w) level_w[n] = W;
    ++n;
  }
  return n;
}

extern "C" int64_t dr_texture_mip_size(int Nt, int H, int W, int C, int L) {
  int64_t s = 0;
  for (int k = 1; k < L; ++k) {
    H /= 2;
    W /= 2;
    s += (int64_t)Nt * H * W * C;
  }
  return s;
}

extern "C" int dr_texture_build_mip(const float* tex, int Nt, int H, int W, int C, int L,
                                    float* pyramid, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  DR_CHECK_ARG(tex && Nt >= 1 && C >= 1, "texture_build_mip: bad arguments");
  MipDesc md;
  int st = build_desc(H, W, C, Nt, L, md);
  if (st) return st;
  if (L > 1) DR_CHECK_ARG(pyramid != nullptr, "texture_build_mip: null pyramid");
  if (C <= kMipMaxC) {
    for (int sl = 0; sl < L - 1;) {
      const int m = (L - 1 - sl) < 5 ? (L - 1 - sl) : 5;
      const float* src = sl == 0 ? tex : pyramid + md.off[sl];
      const int bs = 1 << m;
      const dim3 grid((unsigned)((md.h[sl] / bs) * (md.w[sl] / bs)), (unsigned)Nt);
      {
        DR_TIMED("k_mip_block", stream);
        if (C == 4 && (((uintptr_t)src | (uintptr_t)pyramid) & 15) == 0)
          hipLaunchKernelGGL(k_mip_block_c4, grid, dim3(256), 0, stream, src, pyramid, md, sl, m);
        else
          hipLaunchKernelGGL(k_mip_block, grid, dim3(256), 0, stream, src, pyramid, md, sl, m, Nt,
                             C);
      }
      DR_CHECK_LAUNCH();
      sl += m;
    }
    return DR_OK;
  }
  for (int k = 1; k < L; ++k) {
    const float* src = k == 1 ? tex : pyramid + md.off[k - 1];
    const int64_t n = (int64_t)Nt * md.h[k] * md.w[k] * C;
    DR_TIMED("k_mip_down", stream);
    hipLaunchKernelGGL(k_mip_down, dim3(grid_for(n, 256)), dim3(256), 0, stream, src,
                       pyramid + md.off[k], Nt, md.h[k - 1], md.w[k - 1], C);
    DR_CHECK_LAUNCH();
  }
  return DR_OK;
}

static int check_tex(const float* tex, const float* pyr, int Nt, int N, int Ht, int Wt, int C,
                     int L, const float* uv, const float* uv_da, int filter, int boundary,
                     MipDesc& md) {
  DR_CHECK_ARG(tex && uv && N >= 1 && Ht >= 1 && Wt >= 1 && C >= 1, "texture: bad arguments");
  DR_CHECK_ARG(Nt == 1 || Nt == N, "texture: tex batch dim incompatible with uv batch");
  DR_CHECK_ARG(filter >= 0 && filter <= 3 && boundary >= 0 && boundary <= 3,
               "texture: bad filter / boundary");
  const bool cube = boundary == DR_BOUNDARY_CUBE;
  DR_CHECK_ARG(!cube || filter != DR_FILTER_NEAREST,
               "texture: cube textures support the linear and mipmap filterModes");
  const int ntex = cube ? Nt * 6 : Nt;  // a cube map is six face textures
  const bool mip = filter >= DR_FILTER_LINEAR_MIPMAP_NEAREST;
  if (mip) {
    DR_CHECK_ARG(uv_da != nullptr, "texture: mipmap filterModes require uvDA");
    DR_CHECK_ARG(L == 1 || pyr != nullptr, "texture: mip pyramid missing");
    return build_desc(Ht, Wt, C, ntex, L, md);
  }
  return build_desc(Ht, Wt, C, ntex, 1, md);
}

#define DR_TEX_C_DISPATCH(KERNEL, F, BNDV, GRID, ...)                                        \
  do {                                                                                        \
    switch (C) {                                                                              \
      case 1: hipLaunchKernelGGL((KERNEL<F, BNDV, 1>), GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      case 2: hipLaunchKernelGGL((KERNEL<F, BNDV, 2>), GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      case 3: hipLaunchKernelGGL((KERNEL<F, BNDV, 3>), GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      case 4: hipLaunchKernelGGL((KERNEL<F, BNDV, 4>), GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      default: hipLaunchKernelGGL((KERNEL<F, BNDV, 0>), GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
    }                                                                                         \
  } while (0)

#define DR_TEX_B_DISPATCH(KERNEL, F, GRID, ...)                                                          \
  do {                                                                                                  \
    if (boundary == DR_BOUNDARY_CLAMP) DR_TEX_C_DISPATCH(KERNEL, F, DR_BOUNDARY_CLAMP, GRID, __VA_ARGS__); \
    else if (boundary == DR_BOUNDARY_WRAP) DR_TEX_C_DISPATCH(KERNEL, F, DR_BOUNDARY_WRAP, GRID, __VA_ARGS__); \
    else DR_TEX_C_DISPATCH(KERNEL, F, DR_BOUNDARY_ZERO, GRID, __VA_ARGS__);                             \
  } while (0)

#define DR_TEX_DISPATCH(KERNEL, GRID, ...)                                                              \
  do {                                                                                                  \
    if (boundary == DR_BOUNDARY_CUBE) DR_TEX_C_DISPATCH(KERNEL, DR_FILTER_LINEAR, DR_BOUNDARY_CUBE, GRID, __VA_ARGS__); \
    else if (filter == DR_FILTER_NEAREST) DR_TEX_B_DISPATCH(KERNEL, DR_FILTER_NEAREST, GRID, __VA_ARGS__); \
    else if (filter == DR_FILTER_LINEAR) DR_TEX_B_DISPATCH(KERNEL, DR_FILTER_LINEAR, GRID, __VA_ARGS__); \
    else if (filter == DR_FILTER_LINEAR_MIPMAP_NEAREST) DR_TEX_B_DISPATCH(KERNEL, DR_FILTER_LINEAR_MIPMAP_NEAREST, GRID, __VA_ARGS__); \
    else DR_TEX_B_DISPATCH(KERNEL, DR_FILTER_LINEAR_MIPMAP_LINEAR, GRID, __VA_ARGS__);   \
  } while (0)

// d_tex += the pyramid's gradient (the backward of the 2x2 means).
static int mip_collapse(float* d_pyr, const MipDesc& md, int ntex, int Ht, int Wt, int C,
                        float* d_tex, hipStream_t stream) {
  DR_TIMED("k_mip_collapse", stream);
  if (C == 4 && (((uintptr_t)d_pyr | (uintptr_t)d_tex) & 15) == 0) {
    if (md.L >= 3) {
      const int64_t n1 = (int64_t)ntex * md.h[1] * md.w[1];
      hipLaunchKernelGGL(k_mip_collapse1_c4, dim3(grid_for(n1, 256)), dim3(256), 0, stream,
                         d_pyr, md, n1);
      DR_CHECK_LAUNCH();
    }
    const int64_t n0 = (int64_t)ntex * Ht * Wt;
    hipLaunchKernelGGL(k_mip_collapse0_c4, dim3(grid_for(n0, 256)), dim3(256), 0, stream, d_pyr,
                       md, n0, d_tex);
    DR_CHECK_LAUNCH();
    return DR_OK;
  }
  const int bpr = (Wt + 255) / 256;
  hipLaunchKernelGGL(k_mip_collapse, dim3((unsigned)((int64_t)ntex * Ht * bpr)), dim3(256), 0,
                     stream, d_pyr, md, C, bpr, d_tex);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

static CubeArgs cube_args(const float* tex, const float* pyr, const MipDesc& md,
                          int64_t tex_stride, int Ht, int Wt, int C, const float* dir,
                          const float* dir_da, const float* bias_map, float scale_bias,
                          int has_bias, int64_t P, int HWi) {
  CubeArgs A{};
  A.tex = tex;
  A.pyr = pyr;
  A.md = md;
  A.tex_stride = tex_stride;
  A.Ht = Ht;
  A.Wt = Wt;
  A.C = C;
  A.dir = dir;
  A.dir_da = dir_da;
  A.bias_map = bias_map;
  A.scale_bias = scale_bias;
  A.has_bias = has_bias;
  A.P = P;
  A.HWi = HWi;
  return A;
}

#define DR_CUBE_DISPATCH(KERNEL, MODE, GRID, ARGS)                                           \
  do {                                                                                        \
    switch (C) {                                                                              \
      case 1: hipLaunchKernelGGL((KERNEL<MODE, 1>), GRID, dim3(256), 0, stream, ARGS); break; \
      case 2: hipLaunchKernelGGL((KERNEL<MODE, 2>), GRID, dim3(256), 0, stream, ARGS); break; \
      case 3: hipLaunchKernelGGL((KERNEL<MODE, 3>), GRID, dim3(256), 0, stream, ARGS); break; \
      case 4: hipLaunchKernelGGL((KERNEL<MODE, 4>), GRID, dim3(256), 0, stream, ARGS); break; \
      default: hipLaunchKernelGGL((KERNEL<MODE, 0>), GRID, dim3(256), 0, stream, ARGS); break; \
    }                                                                                         \
  } while (0)

extern "C" int dr_texture_fwd(const float* tex, const float* pyramid, int Nt, int Ht, int Wt,
                              int C, int L, const float* uv, const float* uv_da,
                              const float* bias_map, float bias, int filter, int boundary, int N,
                              int Hi, int Wi, float* out, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  MipDesc md;
  int st = check_tex(tex, pyramid, Nt, N, Ht, Wt, C, L, uv, uv_da, filter, boundary, md);
  if (st) return st;
  DR_CHECK_ARG(out != nullptr && Hi >= 1 && Wi >= 1, "texture: bad output");
  const bool cube = boundary == DR_BOUNDARY_CUBE;
  const int64_t tex_stride = Nt == 1 ? 0 : (int64_t)(cube ? 6 : 1) * Ht * Wt * C;
  const int64_t P = (int64_t)N * Hi * Wi;
  const float scale_bias = exp2f(bias);
  const int has_bias = bias != 0.0f;
  const dim3 grid(grid_for(P, 256));
  if (cube && filter >= DR_FILTER_LINEAR_MIPMAP_NEAREST) {
    CubeArgs A = cube_args(tex, pyramid, md, tex_stride, Ht, Wt, C, uv, uv_da, bias_map,
                           scale_bias, has_bias, P, Hi * Wi);
    A.out = out;
    A.Wi = Wi;
    const int64_t tiles = (int64_t)N * ((Hi + 15) / 16) * ((Wi + 15) / 16);
    DR_CHECK_ARG(tiles <= INT32_MAX, "texture: too many pixel tiles");
    const dim3 tgrid((unsigned)tiles);
    DR_TIMED("k_cube_fwd", stream);
    if (filter == DR_FILTER_LINEAR_MIPMAP_LINEAR) DR_CUBE_DISPATCH(k_cube_fwd, 2, tgrid, A);
    else DR_CUBE_DISPATCH(k_cube_fwd, 1, tgrid, A);
    DR_CHECK_LAUNCH();
    return DR_OK;
  }
  const int64_t px_tiles = (int64_t)N * ((Hi + 15) / 16) * ((Wi + 15) / 16);
  DR_CHECK_ARG(px_tiles < ((int64_t)1 << 31), "texture: too many pixels");
  DR_TIMED("k_tex_fwd", stream);
  DR_TEX_DISPATCH(k_tex_fwd, dim3((unsigned)px_tiles), tex, pyramid, md, tex_stride, Ht, Wt, C, uv,
                  uv_da, bias_map, scale_bias, has_bias, P, Hi, Wi, out);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

// The cube backward's persistent tiles: as many workgroups as fit at once.
template <int MODE, int CT>
static hipError_t launch_cube_bwd(const CubeArgs& A, int Hi, int Wi, int ntx, int total_tiles,
                                  hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_cube_bwd<MODE, CT>, 256, 0) !=
            hipSuccess ||
        b <= 0)
      b = 2;
    per_cu = b;
  }
  const int64_t resident = (int64_t)device_cu_count() * per_cu;
  const unsigned grid = (unsigned)(total_tiles < resident ? total_tiles : resident);
  hipLaunchKernelGGL((k_cube_bwd<MODE, CT>), dim3(grid), dim3(256), 0, stream, A, Hi, Wi, ntx,
                     total_tiles);
  return hipGetLastError();
}

// Where the backward keeps the mip pyramid's gradient: the library's
// per-stream scratch (grown with hipMalloc as needed), or a fixed buffer of
// `cap` floats (dr_texture_bwd_noalloc).
struct DPyrBuf {
  float* fixed;
  int64_t cap;
};

static int dpyr_get(const DPyrBuf& buf, int64_t np, hipStream_t stream, float*& d_pyr) {
  if (buf.fixed) {
    DR_CHECK_ARG(np <= buf.cap, "texture_bwd_noalloc: the mip pyramid gradient needs " +
                                    std::to_string(np) + " floats, above the fixed " +
                                    std::to_string(buf.cap) + " (use dr_texture_bwd)");
    d_pyr = buf.fixed;
    return DR_OK;
  }
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  d_pyr = (float*)scratch_get(sc, stream, SLOT_DPYR, (size_t)np * sizeof(float));
  return d_pyr ? DR_OK : scratch_fail();
}

// The cube extension's backward: one thread per pixel, d_tex / d_pyramid by
// global atomics, then the pyramid collapse over the Nt*6 faces.  The first
// `zero_tex` floats of d_tex are cleared first (0: accumulate), after the
// pyramid gradient's buffer is known to fit, so a refused call leaves d_tex
// untouched.
static int cube_bwd(const float* tex, const float* pyramid, const MipDesc& md, int64_t tex_stride,
                    int Nt, int Ht, int Wt, int C, const float* dir, const float* dir_da,
                    const float* bias_map, float bias, int filter, int N, int Hi, int Wi,
                    const float* d_out, float* d_tex, int64_t zero_tex, float* d_dir,
                    float* d_dir_da, float* d_bias_map, unsigned flags, const DPyrBuf& pbuf,
                    hipStream_t stream) {
  const bool mip = filter >= DR_FILTER_LINEAR_MIPMAP_NEAREST;
  float* d_pyr = nullptr;
  if (mip && md.L > 1) {
    const int64_t np = dr_texture_mip_size(Nt * 6, Ht, Wt, C, md.L);
    const int st = dpyr_get(pbuf, np, stream, d_pyr);
    if (st) return st;
    if (zero_tex) DR_CHECK_HIP(fill2_async(d_tex, zero_tex, d_pyr, np, 0.0f, stream));
    else DR_CHECK_HIP(fill_async(d_pyr, 0.0f, np, stream));
  } else if (zero_tex) {
    DR_CHECK_HIP(fill_async(d_tex, 0.0f, zero_tex, stream));
  }
  const int64_t P = (int64_t)N * Hi * Wi;
  CubeArgs A = cube_args(tex, pyramid, md, tex_stride, Ht, Wt, C, dir, dir_da, bias_map,
                         exp2f(bias), bias != 0.0f, P, Hi * Wi);
  A.d_out = d_out;
  A.d_tex = d_tex;
  A.d_pyr = d_pyr;
  A.d_dir = d_dir;
  A.dir_grad = (flags & DR_CUBE_DIR_GRAD) ? 1 : 0;
  A.d_dir_da = mip ? d_dir_da : nullptr;
  A.d_bias = mip ? d_bias_map : nullptr;
  const int ntx = (Wi + 15) / 16;
  const int64_t total_tiles = (int64_t)N * ntx * ((Hi + 15) / 16);
  DR_CHECK_ARG(total_tiles < ((int64_t)1 << 31), "texture_bwd: too many pixels");
  {
    DR_TIMED("k_cube_bwd", stream);
    hipError_t e = hipSuccess;
#define DR_CB(MODEV, CTV) e = launch_cube_bwd<MODEV, CTV>(A, Hi, Wi, ntx, (int)total_tiles, stream)
#define DR_CB_C(MODEV)                 \
  switch (C) {                         \
    case 1: DR_CB(MODEV, 1); break;    \
    case 2: DR_CB(MODEV, 2); break;    \
    case 3: DR_CB(MODEV, 3); break;    \
    case 4: DR_CB(MODEV, 4); break;    \
    default: DR_CB(MODEV, 0); break;   \
  }
    if (filter == DR_FILTER_LINEAR_MIPMAP_LINEAR) DR_CB_C(2)
    else if (filter == DR_FILTER_LINEAR_MIPMAP_NEAREST) DR_CB_C(1)
    else DR_CB_C(0)
#undef DR_CB_C
#undef DR_CB
    DR_CHECK_HIP(e);
  }
  DR_CHECK_LAUNCH();
  if (d_pyr) return mip_collapse(d_pyr, md, Nt * 6, Ht, Wt, C, d_tex, stream);
  return DR_OK;
}

static int texture_bwd(const float* tex, const float* pyramid, int Nt, int Ht, int Wt, int C,
                       int L, const float* uv, const float* uv_da, const float* bias_map,
                       float bias, int filter, int boundary, int N, int Hi, int Wi,
                       const float* d_out, float* d_tex, float* d_uv, float* d_uv_da,
                       float* d_bias_map, unsigned flags, const DPyrBuf& pbuf,
                       hipStream_t stream) {
  (void)hipGetLastError();
  MipDesc md;
  int st = check_tex(tex, pyramid, Nt, N, Ht, Wt, C, L, uv, uv_da, filter, boundary, md);
  if (st) return st;
  DR_CHECK_ARG(d_out && d_tex && Hi >= 1 && Wi >= 1, "texture_bwd: null tensor");
  const bool cube = boundary == DR_BOUNDARY_CUBE;
  const int64_t tex_stride = Nt == 1 ? 0 : (int64_t)(cube ? 6 : 1) * Ht * Wt * C;
  const int64_t ntex = (int64_t)Nt * (cube ? 6 : 1) * Ht * Wt * C;
  const bool zero_tex = !(flags & DR_ACCUMULATE);
  if (cube && (filter >= DR_FILTER_LINEAR_MIPMAP_NEAREST || (flags & DR_CUBE_DIR_GRAD))) {
    return cube_bwd(tex, pyramid, md, tex_stride, Nt, Ht, Wt, C, uv, uv_da, bias_map, bias,
                    filter, N, Hi, Wi, d_out, d_tex, zero_tex ? ntex : 0, d_uv, d_uv_da,
                    d_bias_map, flags, pbuf, stream);
  }
  const bool mip = !cube && filter >= DR_FILTER_LINEAR_MIPMAP_NEAREST;
  float* d_pyr = nullptr;
  if (mip && md.L > 1) {
    const int64_t np = dr_texture_mip_size(Nt, Ht, Wt, C, md.L);
    st = dpyr_get(pbuf, np, stream, d_pyr);
    if (st) return st;
    // d_tex and the coarser levels' accumulator are zeroed in one launch
    if (zero_tex) DR_CHECK_HIP(fill2_async(d_tex, ntex, d_pyr, np, 0.0f, stream));
    else DR_CHECK_HIP(fill_async(d_pyr, 0.0f, np, stream));
  } else if (zero_tex) {
    DR_CHECK_HIP(fill_async(d_tex, 0.0f, ntex, stream));
  }
  const int ntx = (Wi + 15) / 16, nty = (Hi + 15) / 16;
  TexBwdArgs args;
  args.tex = tex;
  args.pyr = pyramid;
  args.md = md;
  args.tex_stride = tex_stride;
  args.Ht = Ht;
  args.Wt = Wt;
  args.C = C;
  args.boundary = boundary;
  args.has_bias = bias != 0.0f;
  args.uv = uv;
  args.uv_da = uv_da;
  args.bias_map = bias_map;
  args.scale_bias = exp2f(bias);
  args.N = N;
  args.Hi = Hi;
  args.Wi = Wi;
  args.ntx = ntx;
  args.nty = nty;
  args.d_out = d_out;
  args.d_tex = d_tex;
  args.d_pyr = d_pyr;
  args.d_uv = d_uv;
  args.d_uv_da = mip ? d_uv_da : nullptr;
  args.d_bias = mip ? d_bias_map : nullptr;
  const int64_t total_tiles = (int64_t)N * ntx * nty;
  DR_CHECK_ARG(total_tiles < (int64_t)1 << 31, "texture_bwd: too many pixels");
  // Persistent tiles: each wave keeps its footprint accumulator across the
  // tiles it visits.
  {
    DR_TIMED("k_tex_bwd", stream);
    hipError_t e = hipSuccess;
#define DR_TB(F, CUBEV, CTV) e = launch_tex_bwd<F, CUBEV, CTV>(args, (int)total_tiles, stream)
#define DR_TB_C(F, CUBEV)                  \
  switch (C) {                             \
    case 1: DR_TB(F, CUBEV, 1); break;     \
    case 2: DR_TB(F, CUBEV, 2); break;     \
    case 3: DR_TB(F, CUBEV, 3); break;     \
    case 4: DR_TB(F, CUBEV, 4); break;     \
    default: DR_TB(F, CUBEV, 0); break;    \
  }
    // the windowed kernel's tiles are 16 x (4 * kWinWaves) pixels
    TexBwdArgs wargs = args;
    wargs.nty = (Hi + 4 * kWinWaves - 1) / (4 * kWinWaves);
    const int wtiles = (int)((int64_t)N * ntx * wargs.nty);
#define DR_TW(F)                                                   \
  switch (C) {                                                     \
    case 1: e = launch_tex_bwd_win<F, 1>(wargs, wtiles, stream); break; \
    case 2: e = launch_tex_bwd_win<F, 2>(wargs, wtiles, stream); break; \
    case 3: e = launch_tex_bwd_win<F, 3>(wargs, wtiles, stream); break; \
    default: e = launch_tex_bwd_win<F, 4>(wargs, wtiles, stream); break; \
  }
    const bool windowed = !cube && filter != DR_FILTER_NEAREST && C >= 1 && C <= 4 &&
                          Wt <= 32767 && Ht <= 32767;  // window boxes use 16-bit texel coordinates
    if (windowed && filter == DR_FILTER_LINEAR) DR_TW(DR_FILTER_LINEAR)
    else if (windowed && filter == DR_FILTER_LINEAR_MIPMAP_NEAREST) DR_TW(DR_FILTER_LINEAR_MIPMAP_NEAREST)
    else if (windowed) DR_TW(DR_FILTER_LINEAR_MIPMAP_LINEAR)
    else if (cube) DR_TB_C(DR_FILTER_LINEAR, true)
    else if (filter == DR_FILTER_NEAREST) DR_TB_C(DR_FILTER_NEAREST, false)
    else if (filter == DR_FILTER_LINEAR) DR_TB_C(DR_FILTER_LINEAR, false)
    else if (filter == DR_FILTER_LINEAR_MIPMAP_NEAREST) DR_TB_C(DR_FILTER_LINEAR_MIPMAP_NEAREST, false)
    else DR_TB_C(DR_FILTER_LINEAR_MIPMAP_LINEAR, false)
#undef DR_TW
#undef DR_TB_C
#undef DR_TB
    DR_CHECK_HIP(e);
  }
  if (d_pyr) return mip_collapse(d_pyr, md, Nt, Ht, Wt, C, d_tex, stream);
  return DR_OK;
}

extern "C" int dr_texture_bwd(const float* tex, const float* pyramid, int Nt, int Ht, int Wt,
                              int C, int L, const float* uv, const float* uv_da,
                              const float* bias_map, float bias, int filter, int boundary, int N,
                              int Hi, int Wi, const float* d_out, float* d_tex, float* d_uv,
                              float* d_uv_da, float* d_bias_map, unsigned flags,
                              dr_stream_t stream_) {
  return texture_bwd(tex, pyramid, Nt, Ht, Wt, C, L, uv, uv_da, bias_map, bias, filter, boundary,
                     N, Hi, Wi, d_out, d_tex, d_uv, d_uv_da, d_bias_map, flags,
                     DPyrBuf{nullptr, 0}, (hipStream_t)stream_);
}

// ---- dr_texture_bwd without allocation --------------------------------------
// The pyramid gradient lives in one fixed device array instead of the
// library's per-stream scratch.  In host code `scratch` names a host-side
// stand-in: its device address on each GPU comes from hipGetSymbolAddress
// (with that GPU current), kept per device, and only that address is used.

static __device__ __align__(256) float scratch[DR_TEXTURE_BWD_NOALLOC_FLOATS];

static std::mutex g_noalloc_mu;
static float* g_noalloc_ptr[64] = {};

static int noalloc_scratch(float*& ptr) {
  int dev = 0;
  DR_CHECK_HIP(hipGetDevice(&dev));
  DR_CHECK_ARG(dev >= 0 && dev < 64, "texture_bwd_noalloc: device index above 63");
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    DR_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    DR_CHECK_ARG(p != nullptr, "texture_bwd_noalloc: no device address for the scratch array");
    g_noalloc_ptr[dev] = (float*)p;
  }
  ptr = g_noalloc_ptr[dev];
  return DR_OK;
}

extern "C" int dr_texture_bwd_noalloc(const float* tex, const float* pyramid, int Nt, int Ht,
                                      int Wt, int C, int L, const float* uv, const float* uv_da,
                                      const float* bias_map, float bias, int filter, int boundary,
                                      int N, int Hi, int Wi, const float* d_out, float* d_tex,
                                      float* d_uv, float* d_uv_da, float* d_bias_map,
                                      unsigned flags, dr_stream_t stream_) {
  float* ptr = nullptr;
  const int st = noalloc_scratch(ptr);
  if (st) return st;
  return texture_bwd(tex, pyramid, Nt, Ht, Wt, C, L, uv, uv_da, bias_map, bias, filter, boundary,
                     N, Hi, Wi, d_out, d_tex, d_uv, d_uv_da, d_bias_map, flags,
                     DPyrBuf{ptr, (int64_t)DR_TEXTURE_BWD_NOALLOC_FLOATS}, (hipStream_t)stream_);
}
