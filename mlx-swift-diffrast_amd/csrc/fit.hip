// The loss and optimizer step of the reference's inverse-rendering samples:
//   MSE loss and its gradient  Sources/ColorFitExample/main.swift:62-66,
//                              PoseFitExample/main.swift:93-97,
//                              MeshFitExample/main.swift:87-91
//   Adam step                  Sources/MLXDiffRastExamples/Adam.swift:36-43
#include "common.h"

#include <cmath>

namespace dr {

// Number of partial sums of the loss (fixed, so the summation order and
// hence the loss are the same on every call).
constexpr int kMseBlocks = 1024;

__device__ __forceinline__ double block_sum(double v, double* lds) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) lds[w] = v;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0)
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += lds[i];
  return s;
}

// (out - target)^2 summed per block in fp64 from the fp32 squares, and the
// gradient of mean((out - target)^2): the reference's autodiff takes
// d(mean) = cotangent * (1/n), then d(diff * diff) = g*diff + g*diff.
// VEC: out, target and d_out are 16-byte aligned (float4 loads and stores).
template <bool VEC>
__global__ __launch_bounds__(256) void k_mse(const float* __restrict__ out,
                                             const float* __restrict__ target, int64_t n,
                                             float inv_n, float* __restrict__ d_out,
                                             double* __restrict__ partial) {
  __shared__ double lds[4];
  double acc = 0.0;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t head = 0;
  if (VEC) {
    const int64_t n4 = n >> 2;
    const float4* o4 = reinterpret_cast<const float4*>(out);
    for (int64_t i = tid; i < n4; i += stride) {
      // the target is streamed once a call (non-temporal): 1.133 -> 1.127 ms
      // a step at 8 x 1024^2, whose antialias output `out` is still in cache
      const float4 a = o4[i], b = ld_nt4(target + 4 * i);
      const float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z, dw = a.w - b.w;
      const float sx = dx * dx, sy = dy * dy, sz = dz * dz, sw = dw * dw;
      acc += (double)sx + (double)sy + (double)sz + (double)sw;
      if (d_out) {
        const float gx = dx * inv_n, gy = dy * inv_n, gz = dz * inv_n, gw = dw * inv_n;
        reinterpret_cast<float4*>(d_out)[i] = make_float4(gx + gx, gy + gy, gz + gz, gw + gw);
      }
    }
    head = n4 << 2;
  }
  for (int64_t i = head + tid; i < n; i += stride) {
    const float d = out[i] - target[i];
    const float s = d * d;
    acc += (double)s;
    if (d_out) {
      const float g = d * inv_n;
      d_out[i] = g + g;
    }
  }
  const double s = block_sum(acc, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

// Sums the partials in a fixed order; loss = (float)sum * (1/n).
__global__ __launch_bounds__(256) void k_mse_final(const double* __restrict__ partial, int nb,
                                                   float inv_n, float* __restrict__ loss) {
  __shared__ double lds[4];
  double acc = 0.0;
  for (int i = threadIdx.x; i < nb; i += blockDim.x) acc += partial[i];
  const double s = block_sum(acc, lds);
  if (threadIdx.x == 0) loss[0] = (float)s * inv_n;
}

// One Adam step (Adam.swift:36-43), every operation rounded to fp32 in the
// order written there:
//   m = beta1*m + (1-beta1)*g ;  v = beta2*v + (1-beta2)*(g*g)
//   param - lr * (m / c1) / (sqrt(v / c2) + eps),  c = 1 - beta^t.
// g = grad * grad_mask when a mask is given (the samples' gradient masks).
__global__ __launch_bounds__(256) void k_adam(const float* param,
                                              const float* __restrict__ grad,
                                              const float* __restrict__ grad_mask,
                                              float* __restrict__ m, float* __restrict__ v,
                                              float* param_out, int64_t n, float lr, float b1,
                                              float b2, float omb1, float omb2, float c1,
                                              float c2, float eps) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float g = grad[i];
    if (grad_mask) g = g * grad_mask[i];
    const float mi = b1 * m[i] + omb1 * g;
    const float vi = b2 * v[i] + omb2 * (g * g);
    m[i] = mi;
    v[i] = vi;
    const float mh = mi / c1;
    const float vh = vi / c2;
    const float p = param[i];
    param_out[i] = p - lr * mh / (sqrtf(vh) + eps);
  }
}

}  // namespace dr

using namespace dr;

extern "C" int dr_mse_loss(const float* out, const float* target, int64_t n, float* loss,
                           float* d_out, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  DR_CHECK_ARG(n >= 1, "mse_loss: n must be >= 1");
  DR_CHECK_ARG(out && target && loss, "mse_loss: null tensor");
  Scratch* sc = scratch_for(stream);
  if (!sc) return scratch_fail();
  double* partial = (double*)scratch_get(sc, stream, SLOT_LOSS, kMseBlocks * sizeof(double));
  if (!partial) return scratch_fail();
  const float inv_n = 1.0f / (float)n;
  const bool vec =
      (((uintptr_t)out | (uintptr_t)target | (uintptr_t)(d_out ? d_out : out)) & 15) == 0;
  const int64_t units = vec ? (n + 3) / 4 : n;
  const int nb = (int)std::min<int64_t>(kMseBlocks, std::max<int64_t>(1, (units + 255) / 256));
  {
    DR_TIMED("k_mse", stream);
    if (vec)
      hipLaunchKernelGGL(k_mse<true>, dim3(nb), dim3(256), 0, stream, out, target, n, inv_n,
                         d_out, partial);
    else
      hipLaunchKernelGGL(k_mse<false>, dim3(nb), dim3(256), 0, stream, out, target, n, inv_n,
                         d_out, partial);
  }
  DR_CHECK_LAUNCH();
  hipLaunchKernelGGL(k_mse_final, dim3(1), dim3(256), 0, stream, partial, nb, inv_n, loss);
  DR_CHECK_LAUNCH();
  return DR_OK;
}

extern "C" int dr_adam_step(const float* param, const float* grad, const float* grad_mask,
                            float* m, float* v, float* param_out, int64_t n, int step, float lr,
                            float beta1, float beta2, float eps, dr_stream_t stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  (void)hipGetLastError();
  DR_CHECK_ARG(n >= 0 && step >= 1, "adam_step: n must be >= 0 and step >= 1");
  DR_CHECK_ARG(param && grad && m && v && param_out, "adam_step: null tensor");
  if (n == 0) return DR_OK;
  // bias corrections in fp32, as the reference's `1 - pow(Float(beta), Float(t))`;
  // beta^t is rounded once to fp32 from a double evaluation
  const float c1 = 1.0f - (float)pow((double)beta1, (double)step);
  const float c2 = 1.0f - (float)pow((double)beta2, (double)step);
  const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
  const int nb = (int)std::min<int64_t>(4096, (n + 255) / 256);
  DR_TIMED("k_adam", stream);
  hipLaunchKernelGGL(k_adam, dim3(nb), dim3(256), 0, stream, param, grad, grad_mask, m, v,
                     param_out, n, lr, beta1, beta2, omb1, omb2, c1, c2, eps);
  DR_CHECK_LAUNCH();
  return DR_OK;
}
