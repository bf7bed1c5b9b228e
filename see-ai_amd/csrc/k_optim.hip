// k_optim.hip -- gradient conditioning and the in-place optimizer steps on
// gfx950 (runtime/executor/optimizer.cc:19-132).
//
// The L2 norm is two kernels: a fixed grid of workgroups each sums a fixed
// contiguous chunk in double, then one workgroup combines the partials in
// chunk order -- bitwise reproducible at any CU count, no atomics.  The
// clip factor and the refusal verdict are computed on the device and
// written to a device scale slot and a device refusal word; every kernel
// that writes parameters, moments or gradients reads the word first and
// writes nothing once it is set (the range's Flush reports the refusal).
// AdamW takes its two bias-correction reciprocals from the host, which
// evaluates them with the reference's own powf expression, so every element
// update is the reference's expression on the reference's operands.
#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;
constexpr int kNormBlocks = 1024;

__global__ void __launch_bounds__(kThreads)
SqPartialKernel(const float* __restrict__ g, size_t n, double* __restrict__ partials) {
  __shared__ double red[kThreads / kWave];
  const size_t chunk = (n + kNormBlocks - 1) / kNormBlocks;
  const size_t b = static_cast<size_t>(blockIdx.x) * chunk;
  const size_t e = b + chunk < n ? b + chunk : n;
  double sq = 0.0;
  for (size_t i = b + threadIdx.x; i < e; i += kThreads) {
    const double v = static_cast<double>(g[i]);
    sq += v * v;
  }
  sq = BlockSumD<kThreads>(sq, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = sq;
}

__device__ double SumPartials(const double* partials, double* red) {
  double s = 0.0;
  for (int i = threadIdx.x; i < kNormBlocks; i += kThreads) s += partials[i];
  return BlockSumD<kThreads>(s, red);
}

// optimizer.cc:40-50 (ClipScale) and :54-68 (ClipNorm's verdicts).
__global__ void __launch_bounds__(kThreads)
ClipFactorKernel(const double* __restrict__ partials, float max_norm, float* __restrict__ scale,
                 int* __restrict__ flag) {
  __shared__ double red[kThreads / kWave];
  const double sq = SumPartials(partials, red);
  if (threadIdx.x != 0) return;
  float s = 1.0f;
  const double norm = sqrt(sq);
  if (!isfinite(norm)) {
    *flag = 1;
  } else if (!(norm <= static_cast<double>(max_norm) || norm == 0.0)) {
    s = static_cast<float>(static_cast<double>(max_norm) / norm);
  }
  *scale = s;
}

// optimizer.cc:70-72: acc[0] = f32(double(acc[0]) + ||g||^2).
__global__ void __launch_bounds__(kThreads)
SqAccumKernel(const double* __restrict__ partials, float* __restrict__ acc) {
  __shared__ double red[kThreads / kWave];
  const double sq = SumPartials(partials, red);
  if (threadIdx.x == 0) acc[0] = static_cast<float>(static_cast<double>(acc[0]) + sq);
}

// optimizer.cc:74-85: the factor the global accumulator implies.
__global__ void GlobalFactorKernel(const float* __restrict__ acc, float max_norm,
                                   float* __restrict__ scale, int* __restrict__ flag) {
  float s = 1.0f;
  const double norm = sqrt(static_cast<double>(acc[0]));
  if (!isfinite(norm)) {
    *flag = 1;
  } else if (!(norm <= static_cast<double>(max_norm) || norm == 0.0)) {
    s = static_cast<float>(static_cast<double>(max_norm) / norm);
  }
  *scale = s;
}

__global__ void __launch_bounds__(kThreads)
ScaleByFactorKernel(float* __restrict__ g, size_t n, const float* __restrict__ scale,
                    const int* __restrict__ flag) {
  if (*flag) return;
  const float s = *scale;
  if (s == 1.0f) return;  // the reference leaves g untouched below the cap
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    g[i] *= s;
}

// optimizer.cc:104-132, per element.
__device__ __forceinline__ void AdamWElement(float* __restrict__ p, const float* __restrict__ g,
                                             float* __restrict__ m, float* __restrict__ v, size_t i,
                                             float s, float lr, float beta1, float beta2, float eps,
                                             float wd, float inv_bc1, float inv_bc2) {
  const float om_b1 = 1.0f - beta1;
  const float om_b2 = 1.0f - beta2;
  const float gi = g[i] * s;
  const float mi = beta1 * m[i] + om_b1 * gi;
  const float vi = beta2 * v[i] + om_b2 * gi * gi;
  m[i] = mi;
  v[i] = vi;
  const float m_hat = mi * inv_bc1;
  const float v_hat = vi * inv_bc2;
  const float pi = p[i];
  p[i] = pi - lr * (m_hat / (sqrtf(v_hat) + eps) + wd * pi);
}

__global__ void __launch_bounds__(kThreads)
AdamWKernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
            float* __restrict__ v, size_t n, float lr, float beta1, float beta2, float eps,
            float wd, float inv_bc1, float inv_bc2, const float* __restrict__ scale_p,
            const int* __restrict__ flag, const float* __restrict__ hyper) {
  if (*flag) return;
  if (hyper) lr = hyper[0], inv_bc1 = hyper[1], inv_bc2 = hyper[2];
  const float s = scale_p ? *scale_p : 1.0f;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    AdamWElement(p, g, m, v, i, s, lr, beta1, beta2, eps, wd, inv_bc1, inv_bc2);
}

// Adjacent kAdamWStep instructions of a range (no clip) as one launch: the
// workgroups of tensor t are blocks [first[t], first[t + 1]) of the grid,
// each running the per-element update of AdamWKernel on its slice.
__global__ void __launch_bounds__(kThreads)
AdamWMultiKernel(AdamWTable tab, float lr, float beta1, float beta2, float eps, float wd,
                 float inv_bc1, float inv_bc2, const int* __restrict__ flag,
                 const float* __restrict__ hyper) {
  if (*flag) return;
  if (hyper) lr = hyper[0], inv_bc1 = hyper[1], inv_bc2 = hyper[2];
  int t = 0;
  while (t + 1 < tab.count && static_cast<int>(blockIdx.x) >= tab.first[t + 1]) ++t;
  const AdamWTensor& x = tab.t[t];
  const size_t blocks = static_cast<size_t>(tab.first[t + 1] - tab.first[t]);
  const size_t stride = blocks * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x - tab.first[t]) * kThreads + threadIdx.x; i < x.n;
       i += stride)
    AdamWElement(x.p, x.g, x.m, x.v, i, 1.0f, lr, beta1, beta2, eps, wd, inv_bc1, inv_bc2);
}

// optimizer.cc:91-102
__global__ void __launch_bounds__(kThreads)
SgdKernel(float* __restrict__ p, const float* __restrict__ g, size_t n, float lr, float wd,
          const float* __restrict__ scale_p, const int* __restrict__ flag,
          const float* __restrict__ hyper) {
  if (*flag) return;
  if (hyper) lr = hyper[0];
  const float s = scale_p ? *scale_p : 1.0f;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    const float gi = g[i] * s;
    const float pi = p[i];
    p[i] = pi - lr * (gi + wd * pi);
  }
}

hipError_t LaunchPartials(const float* g, size_t n, void* ws, hipStream_t s) {
  hipLaunchKernelGGL(SqPartialKernel, dim3(kNormBlocks), dim3(kThreads), 0, s, g, n,
                     static_cast<double*>(ws));
  return hipGetLastError();
}

}  // namespace

hipError_t LaunchClipFactor(const float* g, size_t n, float max_norm, float* scale, int* flag,
                            void* ws, hipStream_t s) {
  if (hipError_t e = LaunchPartials(g, n, ws, s); e != hipSuccess) return e;
  hipLaunchKernelGGL(ClipFactorKernel, dim3(1), dim3(kThreads), 0, s,
                     static_cast<const double*>(ws), max_norm, scale, flag);
  return hipGetLastError();
}

hipError_t LaunchSqNormAccum(const float* g, size_t n, float* acc, void* ws, hipStream_t s) {
  if (hipError_t e = LaunchPartials(g, n, ws, s); e != hipSuccess) return e;
  hipLaunchKernelGGL(SqAccumKernel, dim3(1), dim3(kThreads), 0, s,
                     static_cast<const double*>(ws), acc);
  return hipGetLastError();
}

hipError_t LaunchGlobalClipFactor(const float* acc, float max_norm, float* scale, int* flag,
                                  hipStream_t s) {
  hipLaunchKernelGGL(GlobalFactorKernel, dim3(1), dim3(1), 0, s, acc, max_norm, scale, flag);
  return hipGetLastError();
}

hipError_t LaunchScaleByFactor(float* g, size_t n, const float* scale, const int* flag,
                               hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(ScaleByFactorKernel, dim3(GridFor(n, kThreads, 4096)), dim3(kThreads), 0, s, g,
                     n, scale, flag);
  return hipGetLastError();
}

hipError_t LaunchAdamW(float* p, const float* g, float* m, float* v, size_t n, float lr,
                       float beta1, float beta2, float eps, float wd, float inv_bc1,
                       float inv_bc2, const float* scale, const int* flag, hipStream_t s,
                       const float* hyper) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(AdamWKernel, dim3(GridFor(n, kThreads, 4096)), dim3(kThreads), 0, s, p, g, m,
                     v, n, lr, beta1, beta2, eps, wd, inv_bc1, inv_bc2, scale, flag, hyper);
  return hipGetLastError();
}

hipError_t LaunchAdamWMulti(const AdamWTable& tab, float lr, float beta1, float beta2, float eps,
                            float wd, float inv_bc1, float inv_bc2, const int* flag, hipStream_t s,
                            const float* hyper) {
  if (tab.count <= 0 || tab.count > kAdamWMulti) return hipErrorInvalidValue;
  AdamWTable t = tab;
  int blocks = 0;
  for (int i = 0; i < t.count; ++i) {
    t.first[i] = blocks;
    blocks += static_cast<int>(GridFor(t.t[i].n ? t.t[i].n : 1, kThreads, 4096));
  }
  t.first[t.count] = blocks;
  hipLaunchKernelGGL(AdamWMultiKernel, dim3(blocks), dim3(kThreads), 0, s, t, lr, beta1, beta2,
                     eps, wd, inv_bc1, inv_bc2, flag, hyper);
  return hipGetLastError();
}

hipError_t LaunchSgd(float* p, const float* g, size_t n, float lr, float wd, const float* scale,
                     const int* flag, hipStream_t s, const float* hyper) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(SgdKernel, dim3(GridFor(n, kThreads, 4096)), dim3(kThreads), 0, s, p, g, n, lr,
                     wd, scale, flag, hyper);
  return hipGetLastError();
}

}  // namespace seeai
