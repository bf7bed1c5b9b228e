// k_loss.hip -- softmax cross-entropy forward / backward (and the masked
// pair) on gfx950 (runtime/executor/loss.cc:21-126).
//
// Forward: one 1024-lane workgroup per row holds the row in registers (up
// to 32 floats a lane, so a 32k vocabulary is read from HBM exactly once),
// reduces the max and the exp-sum in a fixed butterfly order, writes the
// probabilities once, and leaves the row's -log p[label] as a double.  A
// second one-workgroup kernel sums those doubles in a fixed tree and writes
// the f32 mean into the loss slot -- deterministic at any grid, no atomics.
// Backward: scale = seed / N (or / T) divided on the device exactly as the
// reference divides it, then one coalesced pass.
#include "common.h"

namespace seeai {
namespace {

constexpr int kRowThreads = 1024;
constexpr int kPerLane = 32;  // register-resident row up to 32768 classes

__global__ void __launch_bounds__(kRowThreads)
XEntFwdRowKernel(const float* __restrict__ logits, const int32_t* __restrict__ labels,
                 float* __restrict__ probs, double* __restrict__ row_loss, size_t C, int masked) {
  __shared__ float redf[kRowThreads / kWave];
  const size_t r = blockIdx.x;
  const float* x = logits + r * C;
  float* p = probs + r * C;
  const bool resident = C <= static_cast<size_t>(kRowThreads) * kPerLane;
  float v[kPerLane];
  float mx = -INFINITY;
  bool any = false;
  if (resident) {
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const size_t c = threadIdx.x + static_cast<size_t>(i) * kRowThreads;
      v[i] = c < C ? x[c] : -INFINITY;
      if (c < C) {
        mx = any ? fmaxf(mx, v[i]) : v[i];
        any = true;
      }
    }
  } else {
    for (size_t c = threadIdx.x; c < C; c += kRowThreads) {
      mx = any ? fmaxf(mx, x[c]) : x[c];
      any = true;
    }
  }
  // fmax ignores NaN exactly as the reference's std::fmax chain does.
  if (!any) mx = NAN;  // no element on this lane: the identity of fmax
  mx = BlockMaxF<kRowThreads>(mx, redf);
  float sum = 0.0f;
  if (resident) {
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const size_t c = threadIdx.x + static_cast<size_t>(i) * kRowThreads;
      if (c < C) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
      }
    }
  } else {
    for (size_t c = threadIdx.x; c < C; c += kRowThreads) sum += expf(x[c] - mx);
  }
  sum = BlockSumF<kRowThreads>(sum, redf);
  const float inv_sum = 1.0f / sum;
  if (resident) {
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const size_t c = threadIdx.x + static_cast<size_t>(i) * kRowThreads;
      if (c < C) p[c] = v[i] * inv_sum;
    }
  } else {
    for (size_t c = threadIdx.x; c < C; c += kRowThreads) p[c] = expf(x[c] - mx) * inv_sum;
  }
  if (threadIdx.x == 0) {
    const int32_t lab = labels[r];
    double term = 0.0;
    if (!(masked && lab < 0)) {
      // The label's probability as this workgroup computed and stored it;
      // NaN propagates, the clamp only rescues underflow (loss.cc:45-51).
      const size_t c = static_cast<size_t>(lab);
      const float pl = expf(x[c] - mx) * inv_sum;
      const double safe = pl != pl ? static_cast<double>(pl) : static_cast<double>(fmaxf(pl, 1e-12f));
      term = -log(safe);
    }
    row_loss[r] = term;
  }
}

// Fixed-order mean of the per-row terms (and, masked, the target count).
__global__ void __launch_bounds__(1024)
XEntFinishKernel(const double* __restrict__ row_loss, const int32_t* __restrict__ labels,
                 float* __restrict__ loss, size_t N, int masked) {
  __shared__ double red[1024 / kWave];
  double total = 0.0, targets = 0.0;
  for (size_t r = threadIdx.x; r < N; r += 1024) {
    total += row_loss[r];
    if (!masked || labels[r] >= 0) targets += 1.0;
  }
  total = BlockSumD<1024>(total, red);
  targets = BlockSumD<1024>(targets, red);
  if (threadIdx.x == 0) {
    if (masked)
      *loss = targets > 0.0 ? static_cast<float>(total / targets) : 0.0f;
    else
      *loss = static_cast<float>(total / static_cast<double>(N));
  }
}

// The backward scale: seed / N, or seed / T over the target rows (masked).
__global__ void __launch_bounds__(1024)
XEntScaleKernel(const int32_t* __restrict__ labels, const float* __restrict__ seed,
                float* __restrict__ scale, size_t N, int masked) {
  __shared__ double red[1024 / kWave];
  double t = 0.0;
  if (masked)
    for (size_t r = threadIdx.x; r < N; r += 1024) t += labels[r] >= 0 ? 1.0 : 0.0;
  t = BlockSumD<1024>(t, red);
  if (threadIdx.x == 0) {
    if (masked) {
      const uint64_t T = static_cast<uint64_t>(t);
      *scale = T ? *seed / static_cast<float>(T) : 0.0f;
    } else {
      *scale = *seed / static_cast<float>(N);
    }
  }
}

__global__ void __launch_bounds__(256)
XEntBwdKernel(const float* __restrict__ probs, const int32_t* __restrict__ labels,
              const float* __restrict__ scale_p, float* __restrict__ dl, size_t N, size_t C,
              int masked) {
  const float scale = *scale_p;
  const size_t total = N * C;
  const size_t stride = static_cast<size_t>(gridDim.x) * 256;
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    const size_t r = i / C, c = i % C;
    const int32_t lab = labels[r];
    if (masked && lab < 0) {
      dl[i] = 0.0f;
      continue;
    }
    float v = scale * probs[i];
    if (static_cast<size_t>(lab) == c) v -= scale;
    dl[i] = v;
  }
}

}  // namespace

hipError_t LaunchXEntFwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                         size_t N, size_t C, int masked, void* ws, hipStream_t s) {
  if (N == 0) return hipSuccess;
  double* row_loss = static_cast<double*>(ws);
  hipLaunchKernelGGL(XEntFwdRowKernel, dim3(static_cast<unsigned>(N)), dim3(kRowThreads), 0, s,
                     logits, labels, probs, row_loss, C, masked);
  hipLaunchKernelGGL(XEntFinishKernel, dim3(1), dim3(1024), 0, s, row_loss, labels, loss, N, masked);
  return hipGetLastError();
}

hipError_t LaunchXEntBwd(const float* probs, const int32_t* labels, const float* seed,
                         float* dlogits, size_t N, size_t C, int masked, void* ws,
                         hipStream_t s) {
  if (N == 0) return hipSuccess;
  float* scale = static_cast<float*>(ws);
  hipLaunchKernelGGL(XEntScaleKernel, dim3(1), dim3(1024), 0, s, labels, seed, scale, N, masked);
  hipLaunchKernelGGL(XEntBwdKernel, dim3(GridFor(N * C, 256, 16384)), dim3(256), 0, s, probs,
                     labels, scale, dlogits, N, C, masked);
  return hipGetLastError();
}

}  // namespace seeai
