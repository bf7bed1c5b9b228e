// k_attention.hip -- causal scaled-dot-product attention on gfx950: the
// tiled family's four opcodes (kAttnFwdTiled / DQ / DK / DV, with the
// segment mask and the 4-float stats row, source/plan/instruction.h:
// 158-259) on MFMA, plus the cached family (kAttnFwd / DP / DV /
// SoftmaxRowsBwd / DQ / DK) for plan completeness.
//
// Layout (runtime/executor/update_kernels.h:150-154): q, k, v, o are
// [B*S, H*d] row-major with heads interleaved along the row; stats is
// [B*H*S, 4] = (row max m, 1/l, delta, clamped document start).
//
// Head widths 64 and 128 on 16-byte aligned operands run the exact family
// of k_attn32.hip (f32 MFMA, the other side staged through LDS); with the
// relaxed grant and the backend on bf16 attention, the flash kernels of
// k_flash.hip (bf16 MFMA) or, in plans at width 64, k_attn16.hip.  Other
// head widths run the per-row kernels below (double dots, the reference's
// loop order).
#include <cstdlib>

#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;
__device__ __forceinline__ size_t AttnStart(float stored, size_t i) {
  // instruction.h:246-250: clamped into [0, i], NaN to 0.
  if (!(stored > 0.0f)) return 0;
  const float cap = static_cast<float>(i);
  return stored >= cap ? i : static_cast<size_t>(stored);
}

// ---------------------------------------------------------------------------
// Per-row kernels: any head width, the reference's loops and double dots.
// One lane per (b, h, row) unit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double DotD(const float* a, const float* b, size_t d) {
  double acc = 0.0;
  for (size_t x = 0; x < d; ++x) acc += static_cast<double>(a[x]) * static_cast<double>(b[x]);
  return acc;
}

__global__ void __launch_bounds__(kThreads)
AttnFwdRowKernel(const float* __restrict__ q, const float* __restrict__ k,
                 const float* __restrict__ v, float* __restrict__ o, float* __restrict__ stats,
                 float* __restrict__ probs, size_t B, size_t S, size_t H, size_t d,
                 const int32_t* __restrict__ starts) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, i = u % S;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(d));
  const float* qi = q + (b * S + i) * D + h * d;
  size_t j0 = 0;
  if (starts) {
    const int32_t s0 = starts[b * S + i];
    j0 = s0 <= 0 ? 0 : (static_cast<size_t>(s0) < i ? static_cast<size_t>(s0) : i);
  }
  float row_max = -INFINITY;
  for (size_t j = j0; j <= i; ++j) {
    const float s = static_cast<float>(DotD(qi, k + (b * S + j) * D + h * d, d)) * inv_sqrt_d;
    if (s > row_max) row_max = s;
  }
  double denom = 0.0;
  for (size_t j = j0; j <= i; ++j) {
    const float s = static_cast<float>(DotD(qi, k + (b * S + j) * D + h * d, d)) * inv_sqrt_d;
    denom += expf(s - row_max);
  }
  const float inv_denom = 1.0f / static_cast<float>(denom);
  float* oi = o + (b * S + i) * D + h * d;
  for (size_t x = 0; x < d; ++x) oi[x] = 0.0f;
  if (probs)
    for (size_t j = 0; j < S; ++j) probs[u * S + j] = 0.0f;
  for (size_t j = j0; j <= i; ++j) {
    const float s = static_cast<float>(DotD(qi, k + (b * S + j) * D + h * d, d)) * inv_sqrt_d;
    const float p = expf(s - row_max) * inv_denom;
    if (probs) probs[u * S + j] = p;
    const float* vj = v + (b * S + j) * D + h * d;
    for (size_t x = 0; x < d; ++x) oi[x] += p * vj[x];
  }
  if (stats) {
    float* st = stats + u * 4;
    st[0] = row_max;
    st[1] = inv_denom;
    st[2] = 0.0f;
    st[3] = static_cast<float>(j0);
  }
}

__global__ void __launch_bounds__(kThreads)
AttnDQRowKernel(const float* __restrict__ q, const float* __restrict__ k,
                const float* __restrict__ v, const float* __restrict__ dout,
                float* __restrict__ stats, float* __restrict__ dq, size_t B, size_t S, size_t H,
                size_t d) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, i = u % S;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(d));
  const float* qi = q + (b * S + i) * D + h * d;
  const float* doi = dout + (b * S + i) * D + h * d;
  float* st = stats + u * 4;
  const size_t j0 = AttnStart(st[3], i);
  double dot = 0.0;
  for (size_t j = j0; j <= i; ++j) {
    const float s = static_cast<float>(DotD(qi, k + (b * S + j) * D + h * d, d)) * inv_sqrt_d;
    const float p = expf(s - st[0]) * st[1];
    const float dp = static_cast<float>(DotD(doi, v + (b * S + j) * D + h * d, d));
    dot += static_cast<double>(dp) * p;
  }
  const float delta = static_cast<float>(dot);
  float* dqi = dq + (b * S + i) * D + h * d;
  for (size_t x = 0; x < d; ++x) dqi[x] = 0.0f;
  for (size_t j = j0; j <= i; ++j) {
    const float s = static_cast<float>(DotD(qi, k + (b * S + j) * D + h * d, d)) * inv_sqrt_d;
    const float p = expf(s - st[0]) * st[1];
    const float dp = static_cast<float>(DotD(doi, v + (b * S + j) * D + h * d, d));
    const float gg = (p * (dp - delta)) * inv_sqrt_d;
    const float* kj = k + (b * S + j) * D + h * d;
    for (size_t x = 0; x < d; ++x) dqi[x] += gg * kj[x];
  }
  st[2] = delta;
}

template <bool kDV>
__global__ void __launch_bounds__(kThreads)
AttnDKDVRowKernel(const float* __restrict__ q, const float* __restrict__ k,
                  const float* __restrict__ v, const float* __restrict__ dout,
                  const float* __restrict__ stats, float* __restrict__ out, size_t B, size_t S,
                  size_t H, size_t d) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, j = u % S;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(d));
  const float* kj = k + (b * S + j) * D + h * d;
  const float* vj = v + (b * S + j) * D + h * d;
  float* oj = out + (b * S + j) * D + h * d;
  for (size_t x = 0; x < d; ++x) oj[x] = 0.0f;
  for (size_t i = j; i < S; ++i) {
    const float* qi = q + (b * S + i) * D + h * d;
    const float* doi = dout + (b * S + i) * D + h * d;
    const float* st = stats + ((b * H + h) * S + i) * 4;
    if (j < AttnStart(st[3], i)) continue;
    const float s = static_cast<float>(DotD(qi, kj, d)) * inv_sqrt_d;
    const float p = expf(s - st[0]) * st[1];
    if (kDV) {
      for (size_t x = 0; x < d; ++x) oj[x] += p * doi[x];
    } else {
      const float dp = static_cast<float>(DotD(doi, vj, d));
      const float gg = (p * (dp - st[2])) * inv_sqrt_d;
      for (size_t x = 0; x < d; ++x) oj[x] += gg * qi[x];
    }
  }
}

// Cached-family backward primitives (attention.cc:243-343).
__global__ void __launch_bounds__(kThreads)
AttnDPRowKernel(const float* __restrict__ dout, const float* __restrict__ v, float* __restrict__ dp,
                size_t B, size_t S, size_t H, size_t d) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, i = u % S;
  const float* doi = dout + (b * S + i) * D + h * d;
  for (size_t j = 0; j < S; ++j)
    dp[u * S + j] = j <= i ? static_cast<float>(DotD(doi, v + (b * S + j) * D + h * d, d)) : 0.0f;
}

__global__ void __launch_bounds__(kThreads)
AttnDVCachedRowKernel(const float* __restrict__ probs, const float* __restrict__ dout,
                      float* __restrict__ dv, size_t B, size_t S, size_t H, size_t d) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, j = u % S;
  float* dvj = dv + (b * S + j) * D + h * d;
  for (size_t x = 0; x < d; ++x) dvj[x] = 0.0f;
  for (size_t i = j; i < S; ++i) {
    const float p = probs[((b * H + h) * S + i) * S + j];
    const float* doi = dout + (b * S + i) * D + h * d;
    for (size_t x = 0; x < d; ++x) dvj[x] += p * doi[x];
  }
}

__global__ void __launch_bounds__(kThreads)
SoftmaxRowsBwdKernel(const float* __restrict__ probs, const float* __restrict__ dp,
                     float* __restrict__ ds, size_t cols) {
  __shared__ double red[kThreads / kWave];
  const size_t r = blockIdx.x;
  const float* pr = probs + r * cols;
  const float* dpr = dp + r * cols;
  double dot = 0.0;
  for (size_t x = threadIdx.x; x < cols; x += kThreads) dot += static_cast<double>(dpr[x]) * pr[x];
  dot = BlockSumD<kThreads>(dot, red);
  const float sum = static_cast<float>(dot);
  for (size_t x = threadIdx.x; x < cols; x += kThreads) ds[r * cols + x] = pr[x] * (dpr[x] - sum);
}

template <bool kDK>
__global__ void __launch_bounds__(kThreads)
AttnDQDKCachedRowKernel(const float* __restrict__ ds, const float* __restrict__ x,
                        float* __restrict__ out, size_t B, size_t S, size_t H, size_t d) {
  const size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= B * H * S) return;
  const size_t D = H * d, b = u / (H * S), h = (u / S) % H, t = u % S;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(d));
  float* ot = out + (b * S + t) * D + h * d;
  for (size_t y = 0; y < d; ++y) ot[y] = 0.0f;
  if (!kDK) {
    for (size_t j = 0; j <= t; ++j) {
      const float gg = ds[u * S + j] * inv_sqrt_d;
      const float* xj = x + (b * S + j) * D + h * d;
      for (size_t y = 0; y < d; ++y) ot[y] += gg * xj[y];
    }
  } else {
    for (size_t i = t; i < S; ++i) {
      const float gg = ds[((b * H + h) * S + i) * S + t] * inv_sqrt_d;
      const float* xi = x + (b * S + i) * D + h * d;
      for (size_t y = 0; y < d; ++y) ot[y] += gg * xi[y];
    }
  }
}

bool MfmaShape(size_t d, const void* a, const void* b) {
  return (d == 64 || d == 128) && (reinterpret_cast<uintptr_t>(a) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(b) & 15) == 0;
}

inline unsigned UnitsGrid(size_t n) { return GridFor(n, kThreads, 1u << 30); }

}  // namespace

hipError_t LaunchAttnFwdTiled(int dtype, const float* q, const float* k, const float* v, float* o,
                              float* stats, size_t B, size_t S, size_t H, size_t d,
                              const int32_t* starts, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (dtype && MfmaShape(d, q, k) && MfmaShape(d, v, o) && FlashFits(B, S, H, d))
    return LaunchFlashFwd(q, k, v, o, stats, B, S, H, d, starts, s);
  if (Attn32Fits(B, S, H, d, {q, k, v, o, stats}))
    return LaunchAttn32Fwd(q, k, v, o, stats, B, S, H, d, starts, s);
  hipLaunchKernelGGL(AttnFwdRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q, k, v, o,
                     stats, static_cast<float*>(nullptr), B, S, H, d, starts);
  return hipGetLastError();
}

// The relaxed dQ runs in one pass (dQ = K^T (p dP) - delta K^T p) unless
// SEEAI_DQ_TWO_PASS=1 selects the two-pass form (delta first), kept for
// comparison.
int FlashDQOnePass() {
  static const int one = [] {
    const char* e = std::getenv("SEEAI_DQ_TWO_PASS");
    return e && e[0] == '1' ? 0 : 1;
  }();
  return one;
}

hipError_t LaunchAttnDQTiled(int dtype, const float* q, const float* k, const float* v,
                             const float* dout, float* stats, float* dq, size_t B, size_t S,
                             size_t H, size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (dtype && MfmaShape(d, q, k) && MfmaShape(d, v, dout) && MfmaShape(d, dq, q) &&
      FlashFits(B, S, H, d))
    return LaunchFlashDQ(q, k, v, dout, stats, dq, B, S, H, d, FlashDQOnePass(), s);
  if (Attn32Fits(B, S, H, d, {q, k, v, dout, stats, dq}))
    return LaunchAttn32DQ(q, k, v, dout, stats, dq, B, S, H, d, s);
  hipLaunchKernelGGL(AttnDQRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q, k, v,
                     dout, stats, dq, B, S, H, d);
  return hipGetLastError();
}

hipError_t LaunchAttnDKTiled(int dtype, const float* q, const float* k, const float* v,
                             const float* dout, const float* stats, float* dk, size_t B,
                             size_t S, size_t H, size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (dtype && MfmaShape(d, q, k) && MfmaShape(d, v, dout) && MfmaShape(d, dk, q) &&
      FlashFits(B, S, H, d))
    return LaunchFlashDKDV(q, k, v, dout, stats, dk, nullptr, B, S, H, d, s);
  if (Attn32Fits(B, S, H, d, {q, k, v, dout, stats, dk}))
    return LaunchAttn32DKDV(q, k, v, dout, stats, dk, nullptr, B, S, H, d, s);
  hipLaunchKernelGGL(AttnDKDVRowKernel<false>, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q,
                     k, v, dout, stats, dk, B, S, H, d);
  return hipGetLastError();
}

hipError_t LaunchAttnDVTiled(int dtype, const float* q, const float* k, const float* dout,
                             const float* stats, float* dv, size_t B, size_t S, size_t H,
                             size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (dtype && MfmaShape(d, q, k) && MfmaShape(d, dout, dv) && FlashFits(B, S, H, d))
    return LaunchFlashDKDV(q, k, nullptr, dout, stats, nullptr, dv, B, S, H, d, s);
  if (Attn32Fits(B, S, H, d, {q, k, dout, stats, dv}))
    return LaunchAttn32DKDV(q, k, nullptr, dout, stats, nullptr, dv, B, S, H, d, s);
  hipLaunchKernelGGL(AttnDKDVRowKernel<true>, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q,
                     k, static_cast<const float*>(nullptr), dout, stats, dv, B, S, H, d);
  return hipGetLastError();
}

// dK and dV of one attention in a single pass: the relaxed family only,
// where the flash kernels take the shape and fuse at this head size.
bool AttnDKDVFusable(const float* q, const float* k, const float* v, const float* dout,
                     const float* dk, const float* dv, size_t B, size_t S, size_t H, size_t d) {
  return B * H * S > 0 && MfmaShape(d, q, k) && MfmaShape(d, v, dout) && MfmaShape(d, dk, dv) &&
         FlashFits(B, S, H, d) && FlashFusedDKDV(d);
}

// dK and dV of the exact family in one pass: each output computed by the
// instructions its own pass would run (k_attn32.hip's DK / DV template).
bool AttnDKDVExactFusable(const float* q, const float* k, const float* v, const float* dout,
                          const float* stats, const float* dk, const float* dv, size_t B, size_t S,
                          size_t H, size_t d) {
  return B * H * S > 0 && Attn32Fits(B, S, H, d, {q, k, v, dout, stats, dk, dv});
}

hipError_t LaunchAttnDKDVExact(const float* q, const float* k, const float* v, const float* dout,
                               const float* stats, float* dk, float* dv, size_t B, size_t S,
                               size_t H, size_t d, hipStream_t s) {
  if (!AttnDKDVExactFusable(q, k, v, dout, stats, dk, dv, B, S, H, d)) return hipErrorNotSupported;
  return LaunchAttn32DKDV(q, k, v, dout, stats, dk, dv, B, S, H, d, s);
}

hipError_t LaunchAttnDKDVFused(const float* q, const float* k, const float* v, const float* dout,
                               const float* stats, float* dk, float* dv, size_t B, size_t S,
                               size_t H, size_t d, hipStream_t s) {
  if (!AttnDKDVFusable(q, k, v, dout, dk, dv, B, S, H, d)) return hipErrorNotSupported;
  return LaunchFlashDKDV(q, k, v, dout, stats, dk, dv, B, S, H, d, s);
}

hipError_t LaunchAttnFwdCached(const float* q, const float* k, const float* v, float* o,
                               float* probs, size_t B, size_t S, size_t H, size_t d,
                               const int32_t* starts, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  hipLaunchKernelGGL(AttnFwdRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q, k, v, o,
                     static_cast<float*>(nullptr), probs, B, S, H, d, starts);
  return hipGetLastError();
}
hipError_t LaunchAttnDP(const float* dout, const float* v, float* dp, size_t B, size_t S,
                        size_t H, size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  hipLaunchKernelGGL(AttnDPRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, dout, v, dp,
                     B, S, H, d);
  return hipGetLastError();
}
hipError_t LaunchAttnDV(const float* probs, const float* dout, float* dv, size_t B, size_t S,
                        size_t H, size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  hipLaunchKernelGGL(AttnDVCachedRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, probs,
                     dout, dv, B, S, H, d);
  return hipGetLastError();
}
hipError_t LaunchSoftmaxRowsBwd(const float* probs, const float* dp, float* ds, size_t rows,
                                size_t cols, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(SoftmaxRowsBwdKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                     probs, dp, ds, cols);
  return hipGetLastError();
}
hipError_t LaunchAttnDQ(const float* ds, const float* k, float* dq, size_t B, size_t S, size_t H,
                        size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  hipLaunchKernelGGL(AttnDQDKCachedRowKernel<false>, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0,
                     s, ds, k, dq, B, S, H, d);
  return hipGetLastError();
}
hipError_t LaunchAttnDK(const float* ds, const float* q, float* dk, size_t B, size_t S, size_t H,
                        size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  hipLaunchKernelGGL(AttnDQDKCachedRowKernel<true>, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0,
                     s, ds, q, dk, B, S, H, d);
  return hipGetLastError();
}

}  // namespace seeai
