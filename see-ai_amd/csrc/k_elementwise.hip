// k_elementwise.hip -- the HBM-bound plan-completeness family on gfx950:
// pointwise arithmetic and activations, the bias broadcast, the column
// reduction, fused elementwise chains, the embedding gather, LayerNorm,
// RMSNorm, RoPE and the eval argmax.
//
// Pointwise kernels are one element per lane over a grid-stride loop with
// 16-byte loads where the tensor allows; every element has one writer, so
// results never depend on the grid.  Row kernels (norms, argmax) give one
// 256-lane workgroup to a row and reduce in a fixed butterfly + wave order.
// Every expression is the reference's own (built -ffp-contract=off), so the
// arithmetic kernels reproduce the reference's bits wherever no libm call
// is involved.
#include <algorithm>

#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;

template <typename F>
__global__ void __launch_bounds__(kThreads) MapKernel(size_t n, F f) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    f(i);
}

template <typename F>
hipError_t Map(size_t n, hipStream_t s, F f) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(MapKernel<F>, dim3(GridFor(n, kThreads, 8192)), dim3(kThreads), 0, s, n, f);
  return hipGetLastError();
}

// elementwise.cc:16-27 / 38-48 as 4-wide vectors when n and the pointers
// allow (the same per-element expression; vectors only widen the access).
__global__ void __launch_bounds__(kThreads)
AddEW4(const float4* __restrict__ x, const float4* __restrict__ y, float4* __restrict__ o, size_t n4,
       Bf16Sink sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 a = x[i], b = y[i];
    const float4 v = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    if (sink.store_f32) o[i] = v;
    if (sink.out) SinkStore4(sink, 4 * i, v);
  }
}

// A normalisation's output row: float4 where the row allows it (the same
// per-element expression), with the sink; element by element otherwise.
// With a residual row rr, the row stored is rr + the element (a residual
// add fused behind the normalisation).
template <class F>
__device__ __forceinline__ void NormRowOut(float* yr, size_t row0, size_t cols, bool vec,
                                           const Bf16Sink& sink, const float* rr, F&& elem) {
  if (vec) {
    for (size_t c = threadIdx.x * 4; c < cols; c += kThreads * 4) {
      float4 v = make_float4(elem(c), elem(c + 1), elem(c + 2), elem(c + 3));
      if (rr) {
        const float4 r = *reinterpret_cast<const float4*>(rr + c);
        v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
      }
      if (sink.store_f32) *reinterpret_cast<float4*>(yr + c) = v;
      if (sink.out) SinkStore4(sink, row0 + c, v);
    }
  } else {
    for (size_t c = threadIdx.x; c < cols; c += kThreads) yr[c] = rr ? rr[c] + elem(c) : elem(c);
  }
}

inline bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// kFusedMap (elementwise.cc:56-149, instruction.h:270-297).
struct FusedProgram {
  uint8_t stage[4];
  int count;
};

__global__ void __launch_bounds__(kThreads)
FusedMapKernel(const float* __restrict__ x, const float* __restrict__ o1,
               const float* __restrict__ o2, float* __restrict__ out, size_t n,
               FusedProgram prog, float imm0, float imm1) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    float run = x[i];
    for (int s = 0; s < prog.count; ++s) {
      const uint8_t st = prog.stage[s];
      const int arg = (st >> 4) & 3;
      const bool right = (st & 0x80) != 0;
      const float* other = arg == 1 ? o1 : o2;
      switch (st & 0x0F) {
        case 1: run = right ? other[i] + run : run + other[i]; break;
        case 2: run = right ? other[i] * run : run * other[i]; break;
        case 3: run = (arg == 0 ? imm0 : imm1) * run; break;
        case 4: run = ReluExpr(run); break;
        case 5: run = GeluExpr(run); break;
        case 6: run = SiluExpr(run); break;
        default: break;
      }
    }
    out[i] = run;
  }
}

// ReduceRows (elementwise.cc:160-187): one lane per column walking the rows
// in order -- the reference's per-column association exactly.
__global__ void __launch_bounds__(kThreads)
ReduceRowsKernel(const float* __restrict__ dy, float* __restrict__ db, size_t rows, size_t cols) {
  const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.0f;
  for (size_t r = 0; r < rows; ++r) acc += dy[r * cols + c];
  db[c] = acc;
}

// EmbedFwd (elementwise.cc:151-158): one workgroup per token row.
__global__ void __launch_bounds__(kThreads)
EmbedKernel(const int32_t* __restrict__ tokens, const float* __restrict__ table,
            float* __restrict__ out, size_t dim) {
  const size_t r = blockIdx.x;
  const float* src = table + static_cast<size_t>(tokens[r]) * dim;
  float* dst = out + r * dim;
  for (size_t c = threadIdx.x; c < dim; c += kThreads) dst[c] = src[c];
}

// LayerNorm forward (normalization.cc:17-45): double row sums, f32 stats.
__global__ void __launch_bounds__(kThreads)
LayerNormFwdKernel(const float* __restrict__ x, const float* __restrict__ g,
                   const float* __restrict__ b, float* __restrict__ y, float* __restrict__ mean,
                   float* __restrict__ rstd, size_t cols, float eps, int vec, Bf16Sink sink) {
  __shared__ double red[kThreads / kWave];
  const size_t r = blockIdx.x;
  const float* xr = x + r * cols;
  double sum = 0.0;
  for (size_t c = threadIdx.x; c < cols; c += kThreads) sum += xr[c];
  sum = BlockSumD<kThreads>(sum, red);
  const float mu = static_cast<float>(sum / static_cast<double>(cols));
  double var = 0.0;
  for (size_t c = threadIdx.x; c < cols; c += kThreads) {
    const double d = static_cast<double>(xr[c]) - mu;
    var += d * d;
  }
  var = BlockSumD<kThreads>(var, red);
  const float rs = 1.0f / sqrtf(static_cast<float>(var / static_cast<double>(cols)) + eps);
  if (threadIdx.x == 0) {
    mean[r] = mu;
    rstd[r] = rs;
  }
  NormRowOut(y + r * cols, r * cols, cols, vec, sink, nullptr,
             [&](size_t c) { return (xr[c] - mu) * rs * g[c] + b[c]; });
}

// LayerNorm backward (normalization.cc:47-78).
__global__ void __launch_bounds__(kThreads)
LayerNormBwdKernel(const float* __restrict__ dy, const float* __restrict__ x,
                   const float* __restrict__ g, const float* __restrict__ mean,
                   const float* __restrict__ rstd, float* dx, size_t cols, int vec,
                   Bf16Sink sink, const float* res) {
  __shared__ double red[kThreads / kWave];
  const size_t r = blockIdx.x;
  const float* dyr = dy + r * cols;
  const float* xr = x + r * cols;
  const float mu = mean[r], rs = rstd[r];
  double sg = 0.0, sgx = 0.0;
  for (size_t c = threadIdx.x; c < cols; c += kThreads) {
    const float xhat = (xr[c] - mu) * rs;
    const float gg = dyr[c] * g[c];
    sg += gg;
    sgx += static_cast<double>(gg) * xhat;
  }
  sg = BlockSumD<kThreads>(sg, red);
  sgx = BlockSumD<kThreads>(sgx, red);
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float mg = static_cast<float>(sg) * inv_d;
  const float mgx = static_cast<float>(sgx) * inv_d;
  NormRowOut(dx + r * cols, r * cols, cols, vec, sink, res ? res + r * cols : nullptr, [&](size_t c) {
    const float xhat = (xr[c] - mu) * rs;
    const float gg = dyr[c] * g[c];
    return rs * (gg - mg - xhat * mgx);
  });
}

// RMSNorm forward / backward (normalization.cc:80-113).
__global__ void __launch_bounds__(kThreads)
RmsNormFwdKernel(const float* __restrict__ x, const float* __restrict__ g, float* __restrict__ y,
                 float* __restrict__ rstd, size_t cols, float eps, int vec, Bf16Sink sink) {
  __shared__ double red[kThreads / kWave];
  const size_t r = blockIdx.x;
  const float* xr = x + r * cols;
  double ss = 0.0;
  for (size_t c = threadIdx.x; c < cols; c += kThreads) ss += static_cast<double>(xr[c]) * xr[c];
  ss = BlockSumD<kThreads>(ss, red);
  const float rs = 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(cols)) + eps);
  if (threadIdx.x == 0) rstd[r] = rs;
  NormRowOut(y + r * cols, r * cols, cols, vec, sink, nullptr,
             [&](size_t c) { return xr[c] * rs * g[c]; });
}

__global__ void __launch_bounds__(kThreads)
RmsNormBwdKernel(const float* __restrict__ dy, const float* __restrict__ x,
                 const float* __restrict__ g, const float* __restrict__ rstd,
                 float* dx, size_t cols, int vec, Bf16Sink sink, const float* res) {
  __shared__ double red[kThreads / kWave];
  const size_t r = blockIdx.x;
  const float* dyr = dy + r * cols;
  const float* xr = x + r * cols;
  const float rs = rstd[r];
  double sgx = 0.0;
  for (size_t c = threadIdx.x; c < cols; c += kThreads)
    sgx += static_cast<double>(dyr[c] * g[c]) * xr[c];
  sgx = BlockSumD<kThreads>(sgx, red);
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float mgx = static_cast<float>(sgx) * inv_d;
  NormRowOut(dx + r * cols, r * cols, cols, vec, sink, res ? res + r * cols : nullptr,
             [&](size_t c) { return rs * (dyr[c] * g[c] - xr[c] * rs * rs * mgx); });
}

// The normalisations with a row per wave (rows of at most 256 kV floats,
// a multiple of 4, 16-byte aligned operands): lane l holds float4 l + 64 j
// of its row in registers, so the row is read once; the double sums are
// wave reductions (the same sums as the block kernels above, in another
// association -- f32 stats within an ulp of them), and the outputs are the
// block kernels' per-element expressions, with the sink and the residual.
template <int kV>
__device__ __forceinline__ void LoadRow4(const float* __restrict__ p, int lane, size_t cols,
                                         float4 (&v)[kV]) {
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const size_t c = 4 * static_cast<size_t>(lane + kWave * j);
    v[j] = c < cols ? *reinterpret_cast<const float4*>(p + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// With `has_res`, rv holds the residual row (loaded with the row's operands,
// so its latency hides behind the sums).
template <int kV, class F>
__device__ __forceinline__ void StoreRow4(float* yr, size_t row0, size_t cols, int lane,
                                          const Bf16Sink& sink, bool has_res,
                                          const float4 (&rv)[kV], F&& elem) {
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const size_t c = 4 * static_cast<size_t>(lane + kWave * j);
    if (c >= cols) continue;
    float4 v = make_float4(elem(j, 0), elem(j, 1), elem(j, 2), elem(j, 3));
    if (has_res) {
      const float4 r = rv[j];
      v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
    }
    if (sink.store_f32) *reinterpret_cast<float4*>(yr + c) = v;
    if (sink.out) SinkStore4(sink, row0 + c, v);
  }
}

__device__ __forceinline__ float Comp(const float4& v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

template <int kV>
__global__ void __launch_bounds__(kThreads)
LayerNormFwdRows(const float* __restrict__ x, const float* __restrict__ g,
                 const float* __restrict__ b, float* __restrict__ y, float* __restrict__ mean,
                 float* __restrict__ rstd, size_t rows, size_t cols, float eps, Bf16Sink sink) {
  const int lane = threadIdx.x % kWave;
  const size_t r = static_cast<size_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float4 xv[kV];
  LoadRow4<kV>(x + r * cols, lane, cols, xv);
  double sum = 0.0;
#pragma unroll
  for (int j = 0; j < kV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += Comp(xv[j], e);
  sum = WaveSumD(sum);
  const float mu = static_cast<float>(sum / static_cast<double>(cols));
  double var = 0.0;
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    if (4 * static_cast<size_t>(lane + kWave * j) >= cols) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const double d = static_cast<double>(Comp(xv[j], e)) - mu;
      var += d * d;
    }
  }
  var = WaveSumD(var);
  const float rs = 1.0f / sqrtf(static_cast<float>(var / static_cast<double>(cols)) + eps);
  if (lane == 0) {
    mean[r] = mu;
    rstd[r] = rs;
  }
  StoreRow4<kV>(y + r * cols, r * cols, cols, lane, sink, false, xv, [&](int j, int e) {
    const size_t c = 4 * static_cast<size_t>(lane + kWave * j) + e;
    return (Comp(xv[j], e) - mu) * rs * g[c] + b[c];
  });
}

template <int kV>
__global__ void __launch_bounds__(kThreads)
LayerNormBwdRows(const float* __restrict__ dy, const float* __restrict__ x,
                 const float* __restrict__ g, const float* __restrict__ mean,
                 const float* __restrict__ rstd, float* dx, size_t rows, size_t cols,
                 Bf16Sink sink, const float* res) {
  const int lane = threadIdx.x % kWave;
  const size_t r = static_cast<size_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float4 xv[kV], dv[kV], rv[kV];
  LoadRow4<kV>(x + r * cols, lane, cols, xv);
  LoadRow4<kV>(dy + r * cols, lane, cols, dv);
  if (res) LoadRow4<kV>(res + r * cols, lane, cols, rv);
  const float mu = mean[r], rs = rstd[r];
  double sg = 0.0, sgx = 0.0;
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const size_t c0 = 4 * static_cast<size_t>(lane + kWave * j);
    if (c0 >= cols) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xhat = (Comp(xv[j], e) - mu) * rs;
      const float gg = Comp(dv[j], e) * g[c0 + e];
      sg += gg;
      sgx += static_cast<double>(gg) * xhat;
    }
  }
  sg = WaveSumD(sg);
  sgx = WaveSumD(sgx);
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float mg = static_cast<float>(sg) * inv_d;
  const float mgx = static_cast<float>(sgx) * inv_d;
  StoreRow4<kV>(dx + r * cols, r * cols, cols, lane, sink, res != nullptr, rv,
                [&](int j, int e) {
                  const size_t c = 4 * static_cast<size_t>(lane + kWave * j) + e;
                  const float xhat = (Comp(xv[j], e) - mu) * rs;
                  const float gg = Comp(dv[j], e) * g[c];
                  return rs * (gg - mg - xhat * mgx);
                });
}

template <int kV>
__global__ void __launch_bounds__(kThreads)
RmsNormFwdRows(const float* __restrict__ x, const float* __restrict__ g, float* __restrict__ y,
               float* __restrict__ rstd, size_t rows, size_t cols, float eps, Bf16Sink sink) {
  const int lane = threadIdx.x % kWave;
  const size_t r = static_cast<size_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float4 xv[kV];
  LoadRow4<kV>(x + r * cols, lane, cols, xv);
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < kV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += static_cast<double>(Comp(xv[j], e)) * Comp(xv[j], e);
  ss = WaveSumD(ss);
  const float rs = 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(cols)) + eps);
  if (lane == 0) rstd[r] = rs;
  StoreRow4<kV>(y + r * cols, r * cols, cols, lane, sink, false, xv, [&](int j, int e) {
    const size_t c = 4 * static_cast<size_t>(lane + kWave * j) + e;
    return Comp(xv[j], e) * rs * g[c];
  });
}

template <int kV>
__global__ void __launch_bounds__(kThreads)
RmsNormBwdRows(const float* __restrict__ dy, const float* __restrict__ x,
               const float* __restrict__ g, const float* __restrict__ rstd, float* dx,
               size_t rows, size_t cols, Bf16Sink sink, const float* res) {
  const int lane = threadIdx.x % kWave;
  const size_t r = static_cast<size_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float4 xv[kV], dv[kV], rv[kV];
  LoadRow4<kV>(x + r * cols, lane, cols, xv);
  LoadRow4<kV>(dy + r * cols, lane, cols, dv);
  if (res) LoadRow4<kV>(res + r * cols, lane, cols, rv);
  const float rs = rstd[r];
  double sgx = 0.0;
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const size_t c0 = 4 * static_cast<size_t>(lane + kWave * j);
    if (c0 >= cols) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      sgx += static_cast<double>(Comp(dv[j], e) * g[c0 + e]) * Comp(xv[j], e);
  }
  sgx = WaveSumD(sgx);
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float mgx = static_cast<float>(sgx) * inv_d;
  StoreRow4<kV>(dx + r * cols, r * cols, cols, lane, sink, res != nullptr, rv,
                [&](int j, int e) {
                  const size_t c = 4 * static_cast<size_t>(lane + kWave * j) + e;
                  return rs * (Comp(dv[j], e) * g[c] - Comp(xv[j], e) * rs * rs * mgx);
                });
}

// The float4 slots per lane for a row of `cols` (0: the row kernels do not
// take it -- over 4096 floats).
int RowSlots(size_t cols) {
  for (int v : {1, 2, 3, 4, 8, 16})
    if (static_cast<size_t>(v) * 256 >= cols) return v;
  return 0;
}

#define SEEAI_ROWS_SWITCH(KERNEL, ...)                                                        \
  switch (RowSlots(cols)) {                                                                  \
    case 1: hipLaunchKernelGGL((KERNEL<1>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break;  \
    case 2: hipLaunchKernelGGL((KERNEL<2>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break;  \
    case 3: hipLaunchKernelGGL((KERNEL<3>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break;  \
    case 4: hipLaunchKernelGGL((KERNEL<4>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break;  \
    case 8: hipLaunchKernelGGL((KERNEL<8>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break;  \
    default: hipLaunchKernelGGL((KERNEL<16>), grid, dim3(kThreads), 0, s, __VA_ARGS__); break; \
  }

// RoPE (attention.cc:103-174): one lane per interleaved pair (c, c+1) of a
// (b, s, h) head segment, so a wave moves 512 contiguous bytes in and out
// (float2 where the operands are 8-byte aligned).  The rotation is the
// reference's expression per pair.  Without a table the lane forms its
// pair's frequency by the reference's recurrence from 1 (c/2 products of
// `step`, rounded in order), so every angle is the reference's float;
// cos/sin are the device's.
template <bool kVec>
__global__ void __launch_bounds__(kThreads)
RopeKernel(const float* __restrict__ x, float* __restrict__ y, size_t B, size_t S, size_t H,
           size_t d, float step, const float* __restrict__ table, int backward) {
  const size_t half = d / 2, n = B * S * H * half;
  for (size_t u = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; u < n;
       u += static_cast<size_t>(gridDim.x) * kThreads) {
  const size_t p = u % half, seg = u / half;  // seg = (b s) H + h
  const size_t s = (seg / H) % S;
  const size_t at = seg * d + 2 * p;           // [B S, H d] row-major: seg * d
  float cs, sn;
  if (table) {
    const float* row = table + s * half * 2 + 2 * p;
    cs = row[0];
    sn = row[1];
  } else {
    float freq = 1.0f;
    for (size_t c = 0; c < p; ++c) freq *= step;
    const float theta = static_cast<float>(s) * freq;
    cs = cosf(theta);
    sn = sinf(theta);
  }
  float a, b2;
  if constexpr (kVec) {
    const float2 v = *reinterpret_cast<const float2*>(x + at);
    a = v.x;
    b2 = v.y;
  } else {
    a = x[at];
    b2 = x[at + 1];
  }
  float o0, o1;
  if (backward) {
    o0 = a * cs + b2 * sn;
    o1 = -a * sn + b2 * cs;
  } else {
    o0 = a * cs - b2 * sn;
    o1 = a * sn + b2 * cs;
  }
  if constexpr (kVec) {
    *reinterpret_cast<float2*>(y + at) = make_float2(o0, o1);
  } else {
    y[at] = o0;
    y[at + 1] = o1;
  }
  }
}

// RoPE with the table, rows of the [B S, H d] activation on the grid: the
// row's position s = row mod S is uniform across the workgroup, and a lane
// rotates two pairs -- one 16-byte read of x and one of the table row
// (cos p, sin p, cos p+1, sin p+1), 32-bit column arithmetic.  The same
// expressions as RopeKernel.  d % 4 == 0, x, y and the table 16-byte aligned.
__global__ void __launch_bounds__(kThreads)
RopeRowsKernel(const float* __restrict__ x, float* __restrict__ y, unsigned rows, unsigned S,
               unsigned width, unsigned d, const float* __restrict__ table, int backward,
               Bf16Sink sink) {
  for (unsigned r = blockIdx.y; r < rows; r += gridDim.y) {
    const unsigned s = r % S;
    const float* __restrict__ trow = table + static_cast<size_t>(s) * d;  // d/2 pairs x 2
    const size_t base = static_cast<size_t>(r) * width;
    for (unsigned c = (blockIdx.x * kThreads + threadIdx.x) * 4; c < width;
         c += gridDim.x * kThreads * 4) {
      const unsigned j = c % d;  // 2p: the pair index times two
      const float4 v = *reinterpret_cast<const float4*>(x + base + c);
      const float4 t = *reinterpret_cast<const float4*>(trow + j);
      float4 o;
      if (backward) {
        o.x = v.x * t.x + v.y * t.y;
        o.y = -v.x * t.y + v.y * t.x;
        o.z = v.z * t.z + v.w * t.w;
        o.w = -v.z * t.w + v.w * t.z;
      } else {
        o.x = v.x * t.x - v.y * t.y;
        o.y = v.x * t.y + v.y * t.x;
        o.z = v.z * t.z - v.w * t.w;
        o.w = v.z * t.w + v.w * t.z;
      }
      if (sink.store_f32) *reinterpret_cast<float4*>(y + base + c) = o;
      // y's bf16 copy: the attention's (plain), or a product's (its scales)
      if (sink.out) SinkStore4(sink, base + c, o);
    }
  }
}

__global__ void __launch_bounds__(kThreads)
RopeTableKernel(float* __restrict__ table, size_t S, size_t d, float step) {
  const size_t s = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (s >= S) return;
  const size_t half = d / 2;
  float* row = table + s * half * 2;
  float freq = 1.0f;
  for (size_t c = 0; c < half; ++c) {
    const float theta = static_cast<float>(s) * freq;
    row[2 * c] = cosf(theta);
    row[2 * c + 1] = sinf(theta);
    freq *= step;
  }
}

// SegmentStarts (attention.cc:176-185): a sequential scan per window.
__global__ void SegmentStartsKernel(const int32_t* __restrict__ tokens, int32_t* __restrict__ starts,
                                    size_t B, size_t S, int32_t eos) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int32_t start = 0;
  for (size_t t = 0; t < S; ++t) {
    starts[b * S + t] = start;
    if (tokens[b * S + t] == eos) start = static_cast<int32_t>(t + 1);
  }
}

// Eval argmax (update_engine.cc:552-560): the first maximum wins; a NaN
// never wins, and a NaN in column 0 keeps index 0 (no comparison beats it).
// One 256-lane workgroup per row; every lane gets the row's index.
__device__ int RowArgmax(const float* __restrict__ row, size_t cols) {
  __shared__ float bv[kThreads];
  __shared__ int bi[kThreads];
  float best = -INFINITY;
  int idx = -1;
  for (size_t c = threadIdx.x; c < cols; c += kThreads) {
    const float v = row[c];
    if (v == v && (idx < 0 || v > best)) {
      best = v;
      idx = static_cast<int>(c);
    }
  }
  bv[threadIdx.x] = best;
  bi[threadIdx.x] = idx;
  __syncthreads();
  for (int o = kThreads / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float v2 = bv[threadIdx.x + o];
      const int i2 = bi[threadIdx.x + o];
      const int i1 = bi[threadIdx.x];
      if (i2 >= 0 && (i1 < 0 || v2 > bv[threadIdx.x] || (v2 == bv[threadIdx.x] && i2 < i1))) {
        bv[threadIdx.x] = v2;
        bi[threadIdx.x] = i2;
      }
    }
    __syncthreads();
  }
  const float v0 = row[0];
  return (v0 != v0 || bi[0] < 0) ? 0 : bi[0];
}

__global__ void __launch_bounds__(kThreads)
ArgmaxKernel(const float* __restrict__ probs, size_t cols, int32_t* __restrict__ out) {
  const int am = RowArgmax(probs + static_cast<size_t>(blockIdx.x) * cols, cols);
  if (threadIdx.x == 0) out[blockIdx.x] = am;
}

// The eval accuracy tally (update_engine.cc:537-565): over the rows whose
// label is not -1, how many have their label as the argmax, and how many
// were judged.  Integer counts, so the order of the additions cannot change
// them; counts[0] = hits, counts[1] = judged rows, zeroed by ZeroCounts on
// the same stream first (a kernel, not a memset, so a captured graph may
// hold it).
__global__ void ZeroCounts(unsigned long long* __restrict__ counts) {
  if (threadIdx.x < 2) counts[threadIdx.x] = 0;
}

__global__ void __launch_bounds__(kThreads)
ArgmaxTallyKernel(const float* __restrict__ probs, const int32_t* __restrict__ labels, size_t cols,
                  unsigned long long* __restrict__ counts) {
  const int32_t label = labels[blockIdx.x];
  if (label < 0) return;  // uniform over the workgroup: an unjudged row
  const int am = RowArgmax(probs + static_cast<size_t>(blockIdx.x) * cols, cols);
  if (threadIdx.x == 0) {
    if (am == label) atomicAdd(&counts[0], 1ull);
    atomicAdd(&counts[1], 1ull);
  }
}

__global__ void __launch_bounds__(kThreads)
SiluMul4(const float4* __restrict__ x, const float4* __restrict__ u, float4* __restrict__ y,
         float4* __restrict__ h, size_t n4, Bf16Sink sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 a = x[i], b = u[i];
    const float4 g = make_float4(SiluExpr(a.x), SiluExpr(a.y), SiluExpr(a.z), SiluExpr(a.w));
    if (y) y[i] = g;  // null: y is dead after the pass
    const float4 hv = make_float4(g.x * b.x, g.y * b.y, g.z * b.z, g.w * b.w);
    if (sink.store_f32) h[i] = hv;
    if (sink.out) SinkStore4(sink, 4 * i, hv);
  }
}

// kStoreO1 false: the first product is dead after the pass and is not stored.
// `sink` takes dx's bf16 copy, `sink2` the second product's (each with its
// f32 store kept or dropped on its own).  kSiluB2: b2 is SiLU(x), formed
// here from x with the forward's expression rather than read.
template <bool kStoreO1, bool kSiluB2>
__global__ void __launch_bounds__(kThreads)
SwigluBwd4(const float4* __restrict__ a1, const float4* __restrict__ b1, float4* __restrict__ o1,
           const float4* __restrict__ a2, const float4* __restrict__ b2, float4* __restrict__ o2,
           const float4* __restrict__ x, float4* __restrict__ dx, size_t n4, Bf16Sink sink,
           Bf16Sink sink2) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 p = a1[i], q = b1[i], r = a2[i], v = x[i];
    const float4 t = kSiluB2 ? make_float4(SiluExpr(v.x), SiluExpr(v.y), SiluExpr(v.z), SiluExpr(v.w))
                             : b2[i];
    const float4 m1 = make_float4(p.x * q.x, p.y * q.y, p.z * q.z, p.w * q.w);
    if constexpr (kStoreO1) o1[i] = m1;
    const float4 m2 = make_float4(r.x * t.x, r.y * t.y, r.z * t.z, r.w * t.w);
    if (sink2.store_f32) o2[i] = m2;
    if (sink2.out) SinkStore4(sink2, 4 * i, m2);
    const float4 d = make_float4(SiluBwdExpr(m1.x, v.x), SiluBwdExpr(m1.y, v.y),
                                 SiluBwdExpr(m1.z, v.z), SiluBwdExpr(m1.w, v.w));
    if (sink.store_f32) dx[i] = d;
    if (sink.out) SinkStore4(sink, 4 * i, d);
  }
}

// GELU forward and backward (activation.cc's expressions, as the Map forms
// of LaunchUnary / LaunchBinaryBwd compute them) over float4, with a sink.
__device__ __forceinline__ float GeluBwdElem(float dy, float v) {
  const float kC = 0.7978845608028654f, kA = 0.044715f;
  const float u = kC * (v + kA * v * v * v);
  const float t = tanhf(u);
  const float omt2 = 1.0f - t * t;
  const float tail = omt2 == 0.0f ? 0.0f : 0.5f * v * omt2 * (kC * (1.0f + 3.0f * kA * v * v));
  return dy * (0.5f * (1.0f + t) + tail);
}

__global__ void __launch_bounds__(kThreads)
GeluFwd4(const float4* __restrict__ x, float4* __restrict__ out, size_t n4, Bf16Sink sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 a = x[i];
    const float4 g = make_float4(GeluExpr(a.x), GeluExpr(a.y), GeluExpr(a.z), GeluExpr(a.w));
    if (sink.store_f32) out[i] = g;
    if (sink.out) SinkStore4(sink, 4 * i, g);
  }
}

__global__ void __launch_bounds__(kThreads)
GeluBwd4(const float4* __restrict__ dy, const float4* __restrict__ x, float4* __restrict__ dx,
         size_t n4, Bf16Sink sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 d = dy[i], v = x[i];
    const float4 r = make_float4(GeluBwdElem(d.x, v.x), GeluBwdElem(d.y, v.y), GeluBwdElem(d.z, v.z),
                                 GeluBwdElem(d.w, v.w));
    if (sink.store_f32) dx[i] = r;
    if (sink.out) SinkStore4(sink, 4 * i, r);
  }
}

}  // namespace

hipError_t LaunchAddEW(const float* x, const float* y, float* out, size_t n, hipStream_t s,
                       const Bf16Sink& sink) {
  if (n % 4 == 0 && Aligned16(x) && Aligned16(y) && Aligned16(out)) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(AddEW4, dim3(GridFor(n / 4, kThreads, 8192)), dim3(kThreads), 0, s,
                       reinterpret_cast<const float4*>(x), reinterpret_cast<const float4*>(y),
                       reinterpret_cast<float4*>(out), n / 4, sink);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32) return hipErrorInvalidValue;
  return Map(n, s, [=] __device__(size_t i) { out[i] = x[i] + y[i]; });
}
bool SwigluFits(size_t n, std::initializer_list<const void*> ptrs) {
  if (n % 4 != 0) return false;
  for (const void* p : ptrs)
    if (!Aligned16(p)) return false;
  return true;
}

hipError_t LaunchSiluMul(const float* x, const float* u, float* y, float* h, size_t n,
                         hipStream_t s, const Bf16Sink& sink) {
  if (SwigluFits(n, {x, u, y, h})) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(SiluMul4, dim3(GridFor(n / 4, kThreads, 8192)), dim3(kThreads), 0, s,
                       reinterpret_cast<const float4*>(x), reinterpret_cast<const float4*>(u),
                       reinterpret_cast<float4*>(y), reinterpret_cast<float4*>(h), n / 4, sink);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32 || !y) return hipErrorInvalidValue;
  return Map(n, s, [=] __device__(size_t i) {
    const float g = SiluExpr(x[i]);
    y[i] = g;
    h[i] = g * u[i];
  });
}
hipError_t LaunchSwigluBwd(const float* a1, const float* b1, float* o1, const float* a2,
                           const float* b2, float* o2, const float* x, float* dx, size_t n,
                           hipStream_t s, const Bf16Sink& sink, const Bf16Sink& sink2,
                           bool silu_b2) {
  if (SwigluFits(n, {a1, b1, o1, a2, b2, o2, x, dx})) {
    if (n == 0) return hipSuccess;
    const auto c4 = [](const float* p) { return reinterpret_cast<const float4*>(p); };
    const auto m4 = [](float* p) { return reinterpret_cast<float4*>(p); };
    const dim3 grid(GridFor(n / 4, kThreads, 8192));
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, c4(a1), c4(b1), m4(o1), c4(a2),
                         c4(b2), m4(o2), c4(x), m4(dx), n / 4, sink, sink2);
    };
    if (o1) silu_b2 ? go(SwigluBwd4<true, true>) : go(SwigluBwd4<true, false>);
    else silu_b2 ? go(SwigluBwd4<false, true>) : go(SwigluBwd4<false, false>);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32 || sink2.out || !sink2.store_f32) return hipErrorInvalidValue;
  return Map(n, s, [=] __device__(size_t i) {
    const float m1 = a1[i] * b1[i];
    if (o1) o1[i] = m1;
    o2[i] = a2[i] * b2[i];
    dx[i] = SiluBwdExpr(m1, x[i]);
  });
}
hipError_t LaunchMulEW(const float* x, const float* y, float* out, size_t n, hipStream_t s) {
  return Map(n, s, [=] __device__(size_t i) { out[i] = x[i] * y[i]; });
}
hipError_t LaunchAddBias(const float* x, const float* b, float* out, size_t rows, size_t cols,
                         hipStream_t s) {
  return Map(rows * cols, s, [=] __device__(size_t i) { out[i] = x[i] + b[i % cols]; });
}
// kind: 1 relu, 2 gelu, 3 silu, 4 scale (out = alpha * x).
bool ElementwiseSinkFits(int kind, size_t n, const void* a, const void* b, const void* out) {
  return kind == 2 && n > 0 && n % 4 == 0 && Aligned16(a) && (!b || Aligned16(b)) && Aligned16(out);
}

hipError_t LaunchUnary(int kind, const float* x, float* out, size_t n, float alpha, hipStream_t s,
                       const Bf16Sink& sink) {
  if (kind == 2 && ElementwiseSinkFits(2, n, x, nullptr, out)) {
    hipLaunchKernelGGL(GeluFwd4, dim3(GridFor(n / 4, kThreads, 8192)), dim3(kThreads), 0, s,
                       reinterpret_cast<const float4*>(x), reinterpret_cast<float4*>(out), n / 4,
                       sink);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32) return hipErrorInvalidValue;
  switch (kind) {
    case 1: return Map(n, s, [=] __device__(size_t i) { out[i] = ReluExpr(x[i]); });
    case 2: return Map(n, s, [=] __device__(size_t i) { out[i] = GeluExpr(x[i]); });
    case 3: return Map(n, s, [=] __device__(size_t i) { out[i] = SiluExpr(x[i]); });
    default: return Map(n, s, [=] __device__(size_t i) { out[i] = alpha * x[i]; });
  }
}
// kind: 1 relu, 2 gelu, 3 silu backward (activation.cc:28-75).
hipError_t LaunchBinaryBwd(int kind, const float* dy, const float* x, float* dx, size_t n,
                           hipStream_t s, const Bf16Sink& sink) {
  if (kind == 2 && ElementwiseSinkFits(2, n, dy, x, dx)) {
    hipLaunchKernelGGL(GeluBwd4, dim3(GridFor(n / 4, kThreads, 8192)), dim3(kThreads), 0, s,
                       reinterpret_cast<const float4*>(dy), reinterpret_cast<const float4*>(x),
                       reinterpret_cast<float4*>(dx), n / 4, sink);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32) return hipErrorInvalidValue;
  switch (kind) {
    case 1:
      return Map(n, s, [=] __device__(size_t i) { dx[i] = x[i] > 0.0f ? dy[i] : 0.0f; });
    case 2:
      return Map(n, s, [=] __device__(size_t i) {
        const float kC = 0.7978845608028654f, kA = 0.044715f;
        const float v = x[i];
        const float u = kC * (v + kA * v * v * v);
        const float t = tanhf(u);
        const float omt2 = 1.0f - t * t;
        const float tail = omt2 == 0.0f ? 0.0f : 0.5f * v * omt2 * (kC * (1.0f + 3.0f * kA * v * v));
        dx[i] = dy[i] * (0.5f * (1.0f + t) + tail);
      });
    default:
      return Map(n, s, [=] __device__(size_t i) {
        dx[i] = SiluBwdExpr(dy[i], x[i]);
      });
  }
}
hipError_t LaunchReduceRows(const float* dy, float* db, size_t rows, size_t cols, hipStream_t s) {
  if (cols == 0) return hipSuccess;
  hipLaunchKernelGGL(ReduceRowsKernel, dim3(GridFor(cols, kThreads)), dim3(kThreads), 0, s, dy, db,
                     rows, cols);
  return hipGetLastError();
}
hipError_t LaunchFill(float* dst, float value, size_t n, hipStream_t s) {
  return Map(n, s, [=] __device__(size_t i) { dst[i] = value; });
}
hipError_t LaunchCopy(const float* src, float* dst, size_t n, hipStream_t s) {
  return Map(n, s, [=] __device__(size_t i) { dst[i] = src[i]; });
}
hipError_t LaunchAccumulate(float* dst, const float* src, size_t n, hipStream_t s) {
  return Map(n, s, [=] __device__(size_t i) { dst[i] += src[i]; });
}
hipError_t LaunchEmbed(const int32_t* tokens, const float* table, float* out, size_t rows,
                       size_t dim, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(EmbedKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, tokens,
                     table, out, dim);
  return hipGetLastError();
}
hipError_t LaunchFusedMap(const float* x, const float* o1, const float* o2, float* out, size_t n,
                          uint64_t stages, float imm0, float imm1, hipStream_t s) {
  FusedProgram p{};
  p.count = 0;
  for (; p.count < 4; ++p.count) {
    p.stage[p.count] = static_cast<uint8_t>(stages >> (8 * p.count));
    if ((p.stage[p.count] & 0x0F) == 0) break;
  }
  if (p.count == 0 || n == 0) return hipSuccess;
  hipLaunchKernelGGL(FusedMapKernel, dim3(GridFor(n, kThreads, 8192)), dim3(kThreads), 0, s, x, o1,
                     o2, out, n, p, imm0, imm1);
  return hipGetLastError();
}
bool NormSinkFits(size_t cols, std::initializer_list<const void*> ptrs) {
  if (cols == 0 || cols % 4 != 0) return false;
  for (const void* p : ptrs)
    if (p && !Aligned16(p)) return false;
  return true;
}
hipError_t LaunchLayerNormFwd(const float* x, const float* g, const float* b, float* y,
                              float* mean, float* rstd, size_t rows, size_t cols, float eps,
                              hipStream_t s, const Bf16Sink& sink) {
  if (rows == 0) return hipSuccess;
  const int vec = NormSinkFits(cols, {x, g, b, y});
  if (!vec && (sink.out || !sink.store_f32)) return hipErrorInvalidValue;
  if (vec && RowSlots(cols) > 0) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    SEEAI_ROWS_SWITCH(LayerNormFwdRows, x, g, b, y, mean, rstd, rows, cols, eps, sink)
    return hipGetLastError();
  }
  hipLaunchKernelGGL(LayerNormFwdKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                     x, g, b, y, mean, rstd, cols, eps, vec, sink);
  return hipGetLastError();
}
hipError_t LaunchLayerNormBwd(const float* dy, const float* x, const float* g,
                              const float* mean, const float* rstd, float* dx, size_t rows,
                              size_t cols, hipStream_t s, const Bf16Sink& sink, const float* res) {
  if (rows == 0) return hipSuccess;
  const int vec = NormSinkFits(cols, {dy, x, g, dx, res});
  if (!vec && (sink.out || !sink.store_f32)) return hipErrorInvalidValue;
  if (vec && RowSlots(cols) > 0) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    SEEAI_ROWS_SWITCH(LayerNormBwdRows, dy, x, g, mean, rstd, dx, rows, cols, sink, res)
    return hipGetLastError();
  }
  hipLaunchKernelGGL(LayerNormBwdKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                     dy, x, g, mean, rstd, dx, cols, vec, sink, res);
  return hipGetLastError();
}
hipError_t LaunchRmsNormFwd(const float* x, const float* g, float* y, float* rstd, size_t rows,
                            size_t cols, float eps, hipStream_t s, const Bf16Sink& sink) {
  if (rows == 0) return hipSuccess;
  const int vec = NormSinkFits(cols, {x, g, y});
  if (!vec && (sink.out || !sink.store_f32)) return hipErrorInvalidValue;
  if (vec && RowSlots(cols) > 0) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    SEEAI_ROWS_SWITCH(RmsNormFwdRows, x, g, y, rstd, rows, cols, eps, sink)
    return hipGetLastError();
  }
  hipLaunchKernelGGL(RmsNormFwdKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, x,
                     g, y, rstd, cols, eps, vec, sink);
  return hipGetLastError();
}
hipError_t LaunchRmsNormBwd(const float* dy, const float* x, const float* g, const float* rstd,
                            float* dx, size_t rows, size_t cols, hipStream_t s,
                            const Bf16Sink& sink, const float* res) {
  if (rows == 0) return hipSuccess;
  const int vec = NormSinkFits(cols, {dy, x, g, dx, res});
  if (!vec && (sink.out || !sink.store_f32)) return hipErrorInvalidValue;
  if (vec && RowSlots(cols) > 0) {
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    SEEAI_ROWS_SWITCH(RmsNormBwdRows, dy, x, g, rstd, dx, rows, cols, sink, res)
    return hipGetLastError();
  }
  hipLaunchKernelGGL(RmsNormBwdKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, dy,
                     x, g, rstd, dx, cols, vec, sink, res);
  return hipGetLastError();
}
bool RopeRowsFits(const float* x, const float* y, size_t B, size_t S, size_t H, size_t d,
                  const float* table) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                       reinterpret_cast<uintptr_t>(table);
  return table && d % 4 == 0 && (al & 15) == 0 && B * S < (size_t{1} << 31) &&
         H * d < (size_t{1} << 31);
}

hipError_t LaunchRope(const float* x, float* y, size_t B, size_t S, size_t H, size_t d,
                      float step, const float* table, int backward, hipStream_t s,
                      const Bf16Sink& sink) {
  const size_t n = B * S * H * (d / 2);
  if (n == 0) return hipSuccess;
  if (RopeRowsFits(x, y, B, S, H, d, table)) {
    const unsigned width = static_cast<unsigned>(H * d), rows = static_cast<unsigned>(B * S);
    const unsigned gx = static_cast<unsigned>(std::min<size_t>((width / 4 + kThreads - 1) / kThreads, 64));
    const dim3 grid(gx, std::min(rows, 65535u));
    hipLaunchKernelGGL(RopeRowsKernel, grid, dim3(kThreads), 0, s, x, y, rows,
                       static_cast<unsigned>(S), width, static_cast<unsigned>(d), table, backward,
                       sink);
    return hipGetLastError();
  }
  if (sink.out || !sink.store_f32) return hipErrorInvalidValue;  // the row kernel's only
  const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 7) == 0;
  if (vec)
    hipLaunchKernelGGL(RopeKernel<true>, dim3(GridFor(n, kThreads)), dim3(kThreads), 0, s, x, y, B,
                       S, H, d, step, table, backward);
  else
    hipLaunchKernelGGL(RopeKernel<false>, dim3(GridFor(n, kThreads)), dim3(kThreads), 0, s, x, y, B,
                       S, H, d, step, table, backward);
  return hipGetLastError();
}
hipError_t LaunchRopeTable(float* table, size_t S, size_t d, float step, hipStream_t s) {
  if (S == 0) return hipSuccess;
  hipLaunchKernelGGL(RopeTableKernel, dim3(GridFor(S, kThreads)), dim3(kThreads), 0, s, table, S,
                     d, step);
  return hipGetLastError();
}
hipError_t LaunchSegmentStarts(const int32_t* tokens, int32_t* starts, size_t B, size_t S,
                               int32_t eos, hipStream_t s) {
  if (B == 0) return hipSuccess;
  hipLaunchKernelGGL(SegmentStartsKernel, dim3(GridFor(B, 64)), dim3(64), 0, s, tokens, starts, B,
                     S, eos);
  return hipGetLastError();
}
hipError_t LaunchArgmaxRows(const float* probs, size_t rows, size_t cols, int32_t* out,
                            hipStream_t s) {
  if (rows == 0 || cols == 0) return hipSuccess;
  hipLaunchKernelGGL(ArgmaxKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, probs,
                     cols, out);
  return hipGetLastError();
}
hipError_t LaunchArgmaxTally(const float* probs, const int32_t* labels, size_t rows, size_t cols,
                             uint64_t* counts, hipStream_t s) {
  auto* c = reinterpret_cast<unsigned long long*>(counts);
  hipLaunchKernelGGL(ZeroCounts, dim3(1), dim3(64), 0, s, c);
  if (rows == 0 || cols == 0) return hipGetLastError();
  hipLaunchKernelGGL(ArgmaxTallyKernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                     probs, labels, cols, c);
  return hipGetLastError();
}

}  // namespace seeai
