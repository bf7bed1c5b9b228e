// k_loss.hip -- softmax cross-entropy forward / backward (and the masked
// pair) on gfx950 (runtime/executor/loss.cc:21-126).
//
// Forward, four kernels: the row max; the exp-sum in the reference's own
// association (a serial f32 chain per row, fed by a parallel exp pass -- at
// a 32k vocabulary a tree sum differs from the reference's chain by more
// than the 1e-5 parity bar); the probabilities with each row's
// -log p[label] as a double; and a one-workgroup kernel summing those
// doubles in a fixed tree into the f32 mean -- deterministic, no atomics.
// Backward: scale = seed / N (or / T) divided on the device exactly as the
// reference divides it, then one coalesced pass.
#include "common.h"

namespace seeai {
namespace {

// --- pass 1: row max (order-free: fmax ignores NaN as std::fmax does) ------
constexpr int kMaxThreads = 256;

// Rows of 16-byte multiples move as float4 with two running maxima per lane.
__host__ __device__ __forceinline__ bool Vec4Rows(const void* p, size_t C) {
  return C % 4 == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

__global__ void __launch_bounds__(kMaxThreads)
XEntRowMaxKernel(const float* __restrict__ logits, float* __restrict__ row_max, size_t C) {
  __shared__ float red[kMaxThreads / kWave];
  const float* x = logits + static_cast<size_t>(blockIdx.x) * C;
  float mx = NAN, mx2 = NAN;  // the identity of fmax
  if (Vec4Rows(logits, C)) {
    // Four 16-byte loads in flight per lane (a 32k-column row is 31 per
    // lane), each into its own running maximum.
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const size_t n4 = C / 4;
    float m4[4] = {NAN, NAN, NAN, NAN};
    size_t c = threadIdx.x;
    for (; c + 3 * kMaxThreads < n4; c += 4 * kMaxThreads) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = x4[c + u * kMaxThreads];
#pragma unroll
      for (int u = 0; u < 4; ++u) m4[u] = fmaxf(m4[u], fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
    }
    for (; c < n4; c += kMaxThreads) {
      const float4 v = x4[c];
      mx = fmaxf(mx, fmaxf(v.x, v.y));
      mx2 = fmaxf(mx2, fmaxf(v.z, v.w));
    }
    mx = fmaxf(mx, fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
  } else {
    for (size_t c = threadIdx.x; c < C; c += kMaxThreads) mx = fmaxf(mx, x[c]);
  }
  mx = BlockMaxF<kMaxThreads>(fmaxf(mx, mx2), red);
  if (threadIdx.x == 0) row_max[blockIdx.x] = mx;
}

// The row max from the partial maxima the producing GEMM's epilogue left
// ([rows, parts], fmax over each group of 64 columns): fmax is exact and
// order-free, so this is pass 1's value without a pass over the logits.
__global__ void __launch_bounds__(kMaxThreads)
XEntRowMaxPartsKernel(const float* __restrict__ parts, size_t P, float* __restrict__ row_max) {
  __shared__ float red[kMaxThreads / kWave];
  const float* p = parts + static_cast<size_t>(blockIdx.x) * P;
  float mx = NAN;
  for (size_t c = threadIdx.x; c < P; c += kMaxThreads) mx = fmaxf(mx, p[c]);
  mx = BlockMaxF<kMaxThreads>(mx, red);
  if (threadIdx.x == 0) row_max[blockIdx.x] = mx;
}

// --- pass 2: the exp-sum in the reference's order ------------------------------
// loss.cc:24-29 sums exp(x - max) in f32, column by column, one chain per
// row.  That association is reproduced exactly, with the chain apart from
// the exps: a workgroup takes 32 rows; waves 1-7 evaluate exp over 32-row x
// 224-column tiles into LDS (16-byte loads, double-buffered) while lane r
// of wave 0 adds row r's previous tile in column order, sixteen LDS values
// read ahead of its adds.  The chain wave does nothing else, so a tile
// costs the longer of its 224 dependent adds and the producers' exps.
// The exps that feed the chain: 2^(x log2 e) on the hardware's exp2 (two
// instructions where the libm expf takes about fifteen).  The rounding of
// x log2 e moves a term by at most |x| 1e-7 of itself (below 2e-6 down to
// x = -30, where a term is 1e-13 of the row's largest one), so the chain's
// sum stays within 1e-6 of expf's; the probabilities themselves are still
// expf(x - max) times 1/sum (pass 3).
__device__ __forceinline__ float SumExp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

constexpr int kSumThreads = 512;
constexpr int kSumRows = 32;
constexpr int kTileCols = 224;                      // 56 float4 per row
constexpr int kTileLd = kTileCols + 4;
constexpr int kProducers = kSumThreads - kWave;     // waves 1-7

__global__ void __launch_bounds__(kSumThreads)
XEntSerialSumKernel(const float* __restrict__ logits, const float* __restrict__ row_max,
                    float* __restrict__ row_sum, size_t N, size_t C) {
  __shared__ __attribute__((aligned(16))) float tile[2][kSumRows][kTileLd];
  const size_t r0 = static_cast<size_t>(blockIdx.x) * kSumRows;
  const int t = threadIdx.x;
  const size_t ntiles = (C + kTileCols - 1) / kTileCols;
  const bool vec = Vec4Rows(logits, C);
  // Producer p fills float4 slots p + 448 i (i < 4): row = slot / 56,
  // column quad = slot % 56 (consecutive lanes read consecutive quads); the
  // four loads are issued before any exp.
  constexpr int kSlots = kSumRows * (kTileCols / 4) / kProducers;
  static_assert(kSlots * kProducers == kSumRows * (kTileCols / 4), "whole slots per producer");
  auto fill = [&](size_t k, int buf) {
    const int p = t - kWave;
    float4 v[kSlots];
    float mx[kSlots];
    bool full[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int f = p + i * kProducers, r = f / (kTileCols / 4), c4 = f % (kTileCols / 4);
      const size_t row = r0 + r, c = k * kTileCols + 4 * c4;
      full[i] = vec && row < N && c + 4 <= C;
      mx[i] = row < N ? row_max[row] : 0.0f;
      v[i] = full[i] ? *reinterpret_cast<const float4*>(logits + row * C + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int f = p + i * kProducers, r = f / (kTileCols / 4), c4 = f % (kTileCols / 4);
      const size_t row = r0 + r, c = k * kTileCols + 4 * c4;
      float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (full[i]) {
        e[0] = SumExp(v[i].x - mx[i]), e[1] = SumExp(v[i].y - mx[i]);
        e[2] = SumExp(v[i].z - mx[i]), e[3] = SumExp(v[i].w - mx[i]);
      } else if (row < N) {
        for (int u = 0; u < 4; ++u)
          if (c + u < C) e[u] = SumExp(logits[row * C + c + u] - mx[i]);
      }
      *reinterpret_cast<float4*>(&tile[buf][r][4 * c4]) = make_float4(e[0], e[1], e[2], e[3]);
    }
  };
  if (t >= kWave) fill(0, 0);
  __syncthreads();
  float sum = 0.0f;
  for (size_t k = 0; k < ntiles; ++k) {
    if (t >= kWave) {
      if (k + 1 < ntiles) fill(k + 1, (k + 1) & 1);
    } else if (t < kSumRows) {
      const float* row = tile[k & 1][t];
      const size_t w = k + 1 < ntiles ? kTileCols : C - k * kTileCols;
      if (w == kTileCols) {
#pragma unroll 2
        for (int j0 = 0; j0 < kTileCols; j0 += 16) {
          float4 v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const float4*>(row + j0 + 4 * q);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            sum += v[q].x;
            sum += v[q].y;
            sum += v[q].z;
            sum += v[q].w;
          }
        }
      } else {
        for (size_t j = 0; j < w; ++j) sum += row[j];
      }
    }
    __syncthreads();
  }
  if (t < kSumRows && r0 + t < N) row_sum[r0 + t] = sum;
}

// --- pass 3: probabilities and the label term ----------------------------------
constexpr int kProbThreads = 256;

// With kBwd (the backward fused behind the forward, every row 16-byte
// aligned): each probability also becomes its gradient, scale * p minus
// scale at the label (zero on a masked row) -- XEntBwdKernel's expression on
// the same f32 p -- stored with the sink; probs is stored only where given.
template <bool kBwd>
__global__ void __launch_bounds__(kProbThreads)
XEntProbsKernel(const float* __restrict__ logits, const int32_t* __restrict__ labels,
                const float* __restrict__ row_max, const float* __restrict__ row_sum,
                float* __restrict__ probs, double* __restrict__ row_loss, size_t C, int masked,
                const float* __restrict__ scale_p, float* __restrict__ dl, Bf16Sink sink) {
  const size_t r = blockIdx.x;
  const float* x = logits + r * C;
  float* p = probs + r * C;
  const float mx = row_max[r];
  const float inv_sum = 1.0f / row_sum[r];  // loss.cc:30
  if constexpr (kBwd) {
    const float scale = *scale_p;
    const int32_t lab = labels[r];
    const bool zero = masked && lab < 0;
    const size_t lc = static_cast<size_t>(lab);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* d4 = reinterpret_cast<float4*>(dl + r * C);
    for (size_t c = threadIdx.x; c < C / 4; c += kProbThreads) {
      const float4 v = x4[c];
      const float4 q = make_float4(expf(v.x - mx) * inv_sum, expf(v.y - mx) * inv_sum,
                                   expf(v.z - mx) * inv_sum, expf(v.w - mx) * inv_sum);
      if (probs) reinterpret_cast<float4*>(p)[c] = q;
      float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
      if (!zero) {
        g = make_float4(scale * q.x, scale * q.y, scale * q.z, scale * q.w);
        if (lc / 4 == c) {
          const size_t l = lc % 4;
          if (l == 0) g.x -= scale;
          else if (l == 1) g.y -= scale;
          else if (l == 2) g.z -= scale;
          else g.w -= scale;
        }
      }
      if (sink.store_f32) d4[c] = g;
      if (sink.out) SinkStore4(sink, r * C + 4 * c, g);
    }
  } else if (Vec4Rows(logits, C) && Vec4Rows(probs, C)) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* p4 = reinterpret_cast<float4*>(p);
    for (size_t c = threadIdx.x; c < C / 4; c += kProbThreads) {
      const float4 v = x4[c];
      p4[c] = make_float4(expf(v.x - mx) * inv_sum, expf(v.y - mx) * inv_sum,
                          expf(v.z - mx) * inv_sum, expf(v.w - mx) * inv_sum);
    }
  } else {
    for (size_t c = threadIdx.x; c < C; c += kProbThreads) p[c] = expf(x[c] - mx) * inv_sum;
  }
  if (threadIdx.x == 0) {
    const int32_t lab = labels[r];
    double term = 0.0;
    if (!(masked && lab < 0)) {
      // The label's probability exactly as stored; NaN propagates, the
      // clamp only rescues underflow (loss.cc:45-51).
      const float pl = expf(x[static_cast<size_t>(lab)] - mx) * inv_sum;
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

// One workgroup per row (grid-stride over rows): the label is read once,
// the row moves as float4 where it can.
__global__ void __launch_bounds__(256)
XEntBwdKernel(const float* __restrict__ probs, const int32_t* __restrict__ labels,
              const float* __restrict__ scale_p, float* __restrict__ dl, size_t N, size_t C,
              int masked, Bf16Sink sink) {
  const float scale = *scale_p;
  const bool vec = Vec4Rows(probs, C) && Vec4Rows(dl, C);  // always, with a sink
  for (size_t r = blockIdx.x; r < N; r += gridDim.x) {
    const int32_t lab = labels[r];
    const float* pr = probs + r * C;
    float* dr = dl + r * C;
    const bool zero = masked && lab < 0;
    const size_t lc = static_cast<size_t>(lab);
    if (vec) {
      const float4* p4 = reinterpret_cast<const float4*>(pr);
      float4* d4 = reinterpret_cast<float4*>(dr);
      for (size_t c = threadIdx.x; c < C / 4; c += 256) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!zero) {
          const float4 q = p4[c];
          v = make_float4(scale * q.x, scale * q.y, scale * q.z, scale * q.w);
          if (lc / 4 == c) {  // the label's element, by component
            const size_t l = lc % 4;
            if (l == 0) v.x -= scale;
            else if (l == 1) v.y -= scale;
            else if (l == 2) v.z -= scale;
            else v.w -= scale;
          }
        }
        if (sink.store_f32) d4[c] = v;
        if (sink.out) SinkStore4(sink, r * C + 4 * c, v);
      }
    } else {
      for (size_t c = threadIdx.x; c < C; c += 256) {
        float v = 0.0f;
        if (!zero) {
          v = scale * pr[c];
          if (lc == c) v -= scale;
        }
        dr[c] = v;
      }
    }
  }
}

// The whole loss turn for a few rows (N <= 1024, N x C <= kSmallFloats, rows
// 16-byte aligned) in one workgroup: the seed's fill, the row max, the
// exps into LDS, the exp-sum chain of each row in column order, the
// probabilities and their gradient, the loss -- every value the
// multi-kernel path's expression in its association (the chain's
// sum += e, the probability e * (1 / sum), XEntFinishKernel's tree over the
// row terms), so the bits are the same.  Small plans run the turn in one
// dispatch instead of six.
constexpr int kSmallThreads = 1024;
constexpr size_t kSmallFloats = 16384;
__global__ void __launch_bounds__(kSmallThreads)
XEntSmallKernel(const float* __restrict__ logits, const int32_t* __restrict__ labels,
                float* __restrict__ loss, float* __restrict__ probs, float* fill_dst,
                uint64_t fill_n, float fill_v, const float* seed, float* __restrict__ dl,
                size_t N, size_t C, int masked, Bf16Sink sink) {
  __shared__ __attribute__((aligned(16))) float e[kSmallFloats];
  __shared__ float smax[kSmallThreads], sinv[kSmallThreads];
  __shared__ double rloss[kSmallThreads];
  __shared__ double red[kSmallThreads / kWave];
  __shared__ float sscale;
  constexpr int kWaves = kSmallThreads / kWave;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  for (uint64_t i = tid; i < fill_n; i += kSmallThreads) fill_dst[i] = fill_v;
  for (size_t r = wave; r < N; r += kWaves) {  // row max, a wave per row
    const float4* x4 = reinterpret_cast<const float4*>(logits + r * C);
    float mx = NAN, mx2 = NAN;
    for (size_t c = lane; c < C / 4; c += kWave) {
      const float4 v = x4[c];
      mx = fmaxf(mx, fmaxf(v.x, v.y));
      mx2 = fmaxf(mx2, fmaxf(v.z, v.w));
    }
    mx = WaveMaxF(fmaxf(mx, mx2));
    if (lane == 0) smax[r] = mx;
  }
  __syncthreads();
  for (size_t i = tid; i < N * C / 4; i += kSmallThreads) {  // the exps
    const float4 v = reinterpret_cast<const float4*>(logits)[i];
    const float mx = smax[4 * i / C];
    reinterpret_cast<float4*>(e)[i] =
        make_float4(expf(v.x - mx), expf(v.y - mx), expf(v.z - mx), expf(v.w - mx));
  }
  __syncthreads();
  if (static_cast<size_t>(tid) < N) {  // each row's chain in column order, on pass 2's exps
    const float* xr = logits + static_cast<size_t>(tid) * C;
    const float mx = smax[tid];
    float sum = 0.0f;
    for (size_t c = 0; c < C; ++c) sum += SumExp(xr[c] - mx);
    sinv[tid] = 1.0f / sum;  // loss.cc:30
  }
  double t = 0.0;
  if (masked)
    for (size_t r = tid; r < N; r += kSmallThreads) t += labels[r] >= 0 ? 1.0 : 0.0;
  t = BlockSumD<kSmallThreads>(t, red);  // also orders the fill and the chains before what follows
  if (tid == 0) {
    if (masked) {
      const uint64_t T = static_cast<uint64_t>(t);
      sscale = T ? *seed / static_cast<float>(T) : 0.0f;
    } else {
      sscale = *seed / static_cast<float>(N);
    }
  }
  __syncthreads();
  const float scale = sscale;
  for (size_t r = wave; r < N; r += kWaves) {  // probabilities, gradient, the row's term
    const float inv_sum = sinv[r];
    const int32_t lab = labels[r];
    const bool zero = masked && lab < 0;
    const size_t lc = static_cast<size_t>(lab);
    const float4* e4 = reinterpret_cast<const float4*>(e + r * C);
    for (size_t c = lane; c < C / 4; c += kWave) {
      const float4 v = e4[c];
      const float4 q = make_float4(v.x * inv_sum, v.y * inv_sum, v.z * inv_sum, v.w * inv_sum);
      if (probs) reinterpret_cast<float4*>(probs + r * C)[c] = q;
      float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
      if (!zero) {
        g = make_float4(scale * q.x, scale * q.y, scale * q.z, scale * q.w);
        if (lc / 4 == c) {
          const size_t l = lc % 4;
          if (l == 0) g.x -= scale;
          else if (l == 1) g.y -= scale;
          else if (l == 2) g.z -= scale;
          else g.w -= scale;
        }
      }
      if (sink.store_f32) reinterpret_cast<float4*>(dl + r * C)[c] = g;
      if (sink.out) SinkStore4(sink, r * C + 4 * c, g);
    }
    if (lane == 0) {
      double term = 0.0;
      if (!zero) {
        const float pl = e[r * C + lc] * inv_sum;
        const double safe = pl != pl ? static_cast<double>(pl) : static_cast<double>(fmaxf(pl, 1e-12f));
        term = -log(safe);
      }
      rloss[r] = term;
    }
  }
  __syncthreads();
  double total = 0.0, targets = 0.0;
  for (size_t r = tid; r < N; r += kSmallThreads) {
    total += rloss[r];
    if (!masked || labels[r] >= 0) targets += 1.0;
  }
  total = BlockSumD<kSmallThreads>(total, red);
  targets = BlockSumD<kSmallThreads>(targets, red);
  if (tid == 0) {
    if (masked)
      *loss = targets > 0.0 ? static_cast<float>(total / targets) : 0.0f;
    else
      *loss = static_cast<float>(total / static_cast<double>(N));
  }
}

}  // namespace

size_t XEntFwdScratchBytes(size_t N) { return N * (8 + 4 + 4) + 256; }

hipError_t LaunchXEntFwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                         size_t N, size_t C, int masked, void* ws, hipStream_t s) {
  if (N == 0) return hipSuccess;
  double* row_loss = static_cast<double*>(ws);
  float* row_max = reinterpret_cast<float*>(row_loss + N);
  float* row_sum = row_max + N;
  const unsigned rows = static_cast<unsigned>(N);
  hipLaunchKernelGGL(XEntRowMaxKernel, dim3(rows), dim3(kMaxThreads), 0, s, logits, row_max, C);
  hipLaunchKernelGGL(XEntSerialSumKernel, dim3(static_cast<unsigned>((N + kSumRows - 1) / kSumRows)),
                     dim3(kSumThreads), 0, s, logits, row_max, row_sum, N, C);
  hipLaunchKernelGGL((XEntProbsKernel<false>), dim3(rows), dim3(kProbThreads), 0, s, logits, labels,
                     row_max, row_sum, probs, row_loss, C, masked, nullptr, nullptr, Bf16Sink{});
  hipLaunchKernelGGL(XEntFinishKernel, dim3(1), dim3(1024), 0, s, row_loss, labels, loss, N, masked);
  return hipGetLastError();
}

bool XEntOneWorkgroup(size_t N, size_t C) {
  return N <= static_cast<size_t>(kSmallThreads) && N * C <= kSmallFloats;
}

bool XEntFusedFits(const float* logits, const float* probs, const float* dlogits, size_t C) {
  return C > 0 && Vec4Rows(logits, C) && (!probs || Vec4Rows(probs, C)) && Vec4Rows(dlogits, C);
}

hipError_t LaunchXEntFwdBwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                            float* fill_dst, uint64_t fill_n, float fill_v, const float* seed,
                            float* dlogits, size_t N, size_t C, int masked, void* ws,
                            hipStream_t s, const Bf16Sink& sink, const float* max_parts) {
  if (N == 0) return hipSuccess;
  if (!XEntFusedFits(logits, probs, dlogits, C)) return hipErrorInvalidValue;
  if (XEntOneWorkgroup(N, C)) {
    hipLaunchKernelGGL(XEntSmallKernel, dim3(1), dim3(kSmallThreads), 0, s, logits, labels, loss,
                       probs, fill_dst, fill_n, fill_v, seed, dlogits, N, C, masked, sink);
    return hipGetLastError();
  }
  if (hipError_t e = LaunchFill(fill_dst, fill_v, fill_n, s); e != hipSuccess) return e;
  double* row_loss = static_cast<double*>(ws);
  float* row_max = reinterpret_cast<float*>(row_loss + N);
  float* row_sum = row_max + N;
  float* scale = row_sum + N;  // in the scratch's spare tail
  const unsigned rows = static_cast<unsigned>(N);
  hipLaunchKernelGGL(XEntScaleKernel, dim3(1), dim3(1024), 0, s, labels, seed, scale, N, masked);
  if (max_parts)
    hipLaunchKernelGGL(XEntRowMaxPartsKernel, dim3(rows), dim3(kMaxThreads), 0, s, max_parts,
                       (C + 63) / 64, row_max);
  else
    hipLaunchKernelGGL(XEntRowMaxKernel, dim3(rows), dim3(kMaxThreads), 0, s, logits, row_max, C);
  hipLaunchKernelGGL(XEntSerialSumKernel, dim3(static_cast<unsigned>((N + kSumRows - 1) / kSumRows)),
                     dim3(kSumThreads), 0, s, logits, row_max, row_sum, N, C);
  hipLaunchKernelGGL((XEntProbsKernel<true>), dim3(rows), dim3(kProbThreads), 0, s, logits, labels,
                     row_max, row_sum, probs, row_loss, C, masked, scale, dlogits, sink);
  hipLaunchKernelGGL(XEntFinishKernel, dim3(1), dim3(1024), 0, s, row_loss, labels, loss, N, masked);
  return hipGetLastError();
}

bool XEntBwdSinkFits(const float* probs, const float* dlogits, size_t C) {
  return C > 0 && Vec4Rows(probs, C) && Vec4Rows(dlogits, C);
}

hipError_t LaunchXEntBwd(const float* probs, const int32_t* labels, const float* seed,
                         float* dlogits, size_t N, size_t C, int masked, void* ws,
                         hipStream_t s, const Bf16Sink& sink) {
  if (N == 0) return hipSuccess;
  if ((sink.out || !sink.store_f32) && !XEntBwdSinkFits(probs, dlogits, C)) return hipErrorInvalidValue;
  float* scale = static_cast<float*>(ws);
  hipLaunchKernelGGL(XEntScaleKernel, dim3(1), dim3(1024), 0, s, labels, seed, scale, N, masked);
  hipLaunchKernelGGL(XEntBwdKernel, dim3(static_cast<unsigned>(N < 65536 ? N : 65536)), dim3(256), 0,
                     s, probs, labels, scale, dlogits, N, C, masked, sink);
  return hipGetLastError();
}

}  // namespace seeai
