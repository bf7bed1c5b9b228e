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
// MFMA kernels: one wave owns a 16-row tile of one (b, h) -- 16 queries for
// the forward and dQ, 16 keys for dK and dV -- and walks the other side in
// 16-wide tiles up to the causal bound, so every output element has exactly
// one writer and every reduction a fixed order (no atomics).  The score tile
// is formed transposed (S^T = K Q^T in the forward / dQ): its accumulator
// layout -- lane (g = lane/16, c = lane%16) holding rows 4g..4g+3 of column
// c -- is exactly the B-operand layout the next product (O^T += V^T P^T)
// wants, so probabilities never leave registers.  The row softmax becomes a
// column reduction: in-lane over 4 values, then two lane swaps.
// These are the exact family (v_mfma_f32_16x16x4_f32 on f32 operands); the
// relaxed family (kFlagRelaxed) at d in {64, 128} runs the bf16 kernels of
// k_flash.hip.
// Other head widths run the per-row kernels below (double dots, the
// reference's loop order).
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

// out[r] = X[xr(4g+r)] . Y[yr(c)] over D dims, where this lane passes the
// row pointers of tile row c: xrow = X row (x0 + c), yrow = Y row (y0 + c).
template <int D>
__device__ __forceinline__ v4f DotTile(const float* __restrict__ xrow,
                                       const float* __restrict__ yrow, int g) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 4; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xrow[4 * s + g], yrow[4 * s + g], acc, 0, 0, 0);
  return acc;
}

// acc[dt] (rows = dims dt*16 + 4g + r, column c) += sum_t Z[z(t)][dim] * W[t][c]
// where this lane holds W[4g + r][c] = w[r] and zrow(t) points at Z row t.
template <int D>
__device__ __forceinline__ void AccumRows(v4f* acc, const float* __restrict__ z, size_t ld,
                                          const float* w, int g, int c, size_t zmax) {
  // Z rows for this lane's four k-values: t = 4g + r (clamped in bounds; the
  // matching w is 0 wherever the row is outside the sequence).
  const float* zr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    size_t t = static_cast<size_t>(4 * g + r);
    zr[r] = z + (t < zmax ? t : 0) * ld;
  }
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(zr[r][dt * 16 + c], w[r], acc[dt], 0, 0, 0);
}

__device__ __forceinline__ float ColMax(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float ColSum(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

// ---------------------------------------------------------------------------
// Forward (attention.cc:448-493 semantics; online softmax over key tiles).
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kThreads)
AttnFwdMfma(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
            float* __restrict__ o, float* __restrict__ stats, int S, int H,
            const int32_t* __restrict__ starts) {
  const int lane = threadIdx.x % kWave, g = lane / 16, c = lane % 16;
  const int i0 = blockIdx.x * 64 + (threadIdx.x / kWave) * 16;
  if (i0 >= S) return;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const float* qb = q + static_cast<size_t>(b) * S * ld + h * D;
  const float* kb = k + static_cast<size_t>(b) * S * ld + h * D;
  const float* vb = v + static_cast<size_t>(b) * S * ld + h * D;
  const int i = i0 + c;  // this lane's query column
  const int ic = i < S ? i : S - 1;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(D));
  int j_start = 0;
  if (starts) {
    const int s0 = starts[static_cast<size_t>(b) * S + ic];
    j_start = s0 <= 0 ? 0 : (s0 < ic ? s0 : ic);
  }
  // The tile's earliest document start bounds the first key tile.
  int tile_lo = j_start;
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 1, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 2, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 4, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 8, kWave));
  const float* qrow = qb + static_cast<size_t>(ic) * ld;

  v4f oacc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = v4f{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;
  const int i_hi = min(i0 + 15, S - 1);
  for (int j0 = (tile_lo / 16) * 16; j0 <= i_hi; j0 += 16) {
    const int jr = min(j0 + c, S - 1);
    const v4f st = DotTile<D>(kb + static_cast<size_t>(jr) * ld, qrow, g);
    float s[4], tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = j0 + 4 * g + r;
      const bool ok = i < S && j <= i && j >= j_start;
      s[r] = ok ? st[r] * inv_sqrt_d : -INFINITY;
      tmax = fmaxf(tmax, s[r]);
    }
    tmax = ColMax(tmax);
    const float m_new = fmaxf(m, tmax);
    const float alpha = (m == -INFINITY) ? 0.0f : expf(m - m_new);
    float p[4], psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = s[r] == -INFINITY ? 0.0f : expf(s[r] - m_new);
      psum += p[r];
    }
    psum = ColSum(psum);
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) oacc[dt] *= alpha;
    AccumRows<D>(oacc, vb + static_cast<size_t>(j0) * ld, ld, p, g, c,
                      static_cast<size_t>(S - j0));
  }
  if (i >= S) return;
  const float inv = 1.0f / l;
  float* orow = o + (static_cast<size_t>(b) * S + i) * ld + h * D;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const float4 val = make_float4(oacc[dt][0] * inv, oacc[dt][1] * inv, oacc[dt][2] * inv,
                                   oacc[dt][3] * inv);
    *reinterpret_cast<float4*>(orow + dt * 16 + 4 * g) = val;
  }
  if (g == 0) {
    float* st = stats + (static_cast<size_t>(bh) * S + i) * 4;
    st[0] = m;
    st[1] = inv;
    st[2] = 0.0f;
    st[3] = static_cast<float>(j_start);
  }
}

// ---------------------------------------------------------------------------
// dQ (attention.cc:495-535): pass 1 forms delta = sum_j p dP over the row,
// pass 2 forms dS = p (dP - delta) and dQ = dS K / sqrt(d).
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kThreads)
AttnDQMfma(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
           const float* __restrict__ dout, float* __restrict__ stats, float* __restrict__ dq,
           int S, int H) {
  const int lane = threadIdx.x % kWave, g = lane / 16, c = lane % 16;
  const int i0 = blockIdx.x * 64 + (threadIdx.x / kWave) * 16;
  if (i0 >= S) return;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t base = static_cast<size_t>(b) * S * ld + h * D;
  const int i = i0 + c;
  const int ic = i < S ? i : S - 1;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(D));
  float* st = stats + (static_cast<size_t>(bh) * S + ic) * 4;
  const float m = st[0], inv = st[1];
  const int j_start = static_cast<int>(AttnStart(st[3], ic));
  int tile_lo = j_start;
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 1, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 2, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 4, kWave));
  tile_lo = min(tile_lo, __shfl_xor(tile_lo, 8, kWave));
  const float* qrow = q + base + static_cast<size_t>(ic) * ld;
  const float* dorow = dout + base + static_cast<size_t>(ic) * ld;
  const int i_hi = min(i0 + 15, S - 1);
  const int jbeg = (tile_lo / 16) * 16;

  auto probs = [&](int j0, float* p, float* dp) {
    const int jr = min(j0 + c, S - 1);
    const v4f sc = DotTile<D>(k + base + static_cast<size_t>(jr) * ld, qrow, g);
    const v4f dpt = DotTile<D>(v + base + static_cast<size_t>(jr) * ld, dorow, g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = j0 + 4 * g + r;
      const bool ok = i < S && j <= i && j >= j_start;
      p[r] = ok ? expf(sc[r] * inv_sqrt_d - m) * inv : 0.0f;
      dp[r] = ok ? dpt[r] : 0.0f;
    }
  };

  float delta = 0.0f;
  for (int j0 = jbeg; j0 <= i_hi; j0 += 16) {
    float p[4], dp[4];
    probs(j0, p, dp);
#pragma unroll
    for (int r = 0; r < 4; ++r) delta += dp[r] * p[r];
  }
  delta = ColSum(delta);

  v4f acc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int j0 = jbeg; j0 <= i_hi; j0 += 16) {
    float p[4], dp[4], w[4];
    probs(j0, p, dp);
#pragma unroll
    for (int r = 0; r < 4; ++r) w[r] = (p[r] * (dp[r] - delta)) * inv_sqrt_d;
    AccumRows<D>(acc, k + base + static_cast<size_t>(j0) * ld, ld, w, g, c,
                      static_cast<size_t>(S - j0));
  }
  if (i >= S) return;
  float* dqrow = dq + base + static_cast<size_t>(i) * ld;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
    *reinterpret_cast<float4*>(dqrow + dt * 16 + 4 * g) =
        make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
  if (g == 0) st[2] = delta;
}

// ---------------------------------------------------------------------------
// dK and dV (attention.cc:537-590): one wave per 16 keys, walking the query
// tiles from the diagonal down; S and dP are formed query-major so that the
// accumulator layout is the B operand of dK^T += Q^T dS (dV^T += dO^T P).
// ---------------------------------------------------------------------------
template <int D, bool kDV>
__global__ void __launch_bounds__(kThreads)
AttnDKDVMfma(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
             const float* __restrict__ dout, const float* __restrict__ stats,
             float* __restrict__ out, int S, int H) {
  const int lane = threadIdx.x % kWave, g = lane / 16, c = lane % 16;
  const int j0 = blockIdx.x * 64 + (threadIdx.x / kWave) * 16;
  if (j0 >= S) return;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t base = static_cast<size_t>(b) * S * ld + h * D;
  const int j = j0 + c;  // this lane's key column
  const int jc = j < S ? j : S - 1;
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(D));
  const float* krow = k + base + static_cast<size_t>(jc) * ld;
  const float* vrow = v + base + static_cast<size_t>(jc) * ld;
  const float* st_bh = stats + static_cast<size_t>(bh) * S * 4;

  v4f acc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int it0 = j0; it0 < S; it0 += 16) {
    // Query rows of this lane's four accumulator entries: i = it0 + 4g + r.
    const int ir = min(it0 + c, S - 1);
    const v4f sc = DotTile<D>(q + base + static_cast<size_t>(ir) * ld, krow, g);
    v4f dpt = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!kDV) dpt = DotTile<D>(dout + base + static_cast<size_t>(ir) * ld, vrow, g);
    float w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = it0 + 4 * g + r;
      float val = 0.0f;
      if (i < S && j < S && j <= i) {
        const float* st = st_bh + static_cast<size_t>(i) * 4;
        if (static_cast<size_t>(j) >= AttnStart(st[3], i)) {
          const float p = expf(sc[r] * inv_sqrt_d - st[0]) * st[1];
          val = kDV ? p : (p * (dpt[r] - st[2])) * inv_sqrt_d;
        }
      }
      w[r] = val;
    }
    AccumRows<D>(acc, (kDV ? dout : q) + base + static_cast<size_t>(it0) * ld, ld, w, g, c,
                      static_cast<size_t>(S - it0));
  }
  if (j >= S) return;
  float* orow = out + base + static_cast<size_t>(j) * ld;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
    *reinterpret_cast<float4*>(orow + dt * 16 + 4 * g) =
        make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
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

template <template <int> class F, typename... Args>
hipError_t ByShape(size_t d, Args... args) {
  return d == 64 ? F<64>::Run(args...) : F<128>::Run(args...);
}

template <int D>
struct FwdL {
  static hipError_t Run(const float* q, const float* k, const float* v, float* o, float* st,
                        size_t B, size_t S, size_t H, const int32_t* starts, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + 63) / 64), static_cast<unsigned>(B * H));
    hipLaunchKernelGGL((AttnFwdMfma<D>), grid, dim3(kThreads), 0, s, q, k, v, o, st,
                       static_cast<int>(S), static_cast<int>(H), starts);
    return hipGetLastError();
  }
};
template <int D>
struct DQL {
  static hipError_t Run(const float* q, const float* k, const float* v, const float* dout,
                        float* st, float* dq, size_t B, size_t S, size_t H, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + 63) / 64), static_cast<unsigned>(B * H));
    hipLaunchKernelGGL((AttnDQMfma<D>), grid, dim3(kThreads), 0, s, q, k, v, dout, st, dq,
                       static_cast<int>(S), static_cast<int>(H));
    return hipGetLastError();
  }
};
template <int D>
struct DKL {
  static hipError_t Run(const float* q, const float* k, const float* v, const float* dout,
                        const float* st, float* out, size_t B, size_t S, size_t H, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + 63) / 64), static_cast<unsigned>(B * H));
    hipLaunchKernelGGL((AttnDKDVMfma<D, false>), grid, dim3(kThreads), 0, s, q, k, v, dout, st,
                       out, static_cast<int>(S), static_cast<int>(H));
    return hipGetLastError();
  }
};
template <int D>
struct DVL {
  static hipError_t Run(const float* q, const float* k, const float* v, const float* dout,
                        const float* st, float* out, size_t B, size_t S, size_t H, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + 63) / 64), static_cast<unsigned>(B * H));
    hipLaunchKernelGGL((AttnDKDVMfma<D, true>), grid, dim3(kThreads), 0, s, q, k, v, dout, st,
                       out, static_cast<int>(S), static_cast<int>(H));
    return hipGetLastError();
  }
};

inline unsigned UnitsGrid(size_t n) { return GridFor(n, kThreads, 1u << 30); }

}  // namespace

hipError_t LaunchAttnFwdTiled(int dtype, const float* q, const float* k, const float* v, float* o,
                              float* stats, size_t B, size_t S, size_t H, size_t d,
                              const int32_t* starts, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (MfmaShape(d, q, k) && MfmaShape(d, v, o))
    return dtype && FlashFits(B, S, H, d) ? LaunchFlashFwd(q, k, v, o, stats, B, S, H, d, starts, s)
                 : ByShape<FwdL>(d, q, k, v, o, stats, B, S, H, starts, s);
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
  if (MfmaShape(d, q, k) && MfmaShape(d, v, dout) && MfmaShape(d, dq, q))
    return dtype && FlashFits(B, S, H, d) ? LaunchFlashDQ(q, k, v, dout, stats, dq, B, S, H, d, FlashDQOnePass(), s)
                 : ByShape<DQL>(d, q, k, v, dout, stats, dq, B, S, H, s);
  hipLaunchKernelGGL(AttnDQRowKernel, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q, k, v,
                     dout, stats, dq, B, S, H, d);
  return hipGetLastError();
}

hipError_t LaunchAttnDKTiled(int dtype, const float* q, const float* k, const float* v,
                             const float* dout, const float* stats, float* dk, size_t B,
                             size_t S, size_t H, size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (MfmaShape(d, q, k) && MfmaShape(d, v, dout) && MfmaShape(d, dk, q))
    return dtype && FlashFits(B, S, H, d) ? LaunchFlashDKDV(q, k, v, dout, stats, dk, nullptr, B, S, H, d, s)
                 : ByShape<DKL>(d, q, k, v, dout, stats, dk, B, S, H, s);
  hipLaunchKernelGGL(AttnDKDVRowKernel<false>, dim3(UnitsGrid(B * H * S)), dim3(kThreads), 0, s, q,
                     k, v, dout, stats, dk, B, S, H, d);
  return hipGetLastError();
}

hipError_t LaunchAttnDVTiled(int dtype, const float* q, const float* k, const float* dout,
                             const float* stats, float* dv, size_t B, size_t S, size_t H,
                             size_t d, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  if (MfmaShape(d, q, k) && MfmaShape(d, dout, dv))
    return dtype && FlashFits(B, S, H, d) ? LaunchFlashDKDV(q, k, nullptr, dout, stats, nullptr, dv, B, S, H, d, s)
                 : ByShape<DVL>(d, q, k, static_cast<const float*>(nullptr), dout, stats,
                                dv, B, S, H, s);
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
