// k_attn32.hip -- the exact family of causal attention (kAttnFwdTiled,
// kAttnDQTiled, kAttnDKTiled, kAttnDVTiled; source/plan/instruction.h:
// 158-259) on f32 operands, on v_mfma_f32_16x16x4f32, head widths 64 and
// 128.  The reference's expressions per score (attention.cc:405-590, the
// oracle's prob_of and unit loops): s = f32(q . k) * (1/sqrt(d)),
// p = exp(s - m) * (1/l), delta = sum_j p dP (accumulated in double),
// dS = p (dP - delta), dQ += (dS / sqrt(d)) k, dK += (dS / sqrt(d)) q,
// dV += p dO -- with the dots of q . k and dO . v as f32 MFMA sums in place
// of the reference's double dots (within 1e-5 of it, per tensor).
//
// Geometry.  A workgroup of four waves owns 128 rows of one (b, h) -- 128
// queries for the forward and dQ, 128 keys for dK / dV -- each wave 32 of
// them (two 16-row MFMA tiles), held in registers as MFMA fragments for the
// whole kernel.  The other side streams through LDS in blocks of 64 rows
// (row stride d + 4 floats, so the 16-byte fragment reads and the 4-byte
// transposed reads are both free of bank conflicts), double-buffered: the
// next block's global loads are in flight in registers while the current
// block is multiplied, one barrier per block.
//
// Products.  With x the workgroup's own rows and y the staged side, a score
// tile is formed with the staged rows as the MFMA's A operand and the own
// rows as B, so the accumulator's rows are staged rows: in the forward and
// dQ, S^T (keys x queries), whose layout is the B operand of O^T += V^T P^T
// and dQ^T += K^T dS^T; in dK / dV, S (queries x keys), the B operand of
// dV^T += dO^T P and dK^T += Q^T dS.  The A operands of those products
// (V^T, K^T, dO^T, Q^T) are read from the row-major staged block one float
// per lane.  A dot's k-steps take the lane's 16 (or 32) consecutive head
// dims, so each fragment is one run of 16-byte reads.
//
// Order and exactness.  Every output element has one writer and every sum a
// fixed order (no atomics): the forward's online softmax and the dQ / dK /
// dV accumulations walk the blocks in order; delta is the double sum of the
// row's p dP, in block order.  dK and dV are one template: the fused pass
// and the separate passes compute each output with the same instructions.
#include <cstdint>

#include "common.h"

namespace seeai {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;  // 256
constexpr int kOwn = 32;                  // own rows per wave
constexpr int kRowsWG = kOwn * kWaves;    // 128
constexpr int kBlk = 64;                  // staged rows per block

__device__ __forceinline__ v4f Mfma(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// instruction.h:240-247: a stored start clamped into [0, i], NaN to 0.
__device__ __forceinline__ int StartOf(float stored, int i) {
  if (!(stored > 0.0f)) return 0;
  const float cap = static_cast<float>(i);
  return stored >= cap ? i : static_cast<int>(stored);
}

// One staged block: kBlk rows x D floats of one (b, h) slice, rows past the
// sequence zero.
template <int D>
struct Block {
  static constexpr int kLd = D + 4;                      // LDS row stride (floats)
  static constexpr int kN = kBlk * (D / 4) / kThreads;   // float4 per thread
  float4 r[kN];

  __device__ __forceinline__ void Load(const float* __restrict__ base, size_t ld, int row0, int S,
                                       int tid) {
#pragma unroll
    for (int e = 0; e < kN; ++e) {
      const int f = tid + e * kThreads;
      const int row = f / (D / 4), ch = f % (D / 4);
      const int gr = row0 + row;
      r[e] = gr < S ? *reinterpret_cast<const float4*>(base + static_cast<size_t>(gr) * ld + ch * 4)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __device__ __forceinline__ void Store(float* lds, int tid) const {
#pragma unroll
    for (int e = 0; e < kN; ++e) {
      const int f = tid + e * kThreads;
      const int row = f / (D / 4), ch = f % (D / 4);
      *reinterpret_cast<float4*>(lds + row * kLd + ch * 4) = r[e];
    }
  }
};

// The fragments of one own 16-row tile: lane (g, c) holds row c's dims
// [g D/4, (g + 1) D/4), the k-steps of a dot in which this lane takes part.
template <int D>
__device__ __forceinline__ void OwnFrags(const float* __restrict__ rowp, int g, float (&f)[D / 4]) {
#pragma unroll
  for (int u = 0; u < D / 16; ++u) {
    const float4 x = *reinterpret_cast<const float4*>(rowp + g * (D / 4) + 4 * u);
    f[4 * u] = x.x, f[4 * u + 1] = x.y, f[4 * u + 2] = x.z, f[4 * u + 3] = x.w;
  }
}

// S tile = staged rows (16, from `lds` row `r0`) . own tile, over D dims:
// lane (g, c) gets staged rows r0 + 4g + r against own row c.
template <int D>
__device__ __forceinline__ v4f DotTile(const float* lds, int r0, const float (&own)[D / 4], int g,
                                       int c) {
  const float* row = lds + (r0 + c) * (D + 4) + g * (D / 4);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < D / 16; ++u) {
    const float4 x = *reinterpret_cast<const float4*>(row + 4 * u);
    acc = Mfma(x.x, own[4 * u], acc);
    acc = Mfma(x.y, own[4 * u + 1], acc);
    acc = Mfma(x.z, own[4 * u + 2], acc);
    acc = Mfma(x.w, own[4 * u + 3], acc);
  }
  return acc;
}

__device__ __forceinline__ float ColMax(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float ColSum(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}
__device__ __forceinline__ double ColSumD(double v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

// Workgroup w -> (unit, row block): heavy row blocks first; when B*H is a
// multiple of 8, every row block of a unit lands on the same XCD (the
// hardware deals workgroups to XCDs round-robin), so a unit's staged side is
// read through one L2.
__device__ __forceinline__ void UnitOf(int w, int units, int nblocks, bool heavy_last, int& unit,
                                       int& blk) {
  unit = w % units;
  const int rank = w / units;
  blk = heavy_last ? nblocks - 1 - rank : rank;
}

// ---------------------------------------------------------------------------
// Forward (attention.cc:448-493): online softmax over 64-key blocks; the
// stats row gets the row max, 1/l, 0 and the clamped start.
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kThreads)
Attn32Fwd(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
          float* __restrict__ o, float* __restrict__ stats, int S, int H,
          const int32_t* __restrict__ starts) {
  __shared__ __attribute__((aligned(16))) float lds[2][2][kBlk * (D + 4)];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, g = lane / 16,
            c = lane % 16;
  const int nblk = (S + kRowsWG - 1) / kRowsWG;
  int unit, rb;
  UnitOf(blockIdx.x, gridDim.x / nblk, nblk, true, unit, rb);
  const int b = unit / H, h = unit % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t off = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int i0 = rb * kRowsWG, iw = i0 + wave * kOwn;
  const float isd = 1.0f / sqrtf(static_cast<float>(D));

  // This lane's two queries (one per tile) and their first keys.
  float qf[2][D / 4];
  int qi[2], qs[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    qi[t] = iw + 16 * t + c;
    const int qc = min(qi[t], S - 1);
    OwnFrags<D>(q + off + static_cast<size_t>(qc) * ld, g, qf[t]);
    int st = 0;
    if (starts) {
      const int s0 = starts[static_cast<size_t>(b) * S + qc];
      st = s0 <= 0 ? 0 : (s0 < qc ? s0 : qc);
    }
    qs[t] = st;
  }
  // The workgroup's key range: its earliest start to its last query.
  int lo = min(qs[0], qs[1]);
  for (int x = 1; x < kWave; x <<= 1) lo = min(lo, __shfl_xor(lo, x, kWave));
  __shared__ int wg_lo[kWaves];
  if (lane == 0) wg_lo[wave] = lo;
  __syncthreads();
  lo = min(min(wg_lo[0], wg_lo[1]), min(wg_lo[2], wg_lo[3]));
  const int kb0 = lo / kBlk, kb1 = min(i0 + kRowsWG - 1, S - 1) / kBlk;
  const int wave_last = min(iw + kOwn - 1, S - 1);

  v4f oacc[2][D / 16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) oacc[t][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};

  Block<D> nk, nv;
  nk.Load(k + off, ld, kb0 * kBlk, S, tid);
  nv.Load(v + off, ld, kb0 * kBlk, S, tid);
  nk.Store(lds[0][0], tid);
  nv.Store(lds[0][1], tid);
  __syncthreads();
  for (int kb = kb0; kb <= kb1; ++kb) {
    const int buf = (kb - kb0) & 1;
    if (kb < kb1) {
      nk.Load(k + off, ld, (kb + 1) * kBlk, S, tid);
      nv.Load(v + off, ld, (kb + 1) * kBlk, S, tid);
    }
    const float* Ks = lds[buf][0];
    const float* Vs = lds[buf][1];
    const int j0 = kb * kBlk;
    if (j0 <= wave_last) {
      float p[4][2][4];
      float tmax[2] = {-INFINITY, -INFINITY};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int jt = j0 + 16 * kt;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const bool live = jt <= iw + 16 * t + 15;  // wave-uniform
          v4f sc = {0.f, 0.f, 0.f, 0.f};
          if (live) sc = DotTile<D>(Ks, 16 * kt, qf[t], g, c);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = jt + 4 * g + r;
            const bool ok = live && j <= qi[t] && j >= qs[t] && qi[t] < S;
            const float s = ok ? sc[r] * isd : -INFINITY;
            p[kt][t][r] = s;
            tmax[t] = fmaxf(tmax[t], s);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float mn = fmaxf(m[t], ColMax(tmax[t]));
        const float alpha = m[t] == -INFINITY ? 0.0f : expf(m[t] - mn);
        float ps = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float e = p[kt][t][r] == -INFINITY ? 0.0f : expf(p[kt][t][r] - mn);
            p[kt][t][r] = e;
            ps += e;
          }
        l[t] = l[t] * alpha + ColSum(ps);
        m[t] = mn;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) oacc[t][dt] *= alpha;
      }
      // O^T += V^T P^T: V^T's fragment is V[j0 + 16 kt + 4g + r][16 dt + c].
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if (j0 + 16 * kt > wave_last) continue;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float vf = Vs[(16 * kt + 4 * g + r) * (D + 4) + 16 * dt + c];
#pragma unroll
            for (int t = 0; t < 2; ++t) oacc[t][dt] = Mfma(vf, p[kt][t][r], oacc[t][dt]);
          }
      }
    }
    if (kb < kb1) {
      nk.Store(lds[buf ^ 1][0], tid);
      nv.Store(lds[buf ^ 1][1], tid);
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (qi[t] >= S) continue;
    const float inv = 1.0f / l[t];
    float* orow = o + off + static_cast<size_t>(qi[t]) * ld;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      *reinterpret_cast<float4*>(orow + 16 * dt + 4 * g) =
          make_float4(oacc[t][dt][0] * inv, oacc[t][dt][1] * inv, oacc[t][dt][2] * inv,
                      oacc[t][dt][3] * inv);
    if (g == 0)
      *reinterpret_cast<float4*>(stats + (static_cast<size_t>(unit) * S + qi[t]) * 4) =
          make_float4(m[t], inv, 0.0f, static_cast<float>(qs[t]));
  }
}

// ---------------------------------------------------------------------------
// dQ (attention.cc:495-535): pass 1 forms delta = sum_j p dP in double over
// the row's keys, pass 2 dS = p (dP - delta) and dQ += (dS / sqrt(d)) k.
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kThreads)
Attn32DQ(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
         const float* __restrict__ dout, float* __restrict__ stats, float* __restrict__ dq, int S,
         int H) {
  __shared__ __attribute__((aligned(16))) float lds[2][2][kBlk * (D + 4)];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, g = lane / 16,
            c = lane % 16;
  const int nblk = (S + kRowsWG - 1) / kRowsWG;
  int unit, rb;
  UnitOf(blockIdx.x, gridDim.x / nblk, nblk, true, unit, rb);
  const int b = unit / H, h = unit % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t off = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int i0 = rb * kRowsWG, iw = i0 + wave * kOwn;
  const float isd = 1.0f / sqrtf(static_cast<float>(D));

  float qf[2][D / 4], df[2][D / 4];
  int qi[2], qs[2];
  float qm[2], qinv[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    qi[t] = iw + 16 * t + c;
    const int qc = min(qi[t], S - 1);
    OwnFrags<D>(q + off + static_cast<size_t>(qc) * ld, g, qf[t]);
    OwnFrags<D>(dout + off + static_cast<size_t>(qc) * ld, g, df[t]);
    const float4 st = *reinterpret_cast<const float4*>(stats + (static_cast<size_t>(unit) * S + qc) * 4);
    qm[t] = st.x, qinv[t] = st.y;
    qs[t] = StartOf(st.w, qc);
  }
  int lo = min(qs[0], qs[1]);
  for (int x = 1; x < kWave; x <<= 1) lo = min(lo, __shfl_xor(lo, x, kWave));
  __shared__ int wg_lo[kWaves];
  if (lane == 0) wg_lo[wave] = lo;
  __syncthreads();
  lo = min(min(wg_lo[0], wg_lo[1]), min(wg_lo[2], wg_lo[3]));
  const int kb0 = lo / kBlk, kb1 = min(i0 + kRowsWG - 1, S - 1) / kBlk;
  const int wave_last = min(iw + kOwn - 1, S - 1);

  // p and dP of key tile kt against query tile t (lane: keys 4g + r).
  auto tile = [&](const float* Ks, const float* Vs, int j0, int kt, int t, float (&p)[4],
                  float (&dp)[4]) {
    const int jt = j0 + 16 * kt;
    const v4f sc = DotTile<D>(Ks, 16 * kt, qf[t], g, c);
    const v4f dpt = DotTile<D>(Vs, 16 * kt, df[t], g, c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = jt + 4 * g + r;
      const bool ok = j <= qi[t] && j >= qs[t] && qi[t] < S;
      p[r] = ok ? expf(sc[r] * isd - qm[t]) * qinv[t] : 0.0f;
      dp[r] = ok ? dpt[r] : 0.0f;
    }
  };

  Block<D> nk, nv;
  double dsum[2] = {0.0, 0.0};
  float delta[2];
  v4f acc[2][D / 16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[t][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  const int nb = kb1 - kb0 + 1;
  // Both passes walk the same blocks in the same order: step s < nb is
  // pass 1's block kb0 + s, step s >= nb pass 2's block kb0 + s - nb.
  nk.Load(k + off, ld, kb0 * kBlk, S, tid);
  nv.Load(v + off, ld, kb0 * kBlk, S, tid);
  nk.Store(lds[0][0], tid);
  nv.Store(lds[0][1], tid);
  __syncthreads();
  for (int s = 0; s < 2 * nb; ++s) {
    const int buf = s & 1;
    const bool second = s >= nb;
    const int kb = kb0 + (second ? s - nb : s);
    if (s + 1 < 2 * nb) {
      const int nkb = kb0 + (s + 1 >= nb ? s + 1 - nb : s + 1);
      nk.Load(k + off, ld, nkb * kBlk, S, tid);
      nv.Load(v + off, ld, nkb * kBlk, S, tid);
    }
    const float* Ks = lds[buf][0];
    const float* Vs = lds[buf][1];
    const int j0 = kb * kBlk;
    if (s == nb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) delta[t] = static_cast<float>(ColSumD(dsum[t]));
    }
    if (j0 <= wave_last) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if (j0 + 16 * kt > wave_last) continue;
        float gq[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (j0 + 16 * kt > iw + 16 * t + 15) {  // wave-uniform: tile above the diagonal
#pragma unroll
            for (int r = 0; r < 4; ++r) gq[t][r] = 0.0f;
            continue;
          }
          float p[4], dp[4];
          tile(Ks, Vs, j0, kt, t, p, dp);
          if (!second) {
#pragma unroll
            for (int r = 0; r < 4; ++r) dsum[t] += static_cast<double>(dp[r]) * p[r];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) gq[t][r] = (p[r] * (dp[r] - delta[t])) * isd;
          }
        }
        if (second) {
          // dQ^T += K^T dS^T: K^T's fragment is K[j0 + 16 kt + 4g + r][16 dt + c].
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float kf = Ks[(16 * kt + 4 * g + r) * (D + 4) + 16 * dt + c];
#pragma unroll
              for (int t = 0; t < 2; ++t) acc[t][dt] = Mfma(kf, gq[t][r], acc[t][dt]);
            }
        }
      }
    }
    if (s + 1 < 2 * nb) {
      nk.Store(lds[buf ^ 1][0], tid);
      nv.Store(lds[buf ^ 1][1], tid);
    }
    __syncthreads();
  }
  if (nb == 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) delta[t] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (qi[t] >= S) continue;
    float* row = dq + off + static_cast<size_t>(qi[t]) * ld;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      *reinterpret_cast<float4*>(row + 16 * dt + 4 * g) =
          make_float4(acc[t][dt][0], acc[t][dt][1], acc[t][dt][2], acc[t][dt][3]);
    if (g == 0) stats[(static_cast<size_t>(unit) * S + qi[t]) * 4 + 2] = delta[t];
  }
}

// ---------------------------------------------------------------------------
// dK and dV (attention.cc:537-590): each wave's 32 keys against 64-query
// blocks from the diagonal down.  kDK / kDV pick the outputs; each output's
// arithmetic is the same whichever else is formed.
// ---------------------------------------------------------------------------
template <int D, bool kDK, bool kDV>
__global__ void __launch_bounds__(kThreads)
Attn32DKDV(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
           const float* __restrict__ dout, const float* __restrict__ stats, float* __restrict__ dk,
           float* __restrict__ dv, int S, int H) {
  __shared__ __attribute__((aligned(16))) float lds[2][2][kBlk * (D + 4)];
  __shared__ float4 sst[2][kBlk];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, g = lane / 16,
            c = lane % 16;
  const int nblk = (S + kRowsWG - 1) / kRowsWG;
  int unit, rb;
  UnitOf(blockIdx.x, gridDim.x / nblk, nblk, false, unit, rb);
  const int b = unit / H, h = unit % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t off = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int j0w = rb * kRowsWG + wave * kOwn;
  const float isd = 1.0f / sqrtf(static_cast<float>(D));
  const float* st_unit = stats + static_cast<size_t>(unit) * S * 4;

  float kf[2][D / 4], vf[2][D / 4];
  int kj[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    kj[t] = j0w + 16 * t + c;
    const int kc = min(kj[t], S - 1);
    OwnFrags<D>(k + off + static_cast<size_t>(kc) * ld, g, kf[t]);
    if (kDK) OwnFrags<D>(v + off + static_cast<size_t>(kc) * ld, g, vf[t]);
  }
  v4f dka[2][D / 16], dva[2][D / 16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) dka[t][dt] = dva[t][dt] = v4f{0.f, 0.f, 0.f, 0.f};

  const int qb0 = (rb * kRowsWG) / kBlk, qb1 = (S - 1) / kBlk;
  Block<D> nq, nd;
  float4 nst = make_float4(0.f, 0.f, 0.f, 0.f);
  auto load = [&](int qb) {
    nq.Load(q + off, ld, qb * kBlk, S, tid);
    nd.Load(dout + off, ld, qb * kBlk, S, tid);
    const int r = qb * kBlk + tid;
    if (tid < kBlk) nst = r < S ? *reinterpret_cast<const float4*>(st_unit + static_cast<size_t>(r) * 4)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto store = [&](int buf) {
    nq.Store(lds[buf][0], tid);
    nd.Store(lds[buf][1], tid);
    if (tid < kBlk) sst[buf][tid] = nst;
  };
  load(qb0);
  store(0);
  __syncthreads();
  for (int qb = qb0; qb <= qb1; ++qb) {
    const int buf = (qb - qb0) & 1;
    if (qb < qb1) load(qb + 1);
    const float* Qs = lds[buf][0];
    const float* Ds = lds[buf][1];
    const int i0 = qb * kBlk;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int ib = i0 + 16 * it;
      if (ib >= S || ib + 15 < j0w) continue;  // wave-uniform: no query of the tile sees a key
      // This lane's four queries: ib + 4g + r.
      float4 qst[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) qst[r] = sst[buf][16 * it + 4 * g + r];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (ib + 15 < j0w + 16 * t) continue;  // wave-uniform
        const v4f sc = DotTile<D>(Qs, 16 * it, kf[t], g, c);
        v4f dpt = {0.f, 0.f, 0.f, 0.f};
        if (kDK) dpt = DotTile<D>(Ds, 16 * it, vf[t], g, c);
        float p[4], w[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = ib + 4 * g + r;
          const bool ok = i < S && kj[t] <= i && kj[t] >= StartOf(qst[r].w, i);
          const float pr = ok ? expf(sc[r] * isd - qst[r].x) * qst[r].y : 0.0f;
          p[r] = pr;
          w[r] = (pr * (dpt[r] - qst[r].z)) * isd;
        }
        // dV^T += dO^T P, dK^T += Q^T dS: the A fragments are dO / Q
        // [ib + 4g + r][16 dt + c].
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int at = (16 * it + 4 * g + r) * (D + 4) + 16 * dt + c;
            if (kDV) dva[t][dt] = Mfma(Ds[at], p[r], dva[t][dt]);
            if (kDK) dka[t][dt] = Mfma(Qs[at], w[r], dka[t][dt]);
          }
      }
    }
    if (qb < qb1) store(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (kj[t] >= S) continue;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const size_t at = off + static_cast<size_t>(kj[t]) * ld + 16 * dt + 4 * g;
      if (kDK)
        *reinterpret_cast<float4*>(dk + at) =
            make_float4(dka[t][dt][0], dka[t][dt][1], dka[t][dt][2], dka[t][dt][3]);
      if (kDV)
        *reinterpret_cast<float4*>(dv + at) =
            make_float4(dva[t][dt][0], dva[t][dt][1], dva[t][dt][2], dva[t][dt][3]);
    }
  }
}

dim3 GridOf(size_t B, size_t S, size_t H) {
  return dim3(static_cast<unsigned>((S + kRowsWG - 1) / kRowsWG * B * H));
}

}  // namespace

bool Attn32Fits(size_t B, size_t S, size_t H, size_t d, std::initializer_list<const void*> ptrs) {
  if (!(d == 64 || d == 128) || S == 0 || B * H == 0) return false;
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15) != 0) return false;
  return (S + kRowsWG - 1) / kRowsWG * B * H < (size_t{1} << 31) && B * H < (size_t{1} << 31) &&
         S < (size_t{1} << 30) && H * d < (size_t{1} << 30);
}

hipError_t LaunchAttn32Fwd(const float* q, const float* k, const float* v, float* o, float* stats,
                           size_t B, size_t S, size_t H, size_t d, const int32_t* starts,
                           hipStream_t s) {
  const int Si = static_cast<int>(S), Hi = static_cast<int>(H);
  if (d == 64)
    hipLaunchKernelGGL(Attn32Fwd<64>, GridOf(B, S, H), dim3(kThreads), 0, s, q, k, v, o, stats, Si,
                       Hi, starts);
  else
    hipLaunchKernelGGL(Attn32Fwd<128>, GridOf(B, S, H), dim3(kThreads), 0, s, q, k, v, o, stats,
                       Si, Hi, starts);
  return hipGetLastError();
}

hipError_t LaunchAttn32DQ(const float* q, const float* k, const float* v, const float* dout,
                          float* stats, float* dq, size_t B, size_t S, size_t H, size_t d,
                          hipStream_t s) {
  const int Si = static_cast<int>(S), Hi = static_cast<int>(H);
  if (d == 64)
    hipLaunchKernelGGL(Attn32DQ<64>, GridOf(B, S, H), dim3(kThreads), 0, s, q, k, v, dout, stats,
                       dq, Si, Hi);
  else
    hipLaunchKernelGGL(Attn32DQ<128>, GridOf(B, S, H), dim3(kThreads), 0, s, q, k, v, dout, stats,
                       dq, Si, Hi);
  return hipGetLastError();
}

hipError_t LaunchAttn32DKDV(const float* q, const float* k, const float* v, const float* dout,
                            const float* stats, float* dk, float* dv, size_t B, size_t S, size_t H,
                            size_t d, hipStream_t s) {
  const int Si = static_cast<int>(S), Hi = static_cast<int>(H);
  const dim3 grid = GridOf(B, S, H), blk(kThreads);
#define SEEAI_DKDV(DD, A, Bv) \
  hipLaunchKernelGGL((Attn32DKDV<DD, A, Bv>), grid, blk, 0, s, q, k, v, dout, stats, dk, dv, Si, Hi)
  if (d == 64) {
    if (dk && dv) SEEAI_DKDV(64, true, true);
    else if (dk) SEEAI_DKDV(64, true, false);
    else SEEAI_DKDV(64, false, true);
  } else {
    if (dk && dv) SEEAI_DKDV(128, true, true);
    else if (dk) SEEAI_DKDV(128, true, false);
    else SEEAI_DKDV(128, false, true);
  }
#undef SEEAI_DKDV
  return hipGetLastError();
}

}  // namespace seeai
