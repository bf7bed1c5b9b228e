// k_flash.hip -- the bf16-operand tiled attention family on CDNA4 bf16
// MFMA: forward, dQ, dK and dV over the stats-row contract of the exact
// family (instruction.h:174-190, 234-259).  It runs relaxed (kFlagRelaxed,
// instruction.h:356-390) attention where the backend is switched to bf16
// attention (seeai_set_attention_bf16: the BASELINE bf16 configurations).
// Operands arrive as f32 and are rounded to bf16 (RNE) as they are staged,
// unscaled, so bf16-valued inputs enter the products exactly; products
// accumulate in f32; the 1/sqrt(d) and log2(e) factors multiply the f32
// scores; softmax runs in f32 in the base-2 domain.
//
// Geometry: one workgroup = 4 waves = 128 rows of one (b, h) -- queries for
// the forward and dQ, keys for dK/dV -- each wave owning 32 rows; the other
// side streams through LDS in blocks of 64, double buffered, converted to
// bf16 once per block and stored in both the row layout (A operand of the
// score product) and the transposed layout (operand of the accumulation).
// Scores are formed transposed -- S^T = K Q^T (forward, dQ) or S = Q K^T
// (dK/dV) -- so the v_mfma_f32_32x32x16_bf16 accumulator layout (lane
// (g = lane/32, c = lane%32) holds rows 8q + 4g + e, q < 4, e < 4, of
// column c) is exactly the operand layout of the next product: the
// probabilities never leave registers.  Row reductions over the streamed
// side are in-lane plus one lane swap.  Every output element has one
// writer; no atomics.
#include "common.h"

namespace seeai {
namespace {

constexpr int kFThreads = 256;   // 4 waves
constexpr int kRows = 128;       // rows owned per workgroup (32 per wave)
constexpr int kBlk = 64;         // streamed rows per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Word 3 of a raw (stride 0) buffer resource on CDNA: 32-bit data format,
// out-of-range reads return zero.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ v16f Mfma(const bf16x8& a, const bf16x8& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x4 Cvt4(float4 v) {
  return bf16x4{static_cast<__bf16>(v.x), static_cast<__bf16>(v.y), static_cast<__bf16>(v.z),
                static_cast<__bf16>(v.w)};
}

__device__ __forceinline__ size_t StatsStart(float stored, int i) {
  if (!(stored > 0.0f)) return 0;
  const float cap = static_cast<float>(i);
  return stored >= cap ? static_cast<size_t>(i) : static_cast<size_t>(stored);
}

// One streamed block of 64 rows x D dims (f32 in HBM) staged as bf16 into
// a row tile [64][D + 8] and, optionally, a transposed tile [D][64 + 4].
// Lane t handles 4 rows x 4 dims per pass: 16 lanes cover one row's 64
// dims (256 contiguous bytes), the 4 x 4 block transposes in registers.
// Rows are read through a buffer resource spanning the valid rows of the
// (b, h) slice, so rows past the sequence end read as zeros without a
// branch; the per-lane byte offsets are fixed, the block start moves the
// resource base.
template <int D>
struct Stager {
  static constexpr int RLD = D + 8;        // row tile stride (bf16)
  static constexpr int TLD = kBlk + 4;     // transposed tile stride (bf16)
  static constexpr int kD4 = D / 4;
  static constexpr int kPasses = (kBlk / 4) * kD4 / kFThreads;  // 1 (D=64) or 2 (D=128)
  static constexpr int kPassRows = kBlk / kPasses;                 // rows one pass covers
  float4 reg[kPasses][4];
  uint32_t voff[kPasses][4];

  __device__ __forceinline__ explicit Stager(uint32_t ld) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int t = threadIdx.x + p * kFThreads;
      const int d4 = t % kD4, rg = t / kD4;
#pragma unroll
      for (int k = 0; k < 4; ++k) voff[p][k] = ((rg * 4 + k) * ld + d4 * 4) * 4u;
    }
  }
  __device__ __forceinline__ void load(const float* slice, uint32_t slice_bytes, uint32_t ld,
                                       int row0) {
    const uint32_t skip = static_cast<uint32_t>(row0) * ld * 4u;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(slice) + static_cast<size_t>(row0) * ld, 0,
        Uniform(static_cast<int>(slice_bytes - skip)), kRsrcWord3);
#pragma unroll
    for (int p = 0; p < kPasses; ++p)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff[p][k], 0, 0);
        reg[p][k] = *reinterpret_cast<const float4*>(&v);
      }
  }
  __device__ __forceinline__ void store(__bf16* __restrict__ rows, __bf16* __restrict__ trans) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int t = threadIdx.x + p * kFThreads;
      const int d4 = t % kD4, rg = t / kD4;
      if (rows) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          *reinterpret_cast<bf16x4*>(rows + (rg * 4 + k) * RLD + d4 * 4) = Cvt4(reg[p][k]);
      }
      if (trans) {
        const float* f = reinterpret_cast<const float*>(&reg[p][0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x4 col = {static_cast<__bf16>(f[0 * 4 + e]), static_cast<__bf16>(f[1 * 4 + e]),
                              static_cast<__bf16>(f[2 * 4 + e]), static_cast<__bf16>(f[3 * 4 + e])};
          *reinterpret_cast<bf16x4*>(trans + (d4 * 4 + e) * TLD + rg * 4) = col;
        }
      }
    }
  }
};

// This lane's 32 owned rows as a B (or A) operand over D dims, scaled by
// `scale` before rounding: row c of the wave's tile, dims 16s + 8g .. +8.
template <int D>
__device__ __forceinline__ void LoadOwned(const float* __restrict__ row, int g, float scale,
                                          bf16x8* out) {
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const float4 a = *reinterpret_cast<const float4*>(row + 16 * s + 8 * g);
    const float4 b = *reinterpret_cast<const float4*>(row + 16 * s + 8 * g + 4);
    out[s] = bf16x8{static_cast<__bf16>(a.x * scale), static_cast<__bf16>(a.y * scale),
                    static_cast<__bf16>(a.z * scale), static_cast<__bf16>(a.w * scale),
                    static_cast<__bf16>(b.x * scale), static_cast<__bf16>(b.y * scale),
                    static_cast<__bf16>(b.z * scale), static_cast<__bf16>(b.w * scale)};
  }
}

// acc = init + rowtile[kt*32 + c] . owned[c] over D dims: 32 streamed rows
// kt*32.. of the block x this wave's 32 owned columns.  The accumulator
// starts from `init`, which carries each element's offset (the softmax
// row offset, or -delta) so the product arrives already shifted.
template <int D>
__device__ __forceinline__ v16f ScoreTile(const __bf16* __restrict__ tile, const bf16x8* owned,
                                          int lane, int kt, const v16f& init) {
  constexpr int RLD = D + 8;
  const int g = lane / 32, c = lane % 32;
  v16f a = init;
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const bf16x8 kf = *reinterpret_cast<const bf16x8*>(tile + (kt * 32 + c) * RLD + 16 * s + 8 * g);
    a = Mfma(kf, owned[s], a);
  }
  return a;
}

__device__ __forceinline__ v16f Splat(float x) {
  v16f v;
#pragma unroll
  for (int r = 0; r < 16; ++r) v[r] = x;
  return v;
}

// The weights of one 32-row score tile kt (this lane's 16 values, rows
// 8q + 4g + e in w[4q + e]) as the two B operands of AccumTiles.
__device__ __forceinline__ void PackTile(const float* w, bf16x8* out) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
    out[h] = bf16x8{static_cast<__bf16>(w[8 * h + 0]), static_cast<__bf16>(w[8 * h + 1]),
                    static_cast<__bf16>(w[8 * h + 2]), static_cast<__bf16>(w[8 * h + 3]),
                    static_cast<__bf16>(w[8 * h + 4]), static_cast<__bf16>(w[8 * h + 5]),
                    static_cast<__bf16>(w[8 * h + 6]), static_cast<__bf16>(w[8 * h + 7])};
}

// out[dt] (dims dt*32 + 8q + 4g + e, column c) += sum over the 64 streamed
// rows of trans[dim][row] * w(row, c), with w packed by PackTile: bw[s]
// holds rows 16s + 4g + {0..3} and 16s + 8 + 4g + {0..3}.  The k order of
// the product is permuted alike on both operands.
template <int D>
__device__ __forceinline__ void AccumTiles(const __bf16* __restrict__ trans, const bf16x8* bw,
                                           int lane, v16f* out) {
  constexpr int TLD = kBlk + 4;
  const int g = lane / 32, c = lane % 32;
#pragma unroll
  for (int s = 0; s < kBlk / 16; ++s) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const __bf16* r = trans + (dt * 32 + c) * TLD + 16 * s + 4 * g;
      const bf16x4 lo = *reinterpret_cast<const bf16x4*>(r);
      const bf16x4 hi = *reinterpret_cast<const bf16x4*>(r + 8);
      const bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      out[dt] = Mfma(av, bw[s], out[dt]);
    }
  }
}

__device__ __forceinline__ float SwapMax(float v) { return fmaxf(v, __shfl_xor(v, 32, kWave)); }
__device__ __forceinline__ float SwapSum(float v) { return v + __shfl_xor(v, 32, kWave); }
// Wave maximum, returned as a scalar (the value is the same in every lane).
__device__ __forceinline__ int WaveMaxI(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
  return __builtin_amdgcn_readfirstlane(v);
}


// Streamed row of score element r of tile kt, relative to the block start;
// RowConst is its lane-independent part (the lane adds 4g).
__device__ __forceinline__ int RowOf(int kt, int r, int g) { return kt * 32 + 8 * (r / 4) + 4 * g + (r % 4); }
__device__ __forceinline__ constexpr int RowConst(int kt, int r) { return kt * 32 + 8 * (r / 4) + (r % 4); }

// Masks built from sign bits rather than comparisons, so the 32 per-element
// tests of a diagonal block stay in vector registers: all ones when a < 0
// or b < 0.
__device__ __forceinline__ int Outside(int a, int b) { return (a | b) >> 31; }
// x where the mask is clear, -inf where it is set.
__device__ __forceinline__ float OrNegInf(float x, int bad) {
  return __int_as_float((__float_as_int(x) & ~bad) | (static_cast<int>(0xff800000u) & bad));
}
// x where the mask is clear, +0 where it is set.
__device__ __forceinline__ float OrZero(float x, int bad) { return __int_as_float(__float_as_int(x) & ~bad); }

// Work unit of this workgroup: (bh, rank) with rank 0 the heaviest of the
// nq row blocks of one (b, h).  Consecutive workgroup ids land on the 8 XCDs
// in turn, so ids are regrouped to give each XCD whole (b, h) slices, heavy
// blocks first: the K / V (or Q / dO) of a slice is then read into one L2.
__device__ __forceinline__ void UnitOf(int nq, int& bh, int& rank) {
  const int w = blockIdx.x, total = gridDim.x;
  const int t = total % 8 == 0 ? (w % 8) * (total / 8) + w / 8 : w;
  bh = t / nq;
  rank = t % nq;
}

// ---------------------------------------------------------------------------
// Forward: O = softmax(mask(Q K^T / sqrt d)) V and the stats row.
//
// Q is staged unscaled; a score tile's accumulator starts at -m_use / c with
// c = log2(e)/sqrt(d), so c times the tile is s' - m_use in base-2 units and
// one v_exp gives the weight.  m_use moves only when a
// block's maximum exceeds it by more than 2^8 (weights stay below 2^8 in
// f32) or on the first block a row sees; the true row maximum is tracked
// beside it and the stats row is stated against it, so (m, 1/l) is the
// reference's.  l sums the bf16-rounded weights that the P V product uses.
// ---------------------------------------------------------------------------
constexpr float kLazy = 8.0f;

template <int D>
__global__ void __launch_bounds__(kFThreads)
FlashFwd(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
         float* __restrict__ o, float* __restrict__ stats, int S, int H,
         const int32_t* __restrict__ starts) {
  using St = Stager<D>;
  __shared__ __attribute__((aligned(16))) __bf16 Ks[2][kBlk * St::RLD];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[2][D * St::TLD];
  __shared__ int min_start;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 32, c = lane % 32;
  const int nq = (S + kRows - 1) / kRows;
  int bh, rank;
  UnitOf(nq, bh, rank);
  const int qblk = nq - 1 - rank;
  const int b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int i0 = qblk * kRows + wave * 32;
  const int i = i0 + c;
  const int ic = min(i, S - 1);
  int j_start = 0;
  if (starts) {
    const int s0 = starts[static_cast<size_t>(b) * S + ic];
    j_start = s0 <= 0 ? 0 : min(s0, ic);
  }
  if (threadIdx.x == 0) min_start = S;
  __syncthreads();
  atomicMin(&min_start, j_start);  // integer min: order-independent
  __syncthreads();
  const int wave_max_start = WaveMaxI(j_start);
  const int blk_lo = Uniform(min_start) / kBlk;
  const int q_hi = min(qblk * kRows + kRows - 1, S - 1);
  const int nblk = q_hi / kBlk + 1 - blk_lo;

  bf16x8 qf[D / 16];
  LoadOwned<D>(q + base + static_cast<size_t>(ic) * ld, g, 1.0f, qf);
  const float scl = kLog2e / sqrtf(static_cast<float>(D)), inv_scl = 1.0f / scl;

  v16f oacc[D / 32] = {};
  float m_use = 0.0f, m_true = -INFINITY, l = 0.0f;
  v16f cneg = {};  // splat(-m_use / c)
  const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  const uint32_t ld32 = static_cast<uint32_t>(ld);
  const uint32_t slice_bytes = static_cast<uint32_t>(((S - 1) * ld + D) * 4);
  St sk(ld32), sv(ld32);
  auto load = [&](int jb) {
    const int j0 = (blk_lo + jb) * kBlk;
    sk.load(k + base, slice_bytes, ld32, j0);
    sv.load(v + base, slice_bytes, ld32, j0);
  };
  auto block = [&](auto masked, int buf, int j0) {
    constexpr bool kMask = decltype(masked)::value;
    const int hi_rel = i - j0 - 4 * g, lo_rel = j_start - j0 - 4 * g;
    v16f st[2];
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      st[kt] = ScoreTile<D>(Ks[buf], qf, lane, kt, cneg);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        st[kt][r] *= scl;
        if constexpr (kMask)  // keep j0 + row in [j_start, i]
          st[kt][r] = OrNegInf(st[kt][r], Outside(hi_rel - RowConst(kt, r), RowConst(kt, r) - lo_rel));
        bmax = fmaxf(bmax, st[kt][r]);
      }
    }
    bmax = SwapMax(bmax);  // relative to m_use
    const bool first = m_true == -INFINITY;
    if (bmax != -INFINITY) m_true = fmaxf(m_true, m_use + bmax);
    const bool need = first ? bmax != -INFINITY : bmax > kLazy;
    if (__any(need)) {
      const float shift = need ? bmax : 0.0f;
      const float alpha = first ? 0.0f : Exp2(-shift);
      m_use += shift;
      cneg = Splat(-m_use * inv_scl);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) oacc[dt] *= alpha;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) st[kt] -= shift;
    }
    bf16x8 pb[4];
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = Exp2(st[kt][r]);
      PackTile(p, pb + 2 * kt);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          psum = __builtin_amdgcn_fdot2_f32_bf16(
              bf16x2{pb[2 * kt + h2][2 * e], pb[2 * kt + h2][2 * e + 1]}, ones, psum, false);
    }
    l += SwapSum(psum);
    AccumTiles<D>(Vt[buf], pb, lane, oacc);
  };

  load(0);
  sk.store(Ks[0], nullptr);
  sv.store(nullptr, Vt[0]);
  __syncthreads();
  for (int jb = 0; jb < nblk; ++jb) {
    const int buf = jb & 1;
    if (jb + 1 < nblk) load(jb + 1);
    const int j0 = (blk_lo + jb) * kBlk;
    if (j0 + kBlk - 1 <= i0 && j0 >= wave_max_start)
      block(std::false_type{}, buf, j0);
    else if (j0 <= i0 + 31)  // a block wholly after this wave's queries is masked
      block(std::true_type{}, buf, j0);
    if (jb + 1 < nblk) {
      sk.store(Ks[buf ^ 1], nullptr);
      sv.store(nullptr, Vt[buf ^ 1]);
    }
    __syncthreads();
  }
  if (i >= S) return;
  const float inv = 1.0f / l;
  float* orow = o + base + static_cast<size_t>(i) * ld;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<float4*>(orow + dt * 32 + 8 * qq + 4 * g) =
          make_float4(oacc[dt][4 * qq] * inv, oacc[dt][4 * qq + 1] * inv, oacc[dt][4 * qq + 2] * inv,
                      oacc[dt][4 * qq + 3] * inv);
  if (g == 0) {
    float* st = stats + (static_cast<size_t>(bh) * S + i) * 4;
    st[0] = m_true * kLn2;
    st[1] = inv * Exp2(m_true - m_use);  // 1 / sum exp(s - m_true)
    st[2] = 0.0f;
    st[3] = static_cast<float>(j_start);
  }
}

// Row offset of the base-2 exponent: p = 2^(s' - mm) with s' = s log2(e)
// and mm = m log2(e) + log2(l), from the stats row (m, 1/l).
__device__ __forceinline__ float RowOffset(float m, float inv) { return m * kLog2e - log2f(inv); }

// ---------------------------------------------------------------------------
// dQ and the stats row's delta = sum_j p dP.  Q is staged unscaled as in the
// forward and the score accumulators start at -mm / c (p = 2^(c score)).
//
// kOnePass: dS = p (dP - delta) is linear in delta, so
//   dQ^T = K^T (p dP)^T - delta K^T p^T,
// and delta itself accumulates in the same pass: one walk over K / V, four
// products per block (S, dP and the two accumulations) and one exponential
// per score.  The bf16 operands are p dP and p instead of p (dP - delta),
// so each term's rounding is relative to |dP| + |delta| rather than
// |dP - delta|.
// Otherwise two walks: delta first (S and dP), then S, dP and
// dQ^T += K^T dS^T with the dP accumulators started at -delta: five
// products and two exponentials per score.
// dQ is scaled by 1/sqrt d once, at the end.
// ---------------------------------------------------------------------------
template <int D, bool kOnePass>
__global__ void __launch_bounds__(kFThreads)
FlashDQ(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
        const float* __restrict__ dout, float* __restrict__ stats, float* __restrict__ dq, int S,
        int H) {
  using St = Stager<D>;
  __shared__ __attribute__((aligned(16))) __bf16 Ks[2][kBlk * St::RLD];
  __shared__ __attribute__((aligned(16))) __bf16 Kt[2][D * St::TLD];
  __shared__ __attribute__((aligned(16))) __bf16 Vs[2][kBlk * St::RLD];
  __shared__ int min_start;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 32, c = lane % 32;
  const int nq = (S + kRows - 1) / kRows;
  int bh, rank;
  UnitOf(nq, bh, rank);
  const int qblk = nq - 1 - rank;
  const int b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int i0 = qblk * kRows + wave * 32;
  const int i = i0 + c;
  const int ic = min(i, S - 1);
  float* st = stats + (static_cast<size_t>(bh) * S + ic) * 4;
  const float isd = 1.0f / sqrtf(static_cast<float>(D));
  const float scl = kLog2e * isd;
  const v16f cs = Splat(-RowOffset(st[0], st[1]) / scl);
  const int j_start = static_cast<int>(StatsStart(st[3], ic));
  if (threadIdx.x == 0) min_start = S;
  __syncthreads();
  atomicMin(&min_start, j_start);
  __syncthreads();
  const int wave_max_start = WaveMaxI(j_start);
  const int blk_lo = Uniform(min_start) / kBlk;
  const int q_hi = min(qblk * kRows + kRows - 1, S - 1);
  const int nblk = q_hi / kBlk + 1 - blk_lo;

  bf16x8 qf[D / 16], df[D / 16];
  LoadOwned<D>(q + base + static_cast<size_t>(ic) * ld, g, 1.0f, qf);
  LoadOwned<D>(dout + base + static_cast<size_t>(ic) * ld, g, 1.0f, df);

  const uint32_t ld32 = static_cast<uint32_t>(ld);
  const uint32_t slice_bytes = static_cast<uint32_t>(((S - 1) * ld + D) * 4);
  St sk(ld32), sv(ld32);
  auto load = [&](int jb) {
    const int j0 = (blk_lo + jb) * kBlk;
    sk.load(k + base, slice_bytes, ld32, j0);
    sv.load(v + base, slice_bytes, ld32, j0);
  };

  float delta = 0.0f;
  v16f acc[D / 32], acc_p[kOnePass ? D / 32 : 1];
  // pass 0: delta only; pass 1: dQ (and, in one pass, delta beside it)
  for (int pass = kOnePass ? 1 : 0; pass < 2; ++pass) {
    const v16f cp = Splat(kOnePass ? 0.0f : -delta);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = v16f{};
    if constexpr (kOnePass) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) acc_p[dt] = v16f{};
    }
    auto run = [&](auto masked, int buf, int j0) {
      constexpr bool kMask = decltype(masked)::value;
      const int hi_rel = i - j0 - 4 * g, lo_rel = j_start - j0 - 4 * g;
      bf16x8 wb[4], pb[kOnePass ? 4 : 1];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const v16f sc = ScoreTile<D>(Ks[buf], qf, lane, kt, cs);
        const v16f dpt = ScoreTile<D>(Vs[buf], df, lane, kt, cp);
        float w[16], p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float e = Exp2(sc[r] * scl);
          if constexpr (kMask)  // keep j0 + row in [j_start, i]
            e = OrZero(e, Outside(hi_rel - RowConst(kt, r), RowConst(kt, r) - lo_rel));
          if (kOnePass || pass == 0) delta = __builtin_fmaf(dpt[r], e, delta);
          if (pass == 1) w[r] = e * dpt[r];
          p[r] = e;
        }
        if (pass == 1) PackTile(w, wb + 2 * kt);
        if (kOnePass) PackTile(p, pb + 2 * kt);
      }
      if (pass == 1) AccumTiles<D>(Kt[buf], wb, lane, acc);
      if (kOnePass) AccumTiles<D>(Kt[buf], pb, lane, acc_p);
    };
    load(0);
    sk.store(Ks[0], pass ? Kt[0] : nullptr);
    sv.store(Vs[0], nullptr);
    __syncthreads();
    for (int jb = 0; jb < nblk; ++jb) {
      const int buf = jb & 1;
      if (jb + 1 < nblk) load(jb + 1);
      const int j0 = (blk_lo + jb) * kBlk;
      if (j0 + kBlk - 1 <= i0 && j0 >= wave_max_start)
        run(std::false_type{}, buf, j0);
      else if (j0 <= i0 + 31)
        run(std::true_type{}, buf, j0);
      if (jb + 1 < nblk) {
        sk.store(Ks[buf ^ 1], pass ? Kt[buf ^ 1] : nullptr);
        sv.store(Vs[buf ^ 1], nullptr);
      }
      __syncthreads();
    }
    if (!kOnePass && pass == 0) delta = SwapSum(delta);
  }
  if (kOnePass) delta = SwapSum(delta);
  if (i >= S) return;
  if constexpr (kOnePass) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] -= delta * acc_p[dt];
  }
  float* drow = dq + base + static_cast<size_t>(i) * ld;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<float4*>(drow + dt * 32 + 8 * qq + 4 * g) =
          make_float4(acc[dt][4 * qq] * isd, acc[dt][4 * qq + 1] * isd, acc[dt][4 * qq + 2] * isd,
                      acc[dt][4 * qq + 3] * isd);
  if (g == 0) st[2] = delta;
}

// ---------------------------------------------------------------------------
// dK and / or dV: one wave per 32 keys walking the query blocks from the
// diagonal; S = Q K^T and dP = dO V^T formed query-major, dK^T += Q^T dS
// (times 1/sqrt d at the end), dV^T += dO^T P.  K is staged unscaled; the
// score and dP accumulators start at each query row's -mm / c and -delta,
// read from LDS.  With both outputs (kDK && kDV) one pass forms
// S, P and dP once per block and feeds both accumulations: four products
// per block instead of the five of two passes, one exponential per score
// instead of two.
// ---------------------------------------------------------------------------
template <int D, bool kDK, bool kDV>
__global__ void __launch_bounds__(kFThreads)
FlashDKDV(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
          const float* __restrict__ dout, const float* __restrict__ stats,
          float* __restrict__ out_k, float* __restrict__ out_v, int S, int H) {
  using St = Stager<D>;
  __shared__ __attribute__((aligned(16))) __bf16 Qs[2][kBlk * St::RLD];
  __shared__ __attribute__((aligned(16))) __bf16 Qt[2][kDK ? D * St::TLD : 1];
  __shared__ __attribute__((aligned(16))) __bf16 Ds[2][kDK ? kBlk * St::RLD : 1];
  __shared__ __attribute__((aligned(16))) __bf16 Dt[2][kDV ? D * St::TLD : 1];
  // Per streamed query row: -mm, -delta, document start; and the block's
  // largest start.
  __shared__ __attribute__((aligned(16))) float Smm[2][kBlk];
  __shared__ __attribute__((aligned(16))) float Sdl[2][kBlk];
  __shared__ int Sst[2][kBlk];
  __shared__ int Smax[2];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 32, c = lane % 32;
  const int nk = (S + kRows - 1) / kRows;
  int bh, kblk;
  UnitOf(nk, bh, kblk);  // rank 0 = the first keys, the longest columns
  const int b = bh / H, h = bh % H;
  const size_t ld = static_cast<size_t>(H) * D;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * D;
  const int j0w = kblk * kRows + wave * 32;
  const int j = j0w + c;
  const int jc = min(j, S - 1);
  const float isd = 1.0f / sqrtf(static_cast<float>(D));
  const float scl = kLog2e * isd, inv_scl = 1.0f / scl;
  const float4* st_bh = reinterpret_cast<const float4*>(stats) + static_cast<size_t>(bh) * S;

  bf16x8 kf[D / 16], vf[D / 16];
  LoadOwned<D>(k + base + static_cast<size_t>(jc) * ld, g, 1.0f, kf);
  if (kDK) LoadOwned<D>(v + base + static_cast<size_t>(jc) * ld, g, 1.0f, vf);

  const int blk_first = (kblk * kRows) / kBlk;
  const int nblk = (S + kBlk - 1) / kBlk - blk_first;
  const uint32_t ld32 = static_cast<uint32_t>(ld);
  const uint32_t slice_bytes = static_cast<uint32_t>(((S - 1) * ld + D) * 4);
  St sq(ld32), sd(ld32);
  auto load = [&](int ib) {
    const int r0 = (blk_first + ib) * kBlk;
    sq.load(q + base, slice_bytes, ld32, r0);
    sd.load(dout + base, slice_bytes, ld32, r0);
  };
  auto stage = [&](int buf, int ib) {
    sq.store(Qs[buf], kDK ? Qt[buf] : nullptr);
    sd.store(kDK ? Ds[buf] : nullptr, kDV ? Dt[buf] : nullptr);
    if (threadIdx.x < kBlk) {  // wave 0
      const int t = threadIdx.x, iq = (blk_first + ib) * kBlk + t;
      int start = 0;
      if (iq < S) {
        const float4 s4 = st_bh[iq];
        Smm[buf][t] = -RowOffset(s4.x, s4.y) * inv_scl;
        Sdl[buf][t] = -s4.z;
        start = static_cast<int>(StatsStart(s4.w, iq));
      } else {
        Smm[buf][t] = -INFINITY;  // weight 0 past the sequence end
        Sdl[buf][t] = 0.0f;
      }
      Sst[buf][t] = start;
      const int mx = WaveMaxI(start);
      if (t == 0) Smax[buf] = mx;
    }
  };
  // The 16 per-row values of tile kt for this lane (rows 8q + 4g + e).
  auto rows16 = [&](const float* src, int kt) {
    v16f x;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const float4 f = *reinterpret_cast<const float4*>(src + kt * 32 + 8 * q4 + 4 * g);
      x[4 * q4] = f.x;
      x[4 * q4 + 1] = f.y;
      x[4 * q4 + 2] = f.z;
      x[4 * q4 + 3] = f.w;
    }
    return x;
  };

  v16f acc_k[kDK ? D / 32 : 1] = {}, acc_v[kDV ? D / 32 : 1] = {};
  auto run = [&](auto masked, int buf, int r0) {
    constexpr bool kMask = decltype(masked)::value;
    const int lo_rel = r0 + 4 * g - j;  // query row r0 + il minus this lane's key
    bf16x8 wb[kDK ? 4 : 1], pb[kDV ? 4 : 1];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const v16f sc = ScoreTile<D>(Qs[buf], kf, lane, kt, rows16(Smm[buf], kt));
      v16f dpt;
      if (kDK) dpt = ScoreTile<D>(Ds[buf], vf, lane, kt, rows16(Sdl[buf], kt));
      float p[16], w[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float e = Exp2(sc[r] * scl);
        if constexpr (kMask) {  // keep query row r0 + il >= j and its start <= j
          const int il = RowOf(kt, r, g);
          e = OrZero(e, Outside(lo_rel + RowConst(kt, r), j - Sst[buf][il]));
        }
        p[r] = e;
        if (kDK) w[r] = e * dpt[r];
      }
      if (kDK) PackTile(w, wb + 2 * kt);
      if (kDV) PackTile(p, pb + 2 * kt);
    }
    if (kDK) AccumTiles<D>(Qt[buf], wb, lane, acc_k);
    if (kDV) AccumTiles<D>(Dt[buf], pb, lane, acc_v);
  };

  load(0);
  stage(0, 0);
  __syncthreads();
  for (int ib = 0; ib < nblk; ++ib) {
    const int buf = ib & 1;
    if (ib + 1 < nblk) load(ib + 1);
    const int r0 = (blk_first + ib) * kBlk;
    if (r0 >= j0w + 31 && r0 + kBlk <= S && Uniform(Smax[buf]) <= j0w)
      run(std::false_type{}, buf, r0);
    else if (r0 + kBlk - 1 >= j0w)  // some query of the block reaches this wave's keys
      run(std::true_type{}, buf, r0);
    if (ib + 1 < nblk) stage(buf ^ 1, ib + 1);
    __syncthreads();
  }
  if (j >= S) return;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const size_t at = base + static_cast<size_t>(j) * ld + dt * 32 + 8 * qq + 4 * g;
      if (kDK)
        *reinterpret_cast<float4*>(out_k + at) =
            make_float4(acc_k[dt][4 * qq] * isd, acc_k[dt][4 * qq + 1] * isd,
                        acc_k[dt][4 * qq + 2] * isd, acc_k[dt][4 * qq + 3] * isd);
      if (kDV)
        *reinterpret_cast<float4*>(out_v + at) =
            make_float4(acc_v[dt][4 * qq], acc_v[dt][4 * qq + 1], acc_v[dt][4 * qq + 2],
                        acc_v[dt][4 * qq + 3]);
    }
}

}  // namespace

// The staging reads address one (b, h) slice with 32-bit byte offsets, and
// the grid is one-dimensional.
bool FlashFits(size_t B, size_t S, size_t H, size_t d) {
  return S > 0 && S * H * d * 4 < (size_t{1} << 31) &&
         (S + kRows - 1) / kRows * B * H < (size_t{1} << 31);
}

// One workgroup per (b, h, 128-row block), a 1D grid regrouped per XCD.
inline dim3 FlashGrid(size_t B, size_t S, size_t H) {
  return dim3(static_cast<unsigned>((S + kRows - 1) / kRows * B * H));
}

hipError_t LaunchFlashFwd(const float* q, const float* k, const float* v, float* o, float* stats,
                          size_t B, size_t S, size_t H, size_t d, const int32_t* starts,
                          hipStream_t s) {
  const dim3 grid = FlashGrid(B, S, H);
  if (d == 64)
    hipLaunchKernelGGL(FlashFwd<64>, grid, dim3(kFThreads), 0, s, q, k, v, o, stats,
                       static_cast<int>(S), static_cast<int>(H), starts);
  else
    hipLaunchKernelGGL(FlashFwd<128>, grid, dim3(kFThreads), 0, s, q, k, v, o, stats,
                       static_cast<int>(S), static_cast<int>(H), starts);
  return hipGetLastError();
}

hipError_t LaunchFlashDQ(const float* q, const float* k, const float* v, const float* dout,
                         float* stats, float* dq, size_t B, size_t S, size_t H, size_t d,
                         int one_pass, hipStream_t s) {
  const dim3 grid = FlashGrid(B, S, H);
  const int Si = static_cast<int>(S), Hi = static_cast<int>(H);
#define SEEAI_DQ(DD, OP) \
  hipLaunchKernelGGL((FlashDQ<DD, OP>), grid, dim3(kFThreads), 0, s, q, k, v, dout, stats, dq, Si, Hi)
  if (d == 64) {
    if (one_pass) SEEAI_DQ(64, true);
    else SEEAI_DQ(64, false);
  } else {
    if (one_pass) SEEAI_DQ(128, true);
    else SEEAI_DQ(128, false);
  }
#undef SEEAI_DQ
  return hipGetLastError();
}

hipError_t LaunchFlashDKDV(const float* q, const float* k, const float* v, const float* dout,
                           const float* stats, float* dk, float* dv, size_t B, size_t S, size_t H,
                           size_t d, hipStream_t s) {
  if (!dk && !dv) return hipErrorInvalidValue;
  const dim3 grid = FlashGrid(B, S, H);
  const int Si = static_cast<int>(S), Hi = static_cast<int>(H);
#define SEEAI_DKDV(DD, KK, VV)                                                                    \
  hipLaunchKernelGGL((FlashDKDV<DD, KK, VV>), grid, dim3(kFThreads), 0, s, q, k, v, dout, stats, dk, \
                     dv, Si, Hi)
  if (d == 64) {
    if (dk && dv) SEEAI_DKDV(64, true, true);
    else if (dk) SEEAI_DKDV(64, true, false);
    else SEEAI_DKDV(64, false, true);
  } else {
    // d = 128 runs the two passes apart: both accumulators and both score
    // tiles at once exceed the register file (occupancy 1 with spills).
    if (dk && dv) return hipErrorInvalidValue;
    if (dk) SEEAI_DKDV(128, true, false);
    else SEEAI_DKDV(128, false, true);
  }
#undef SEEAI_DKDV
  return hipGetLastError();
}

bool FlashFusedDKDV(size_t d) { return d == 64; }

}  // namespace seeai
