// k_attn16.hip -- causal attention at head width 64 on bf16 operands held in
// HBM as bf16: forward, dQ and dK / dV over the tiled family's stats-row
// contract (instruction.h:174-190, 234-259), for the models that train in
// bf16 activations (BASELINE configs[2] bf16, [3], [4]).
//
// Staging.  Every tile that enters a product is a 64-row block of one
// (b, h) slice -- 64 rows x 64 dims of bf16 -- copied from HBM straight into
// LDS by buffer_load ... lds (no registers, no conversion).  A tile is two
// halves (dims 0-31, 32-63) of 64-byte rows; chunk c (16 bytes) of row r
// sits at physical chunk (c + r / 4) mod 4, which keeps the MFMA fragment
// reads free of bank conflicts (the W8A8 kernel's measured rotation).  Rows
// past the sequence end read as zeros through the buffer range check.
//
// Products.  v_mfma_f32_32x32x16_bf16 with the scores formed transposed
// (S^T = K Q^T): the accumulator layout -- lane (g = lane / 32, c = lane %
// 32) holding rows 8q + 4g + e of column c -- is then the B operand of the
// next product, so probabilities never leave registers.  Operands whose
// reduction index runs down a tile's rows (V^T in O^T = V^T P^T, K^T in
// dQ^T = K^T dS^T, Q^T and dO^T in dK^T / dV^T) are read with gfx950's
// ds_read_b64_tr_b16, which hands each lane one column of a 4 x 16 block
// gathered from its 16-lane group: no transposed copies.
//
// Every output element has one writer; no atomics; the reductions run in a
// fixed order, so results repeat bit for bit.
#include "common.h"

namespace seeai {
namespace {

constexpr int kD = 64;          // head width
constexpr int kBlkRows = 64;    // rows of a staged tile
constexpr int kTile = kBlkRows * kD * 2;  // bytes of one staged tile (8 KiB)
constexpr int kHalf = kTile / 2;          // one 64-byte-row half
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kRsrcWord3 = 0x00020000;   // raw buffer, 32-bit format, range-checked

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* LdsPtr;
typedef __attribute__((address_space(3))) bf16x4* LdsBf16x4;

__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ v16f Mfma(const bf16x8& a, const bf16x8& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int Phys(int row, int chunk) { return (chunk + row / 4) & 3; }

// s_waitcnt vmcnt(n), the other counters left alone.
template <int n>
__device__ __forceinline__ void WaitVm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

// f(integral_constant<I>) for I = 0 .. N-1, unrolled.
template <int I, int N>
struct Unroll {
  template <class F>
  __device__ __forceinline__ static void Run(F&& f) {
    if constexpr (I < N) {
      f(std::integral_constant<int, I>{});
      Unroll<I + 1, N>::Run(f);
    }
  }
};

// The stage ring of a kernel: kStages buffers of one K-and-V (or Q-and-dO)
// block, each a separate LDS object named at compile time (stage ids are
// template constants after unrolling), so the compiler can tell a fragment
// read of one stage from the DMA into another and does not make the read
// wait for that DMA.
#define SEEAI_STAGE_RING(kStages)                                                          \
  static_assert(kStages >= 2 && kStages <= 4, "2 to 4 stages");                            \
  __shared__ __attribute__((aligned(1024))) uint8_t stage_0[2 * kTile];                    \
  __shared__ __attribute__((aligned(1024))) uint8_t stage_1[2 * kTile];                    \
  __shared__ __attribute__((aligned(1024))) uint8_t stage_2[kStages > 2 ? 2 * kTile : 1];  \
  __shared__ __attribute__((aligned(1024))) uint8_t stage_3[kStages > 3 ? 2 * kTile : 1];  \
  auto stage = [&](auto id) -> uint8_t* {                                                  \
    constexpr int kId = decltype(id)::value % kStages;                                     \
    if constexpr (kId == 0) return stage_0;                                                \
    else if constexpr (kId == 1) return stage_1;                                           \
    else if constexpr (kId == 2) return stage_2;                                           \
    else return stage_3;                                                                   \
  }

// Runs blocks 0 .. nblk-1 through the ring: block jb computes from stage
// jb % kStages while blocks jb + 1 .. jb + kStages - 1 land in the others.
// issue(jb, stage) starts block jb's loads (kLoads per wave); step(jb, stage)
// computes it.  Past the last block the last is loaded again into a stage
// no later block reads, so every wait counts the same number of loads.
template <int kStages, int kLoads, class Issue, class Step, class Stage>
__device__ __forceinline__ void RunRing(int nblk, Issue&& issue, Step&& step, Stage&& stage) {
  const int last = nblk - 1;
  Unroll<0, kStages - 1>::Run([&](auto id) { issue(min(decltype(id)::value, last), stage(id)); });
  for (int jb0 = 0; jb0 < nblk; jb0 += kStages) {
    Unroll<0, kStages>::Run([&](auto id) {
      constexpr int kId = decltype(id)::value;
      const int jb = jb0 + kId;
      if (jb >= nblk) return;
      WaitVm<(kStages - 2) * kLoads>();  // block jb's loads have landed
      __syncthreads();  // ... in every wave, and block jb - 1's stage is free
      issue(min(jb + kStages - 1, last), stage(std::integral_constant<int, kId + kStages - 1>{}));
      step(jb, static_cast<const uint8_t*>(stage(id)));
    });
  }
  WaitVm<0>();  // no load into LDS outlives the workgroup
}

// The (b, h) slice of a [B*S, H*64] bf16 tensor as a buffer resource whose
// first record is row `row0`; rows at or past S are out of range (zeros).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t SliceRsrc(const uint16_t* slice, int ld, int S,
                                                            int row0) {
  const int rows = S - row0;
  const int bytes = rows > 0 ? ((rows - 1) * ld + kD) * 2 : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(slice) +
                                               static_cast<size_t>(row0) * ld,
                                           0, Uniform(bytes), kRsrcWord3);
}

// One wave-load of a tile: 16 rows x 64 bytes of one half, lane l filling
// row r0 + l / 4, physical chunk l % 4.  `u` = half * 4 + row group.
__device__ __forceinline__ int TileLoadOffset(int u, int lane, int ld) {
  const int half = u / 4, row = (u % 4) * 16 + lane / 4;
  const int c = (lane % 4 - row / 4) & 3;
  return row * ld * 2 + half * 64 + c * 16;
}
__device__ __forceinline__ void TileLoad(__amdgpu_buffer_rsrc_t rs, uint8_t* tile, int u,
                                         int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LdsPtr)(tile + (u / 4) * kHalf + (u % 4) * 1024),
                                           16, voff, 0, 0, 0);
}

// Per-lane byte offsets of the two fragment kinds within a tile.  The
// swizzle's phase repeats every 16 rows, so a fragment 16 k rows further
// down (or 32 rows, for the row kind) is the same offset plus a constant:
// the offsets are computed once and the rest folds into the read's
// immediate.
struct FragOffsets {
  int row[2];  // row kind, k-step parity 0 / 1
  int col[2];  // column kind, lo / hi quads
};
__device__ __forceinline__ FragOffsets MakeFragOffsets(int lane) {
  FragOffsets f;
  const int r = lane % 32, g = lane / 32;
#pragma unroll
  for (int p = 0; p < 2; ++p) f.row[p] = r * 64 + Phys(r, 2 * p + g) * 16;
  const int grp = lane / 16, j = lane % 16;
  const int row = 4 * (grp / 2) + j / 4;
  const int byte = 32 * (grp % 2) + 8 * (j % 4);  // within the 64-byte half row
  const int chunk = byte / 16, in = byte % 16;
  f.col[0] = row * 64 + Phys(row, chunk) * 16 + in;
  f.col[1] = (row + 8) * 64 + Phys(row + 8, chunk) * 16 + in;
  return f;
}

// A fragment with the reduction along the tile's columns: lane (g, c) gets
// row `row0 + c` dims 16 s + 8 g .. + 8 (k-step s of the 64 dims); row0 a
// multiple of 32.
__device__ __forceinline__ bf16x8 RowFrag(const uint8_t* tile, const FragOffsets& f, int row0,
                                          int s) {
  return *reinterpret_cast<const bf16x8*>(tile + (s / 2) * kHalf + row0 * 64 + f.row[s % 2]);
}

// A fragment with the reduction down the tile's rows: lane (g, c) gets
// column `32 dt + c` at rows k0 + 4 g + {0..3} (elements 0-3) and
// k0 + 8 + 4 g + {0..3} (elements 4-7) -- the k order PackTile gives the
// register operand it meets; k0 a multiple of 16.  Two transpose reads of
// 4 rows x 16 columns per 16-lane group: lane 16 G + j points at row
// k0 + 4 (G / 2) + j / 4, columns 32 dt + 16 (G % 2) + 4 (j % 4) .. + 4, and
// receives column 32 dt + 16 (G % 2) + j of the group's four rows.
__device__ __forceinline__ bf16x8 ColFrag(const uint8_t* tile, const FragOffsets& f, int dt,
                                          int k0) {
  const uint8_t* base = tile + dt * kHalf + k0 * 64;
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LdsBf16x4)(base + f.col[0]));
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LdsBf16x4)(base + f.col[1]));
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// A 32 x 32 score tile's 16 values in this lane (rows 8q + 4g + e in
// w[4q + e]) as the two B operands of a 16-row-step product over those rows:
// out[h] holds rows 16h + 4g + {0..3} and 16h + 8 + 4g + {0..3}.
__device__ __forceinline__ void PackTile(const float* w, bf16x8* out) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
    out[h] = bf16x8{static_cast<__bf16>(w[8 * h + 0]), static_cast<__bf16>(w[8 * h + 1]),
                    static_cast<__bf16>(w[8 * h + 2]), static_cast<__bf16>(w[8 * h + 3]),
                    static_cast<__bf16>(w[8 * h + 4]), static_cast<__bf16>(w[8 * h + 5]),
                    static_cast<__bf16>(w[8 * h + 6]), static_cast<__bf16>(w[8 * h + 7])};
}

// Lane (g, c)'s 8 dims 16 s + 8 g .. + 8 of one bf16 row, from HBM.
__device__ __forceinline__ bf16x8 OwnedFrag(const uint16_t* row, int s, int lane) {
  return *reinterpret_cast<const bf16x8*>(row + 16 * s + 8 * (lane / 32));
}

// Lanes c and c + 32 combined by v_permlane32_swap (no LDS round trip): the
// swap of v with itself leaves lanes c's value in .x and lane c + 32's in .y
// of both lanes, so the sum is formed in the same order in both.
__device__ __forceinline__ float SwapMax(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float SwapSum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int WaveMaxI(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ int WaveMinI(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return __builtin_amdgcn_readfirstlane(v);
}
// all ones when a < 0 or b < 0
__device__ __forceinline__ int Outside(int a, int b) { return (a | b) >> 31; }
__device__ __forceinline__ float OrNegInf(float x, int bad) {
  return __int_as_float((__float_as_int(x) & ~bad) | (static_cast<int>(0xff800000u) & bad));
}
__device__ __forceinline__ float OrZero(float x, int bad) { return __int_as_float(__float_as_int(x) & ~bad); }
// Row r (0..15) of a lane's accumulator within its 32-row tile, less 4 g.
__device__ __forceinline__ constexpr int RowConst(int r) { return 8 * (r / 4) + (r % 4); }

// Work unit: (bh, rank), rank 0 the heaviest of the nb row blocks of one
// (b, h); consecutive workgroup ids go to the 8 XCDs in turn, so ids are
// regrouped to give each XCD whole (b, h) slices, heavy blocks first.
__device__ __forceinline__ void UnitOf(int nb, int& bh, int& rank) {
  const int w = blockIdx.x, total = gridDim.x;
  const int t = total % 8 == 0 ? (w % 8) * (total / 8) + w / 8 : w;
  bh = t / nb;
  rank = t % nb;
}

// ---------------------------------------------------------------------------
// Forward.  A workgroup of kFwdWaves waves owns kFwdWaves * 32 queries of one
// (b, h), 32 per wave.  Keys stream in 64-row blocks through two stage
// buffers.  The scores arrive as q.k; x = q.k * log2(e)/sqrt(d) - m_use (one
// FMA) is the base-2 exponent of the weight.
//
// Lazy offset.  Lane (g, c) holds 16 of query c's scores per tile, lane
// (1 - g, c) the other 16, and both must weigh against the same m_use.  Each
// half tracks its own maximum; m_use moves only when some half's tile
// maximum passes it by more than 2^8, or on the first tile a half sees --
// rare events, in which the pair first agrees on its maximum by one lane
// swap.  The common tile therefore has no cross-lane traffic: l and the true
// maximum are per half until the end.  The stats row (m, 1/l) is stated
// against the true maximum; l sums the bf16-rounded weights that enter P V.
//
// Every tile runs one body; on the diagonal (and at document starts) a
// uniform branch masks the exponents, so the accumulators keep their
// registers across the branch.
// ---------------------------------------------------------------------------
constexpr float kLazy = 8.0f;

template <int kFwdWaves, int kStages, int kMinBlocks>
__global__ void __launch_bounds__(kFwdWaves * kWave, kMinBlocks)
Attn16Fwd(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
          const uint16_t* __restrict__ v, float* __restrict__ o, float* __restrict__ stats, int S,
          int H, const int32_t* __restrict__ starts, Bf16Sink sink) {
  constexpr int kFwdRows = kFwdWaves * 32;
  SEEAI_STAGE_RING(kStages);
  __shared__ int wave_lo[kFwdWaves];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane / 32, c = lane % 32;
  const int nq = (S + kFwdRows - 1) / kFwdRows;
  int bh, rank;
  UnitOf(nq, bh, rank);
  const int qblk = nq - 1 - rank;
  const int b = bh / H, h = bh % H;
  const int ld = H * kD;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * kD;
  const int qw = qblk * kFwdRows + wave * 32;  // this wave's first query
  const int i = qw + c;
  const int ic = min(i, S - 1);
  int jstart = 0;
  if (starts) {
    const int v0 = starts[static_cast<size_t>(b) * S + ic];
    jstart = v0 <= 0 ? 0 : min(v0, ic);
  }
  const int w_hi_start = WaveMaxI(jstart);
  if (lane == 0) wave_lo[wave] = WaveMinI(jstart);
  __syncthreads();
  int lo = wave_lo[0];
#pragma unroll
  for (int w = 1; w < kFwdWaves; ++w) lo = min(lo, wave_lo[w]);
  const int blk_lo = Uniform(lo) / kBlkRows;
  const int q_hi = min(qblk * kFwdRows + kFwdRows - 1, S - 1);
  const int nblk = q_hi / kBlkRows + 1 - blk_lo;

  bf16x8 qf[4];
  {
    const uint16_t* row = q + base + static_cast<size_t>(ic) * ld;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = OwnedFrag(row, s, lane);
  }
  const float scl = kLog2e * 0.125f;  // log2(e) / sqrt(64)

  // Loads: per stage 16 wave-loads (K then V, 2 halves x 4 row groups); wave
  // w takes u = kFwdWaves j + w.
  constexpr int kLoadsPerWave = 16 / kFwdWaves;
  static_assert(kLoadsPerWave * kFwdWaves == 16, "16 wave-loads per block");
  int voff[kLoadsPerWave];
#pragma unroll
  for (int j = 0; j < kLoadsPerWave; ++j)
    voff[j] = TileLoadOffset((kFwdWaves * j + wave) % 8, lane, ld);
  auto issue = [&](int jb, uint8_t* st) {
    const int j0 = (blk_lo + jb) * kBlkRows;
    const __amdgpu_buffer_rsrc_t rk = SliceRsrc(k + base, ld, S, j0);
    const __amdgpu_buffer_rsrc_t rv = SliceRsrc(v + base, ld, S, j0);
#pragma unroll
    for (int j = 0; j < kLoadsPerWave; ++j) {
      const int u = kFwdWaves * j + wave;
      if (u < 8)
        TileLoad(rk, st, u, voff[j]);
      else
        TileLoad(rv, st + kTile, u - 8, voff[j]);
    }
  };

  const FragOffsets fo = MakeFragOffsets(lane);
  v16f oacc[2] = {};  // [dt]
  float m_use = 0.0f, m_half = -INFINITY, l_half = 0.0f;
  float thr = -INFINITY;  // a half's tile maximum above this moves m_use: -inf until it sees a score

  const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};

  // A 32-key tile kt of a staged block: S^T = K Q^T (four MFMAs) ...
  auto scores = [&](const uint8_t* kt_tile, int kt) {
    v16f sc = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) sc = Mfma(RowFrag(kt_tile, fo, 32 * kt, s), qf[s], sc);
    return sc;
  };
  // ... the softmax weights (VALU) and O^T += V^T P^T (four MFMAs).
  auto weigh = [&](const v16f& sc, bool masked, const uint8_t* vt_tile, int kt, int jt) {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(sc[r], scl, -m_use);
    if (masked) {  // keep key jt + row in [jstart, i]
      const int hi_rel = i - jt - 4 * g, lo_rel = jstart - jt - 4 * g;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        x[r] = OrNegInf(x[r], Outside(hi_rel - RowConst(r), RowConst(r) - lo_rel));
    }
    float hmax = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) hmax = fmaxf(hmax, x[r]);  // relative to m_use
    const float m_prev = m_half;
    m_half = fmaxf(m_half, m_use + hmax);
    if (__any(hmax > thr)) {
      const float bmax = SwapMax(hmax);
      const bool first = SwapMax(m_prev) == -INFINITY;
      const bool need = first ? bmax != -INFINITY : bmax > kLazy;
      const float shift = need ? bmax : 0.0f;
      const float alpha = first ? 0.0f : Exp2(-shift);
      m_use += shift;
      l_half *= alpha;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) oacc[dt] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= shift;
      thr = m_half == -INFINITY ? -INFINITY : kLazy;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = Exp2(x[r]);
    bf16x8 pb[2];
    PackTile(p, pb);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        l_half = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pb[hh][2 * e], pb[hh][2 * e + 1]}, ones,
                                                 l_half, false);
    // O^T += V^T P^T over the tile's 32 keys (two 16-key steps).
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
        oacc[dt] = Mfma(ColFrag(vt_tile, fo, dt, 32 * kt + 16 * hh), pb[hh], oacc[dt]);
  };

  const int qmin = qw, qmax = qw + 31;
  auto step = [&](int jb, const uint8_t* cur) {
    const int j0 = (blk_lo + jb) * kBlkRows;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int jt = j0 + 32 * kt;
      if (jt > qmax) continue;  // keys wholly after this wave's queries
      weigh(scores(cur, kt), !(jt + 31 <= qmin && jt >= w_hi_start), cur + kTile, kt, jt);
    }
  };
  RunRing<kStages, kLoadsPerWave>(nblk, issue, step, stage);

  const float l = SwapSum(l_half);
  const float m_true = SwapMax(m_half);
  if (i >= S) return;
  const float inv = 1.0f / l;
  const size_t orow0 = base + static_cast<size_t>(i) * ld;
  float* orow = o + orow0;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float4 ov = make_float4(oacc[dt][4 * qq] * inv, oacc[dt][4 * qq + 1] * inv,
                                    oacc[dt][4 * qq + 2] * inv, oacc[dt][4 * qq + 3] * inv);
      const int col = dt * 32 + 8 * qq + 4 * g;
      if (sink.store_f32) *reinterpret_cast<float4*>(orow + col) = ov;
      if (sink.out) SinkStore4(sink, orow0 + col, ov);  // the next product's bf16 A'
    }
  if (g == 0) {
    float* sr = stats + (static_cast<size_t>(bh) * S + i) * 4;
    sr[0] = m_true * kLn2;
    sr[1] = inv * Exp2(m_true - m_use);
    sr[2] = 0.0f;
    sr[3] = static_cast<float>(jstart);
  }
}

// Row offset of the base-2 exponent: p = 2^(s c - mm) with c = log2(e)/8
// and mm = m log2(e) + log2(l), from the stats row (m, 1/l).
__device__ __forceinline__ float RowOffset(float m, float inv) { return m * kLog2e - log2f(inv); }

// Stats start column: the document start stored as a float (instruction.h:
// 246-250), clamped to the row.
__device__ __forceinline__ int StatsStart(float stored, int i) {
  if (!(stored > 0.0f)) return 0;
  const float cap = static_cast<float>(i);
  return stored >= cap ? i : static_cast<int>(stored);
}

// ---------------------------------------------------------------------------
// dQ and the stats row's delta = sum_j p dP, in one walk over K / V: with
// dS = p (dP - delta) linear in delta,
//   dQ^T = K^T (p dP)^T - delta K^T p^T,
// and delta accumulates beside the two products (four per tile -- S^T,
// dP^T and the two accumulations -- one exponential per score).  Four waves
// of 32 queries; K and V blocks staged as in the forward, K^T read by
// transpose reads.  dQ is scaled by 1/sqrt(d) once, at the end.
// ---------------------------------------------------------------------------
constexpr int kBwdWaves = 4;
constexpr int kBwdRows = kBwdWaves * 32;

template <int kStages, int kMinBlocks>
__global__ void __launch_bounds__(kBwdWaves * kWave, kMinBlocks)
Attn16DQ(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
         const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
         float* __restrict__ stats, float* __restrict__ dq, int S, int H) {
  SEEAI_STAGE_RING(kStages);
  __shared__ int wave_lo[kBwdWaves];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane / 32;
  const int nq = (S + kBwdRows - 1) / kBwdRows;
  int bh, rank;
  UnitOf(nq, bh, rank);
  const int qblk = nq - 1 - rank;
  const int b = bh / H, h = bh % H;
  const int ld = H * kD;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * kD;
  const int qw = qblk * kBwdRows + wave * 32;
  const int i = qw + lane % 32;
  const int ic = min(i, S - 1);
  float* st = stats + (static_cast<size_t>(bh) * S + ic) * 4;
  const float4 st4 = *reinterpret_cast<const float4*>(st);
  const float mm = RowOffset(st4.x, st4.y);
  const int jstart = StatsStart(st4.w, ic);
  const int w_hi_start = WaveMaxI(jstart);
  if (lane == 0) wave_lo[wave] = WaveMinI(jstart);
  __syncthreads();
  int lo = wave_lo[0];
#pragma unroll
  for (int w = 1; w < kBwdWaves; ++w) lo = min(lo, wave_lo[w]);
  const int blk_lo = Uniform(lo) / kBlkRows;
  const int q_hi = min(qblk * kBwdRows + kBwdRows - 1, S - 1);
  const int nblk = q_hi / kBlkRows + 1 - blk_lo;
  const float scl = kLog2e * 0.125f;

  bf16x8 qf[4], df[4];
  {
    const uint16_t* qrow = q + base + static_cast<size_t>(ic) * ld;
    const uint16_t* drow = dout + base + static_cast<size_t>(ic) * ld;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = OwnedFrag(qrow, s, lane), df[s] = OwnedFrag(drow, s, lane);
  }
  int voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) voff[j] = TileLoadOffset((4 * j + wave) % 8, lane, ld);
  auto issue = [&](int jb, uint8_t* sb) {
    const int j0 = (blk_lo + jb) * kBlkRows;
    const __amdgpu_buffer_rsrc_t rk = SliceRsrc(k + base, ld, S, j0);
    const __amdgpu_buffer_rsrc_t rv = SliceRsrc(v + base, ld, S, j0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = 4 * j + wave;
      if (u < 8)
        TileLoad(rk, sb, u, voff[j]);
      else
        TileLoad(rv, sb + kTile, u - 8, voff[j]);
    }
  };
  const FragOffsets fo = MakeFragOffsets(lane);
  v16f acc[2] = {}, acc_p[2] = {};  // [dt]
  float delta = 0.0f;

  // A 32-key tile kt: S^T = K Q^T and dP^T = V dO^T (eight MFMAs) ...
  auto front = [&](const uint8_t* ktile, const uint8_t* vtile, int kt, v16f& sc, v16f& dp) {
    sc = v16f{};
    dp = v16f{};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sc = Mfma(RowFrag(ktile, fo, 32 * kt, s), qf[s], sc);
      dp = Mfma(RowFrag(vtile, fo, 32 * kt, s), df[s], dp);
    }
  };
  // ... the weights (VALU) and the two accumulations (eight MFMAs).
  auto back = [&](const v16f& sc, const v16f& dp, bool masked, const uint8_t* ktile, int kt,
                  int jt) {
    float w[16], p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = Exp2(__builtin_fmaf(sc[r], scl, -mm));
    if (masked) {  // keep key jt + row in [jstart, i]
      const int hi_rel = i - jt - 4 * g, lo_rel = jstart - jt - 4 * g;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        p[r] = OrZero(p[r], Outside(hi_rel - RowConst(r), RowConst(r) - lo_rel));
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      delta = __builtin_fmaf(dp[r], p[r], delta);
      w[r] = p[r] * dp[r];
    }
    bf16x8 wb[2], pb[2];
    PackTile(w, wb);
    PackTile(p, pb);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x8 kf = ColFrag(ktile, fo, dt, 32 * kt + 16 * hh);
        acc[dt] = Mfma(kf, wb[hh], acc[dt]);
        acc_p[dt] = Mfma(kf, pb[hh], acc_p[dt]);
      }
  };

  const int qmin = qw, qmax = qw + 31;
  auto step = [&](int jb, const uint8_t* cur) {
    const int j0 = (blk_lo + jb) * kBlkRows;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int jt = j0 + 32 * kt;
      if (jt > qmax) continue;
      v16f sc, dp;
      front(cur, cur + kTile, kt, sc, dp);
      back(sc, dp, !(jt + 31 <= qmin && jt >= w_hi_start), cur, kt, jt);
    }
  };
  RunRing<kStages, 4>(nblk, issue, step, stage);
  delta = SwapSum(delta);
  if (i >= S) return;
  const float isd = 0.125f;
  float* drow = dq + base + static_cast<size_t>(i) * ld;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const v16f r = acc[dt] - delta * acc_p[dt];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<float4*>(drow + dt * 32 + 8 * qq + 4 * g) =
          make_float4(r[4 * qq] * isd, r[4 * qq + 1] * isd, r[4 * qq + 2] * isd,
                      r[4 * qq + 3] * isd);
  }
  if (g == 0) st[2] = delta;
}

// ---------------------------------------------------------------------------
// dK and dV: four waves of 32 keys walking the query blocks from the
// diagonal.  S = Q K^T and dP = dO V^T are formed query-major (Q and dO
// tiles as the row operand, K and V held in registers), so the score
// accumulator's layout is the k operand of dV^T = dO^T P and
// dK^T = Q^T dS, whose dO^T and Q^T come by transpose reads.  Per query
// row the exponent offset -mm and -delta come from a row-terms array
// staged beside the tiles; four products per tile, one exponential per
// score.  dK is scaled by 1/sqrt(d) once, at the end.
// ---------------------------------------------------------------------------
template <int kStages, int kMinBlocks>
__global__ void __launch_bounds__(kBwdWaves * kWave, kMinBlocks)
Attn16DKDV(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
           const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
           const float* __restrict__ stats, float* __restrict__ out_k,
           float* __restrict__ out_v, int S, int H, Bf16Sink sink_v) {
  SEEAI_STAGE_RING(kStages);
  // Per streamed query row: -mm, -delta and the document start.  Rows are
  // contiguous, so a lane's 16 rows of a tile (8q + 4g + e) are four 16-byte
  // reads in accumulator order.
  __shared__ __attribute__((aligned(16))) float Smm[2][kBlkRows];
  __shared__ __attribute__((aligned(16))) float Sdl[2][kBlkRows];
  __shared__ int Sst[2][kBlkRows];
  __shared__ int Smax[2];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane / 32;
  const int nk = (S + kBwdRows - 1) / kBwdRows;
  int bh, kblk;
  UnitOf(nk, bh, kblk);  // rank 0 = the first keys, the longest columns
  const int b = bh / H, h = bh % H;
  const int ld = H * kD;
  const size_t base = static_cast<size_t>(b) * S * ld + static_cast<size_t>(h) * kD;
  const int jw = kblk * kBwdRows + wave * 32;
  const int j = jw + lane % 32;
  const int jc = min(j, S - 1);
  const float scl = kLog2e * 0.125f;
  const float4* st_bh = reinterpret_cast<const float4*>(stats) + static_cast<size_t>(bh) * S;

  bf16x8 kf[4], vf[4];
  {
    const uint16_t* krow = k + base + static_cast<size_t>(jc) * ld;
    const uint16_t* vrow = v + base + static_cast<size_t>(jc) * ld;
#pragma unroll
    for (int s = 0; s < 4; ++s) kf[s] = OwnedFrag(krow, s, lane), vf[s] = OwnedFrag(vrow, s, lane);
  }
  const int blk_first = (kblk * kBwdRows) / kBlkRows;
  const int nblk = (S + kBlkRows - 1) / kBlkRows - blk_first;
  int voff[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) voff[jj] = TileLoadOffset((4 * jj + wave) % 8, lane, ld);
  auto issue = [&](int ib, uint8_t* sb) {
    const int r0 = (blk_first + ib) * kBlkRows;
    const __amdgpu_buffer_rsrc_t rq = SliceRsrc(q + base, ld, S, r0);
    const __amdgpu_buffer_rsrc_t rd = SliceRsrc(dout + base, ld, S, r0);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int u = 4 * jj + wave;
      if (u < 8)
        TileLoad(rq, sb, u, voff[jj]);
      else
        TileLoad(rd, sb + kTile, u - 8, voff[jj]);
    }
  };
  // The row terms of block ib, by wave 0 (64 queries): fetched from HBM one
  // block ahead of their store into LDS, so the load's latency hides behind
  // a block's products.
  float4 pend = {};
  auto fetch = [&](int ib) {
    const int iq = (blk_first + ib) * kBlkRows + lane;
    if (iq < S) pend = st_bh[iq];
  };
  auto put = [&](int ib, int buf) {
    const int iq = (blk_first + ib) * kBlkRows + lane;
    int start = 0;
    if (iq < S) {
      Smm[buf][lane] = -RowOffset(pend.x, pend.y);
      Sdl[buf][lane] = -pend.z;
      start = StatsStart(pend.w, iq);
    } else {
      Smm[buf][lane] = -INFINITY;  // weight 0 past the sequence end
      Sdl[buf][lane] = 0.0f;
    }
    Sst[buf][lane] = start;
    const int mx = WaveMaxI(start);
    if (lane == 0) Smax[buf] = mx;
  };
  // This lane's 16 per-row values of tile qt (rows 8q + 4g + e).
  // A lane's 16 values of one row-term array for tile qt, in accumulator
  // order.
  auto rows16 = [&](const float* terms, int qt) {
    v16f r;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const float4 a = *reinterpret_cast<const float4*>(terms + qt * 32 + 8 * q4 + 4 * g);
      r[4 * q4] = a.x, r[4 * q4 + 1] = a.y, r[4 * q4 + 2] = a.z, r[4 * q4 + 3] = a.w;
    }
    return r;
  };
  const FragOffsets fo = MakeFragOffsets(lane);
  v16f acc_k[2] = {}, acc_v[2] = {};  // [dt]

  // A 32-query tile qt: S = Q K^T and dP = dO V^T (eight MFMAs) ...
  // dP starts at -delta, so the product arrives as dP - delta.
  auto front = [&](const uint8_t* qtile, const uint8_t* dtile, int buf, int qt, v16f& sc,
                   v16f& dp) {
    sc = v16f{};
    dp = rows16(Sdl[buf], qt);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sc = Mfma(RowFrag(qtile, fo, 32 * qt, s), kf[s], sc);
      dp = Mfma(RowFrag(dtile, fo, 32 * qt, s), vf[s], dp);
    }
  };
  // ... the weights (VALU) and dK^T += Q^T dS, dV^T += dO^T P (eight MFMAs).
  auto back = [&](const v16f& sc, const v16f& dp, bool masked, const uint8_t* qtile,
                  const uint8_t* dtile, int buf, int qt, int r0) {
    const v16f mmv = rows16(Smm[buf], qt);
    float w[16], p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = Exp2(__builtin_fmaf(sc[r], scl, mmv[r]));
    if (masked) {  // keep query row >= j and its start <= j
      const int lo_rel = r0 + 32 * qt + 4 * g - j;  // query row minus this lane's key
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int il = qt * 32 + RowConst(r) + 4 * g;
        p[r] = OrZero(p[r], Outside(lo_rel + RowConst(r), j - Sst[buf][il]));
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = p[r] * dp[r];
    bf16x8 wb[2], pb[2];
    PackTile(w, wb);
    PackTile(p, pb);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        acc_k[dt] = Mfma(ColFrag(qtile, fo, dt, 32 * qt + 16 * hh), wb[hh], acc_k[dt]);
        acc_v[dt] = Mfma(ColFrag(dtile, fo, dt, 32 * qt + 16 * hh), pb[hh], acc_v[dt]);
      }
  };

  // Row terms run one block ahead of the tiles (two LDS buffers, by
  // parity): block ib's are stored during block ib - 1, from a load issued
  // during block ib - 2.
  if (wave == 0) {
    fetch(0);
    put(0, 0);
    if (1 < nblk) fetch(1);
  }
  auto step = [&](int ib, const uint8_t* cur) {
    const int buf = ib & 1;
    if (wave == 0 && ib + 1 < nblk) {
      put(ib + 1, buf ^ 1);
      if (ib + 2 < nblk) fetch(ib + 2);
    }
    const int r0 = (blk_first + ib) * kBlkRows;
    const int smax = Uniform(Smax[buf]);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int rt = r0 + 32 * qt;
      if (rt + 31 < jw) continue;  // queries wholly before this wave's keys
      v16f sc, dp;
      front(cur, cur + kTile, buf, qt, sc, dp);
      back(sc, dp, !(rt >= jw + 31 && rt + 32 <= S && smax <= jw), cur, cur + kTile, buf, qt, r0);
    }
  };
  RunRing<kStages, 4>(nblk, issue, step, stage);
  if (j >= S) return;
  const float isd = 0.125f;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const size_t at = base + static_cast<size_t>(j) * ld + dt * 32 + 8 * qq + 4 * g;
      if (out_k)
        *reinterpret_cast<float4*>(out_k + at) =
            make_float4(acc_k[dt][4 * qq] * isd, acc_k[dt][4 * qq + 1] * isd,
                        acc_k[dt][4 * qq + 2] * isd, acc_k[dt][4 * qq + 3] * isd);
      if (out_v) {
        const float4 v4 = make_float4(acc_v[dt][4 * qq], acc_v[dt][4 * qq + 1],
                                      acc_v[dt][4 * qq + 2], acc_v[dt][4 * qq + 3]);
        *reinterpret_cast<float4*>(out_v + at) = v4;
        if (sink_v.out) SinkStore4(sink_v, at, v4);  // a later product's copy of dV
      }
    }
}

}  // namespace

bool Attn16Fits(size_t B, size_t S, size_t H, size_t d) {
  return d == kD && S > 0 && (S - 1) * H * kD * 2 + kD * 2 < (size_t{1} << 31) &&
         (S + 127) / 128 * B * H < (size_t{1} << 31);
}

hipError_t LaunchAttn16Fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* o,
                           float* stats, size_t B, size_t S, size_t H, const int32_t* starts,
                           hipStream_t s, const Bf16Sink& sink) {
  if (B * H * S == 0) return hipSuccess;
  // Four waves, two stages, four workgroups per CU (measured against 3-4
  // stages and 8-wave workgroups at B16 H16 S2048).
  const dim3 grid(static_cast<unsigned>((S + 127) / 128 * B * H));
  hipLaunchKernelGGL((Attn16Fwd<4, 2, 4>), grid, dim3(256), 0, s, q, k, v, o, stats,
                     static_cast<int>(S), static_cast<int>(H), starts, sink);
  return hipGetLastError();
}

hipError_t LaunchAttn16DQ(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const uint16_t* dout, float* stats, float* dq, size_t B, size_t S,
                          size_t H, hipStream_t s) {
  if (B * H * S == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((S + kBwdRows - 1) / kBwdRows * B * H));
  // Three stages, three workgroups per CU (160 VGPRs, 48 KiB of LDS each).
  hipLaunchKernelGGL((Attn16DQ<3, 3>), grid, dim3(kBwdWaves * kWave), 0, s, q, k, v, dout, stats,
                     dq, static_cast<int>(S), static_cast<int>(H));
  return hipGetLastError();
}

hipError_t LaunchAttn16DKDV(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* dout, const float* stats, float* dk, float* dv,
                            size_t B, size_t S, size_t H, hipStream_t s, const Bf16Sink& sink_v) {
  if (B * H * S == 0) return hipSuccess;
  if (!dk && !dv) return hipErrorInvalidValue;
  if (sink_v.out && (!dv || !sink_v.store_f32)) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((S + kBwdRows - 1) / kBwdRows * B * H));
  // Two stages, two workgroups per CU (about 200 VGPRs).
  hipLaunchKernelGGL((Attn16DKDV<2, 2>), grid, dim3(kBwdWaves * kWave), 0, s, q, k, v, dout,
                     stats, dk, dv, static_cast<int>(S), static_cast<int>(H), sink_v);
  return hipGetLastError();
}

}  // namespace seeai
