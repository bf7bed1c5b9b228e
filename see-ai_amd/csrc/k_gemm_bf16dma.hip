// k_gemm_bf16dma.hip -- the relaxed family's frozen-weight products
// (kFlagRelaxed on kGemmNN / kGemmNT / kGemmNNQ8 / kGemmNTQ8,
// source/plan/instruction.h:356-384) with both operands in bf16 in HBM,
// staged into LDS by direct-to-LDS buffer loads.
//
// The relaxed family rounds the activations to bf16 once at the GEMM input
// and takes the frozen weight in reduced precision:
//   * ConvertRowsKernel writes A' [M, Kp] bf16 = RNE(alpha * (A * kscale))
//     -- the per-tensor scale (NN) or alpha and the q8 k-scale (NT) multiply
//     A before it rounds, as gemm.cc:626-674 places them -- zero past K;
//   * ShadowKernel writes the weight once as W' [N, Kp] bf16 (K contiguous):
//     f32 rounded, int8 levels and bf16 exactly; a weight in rodata or the
//     source image cannot change until the next bind, so the launcher keeps
//     the shadow and reuses it;
//   * GemmBf16DmaKernel: a BM x BN tile per workgroup of WGM x WGN waves, each
//     a (BM/WGM) x (BN/WGN) block of v_mfma_f32_32x32x16_bf16 accumulators.
//     K moves 64 bytes (32 bf16) per stage through kStages LDS buffers filled
//     by buffer_load ... lds; kStages - 1 stages are in flight while one is
//     multiplied, one barrier per stage.  LDS rows are 64 bytes, four 16-byte
//     chunks; chunk c of row r sits at physical chunk (c + r/4) mod 4, which
//     keeps the fragment reads (lane l: row l % 32, chunk 2ks + l / 32) free
//     of bank conflicts.  The W fragment is the MFMA's first operand, so a
//     lane's accumulators hold four consecutive columns of one row; the
//     epilogue (NN column scale, alpha, addend, accumulate, bias, activation
//     -- the exact family's order) runs on them in registers and C leaves in
//     16-byte stores.  With the low-rank term, or rows whose length is not a
//     multiple of four, the rows pass through LDS instead; the low-rank
//     term's t rows for the whole tile are staged in LDS once, and at rank 8
//     or 16 behind a plain epilogue (column scale and alpha only) the rank
//     is a compile-time constant, so each row pass is straight-line code of
//     four independent chains.
// Rows past M or N read as zeros through the buffer range check; Kp is K
// rounded up to 32.
#include <algorithm>
#include <numeric>
#include <type_traits>
#include <cstdint>

#include "common.h"

namespace seeai {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* LdsPtr;

constexpr int kRowBytes = 64;             // K bytes of one row per stage (32 bf16)
constexpr int kChunks = kRowBytes / 16;   // 16-byte chunks per staged row
constexpr int kRsrcWord3 = 0x00020000;    // raw buffer, out-of-range reads give 0

__device__ __forceinline__ int Phys(int row, int c) { return (c + row / 4) & 3; }

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding).
template <int n>
__device__ __forceinline__ void WaitVm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

// Tile -> workgroup order: the 8 XCDs each take a contiguous run of tiles
// (workgroup b runs on XCD b % 8) walked column-major in bands of kGroupM
// row tiles, so concurrent tiles of one XCD share A row panels and W column
// panels in its L2.
constexpr int kGroupM = 4;
__device__ __forceinline__ void TileOf(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  int t = b;
  if (ntiles % 8 == 0) t = (b % 8) * (ntiles / 8) + b / 8;
  const int per_group = kGroupM * tiles_n;
  const int g = t / per_group;
  const int first_m = g * kGroupM;
  const int rows = min(tiles_m - first_m, kGroupM);
  const int off = t % per_group;
  tm = first_m + off % rows;
  tn = off / rows;
}

__device__ __forceinline__ float ActF(int act, float v) { return act ? ActExpr(act, v) : v; }

__device__ __forceinline__ float MulRn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float AddRn(float a, float b) { return __fadd_rn(a, b); }

// The low-rank term of one output: the rank-r product's exact chain over
// the row's t values and the column's rank-operand values (GemmArgs).
// NN: `t` holds the row's t values already multiplied by alpha (each
// (alpha t) rounded once, as the reference folds alpha into A), shared by
// the row's columns; NT: the raw t, alpha applied to the finished dot.
template <int kLayout>
__device__ __forceinline__ float LowRankDot(const float (&t)[kLowRankMaxK],
                                            const float (&b)[kLowRankMaxK], int r, float alpha) {
  if constexpr (kLayout == 0) {  // quads of (alpha t) b from k = 0 (r % 4 == 0: no tail)
    (void)alpha;
    float c = 0.0f;
#pragma unroll
    for (int k = 0; k < kLowRankMaxK; k += 4) {
      if (k < r)
        c = AddRn(c, AddRn(AddRn(AddRn(MulRn(t[k], b[k]), MulRn(t[k + 1], b[k + 1])),
                                 MulRn(t[k + 2], b[k + 2])), MulRn(t[k + 3], b[k + 3])));
    }
    return c;
  } else {  // eight lanes by k mod 8, added in lane order, then alpha
    // Lane l holds 0 + t[l] b[l] (+ t[l+8] b[l+8]); each lane is formed
    // just before it joins the running sum, so few values are live at once.
    float c = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      float lane = 0.0f;
      if (l < r) lane = AddRn(lane, MulRn(t[l], b[l]));
      if (l + 8 < r) lane = AddRn(lane, MulRn(t[l + 8], b[l + 8]));
      c = l == 0 ? lane : AddRn(c, lane);
    }
    return MulRn(alpha, c);
  }
}

template <int BM, int BN, int WGM, int WGN, int kStages, int kLR>
__global__ void __launch_bounds__(WGM * WGN * kWave)
GemmBf16DmaKernel(const __bf16* __restrict__ A, const __bf16* __restrict__ W, int Kp, GemmArgs g) {
  // kLR: 0 none, 1 NN low-rank epilogue, 2 NT low-rank epilogue.
  constexpr int kWaves = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kRowsPerLoad = kWave / kChunks;           // 16 rows per wave-load
  constexpr int kLoadsA = BM / kRowsPerLoad / kWaves;     // wave-loads per stage, per wave
  constexpr int kLoadsB = BN / kRowsPerLoad / kWaves;
  static_assert(kLoadsA * kRowsPerLoad * kWaves == BM && kLoadsB * kRowsPerLoad * kWaves == BN,
                "loads cover the tile");
  static_assert(kLoadsA <= 4 && kLoadsB <= 4, "voff capacity");
  constexpr int kStageA = BM * kRowBytes;
  constexpr int kStage = (BM + BN) * kRowBytes;
  constexpr int kPerStage = kLoadsA + kLoadsB;            // vmcnt units per stage
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStage];

  const int M = static_cast<int>(g.M), N = static_cast<int>(g.N);
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  int tm, tn;
  TileOf(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kb = Kp * 2;  // row bytes

  // Ranges cover this tile's rows only: offsets stay below BM * kb.
  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(A) + static_cast<size_t>(m0) * Kp, 0, Uniform(min(M - m0, BM) * kb),
      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(W) + static_cast<size_t>(n0) * Kp, 0, Uniform(min(N - n0, BN) * kb),
      kRsrcWord3);
  // This lane's slot in a wave-load: row rbase + lane / 4, physical chunk
  // lane % 4, which holds logical chunk (p - r/4) mod 4.
  int voff_a[4], voff_b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ra = (j * kWaves + wave) * kRowsPerLoad + lane / kChunks;
    voff_a[j] = ra * kb + ((lane % kChunks - ra / 4) & 3) * 16;
    voff_b[j] = voff_a[j];
  }
  auto issue = [&](int st, int buf) {
    uint8_t* sA = smem + buf * kStage;
    uint8_t* sB = sA + kStageA;
    const int k0 = st * kRowBytes;
#pragma unroll
    for (int j = 0; j < kLoadsA; ++j) {
      const int rbase = Uniform((j * kWaves + wave) * kRowsPerLoad);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, (LdsPtr)(sA + rbase * kRowBytes), 16,
                                               voff_a[j], k0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kLoadsB; ++j) {
      const int rbase = Uniform((j * kWaves + wave) * kRowsPerLoad);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, (LdsPtr)(sB + rbase * kRowBytes), 16,
                                               voff_b[j], k0, 0, 0);
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{};

  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
  const int lr = lane % 32, h = lane / 32;
  const int frag0 = lr * kRowBytes + Phys(lr, h) * 16;
  const int frag1 = lr * kRowBytes + Phys(lr, 2 + h) * 16;

  const int nsteps = Kp / 32;
  bf16x8 fa[2][TM], fb[2][TN];
  auto read = [&](int buf, int fo, int slot) {
    const uint8_t* sA = smem + buf * kStage;
    const uint8_t* sB = sA + kStageA;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[slot][i] = *reinterpret_cast<const bf16x8*>(sA + (wm + i * 32) * kRowBytes + fo);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[slot][j] = *reinterpret_cast<const bf16x8*>(sB + (wn + j * 32) * kRowBytes + fo);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[slot][j], fa[slot][i], acc[i][j],
                                                            0, 0, 0);
  };
  // The next k-step's TM + TN LDS reads spread one per MFMA; after the
  // barrier the stage's loads take the last MFMA slots.
  auto interleave = [&]() {
#pragma unroll
    for (int s = 0; s < TM + TN; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int s = TM + TN; s < TM * TN; ++s) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };
  auto interleave_loads = [&]() {
#pragma unroll
    for (int s = 0; s < TM * TN; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (s < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (s >= TM * TN - kPerStage) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  };
  static_assert(TM * TN >= TM + TN && TM * TN >= kPerStage, "MFMA slots for the reads and loads");

  // Every iteration loads one stage; past the last the loads repeat it (in
  // bounds, into a buffer no later stage uses), so the stages in flight at
  // each barrier are always kStages - 3.
  const int last = nsteps - 1;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(min(s, last), s);
  WaitVm<(kStages - 2) * kPerStage>();
  __builtin_amdgcn_s_barrier();
  read(0, frag0, 0);
  for (int it = 0; it < last; ++it) {
    const int buf = it % kStages;
    read(buf, frag1, 1);
    mfmas(0);
    interleave();
    WaitVm<(kStages - 3) * kPerStage>();
    __builtin_amdgcn_s_barrier();
    issue(min(it + kStages - 1, last), (it + kStages - 1) % kStages);
    read((it + 1) % kStages, frag0, 0);
    mfmas(1);
    interleave_loads();
  }
  read(last % kStages, frag1, 1);
  mfmas(0);
  interleave();
  mfmas(1);
  WaitVm<0>();  // the repeated loads past the last stage have landed

  // Accumulator element 4q + e of block (i, j) is C[m][n] at
  // m = m0 + wm + 32 i + lane % 32, n = n0 + wn + 32 j + 8 q + 4 (lane / 32) + e.
  if constexpr (kLR == 0) {
    const bool vec4 = (g.N % 4) == 0 &&
                      ((reinterpret_cast<uintptr_t>(g.C) | reinterpret_cast<uintptr_t>(g.addend) |
                        reinterpret_cast<uintptr_t>(g.b_col_scale) |
                        reinterpret_cast<uintptr_t>(g.bias)) & 15) == 0;
    // Row m's maximum over this wave's 64 columns, from the lane's values
    // `pm` of its half (columns 4 h + 8 q + 32 j) and the other half's, into
    // the partials (WN = 64: the wave's columns are one group).
    auto row_max_out = [&](int m, float pm) {
      if constexpr (WN == 64) {
        pm = fmaxf(pm, __shfl_xor(pm, 32));
        // (a group wholly past the last column has no partial)
        if (h == 0 && m < M && n0 + wn < N)
          g.row_max_part[static_cast<size_t>(m) * ((N + 63) / 64) + (n0 + wn) / 64] = pm;
      }
    };
    // The plain product (the frozen projections): nothing but the stores.
    if (vec4 && !g.b_col_scale && g.alpha_dot == 1.0f && !g.addend && !g.accumulate && !g.bias &&
        !g.act) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm + i * 32 + lr;
        float pm = __builtin_nanf("");  // fmaxf's identity
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn + j * 32 + 8 * q + 4 * h;
            if (m < M && n < N) {
              *reinterpret_cast<float4*>(g.C + static_cast<size_t>(m) * N + n) = make_float4(
                  acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
              if (g.lr_sink) {  // C's bf16 copy for the attention that reads it next
                const float cv[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                     acc[i][j][4 * q + 3]};
                StoreBf16x4(g.lr_sink + static_cast<size_t>(m) * N + n, cv);
              }
              if (g.row_max_part)
                pm = fmaxf(pm, fmaxf(fmaxf(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                     fmaxf(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])));
            }
          }
        if (g.row_max_part) row_max_out(m, pm);
      }
      return;
    }
    if (vec4) {  // the general epilogue on one column quad at a time
      const float alpha = g.alpha_dot;
      const float* __restrict__ cs = g.b_col_scale;
      const float* __restrict__ add = g.addend;
      const float* __restrict__ bias = g.bias;
      float* __restrict__ C = g.C;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm + i * 32 + lr;
        float pm = __builtin_nanf("");
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn + j * 32 + 8 * q + 4 * h;
            if (m < M && n < N) {
              const size_t o = static_cast<size_t>(m) * N + n;
              float x0 = acc[i][j][4 * q], x1 = acc[i][j][4 * q + 1], x2 = acc[i][j][4 * q + 2],
                    x3 = acc[i][j][4 * q + 3];
              if (cs) {
                const float4 s4 = *reinterpret_cast<const float4*>(cs + n);
                x0 = x0 * s4.x, x1 = x1 * s4.y, x2 = x2 * s4.z, x3 = x3 * s4.w;
              }
              if (alpha != 1.0f) x0 = alpha * x0, x1 = alpha * x1, x2 = alpha * x2, x3 = alpha * x3;
              if (add) {
                const float4 a4 = *reinterpret_cast<const float4*>(add + o);
                x0 = a4.x + x0, x1 = a4.y + x1, x2 = a4.z + x2, x3 = a4.w + x3;
              }
              if (g.accumulate) {
                const float4 c4v = *reinterpret_cast<const float4*>(C + o);
                x0 = c4v.x + x0, x1 = c4v.y + x1, x2 = c4v.z + x2, x3 = c4v.w + x3;
              }
              if (bias) {
                const float4 b4 = *reinterpret_cast<const float4*>(bias + n);
                x0 = x0 + b4.x, x1 = x1 + b4.y, x2 = x2 + b4.z, x3 = x3 + b4.w;
              }
              x0 = ActF(g.act, x0), x1 = ActF(g.act, x1), x2 = ActF(g.act, x2), x3 = ActF(g.act, x3);
              *reinterpret_cast<float4*>(C + o) = make_float4(x0, x1, x2, x3);
              if (g.lr_sink) {
                const float cv[4] = {x0, x1, x2, x3};
                StoreBf16x4(g.lr_sink + o, cv);
              }
              if (g.row_max_part) pm = fmaxf(pm, fmaxf(fmaxf(x0, x1), fmaxf(x2, x3)));
            }
          }
        if (g.row_max_part) row_max_out(m, pm);
      }
      return;
    }
  }
  __syncthreads();  // every wave is done with the stage buffers: reuse them for staging

  // The staged epilogue: this wave's 32 x WN slice of LDS, 32 rows at a
  // time, so a lane keeps one column quad (and its rank-operand values).
  constexpr int SLD = WN + 4;
  static_assert(kWaves * 32 * SLD * 4 <= kStages * kStage, "staging fits in LDS");
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * SLD;
  const bool vec = (N % 4) == 0;
  const float alpha = g.alpha_dot;
  const float* __restrict__ cs = g.b_col_scale;
  const float* __restrict__ add = g.addend;
  const float* __restrict__ bias = g.bias;
  float* __restrict__ C = g.C;
  constexpr int kVecRow = WN / 4;
  // A lane keeps one column quad through the epilogue: kRowsPerPass rows of
  // kVecRow quads per pass (lanes past them idle where kVecRow does not
  // divide the wave).
  constexpr int kRowsPerPass = kWave / kVecRow;
  static_assert(kRowsPerPass >= 1 && 32 % kRowsPerPass == 0, "epilogue passes cover 32 rows");
  const int c4 = lane % kVecRow, row0 = lane / kVecRow;
  const bool epi_lane = lane < kRowsPerPass * kVecRow;
  // Low-rank epilogue: this lane's four columns of the rank operand, every k,
  // in registers for the whole epilogue (its column quad never changes).
  float lb[4][kLowRankMaxK];
  const int lr_r = kLR ? g.lr_k : 0;
  // The tile's t rows [BM][kLowRankMaxK] in LDS past the staging slices
  // (NN: already alpha t, each product rounded once), zero past r and M.
  constexpr int kTOff = kWaves * 32 * SLD;
  static_assert((kTOff + BM * kLowRankMaxK) * 4 <= kStages * kStage, "t block fits in LDS");
  float* tl = reinterpret_cast<float*>(smem) + kTOff;
  if constexpr (kLR != 0) {
    for (int e = tid; e < BM * (kLowRankMaxK / 4); e += kWaves * kWave) {
      const int rr = e / (kLowRankMaxK / 4), k = (e % (kLowRankMaxK / 4)) * 4;
      float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k < lr_r && m0 + rr < M)
        q = *reinterpret_cast<const float4*>(g.lr_t + static_cast<size_t>(m0 + rr) * lr_r + k);
      if (kLR == 1 && g.lr_alpha != 1.0f)
        q = make_float4(MulRn(g.lr_alpha, q.x), MulRn(g.lr_alpha, q.y), MulRn(g.lr_alpha, q.z),
                        MulRn(g.lr_alpha, q.w));
      *reinterpret_cast<float4*>(tl + rr * kLowRankMaxK + k) = q;
    }
    const int nl = n0 + wn + c4 * 4;
    const bool b16 = (reinterpret_cast<uintptr_t>(g.lr_b) & 15) == 0;
#pragma unroll
    for (int k = 0; k < kLowRankMaxK; ++k) lb[0][k] = lb[1][k] = lb[2][k] = lb[3][k] = 0.0f;
    if constexpr (kLR == 1) {
#pragma unroll
      for (int k = 0; k < kLowRankMaxK; ++k) {
        float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < lr_r && nl < N)
          b = *reinterpret_cast<const float4*>(g.lr_b + static_cast<size_t>(k) * N + nl);
        lb[0][k] = b.x, lb[1][k] = b.y, lb[2][k] = b.z, lb[3][k] = b.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int k = 0; k < kLowRankMaxK; k += 4) {
          if (k < lr_r && nl < N) {
            const float* src = g.lr_b + static_cast<size_t>(nl + e) * lr_r + k;
            float4 b;
            if (b16) b = *reinterpret_cast<const float4*>(src);
            else b = make_float4(src[0], src[1], src[2], src[3]);
            lb[e][k] = b.x, lb[e][k + 1] = b.y, lb[e][k + 2] = b.z, lb[e][k + 3] = b.w;
          }
        }
    }
    __syncthreads();
  }
  if constexpr (kLR != 0) {
    // Rank 8 or 16 with nothing but the column scale and alpha before the
    // low-rank term (on NT sites also an addend, which adds after alpha as
    // in the general pass -- loaded ahead on 128 x 128 tiles, at its use on
    // 256 x 256, which has no registers to spare for a ring): the rank is a
    // constant, so each pass is one block of four independent chains; a
    // residual behind the site (NN or NT) adds last.
    constexpr bool kAddFast = kLR == 2 && BM * BN <= 128 * 128;
    const bool plain = (!add || kLR == 2) && !g.accumulate && !bias && !g.act;
    auto fast = [&](auto rq_tag) {
      constexpr int RQ = decltype(rq_tag)::value;
      float csq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) csq[e] = 1.0f;
      {
        const int n = n0 + wn + c4 * 4;
        if (cs && n < N) {
          const float4 c4v = *reinterpret_cast<const float4*>(cs + n);
          csq[0] = c4v.x, csq[1] = c4v.y, csq[2] = c4v.z, csq[3] = c4v.w;
        }
      }
      // The residual, kResAhead quads in flight ahead of their use in the
      // lane's sequence of (pass, row) steps (each element read before this
      // lane writes it, also where the output is the residual itself).
      constexpr int kSteps = 32 / kRowsPerPass, kResAhead = kLR == 1 ? 4 : 2;
      float4 rr[kResAhead];
      auto res_load = [&](const float* src, int s) {
        const int m = m0 + wm + (s / kSteps) * 32 + row0 + (s % kSteps) * kRowsPerPass;
        const int n = n0 + wn + c4 * 4;
        return epi_lane && m < M && n < N && s < TM * kSteps
                   ? *reinterpret_cast<const float4*>(src + static_cast<size_t>(m) * N + n)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
      };
      if (g.lr_res) {
#pragma unroll
        for (int s = 0; s < kResAhead; ++s) rr[s] = res_load(g.lr_res, s);
      }
      // The NT site's addend, in flight the same way.
      float4 ra[kAddFast ? kResAhead : 1];
      if constexpr (kAddFast) {
        if (add) {
#pragma unroll
          for (int s = 0; s < kResAhead; ++s) ra[s] = res_load(add, s);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int mb = m0 + wm + i * 32;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            *reinterpret_cast<float4*>(stage + lr * SLD + j * 32 + 8 * q + 4 * h) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                            acc[i][j][4 * q + 3]);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int tt = 0; tt < 32 / kRowsPerPass; ++tt) {
          const int row = row0 + tt * kRowsPerPass;
          const int m = mb + row, n = n0 + wn + c4 * 4;
          if (!epi_lane || m >= M || n >= N) continue;
          const float4 s4 = *reinterpret_cast<const float4*>(stage + row * SLD + c4 * 4);
          float v[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = alpha * (v[e] * csq[e]);  // x 1.0f is exact
          const size_t o = static_cast<size_t>(m) * N + n;
          if constexpr (kLR == 2) {
            if (add) {
              float4 a4;
              if constexpr (kAddFast) {
                const int s = i * kSteps + tt;
                a4 = ra[s % kResAhead];
                if (s + kResAhead < TM * kSteps) ra[s % kResAhead] = res_load(add, s + kResAhead);
              } else {
                a4 = *reinterpret_cast<const float4*>(add + o);
              }
              v[0] = a4.x + v[0], v[1] = a4.y + v[1], v[2] = a4.z + v[2], v[3] = a4.w + v[3];
            }
          }
          if (g.lr_store_c) *reinterpret_cast<float4*>(C + o) = make_float4(v[0], v[1], v[2], v[3]);
          float t[kLowRankMaxK];
          const float* trow = tl + (m - m0) * kLowRankMaxK;
#pragma unroll
          for (int k = 0; k < kLowRankMaxK; k += 4) {
            float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < 4 * RQ) q = *reinterpret_cast<const float4*>(trow + k);
            t[k] = q.x, t[k + 1] = q.y, t[k + 2] = q.z, t[k + 3] = q.w;
          }
          float o4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o4[e] = AddRn(v[e], LowRankDot<kLR - 1>(t, lb[e], 4 * RQ, g.lr_alpha));
          if (g.lr_res) {
            const int s = i * kSteps + tt;
            const float4 r4 = rr[s % kResAhead];
            if (s + kResAhead < TM * kSteps) rr[s % kResAhead] = res_load(g.lr_res, s + kResAhead);
            o4[0] = AddRn(r4.x, o4[0]), o4[1] = AddRn(r4.y, o4[1]);
            o4[2] = AddRn(r4.z, o4[2]), o4[3] = AddRn(r4.w, o4[3]);
          }
          *reinterpret_cast<float4*>(g.lr_out + o) = make_float4(o4[0], o4[1], o4[2], o4[3]);
          if (g.lr_sink) StoreBf16x4(g.lr_sink + o, o4);
        }
        __builtin_amdgcn_wave_barrier();
      }
    };
    if (plain && lr_r == 16) return fast(std::integral_constant<int, 4>{});
    if (plain && lr_r == 8) return fast(std::integral_constant<int, 2>{});
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int mb = m0 + wm + i * 32;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < TN; ++j)  // four consecutive columns: one 16-byte write
        *reinterpret_cast<float4*>(stage + lr * SLD + j * 32 + 8 * q + 4 * h) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < 32 / kRowsPerPass; ++t) {
      const int row = row0 + t * kRowsPerPass;
      const int m = mb + row, n = n0 + wn + c4 * 4;
      if (!epi_lane || m >= M || n >= N) continue;
      float v[4];
      const float4 s4 = *reinterpret_cast<const float4*>(stage + row * SLD + c4 * 4);
      v[0] = s4.x, v[1] = s4.y, v[2] = s4.z, v[3] = s4.w;
      const size_t o = static_cast<size_t>(m) * N + n;
      const int cnt = vec ? 4 : min(4, N - n);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e >= cnt) break;
        float x = v[e];
        if (cs) x = x * cs[n + e];
        if (alpha != 1.0f) x = alpha * x;
        if (add) x = add[o + e] + x;
        if (g.accumulate) x = C[o + e] + x;
        if (bias) x = x + bias[n + e];
        v[e] = ActF(g.act, x);
      }
      if constexpr (kLR != 0) {
        // N % 4 == 0 here: the whole quad is in range.
        if (g.lr_store_c) *reinterpret_cast<float4*>(C + o) = make_float4(v[0], v[1], v[2], v[3]);
        float t[kLowRankMaxK];
        const float* trow = tl + (m - m0) * kLowRankMaxK;
#pragma unroll
        for (int k = 0; k < kLowRankMaxK; k += 4) {
          const float4 q = *reinterpret_cast<const float4*>(trow + k);
          t[k] = q.x, t[k + 1] = q.y, t[k + 2] = q.z, t[k + 3] = q.w;
        }
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o4[e] = AddRn(v[e], LowRankDot<kLR - 1>(t, lb[e], lr_r, g.lr_alpha));
        // (NT sites only here: in the NN instance the extra operand pushes
        // the general pass's 256 x 256 tile into scratch; NN sites with a
        // residual take the constant-rank pass above.)
        if (kLR == 2 && g.lr_res) {
          const float4 r4 = *reinterpret_cast<const float4*>(g.lr_res + o);
          o4[0] = AddRn(r4.x, o4[0]), o4[1] = AddRn(r4.y, o4[1]);
          o4[2] = AddRn(r4.z, o4[2]), o4[3] = AddRn(r4.w, o4[3]);
        }
        *reinterpret_cast<float4*>(g.lr_out + o) = make_float4(o4[0], o4[1], o4[2], o4[3]);
      } else if (vec) {
        *reinterpret_cast<float4*>(C + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        for (int e = 0; e < cnt; ++e) C[o + e] = v[e];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// A' [M, Kp] bf16 = RNE(alpha * (A[m, k] * kscale[k])), zero for k >= K;
// one row per workgroup, eight elements per lane per pass.
constexpr int kCvtThreads = 256;

__global__ void __launch_bounds__(kCvtThreads)
ConvertRowsKernel(const float* __restrict__ A, size_t K, size_t Kp, float alpha,
                  const float* __restrict__ ks, __bf16* __restrict__ out) {
  const size_t m = blockIdx.x;
  const float* row = A + m * K;
  __bf16* orow = out + m * Kp;
  const bool vec = (K % 4) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  for (size_t k = static_cast<size_t>(threadIdx.x) * 8; k < Kp; k += kCvtThreads * 8) {
    float x[8];
    if (vec && k + 8 <= K) {
      const float4 a = *reinterpret_cast<const float4*>(row + k);
      const float4 b = *reinterpret_cast<const float4*>(row + k + 4);
      x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = k + e < K ? row[k + e] : 0.0f;
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = x[e];
      if (ks && k + e < K) v = v * ks[k + e];
      if (alpha != 1.0f) v = alpha * v;
      o[e] = static_cast<__bf16>(v);
    }
    *reinterpret_cast<bf16x8*>(orow + k) = o;
  }
}

// K a multiple of 32 (Kp == K): A' is A element for element, so the rows
// flatten into one array of groups of eight, walked grid-stride by a grid
// of a few workgroups per CU; each lane keeps four groups (eight 16-byte
// loads) in flight per trip.  The k-scale index is the flat index mod K
// (32-bit: fewer than 2^32 groups), its eight values two 16-byte loads.
// kFixedK: the grid's stride is a multiple of K / 8, so a lane's groups all
// share one k-scale group, loaded once (8192 x 5632 on MI355X: 50 -> 42 us;
// the per-group index division and loads dominated).
template <bool kScale, bool kFixedK = false>
__global__ void __launch_bounds__(kCvtThreads)
ConvertFlatKernel(const float* __restrict__ A, unsigned groups, unsigned kgroups, float alpha,
                  const float* __restrict__ ks, __bf16* __restrict__ out) {
  const unsigned stride = gridDim.x * kCvtThreads;
  float fixed_sc[8];
  if constexpr (kScale && kFixedK) {
    const float4* k4 =
        reinterpret_cast<const float4*>(ks + ((blockIdx.x * kCvtThreads + threadIdx.x) % kgroups) * 8);
    const float4 s0 = k4[0], s1 = k4[1];
    fixed_sc[0] = s0.x, fixed_sc[1] = s0.y, fixed_sc[2] = s0.z, fixed_sc[3] = s0.w;
    fixed_sc[4] = s1.x, fixed_sc[5] = s1.y, fixed_sc[6] = s1.z, fixed_sc[7] = s1.w;
  }
  auto convert = [&](unsigned gi, float4 a, float4 b) {
    float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if constexpr (kScale && kFixedK) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = x[e] * fixed_sc[e];
    } else if constexpr (kScale) {
      const float4* k4 = reinterpret_cast<const float4*>(ks + (gi % kgroups) * 8);
      const float4 s0 = k4[0], s1 = k4[1];
      const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = x[e] * sc[e];
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<__bf16>(alpha != 1.0f ? alpha * x[e] : x[e]);
    reinterpret_cast<bf16x8*>(out)[gi] = o;
  };
  const float4* A4 = reinterpret_cast<const float4*>(A);
  unsigned gi = blockIdx.x * kCvtThreads + threadIdx.x;
  for (; gi + 3 * stride < groups; gi += 4 * stride) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[2 * u] = A4[2 * (gi + u * stride)];
      v[2 * u + 1] = A4[2 * (gi + u * stride) + 1];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) convert(gi + u * stride, v[2 * u], v[2 * u + 1]);
  }
  for (; gi < groups; gi += stride) convert(gi, A4[2 * gi], A4[2 * gi + 1]);
}

// W' [N, Kp] bf16 from the weight as the instruction reads it: NN's W[K, N]
// (transposed through a 32 x 32 LDS tile) or NT's W[N, K]; f32 rounded
// (RNE), int8 levels and bf16 exact; zero for k >= K.
template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kCvtThreads)
ShadowKernel(const void* __restrict__ W, size_t N, size_t K, size_t Kp, __bf16* __restrict__ out) {
  __shared__ float tile[32][33];
  const size_t k0 = static_cast<size_t>(blockIdx.x) * 32, n0 = static_cast<size_t>(blockIdx.y) * 32;
  const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 32 x 8
  auto src = [&](size_t n, size_t k) -> float {
    const size_t idx = kLayout == 1 ? n * K + k : k * N + n;
    if constexpr (kBKind == 0) return static_cast<const float*>(W)[idx];
    else if constexpr (kBKind == 1) return static_cast<float>(static_cast<const int8_t*>(W)[idx]);
    else return Bf16ToF32(static_cast<const uint16_t*>(W)[idx]);
  };
  for (int r = ty; r < 32; r += 8) {
    // NN reads along n (coalesced in W[K, N]); NT along k.
    const size_t n = kLayout == 1 ? n0 + r : n0 + tx, k = kLayout == 1 ? k0 + tx : k0 + r;
    const float v = (n < N && k < K) ? src(n, k) : 0.0f;
    if (kLayout == 1) tile[r][tx] = v;  // [n][k]
    else tile[tx][r] = v;               // [n][k]
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const size_t n = n0 + r, k = k0 + tx;
    if (n < N && k < Kp) out[n * Kp + k] = static_cast<__bf16>(tile[r][tx]);
  }
}

template <int BM, int BN, int WGM, int WGN, int kStages>
hipError_t Launch(const __bf16* A, const __bf16* W, size_t Kp, const GemmArgs& g, hipStream_t s) {
  const size_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const dim3 grid(static_cast<unsigned>(tiles)), block(WGM * WGN * kWave);
  if (!g.lr_out)
    hipLaunchKernelGGL((GemmBf16DmaKernel<BM, BN, WGM, WGN, kStages, 0>), grid, block, 0, s, A, W,
                       static_cast<int>(Kp), g);
  else if (g.lr_layout == 0)
    hipLaunchKernelGGL((GemmBf16DmaKernel<BM, BN, WGM, WGN, kStages, 1>), grid, block, 0, s, A, W,
                       static_cast<int>(Kp), g);
  else
    hipLaunchKernelGGL((GemmBf16DmaKernel<BM, BN, WGM, WGN, kStages, 2>), grid, block, 0, s, A, W,
                       static_cast<int>(Kp), g);
  return hipGetLastError();
}

}  // namespace

size_t Bf16DmaKp(size_t K) { return (K + 31) / 32 * 32; }

bool Bf16DmaFits(const GemmArgs& a) {
  if (!a.relaxed || a.layout > 1 || a.b_kind > 2) return false;
  if (a.M < 128 || a.N < 128 || a.K < 64) return false;
  // NT below the tile policy's relaxed_nt_dma_min_k runs the
  // register-staged kernel (at short K the conversion pass can cost more
  // than it saves).
  if (a.layout == 1 && a.K < (a.policy ? a.policy->relaxed_nt_dma_min_k : 768)) return false;
  const size_t Kp = Bf16DmaKp(a.K);
  // 32-bit buffer offsets within a tile and int tile indices.
  if (Kp * 2 * 256 >= (size_t{1} << 31) || a.M >= (size_t{1} << 30) || a.N >= (size_t{1} << 30))
    return false;
  return ((a.M + 127) / 128) * ((a.N + 127) / 128) < (size_t{1} << 31);
}

// The partial row maxima ride the epilogue that stores from registers: no
// low-rank term, whole 16-byte column quads.
bool Bf16DmaRowMaxFits(const GemmArgs& a) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.C) | reinterpret_cast<uintptr_t>(a.addend) |
                       reinterpret_cast<uintptr_t>(a.b_col_scale) |
                       reinterpret_cast<uintptr_t>(a.bias);
  return Bf16DmaFits(a) && !a.lr_out && a.N % 4 == 0 && (al & 15) == 0;
}

// The epilogue's constant-rank pass: rank 8 or 16 behind nothing but the
// column scale and alpha.
bool LowRankConstPass(const GemmArgs& a) {
  return (a.lr_k == 8 || a.lr_k == 16) && !a.addend && !a.bias && !a.act && !a.accumulate;
}

bool Bf16DmaLowRankFits(const GemmArgs& a) {
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return a.lr_out && a.lr_t && a.lr_b && a.lr_layout >= 0 && a.lr_layout <= 1 && a.lr_k >= 1 &&
         a.lr_k <= kLowRankMaxK && a.lr_k % 4 == 0 && a.N % 4 == 0 && !a.accumulate &&
         al16(a.lr_t) && al16(a.lr_out) && al16(a.C) && (a.lr_layout == 1 || al16(a.lr_b)) &&
         al16(a.lr_res) && al16(a.addend) && (reinterpret_cast<uintptr_t>(a.lr_sink) & 7) == 0 &&
         // A residual on an NN site rides the constant-rank pass only (rank 8
         // or 16 with no addend, bias or activation), the general pass adds
         // it on NT sites alone; the bf16 copy of the output rides the
         // constant-rank pass only.
         (!a.lr_res || a.lr_layout == 1 || LowRankConstPass(a)) &&
         (!a.lr_sink || LowRankConstPass(a));
}

hipError_t LaunchConvertRowsBf16(const float* A, size_t M, size_t K, float alpha,
                                 const float* kscale, void* out, int wgs_per_cu, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const size_t groups = M * K / 8;
  if (K % 32 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(kscale) & 15) == 0 && groups < (size_t{1} << 31)) {
    // wgs_per_cu workgroups per CU (tile policy), four groups per lane per trip.
    const unsigned grid = static_cast<unsigned>(
        std::min<size_t>((groups + 4 * kCvtThreads - 1) / (4 * kCvtThreads),
                         static_cast<size_t>(DeviceCUs()) * (wgs_per_cu > 0 ? wgs_per_cu : 8)));
    const unsigned g = static_cast<unsigned>(groups), kg = static_cast<unsigned>(K / 8);
    // A grid whose stride (grid x 256 groups) is a multiple of K / 8 keeps
    // each lane on one k-scale group: the largest such grid not above the
    // default, where one exists.
    const unsigned period = kg / std::gcd(static_cast<unsigned>(kCvtThreads), kg);
    if (kscale && period <= grid)
      hipLaunchKernelGGL((ConvertFlatKernel<true, true>), dim3(grid / period * period),
                         dim3(kCvtThreads), 0, s, A, g, kg, alpha, kscale, static_cast<__bf16*>(out));
    else if (kscale)
      hipLaunchKernelGGL((ConvertFlatKernel<true>), dim3(grid), dim3(kCvtThreads), 0, s, A, g, kg,
                         alpha, kscale, static_cast<__bf16*>(out));
    else
      hipLaunchKernelGGL((ConvertFlatKernel<false>), dim3(grid), dim3(kCvtThreads), 0, s, A, g, kg,
                         alpha, kscale, static_cast<__bf16*>(out));
    return hipGetLastError();
  }
  hipLaunchKernelGGL(ConvertRowsKernel, dim3(static_cast<unsigned>(M)), dim3(kCvtThreads), 0, s, A, K,
                     Bf16DmaKp(K), alpha, kscale, static_cast<__bf16*>(out));
  return hipGetLastError();
}

hipError_t LaunchWeightShadow(const GemmArgs& a, void* out, hipStream_t s) {
  const size_t Kp = Bf16DmaKp(a.K);
  const dim3 grid(static_cast<unsigned>(Kp / 32), static_cast<unsigned>((a.N + 31) / 32));
  __bf16* o = static_cast<__bf16*>(out);
  switch (a.layout * 3 + a.b_kind) {
    case 0: hipLaunchKernelGGL((ShadowKernel<0, 0>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    case 1: hipLaunchKernelGGL((ShadowKernel<0, 1>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    case 2: hipLaunchKernelGGL((ShadowKernel<0, 2>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    case 3: hipLaunchKernelGGL((ShadowKernel<1, 0>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    case 4: hipLaunchKernelGGL((ShadowKernel<1, 1>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    case 5: hipLaunchKernelGGL((ShadowKernel<1, 2>), grid, dim3(kCvtThreads), 0, s, a.B, a.N, a.K, Kp, o); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// 256 x 256 tiles (eight waves of 128 x 64) where the grid has at least the
// policy's relaxed_min_tiles_256 of them (default 256: one per CU) and they
// fill the CUs' last round of tiles to at least relaxed_min_fill_256 percent
// (384 tiles on 256 CUs: 75 %); otherwise
// 128 x 128 (four waves of 64 x 64).  Both accumulate each output over k in
// the same 16-deep MFMA steps: the same bits.
hipError_t LaunchGemmBf16Dma(const void* A, const void* W, const GemmArgs& a, hipStream_t s) {
  // The partial row maxima and (with no low-rank term) C's bf16 copy ride
  // the epilogue that stores from registers.
  if ((a.row_max_part || (a.lr_sink && !a.lr_out)) && !Bf16DmaRowMaxFits(a))
    return hipErrorInvalidValue;
  const size_t Kp = Bf16DmaKp(a.K);
  const auto* Ab = static_cast<const __bf16*>(A);
  const auto* Wb = static_cast<const __bf16*>(W);
  const size_t t256 = ((a.M + 255) / 256) * ((a.N + 255) / 256);
  const size_t min256 = a.policy ? a.policy->relaxed_min_tiles_256 : 256;
  const int fill = a.policy ? a.policy->relaxed_min_fill_256 : 0;
  const size_t cus = static_cast<size_t>(DeviceCUs());
  const size_t rounds = (t256 + cus - 1) / cus;
  const bool full = 100 * t256 >= static_cast<size_t>(fill) * rounds * cus;
  if (t256 >= min256 && full) return Launch<256, 256, 2, 4, 4>(Ab, Wb, Kp, a, s);
  // Below that, 128 x 128; the policy can take 128 x 192 (four waves of
  // 64 x 96, three stages) where it needs fewer rounds of tiles over the CUs
  // per unit of work (8192 x 768: 256 tiles instead of 384) -- measured
  // slower there on MI355X (one wave per SIMD against two workgroups of
  // 128 x 128 per CU), so not by default.
  const size_t t128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
  const size_t t192 = ((a.M + 127) / 128) * ((a.N + 191) / 192);
  const size_t r128 = (t128 + 2 * cus - 1) / (2 * cus), r192 = (t192 + 2 * cus - 1) / (2 * cus);
  const size_t c128 = std::max<size_t>(1, (t128 + cus - 1) / cus) * 2,
               c192 = std::max<size_t>(1, (t192 + cus - 1) / cus) * 3;  // CU-rounds x tile area / 8192
  const int mode = a.policy ? a.policy->relaxed_tile_192 : 2;
  // (The partial row maxima need 64-column wave slices: not on 128 x 192.)
  if (a.N >= 192 && !a.row_max_part &&
      (mode == 3 || (mode == 1 && (c192 < c128 || (c192 == c128 && r192 <= r128)))))
    return Launch<128, 192, 2, 2, 3>(Ab, Wb, Kp, a, s);
  return Launch<128, 128, 2, 2, 4>(Ab, Wb, Kp, a, s);
}

}  // namespace seeai
