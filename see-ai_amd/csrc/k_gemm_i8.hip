// k_gemm_i8.hip -- the W8A8 GEMM on CDNA4 int8 MFMA: per-row symmetric
// int8 activations x per-output-channel symmetric int8 weights, int32
// accumulation, f32 dequant C[m,n] = (f32(acc) * sa[m]) * sw[n].
//
// The reference has no such kernel (its q8 GEMM widens int8 weights into f32
// arithmetic); the quantizer follows the reference's int8 weight packer
// (compiler/backend/allocation/arena_binder.cc:129-177): scale = max|x|/127,
// an all-zero vector takes 1, a subnormal quotient FLT_MIN, levels
// clamp(round(x / scale), -127, 127) by a true division, ties away from zero.
// int8 x int8 products summed in int32 are exact (|sum| <= 127^2 K < 2^31 for
// K <= 133,144), so every accumulation order gives the same bits.
//
// Layout: activations QA [M, K] row-major, weights packed once into
// QWt [N, K] (K contiguous: both MFMA operands then read 16 contiguous
// bytes per lane).
//
// Large M (M, N >= the tile policy's w8a8_large_min, 4096 by default; K a
// multiple of 64): GemmI8DmaKernel, a 256 x 256
// tile per workgroup of eight waves (two per SIMD, blocks of 128 x 64 on
// v_mfma_i32_32x32x32_i8), K staged 64 bytes at a time through four LDS
// buffers filled by direct-to-LDS buffer loads, three stages in flight;
// workgroups are ordered so each XCD's L2 serves a compact block of tiles.
// Other large shapes: GemmI8TileKernel (sixteen waves of 64 x 64, loads
// staged through registers into two padded LDS buffers).
// Small M (decode-like, M <= 64): one 16-column slice of C per workgroup,
// its four waves each reducing a quarter of K on v_mfma_i32_16x16x64_i8
// straight from global memory (each weight byte is read once), then summed
// through LDS -- the weight stream is the whole cost, spread over N/16
// workgroups.
#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cstdlib>

#include "common.h"

namespace seeai {
namespace {

// --- quantizers --------------------------------------------------------------

__device__ __forceinline__ float QuantScale(float max_abs) {
  if (max_abs == 0.0f) return 1.0f;
  const float s = __fdiv_rn(max_abs, 127.0f);
  return s > FLT_MIN ? s : FLT_MIN;
}
__device__ __forceinline__ int8_t QuantLevel(float x, float scale) {
  float r = roundf(__fdiv_rn(x, scale));
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<int8_t>(r);
}

constexpr int kQThreads = 256;

// One workgroup per row.  Rows up to kQThreads * 4 * kQRegs floats stay in
// registers between the max pass and the level pass, so X is read from HBM
// once; longer (or unaligned) rows are read twice.
constexpr int kQRegs = 8;

__device__ __forceinline__ uint32_t PackLevels(float4 v, float s) {
  return static_cast<uint32_t>(static_cast<uint8_t>(QuantLevel(v.x, s))) |
         (static_cast<uint32_t>(static_cast<uint8_t>(QuantLevel(v.y, s))) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(QuantLevel(v.z, s))) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(QuantLevel(v.w, s))) << 24);
}

__global__ void __launch_bounds__(kQThreads)
QuantizeRowsKernel(const float* __restrict__ X, int8_t* __restrict__ Q, float* __restrict__ scale,
                   size_t cols) {
  __shared__ float red[kQThreads / kWave];
  const size_t r = blockIdx.x;
  const float* x = X + r * cols;
  int8_t* q = Q + r * cols;
  const bool vec = (cols % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 3) == 0);
  const bool resident = vec && cols <= static_cast<size_t>(kQThreads) * 4 * kQRegs;
  float mx = 0.0f;
  float4 keep[kQRegs];
  if (resident) {
#pragma unroll
    for (int i = 0; i < kQRegs; ++i) {
      const size_t c = (threadIdx.x + static_cast<size_t>(i) * kQThreads) * 4;
      keep[i] = c < cols ? *reinterpret_cast<const float4*>(x + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(keep[i].x), fabsf(keep[i].y)),
                           fmaxf(fabsf(keep[i].z), fabsf(keep[i].w))));
    }
  } else if (vec) {
    for (size_t c = threadIdx.x * 4; c < cols; c += kQThreads * 4) {
      const float4 v = *reinterpret_cast<const float4*>(x + c);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  } else {
    for (size_t c = threadIdx.x; c < cols; c += kQThreads) mx = fmaxf(mx, fabsf(x[c]));
  }
  mx = BlockMaxF<kQThreads>(mx, red);
  const float s = QuantScale(mx);
  if (threadIdx.x == 0) scale[r] = s;
  if (resident) {
#pragma unroll
    for (int i = 0; i < kQRegs; ++i) {
      const size_t c = (threadIdx.x + static_cast<size_t>(i) * kQThreads) * 4;
      if (c < cols) *reinterpret_cast<uint32_t*>(q + c) = PackLevels(keep[i], s);
    }
  } else if (vec) {
    for (size_t c = threadIdx.x * 4; c < cols; c += kQThreads * 4)
      *reinterpret_cast<uint32_t*>(q + c) = PackLevels(*reinterpret_cast<const float4*>(x + c), s);
  } else {
    for (size_t c = threadIdx.x; c < cols; c += kQThreads) q[c] = QuantLevel(x[c], s);
  }
}

// The level of x at scale s from the reciprocal: a = fl(x * fl(1/s)) is
// within 2^-24 + 2^-24 (relative) of x / s, so for |x / s| <= 128 it lies
// within 2^-15 of the correctly rounded quotient fl(x / s).  Round-half-away
// and the clamp can then only disagree when a is within 2^-15 of a half
// integer; a group of four with any element inside 2^-12 of one is redone by
// the true division (QuantLevel).  So the levels are bitwise QuantLevel(x, s)
// for every |x| <= 128 s, which the row's own max guarantees (NaN and
// infinities give what the division gives: inf * 0 and inf / inf are both
// NaN, clamped alike).
__device__ __forceinline__ uint32_t LevelByteFast(float x, float inv, bool& near) {
  const float a = x * inv;
  near = near || fabsf(fabsf(a - truncf(a)) - 0.5f) < 0x1p-12f;
  const float l = fminf(fmaxf(roundf(a), -127.0f), 127.0f);
  return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(l)));
}

__device__ __forceinline__ uint32_t PackLevelsInv(float4 v, float s, float inv) {
  bool near = false;
  const uint32_t w = LevelByteFast(v.x, inv, near) | (LevelByteFast(v.y, inv, near) << 8) |
                     (LevelByteFast(v.z, inv, near) << 16) | (LevelByteFast(v.w, inv, near) << 24);
  return near ? PackLevels(v, s) : w;
}

// Rows of at most 256 * kR floats (16-byte aligned, a multiple of 4): each
// wave walks rows g, g + W, g + 2W, ... (W waves in the grid) with the next
// row's loads in flight while it quantizes the current one.  Lane l holds
// float4 chunks l, l + 64, ... of a row, read by buffer loads over a range of
// exactly that row: chunks past the row end, and the whole of a row past the
// matrix end (the last prefetch), read as zeros without touching memory, so
// every load is issued unconditionally.  The max is a butterfly inside the
// wave (no LDS, no barrier).
template <int kR>
__device__ __forceinline__ void LoadRowChunks(const float* X, size_t row, size_t rows, size_t cols,
                                              int lane, float4 (&v)[kR]) {
  const size_t r = row < rows ? row : rows;
  const bool live = r < rows;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(X) + (live ? r * cols : 0), 0,
      live ? static_cast<int>(cols * 4) : 0, 0x00020000);
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + i * kWave) * 16, 0, 0);
    v[i] = *reinterpret_cast<const float4*>(&q);
  }
}

template <int kR>
__device__ __forceinline__ void QuantizeRowChunks(const float4 (&v)[kR], int8_t* q, float* scale,
                                                  size_t cols, int lane) {
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  }
  mx = WaveMaxF(mx);
  const float s = QuantScale(mx);
  const float inv = 1.0f / s;
  if (lane == 0) *scale = s;
  // The level bytes leave through a buffer range of exactly this row: the
  // stores of chunks past its end are dropped by the range check.
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(q, 0, static_cast<int>(cols), 0x00020000);
#pragma unroll
  for (int i = 0; i < kR; ++i)
    __builtin_amdgcn_raw_buffer_store_b32(PackLevelsInv(v[i], s, inv), rs, (lane + i * kWave) * 4,
                                          0, 0);
}

template <int kR>
__global__ void __launch_bounds__(kQThreads)
QuantizeRowsWaveKernel(const float* __restrict__ X, int8_t* __restrict__ Q,
                       float* __restrict__ scale, size_t rows, size_t cols) {
  const int lane = threadIdx.x % kWave;
  const size_t W = static_cast<size_t>(gridDim.x) * (kQThreads / kWave);
  // The row index is wave-uniform: kept in scalar registers, so the buffer
  // ranges built from it need no per-lane resolution.
  size_t r = static_cast<size_t>(
      Uniform(static_cast<int>(blockIdx.x * (kQThreads / kWave) + threadIdx.x / kWave)));
  if (r >= rows) return;
  float4 a[kR], b[kR];
  LoadRowChunks<kR>(X, r, rows, cols, lane, a);
  for (;;) {
    LoadRowChunks<kR>(X, r + W, rows, cols, lane, b);
    QuantizeRowChunks<kR>(a, Q + r * cols, scale + r, cols, lane);
    r += W;
    if (r >= rows) break;
    LoadRowChunks<kR>(X, r + W, rows, cols, lane, a);
    QuantizeRowChunks<kR>(b, Q + r * cols, scale + r, cols, lane);
    r += W;
    if (r >= rows) break;
  }
}

// Rows of 1024 kR floats or fewer (16-byte aligned, a multiple of 4): a
// workgroup of four waves per row.  Lane t of the workgroup holds float4
// chunks t, t + 256, ... of the row, read by buffer loads over exactly the
// row (chunks past its end read as zeros and their stores are dropped); the
// row max is a butterfly in each wave, then the four waves' maxima through
// LDS.  Spreading a row over four waves puts more rows' loads in flight per
// CU than the wave-per-row kernel and lets each row's stores start sooner:
// 4096 x 4096 on MI355X 14.3 us against 17.9 us (two waves per row 15.8,
// eight 14.6).  Max-abs is exact in any order and the levels are
// PackLevelsInv's, so the bytes are the wave kernel's.
template <int kR>
__global__ void __launch_bounds__(kQThreads)
QuantizeRowsBlockKernel(const float* __restrict__ X, int8_t* __restrict__ Q,
                        float* __restrict__ scale, size_t cols) {
  constexpr int kWaves = kQThreads / kWave;
  __shared__ float red[kWaves];
  const size_t r = blockIdx.x;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(X) + r * cols, 0, static_cast<int>(cols * 4), 0x00020000);
  float4 v[kR];
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, (t + i * kQThreads) * 16, 0, 0);
    v[i] = *reinterpret_cast<const float4*>(&q);
  }
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < kR; ++i)
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  mx = WaveMaxF(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, red[w]);
  const float s = QuantScale(mx);
  const float inv = 1.0f / s;
  if (t == 0) scale[r] = s;
  const __amdgpu_buffer_rsrc_t ws = __builtin_amdgcn_make_buffer_rsrc(
      Q + r * cols, 0, static_cast<int>(cols), 0x00020000);
#pragma unroll
  for (int i = 0; i < kR; ++i)
    __builtin_amdgcn_raw_buffer_store_b32(PackLevelsInv(v[i], s, inv), ws, (t + i * kQThreads) * 4,
                                          0, 0);
}

// Column max-abs of W [K, N]: one lane per column, coalesced across lanes.
__global__ void __launch_bounds__(kQThreads)
ColumnScaleKernel(const float* __restrict__ W, float* __restrict__ scale, size_t K, size_t N) {
  const size_t n = static_cast<size_t>(blockIdx.x) * kQThreads + threadIdx.x;
  if (n >= N) return;
  float mx = 0.0f;
  for (size_t k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(W[k * N + n]));
  scale[n] = QuantScale(mx);
}

// Quantize and transpose W [K, N] -> Qt [N, K] through a 32 x 32 LDS tile.
__global__ void __launch_bounds__(kQThreads)
PackTransposeKernel(const float* __restrict__ W, const float* __restrict__ scale,
                    int8_t* __restrict__ Qt, size_t K, size_t N) {
  __shared__ int8_t tile[32][33];
  const size_t k0 = static_cast<size_t>(blockIdx.y) * 32, n0 = static_cast<size_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const size_t k = k0 + r, n = n0 + tx;
    tile[r][tx] = (k < K && n < N) ? QuantLevel(W[k * N + n], scale[n]) : 0;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const size_t n = n0 + r, k = k0 + tx;
    if (n < N && k < K) Qt[n * K + k] = tile[tx][r];
  }
}

// --- the large-M GEMM ----------------------------------------------------------

constexpr int kThreads = 256;

// Tile -> workgroup order.  The hardware deals workgroups round-robin over
// the 8 XCDs (workgroup b runs on XCD b % 8), each with its own L2.  When
// the tile count divides by 8, the tiles are renumbered so each XCD owns a
// contiguous run, and the run walks column-major within bands of kGroupM
// row tiles: an XCD's 32 concurrent tiles at 4096^2 share 4 row panels of A
// and 8 column panels of W, so each k-slice of A and W leaves HBM once per
// XCD instead of once per tile row or column.
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

// BM x BN tile per workgroup of WGM x WGN waves, each wave a (BM/WGM) x
// (BN/WGN) block of 32 x 32 x 32 int8 MFMAs.  K advances BK bytes per step
// through two LDS buffers (rows padded by 16 bytes): the next step's global
// loads are issued before the current step's MFMAs and land in the other
// buffer after them, so one barrier per step orders both hazards.
template <int BM, int BN, int BK, int WGM, int WGN>
__global__ void __launch_bounds__(WGM * WGN * kWave)
GemmI8TileKernel(const int8_t* __restrict__ QA, const float* __restrict__ sa,
                 const int8_t* __restrict__ QW, const float* __restrict__ sw,
                 float* __restrict__ C, int32_t* __restrict__ acc_out, int M, int N, int K) {
  constexpr int kT = WGM * WGN * kWave;        // lanes per workgroup
  constexpr int LDK = BK + 16;                 // padded LDS row stride (bytes)
  constexpr int WM = BM / WGM, WN = BN / WGN;  // per-wave block
  constexpr int TM = WM / 32, TN = WN / 32;    // 32 x 32 MFMA tiles per wave
  constexpr int kChunksRow = BK / 16;          // 16-byte chunks per tile row
  constexpr int NA = BM * kChunksRow / kT;
  constexpr int NB = BN * kChunksRow / kT;
  static_assert(NA * kT == BM * kChunksRow && NB * kT == BN * kChunksRow, "tile / lanes");
  // One LDS block: two A buffers then two B buffers (rows padded by 16 B);
  // the epilogue reuses all of it as per-wave staging.
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * (BM + BN) * LDK];
  auto As = [&](int buf) { return smem + buf * (BM * LDK); };
  auto Bs = [&](int buf) { return smem + 2 * BM * LDK + buf * (BN * LDK); };

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
  int tm, tn;
  TileOf(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  v4i ra[NA], rb[NB];
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < NA; ++e) {
      const int c = tid + e * kT;
      const int row = c / kChunksRow, kc = c % kChunksRow;
      const int m = m0 + row, k = k0 + kc * 16;
      ra[e] = (m < M && k < K) ? *reinterpret_cast<const v4i*>(QA + static_cast<size_t>(m) * K + k)
                               : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int e = 0; e < NB; ++e) {
      const int c = tid + e * kT;
      const int row = c / kChunksRow, kc = c % kChunksRow;
      const int n = n0 + row, k = k0 + kc * 16;
      rb[e] = (n < N && k < K) ? *reinterpret_cast<const v4i*>(QW + static_cast<size_t>(n) * K + k)
                               : v4i{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int e = 0; e < NA; ++e) {
      const int c = tid + e * kT;
      *reinterpret_cast<v4i*>(As(buf) + (c / kChunksRow) * LDK + (c % kChunksRow) * 16) = ra[e];
    }
#pragma unroll
    for (int e = 0; e < NB; ++e) {
      const int c = tid + e * kT;
      *reinterpret_cast<v4i*>(Bs(buf) + (c / kChunksRow) * LDK + (c % kChunksRow) * 16) = rb[e];
    }
  };

  const int nsteps = (K + BK - 1) / BK;
  constexpr int KS = BK / 32;  // 32-byte k-steps per LDS buffer
  v4i af[2][TM], bf[2][TN];
  auto read_frags = [&](int buf, int ks, int slot) {
    const int koff = ks * 32 + (lane / 32) * 16;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      af[slot][i] = *reinterpret_cast<const v4i*>(As(buf) + (wm + i * 32 + lane % 32) * LDK + koff);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      bf[slot][j] = *reinterpret_cast<const v4i*>(Bs(buf) + (wn + j * 32 + lane % 32) * LDK + koff);
  };
  load(0);
  store(0);
  __syncthreads();
  for (int it = 0; it < nsteps; ++it) {
    const int buf = it & 1;
    if (it + 1 < nsteps) load((it + 1) * BK);
    // Fragments double-buffered in registers: the next k-step's LDS reads
    // are in flight while the current k-step's MFMAs issue.
    read_frags(buf, 0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_frags(buf, ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks & 1][i], bf[ks & 1][j],
                                                            acc[i][j], 0, 0, 0);
    }
    if (it + 1 < nsteps) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue.  Lane holds column (lane % 32) and rows 8*(r/4) + 4*(lane/32)
  // + r%4 of each 32 x 32 tile.  The dequantized tile goes through this
  // wave's slice of LDS (free now: the loop ended on a barrier) so C leaves
  // in row-contiguous 16-byte stores; the row scales are read once per
  // 4-row group as float4.
  if (acc_out) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
          const int n = n0 + wn + j * 32 + lane % 32;
          if (m < M && n < N) acc_out[static_cast<size_t>(m) * N + n] = acc[i][j][r];
        }
  }
  constexpr int SLD = WN + 4;  // staging row stride (floats)
  static_assert(WGM * WGN * 32 * SLD * 4 <= 2 * (BM + BN) * LDK, "staging fits in LDS");
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * SLD;
  const bool vec_out = (N % 4) == 0;
  float swv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn + j * 32 + lane % 32;
    swv[j] = n < N ? sw[n] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int mb = m0 + wm + i * 32;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m4 = mb + 8 * q + 4 * (lane / 32);
      float sav[4];
      if (m4 + 3 < M && (M % 4) == 0) {
        const float4 v = *reinterpret_cast<const float4*>(sa + m4);
        sav[0] = v.x, sav[1] = v.y, sav[2] = v.z, sav[3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) sav[e] = m4 + e < M ? sa[m4 + e] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 8 * q + 4 * (lane / 32) + e;
          stage[row * SLD + j * 32 + lane % 32] =
              (static_cast<float>(acc[i][j][4 * q + e]) * sav[e]) * swv[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    constexpr int kVecRow = WN / 4;  // float4 per staged row
#pragma unroll
    for (int t = 0; t < 32 * kVecRow / kWave; ++t) {
      const int idx = lane + t * kWave;
      const int row = idx / kVecRow, c4 = idx % kVecRow;
      const int m = mb + row, n = n0 + wn + c4 * 4;
      const float4 v = *reinterpret_cast<const float4*>(stage + row * SLD + c4 * 4);
      if (m >= M) continue;
      float* dst = C + static_cast<size_t>(m) * N + n;
      if (vec_out && n + 3 < N) {
        *reinterpret_cast<float4*>(dst) = v;
      } else {
        if (n < N) dst[0] = v.x;
        if (n + 1 < N) dst[1] = v.y;
        if (n + 2 < N) dst[2] = v.z;
        if (n + 3 < N) dst[3] = v.w;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// --- the large-M GEMM, staged by direct-to-LDS loads -----------------------------
//
// 256 x 256 tile per workgroup of WGM x WGN waves, each a (256/WGM) x
// (256/WGN) block of v_mfma_i32_32x32x32_i8 accumulators.  The launcher runs
// eight waves (two per SIMD, 2 x 4, blocks of 128 x 64: 128 int32
// accumulators per lane), measured 6-7 % faster than four waves of 128 x 128
// (one per SIMD, 256 accumulators) at 4096^3 and 8192^3: the second wave on
// each SIMD issues MFMAs while the first waits on LDS or the barrier.  K moves 64 bytes per stage through kStages LDS buffers (32 KiB
// each: 256 A rows + 256 W rows of 64 bytes) filled by buffer_load ... lds,
// which writes a wave's 64 x 16 bytes to consecutive LDS addresses from M0
// without passing through registers; kStages - 1 stages are in flight while
// one is multiplied.  One barrier per stage: every wave's loads of the
// stage it is about to read have landed (vmcnt), and every wave has
// finished reading the buffer the next load overwrites.
//
// LDS rows are 64 bytes, four 16-byte chunks; chunk c of row r sits at
// physical chunk (c + r/4) mod 4.  The fragment reads (lane l: row l % 32,
// chunk 2ks + l / 32) are then free of bank conflicts -- measured with
// SQ_LDS_BANK_CONFLICT on gfx950 for ds_read_b128, which also counts
// conflicts for rotations that bring in r/8 or r/16.  Loads pick the global
// chunk that belongs at each physical slot.  Rows past M (or N) read as zeros (buffer
// range check); K must be a multiple of 64.
constexpr int kDmaBK = 64;
constexpr int kDmaChunks = kDmaBK / 16;

typedef __attribute__((address_space(3))) void* LdsPtr;

__device__ __forceinline__ int DmaPhys(int row, int c) { return (c + row / 4) & 3; }

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int n>
__device__ __forceinline__ void WaitVm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

template <int kStages, int WGM, int WGN>
__global__ void __launch_bounds__(WGM * WGN * kWave)
GemmI8DmaKernel(const int8_t* __restrict__ QA, const float* __restrict__ sa,
                const int8_t* __restrict__ QW, const float* __restrict__ sw,
                float* __restrict__ C, int32_t* __restrict__ acc_out, int M, int N, int K) {
  constexpr int BM = 256, BN = 256;
  constexpr int kWaves = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;       // per-wave block
  constexpr int TM = WM / 32, TN = WN / 32;         // 32 x 32 accumulators per wave
  constexpr int kRowsPerLoad = kWave / kDmaChunks;  // rows one wave-load fills (16)
  constexpr int kLoads = BM / kRowsPerLoad / kWaves;  // wave-loads per operand, stage, wave
  static_assert(kLoads * kRowsPerLoad * kWaves == BM, "loads cover the tile");
  constexpr int kStageA = BM * kDmaBK;               // bytes
  constexpr int kStage = (BM + BN) * kDmaBK;
  constexpr int kPerStage = 2 * kLoads;              // vmcnt units per stage
  __shared__ __attribute__((aligned(1024))) int8_t smem[kStages * kStage];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  int tm, tn;
  TileOf(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // Operand ranges start at this tile's first row: offsets stay below
  // 256 * K, and rows past the operand's end fall outside num_records.
  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(QA) + static_cast<size_t>(m0) * K, 0,
      Uniform((M - m0) * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(QW) + static_cast<size_t>(n0) * K, 0,
      Uniform((N - n0) * K), 0x00020000);
  // This lane's slot in each wave-load: row rbase + lane / 4, physical chunk
  // lane % 4, which holds logical chunk (p - r/4) mod 4.
  // (Fixed capacity: an array sized by a template-dependent constant and
  // captured by the lambdas below loses the kernel's host-side stub.)
  static_assert(kLoads <= 4, "voff capacity");
  int voff[4];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int row = (j * kWaves + wave) * kRowsPerLoad + lane / kDmaChunks;
    const int c = (lane % kDmaChunks - row / 4) & 3;
    voff[j] = row * K + c * 16;
  }
  auto issue = [&](int st, int buf) {
    int8_t* sA = smem + buf * kStage;
    int8_t* sB = sA + kStageA;
    const int k0 = st * kDmaBK;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int rbase = Uniform((j * kWaves + wave) * kRowsPerLoad);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, (LdsPtr)(sA + rbase * kDmaBK), 16, voff[j],
                                               k0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, (LdsPtr)(sB + rbase * kDmaBK), 16, voff[j],
                                               k0, 0, 0);
    }
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
  const int lr = lane % 32, h = lane / 32;
  // Fragment offsets within a buffer for k-steps 0 and 1 (logical chunks h
  // and 2 + h of row lr; the tile rows wm + 32 i add multiples of 32 rows,
  // which leave the swizzle unchanged).
  const int frag0 = lr * kDmaBK + DmaPhys(lr, h) * 16;
  const int frag1 = lr * kDmaBK + DmaPhys(lr, 2 + h) * 16;

  // Software pipeline, one k-step (32 bytes of K) ahead in registers: while
  // the MFMAs of one k-step issue, the fragments of the next are read from
  // LDS (interleaved two MFMAs per read).  The barrier sits between a
  // stage's two k-steps: after it, stage it + 1 has landed, and every wave
  // has consumed its reads of stage it - 1 (their MFMAs were issued before
  // the barrier), whose buffer then takes the loads of stage
  // it + kStages - 1.
  const int nsteps = K / kDmaBK;
  v4i fa[2][TM], fb[2][TN];
  auto read = [&](int buf, int fo, int slot) {
    const int8_t* sA = smem + buf * kStage;
    const int8_t* sB = sA + kStageA;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[slot][i] = *reinterpret_cast<const v4i*>(sA + (wm + i * 32) * kDmaBK + fo);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[slot][j] = *reinterpret_cast<const v4i*>(sB + (wn + j * 32) * kDmaBK + fo);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[slot][j], fa[slot][i], acc[i][j],
                                                          0, 0, 0);
  };
  // The next k-step's TM + TN LDS reads spread one per MFMA from the start
  // of a k-step's TM x TN MFMAs; after the barrier, the stage's loads take
  // the following MFMA slots.
  auto interleave = [&]() {
#pragma unroll
    for (int g = 0; g < TM + TN; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int g = TM + TN; g < TM * TN; ++g) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };
  auto interleave_loads = [&]() {
#pragma unroll
    for (int g = 0; g < TM * TN; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (g < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (g >= TM * TN - 2 * kLoads) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  };
  static_assert(TM * TN >= TM + TN && TM * TN >= 2 * kLoads, "MFMA slots for the reads and loads");

  // Every iteration loads one stage: past the last stage the loads repeat
  // it (in bounds, into a buffer no later stage uses), so the number of
  // stages in flight at each barrier is always kStages - 3.
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
  WaitVm<0>();  // the repeated loads have landed before the workgroup ends

  // The products are C^T tiles (W fragments as the A operand): lane (h, lr)
  // holds columns n = 32 j + 8 q + 4 h + e, e < 4, of row m = 32 i + lr --
  // four consecutive floats of one C row, stored as 16 bytes straight from
  // registers.
  const bool vec_out = (N % 4) == 0 && ((reinterpret_cast<uintptr_t>(C) |
                                         reinterpret_cast<uintptr_t>(sw) |
                                         reinterpret_cast<uintptr_t>(acc_out)) & 15) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm + i * 32 + lr;
    if (m >= M) continue;
    const float s_a = sa[m];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + j * 32 + 8 * q + 4 * h;
        const size_t at = static_cast<size_t>(m) * N + n;
        const v16i& a = acc[i][j];
        if (vec_out && n + 3 < N) {
          const float4 s4 = *reinterpret_cast<const float4*>(sw + n);
          *reinterpret_cast<float4*>(C + at) =
              make_float4((static_cast<float>(a[4 * q]) * s_a) * s4.x,
                          (static_cast<float>(a[4 * q + 1]) * s_a) * s4.y,
                          (static_cast<float>(a[4 * q + 2]) * s_a) * s4.z,
                          (static_cast<float>(a[4 * q + 3]) * s_a) * s4.w);
          if (acc_out)
            *reinterpret_cast<int4*>(acc_out + at) =
                make_int4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e >= N) continue;
            C[at + e] = (static_cast<float>(a[4 * q + e]) * s_a) * sw[n + e];
            if (acc_out) acc_out[at + e] = a[4 * q + e];
          }
        }
      }
  }
}

// --- the small-M GEMM (decode-like) ---------------------------------------------

// A workgroup per 16 kNT output columns; its kW waves each reduce one
// contiguous K / kW slice (a 16-wave workgroup keeps 64 KB of the weight
// stream in flight per CU), each activation fragment serving kNT weight
// tiles; the int32 partials add exactly in any order.
template <int MT, int kW, int kNT>  // M <= 16 MT rows; kW waves; 16 kNT columns
__global__ void __launch_bounds__(kW * kWave)
GemmI8SkinnyKernel(const int8_t* __restrict__ QA, const float* __restrict__ sa,
                   const int8_t* __restrict__ QW, const float* __restrict__ sw,
                   float* __restrict__ C, int32_t* __restrict__ acc_out, int M, int N, int K) {
  constexpr int kTiles = MT * kNT;
  static_assert(kTiles <= kW, "a reducing wave per tile");
  __shared__ v4i part[kW][kTiles][kWave];
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int n0 = blockIdx.x * 16 * kNT;
  const int kq = K / kW;  // each wave reduces one contiguous slice of K
  const int kb = wave * kq, ke = kb + kq;
  const int kl = (lane / 16) * 16;
  const int8_t* wrow[kNT];
#pragma unroll
  for (int c = 0; c < kNT; ++c) {
    const int col = n0 + c * 16 + lane % 16;
    wrow[c] = QW + static_cast<size_t>(col < N ? col : 0) * K;
  }
  v4i acc[MT][kNT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < kNT; ++c) acc[t][c] = v4i{0, 0, 0, 0};
#pragma unroll 4
  for (int k = kb; k < ke; k += 64) {
    v4i b[kNT];
#pragma unroll
    for (int c = 0; c < kNT; ++c)
      b[c] = n0 + c * 16 + lane % 16 < N ? *reinterpret_cast<const v4i*>(wrow[c] + k + kl)
                                         : v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + lane % 16;
      const v4i a = m < M ? *reinterpret_cast<const v4i*>(QA + static_cast<size_t>(m) * K + k + kl)
                          : v4i{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < kNT; ++c)
        acc[t][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[c], acc[t][c], 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < kNT; ++c) part[wave][t * kNT + c][lane] = acc[t][c];
  __syncthreads();
  if (wave >= kTiles) return;
  // Wave w sums tile w over the K slices (integers: exact in any order).
  const int t = wave / kNT, c = wave % kNT;
  v4i sum = part[0][wave][lane];
#pragma unroll
  for (int w = 1; w < kW; ++w) sum += part[w][wave][lane];
  const int col = n0 + c * 16 + lane % 16;
  if (col >= N) return;
  const float swn = sw[col];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = t * 16 + (lane / 16) * 4 + r;  // lane holds rows 4*(lane/16)+r
    if (m >= M) continue;
    const size_t o = static_cast<size_t>(m) * N + col;
    if (acc_out) acc_out[o] = sum[r];
    C[o] = (static_cast<float>(sum[r]) * sa[m]) * swn;
  }
}

// --- any shape: one lane per output, for K not a multiple of the vector ------

__global__ void __launch_bounds__(kThreads)
GemmI8NaiveKernel(const int8_t* __restrict__ QA, const float* __restrict__ sa,
                  const int8_t* __restrict__ QW, const float* __restrict__ sw,
                  float* __restrict__ C, int32_t* __restrict__ acc_out, size_t M, size_t N,
                  size_t K) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= M * N) return;
  const size_t m = i / N, n = i % N;
  int32_t s = 0;
  for (size_t k = 0; k < K; ++k)
    s += static_cast<int32_t>(QA[m * K + k]) * static_cast<int32_t>(QW[n * K + k]);
  if (acc_out) acc_out[i] = s;
  C[i] = (static_cast<float>(s) * sa[m]) * sw[n];
}

inline bool Aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

int DeviceCUs() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

hipError_t LaunchQuantizeRows(const float* X, int8_t* Q, float* scale, size_t rows, size_t cols,
                              int waves_per_cu, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const bool vec = cols > 0 && cols % 4 == 0 && Aligned(X, 16) && Aligned(Q, 4);
  if (vec && cols > 1024 && cols <= 8 * 1024 && rows < (size_t{1} << 31)) {
    // Long rows: a workgroup of four waves per row.
    const dim3 grid(static_cast<unsigned>(rows));
    if (cols <= 2 * 1024)
      hipLaunchKernelGGL(QuantizeRowsBlockKernel<2>, grid, dim3(kQThreads), 0, s, X, Q, scale, cols);
    else if (cols <= 4 * 1024)
      hipLaunchKernelGGL(QuantizeRowsBlockKernel<4>, grid, dim3(kQThreads), 0, s, X, Q, scale, cols);
    else
      hipLaunchKernelGGL(QuantizeRowsBlockKernel<8>, grid, dim3(kQThreads), 0, s, X, Q, scale, cols);
    return hipGetLastError();
  }
  if (vec && cols <= 16 * 256 && rows < (size_t{1} << 31)) {
    // waves_per_cu waves per compute unit walk the rows (at least one row each).
    const int cus = DeviceCUs();
    const size_t waves = std::min(rows, static_cast<size_t>(cus) * static_cast<size_t>(waves_per_cu > 0 ? waves_per_cu : 32));
    const size_t per_wg = kQThreads / kWave;
    const dim3 grid(static_cast<unsigned>((waves + per_wg - 1) / per_wg));
    if (cols <= 4 * 256)
      hipLaunchKernelGGL(QuantizeRowsWaveKernel<4>, grid, dim3(kQThreads), 0, s, X, Q, scale,
                         rows, cols);
    else if (cols <= 8 * 256)
      hipLaunchKernelGGL(QuantizeRowsWaveKernel<8>, grid, dim3(kQThreads), 0, s, X, Q, scale,
                         rows, cols);
    else
      hipLaunchKernelGGL(QuantizeRowsWaveKernel<16>, grid, dim3(kQThreads), 0, s, X, Q, scale,
                         rows, cols);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(QuantizeRowsKernel, dim3(static_cast<unsigned>(rows)), dim3(kQThreads), 0, s,
                     X, Q, scale, cols);
  return hipGetLastError();
}

hipError_t LaunchPackWeightsI8(const float* W, int8_t* Qt, float* scale, size_t K, size_t N,
                               hipStream_t s) {
  if (N == 0) return hipSuccess;
  hipLaunchKernelGGL(ColumnScaleKernel, dim3(GridFor(N, kQThreads)), dim3(kQThreads), 0, s, W,
                     scale, K, N);
  if (K == 0) return hipGetLastError();
  hipLaunchKernelGGL(PackTransposeKernel,
                     dim3(static_cast<unsigned>((N + 31) / 32), static_cast<unsigned>((K + 31) / 32)),
                     dim3(kQThreads), 0, s, W, scale, Qt, K, N);
  return hipGetLastError();
}

hipError_t LaunchGemmW8A8(const int8_t* QA, const float* sa, const int8_t* QWt, const float* sw,
                          float* C, int32_t* acc, size_t M, size_t N, size_t K,
                          const TilePolicy& policy, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  const bool vec_ok = K % 16 == 0 && Aligned(QA, 16) && Aligned(QWt, 16) && M < (1u << 30) &&
                      N < (1u << 30) && K < (1u << 30) && M * K < (1ull << 31) &&
                      N * K < (1ull << 31);
  if (vec_ok && M <= 64 && K % 256 == 0) {
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const auto grid = [&](int cols) { return dim3(static_cast<unsigned>((N + cols - 1) / cols)); };
    if (K % (64 * 16) == 0) {  // 16 waves of 64-deep steps (two column tiles per
                               // fragment measured slower at 32 x 4096 x 4096)
      if (M <= 32)
        hipLaunchKernelGGL((GemmI8SkinnyKernel<2, 16, 1>), grid(16), dim3(16 * kWave), 0, s, QA, sa,
                           QWt, sw, C, acc, m, n, k);
      else
        hipLaunchKernelGGL((GemmI8SkinnyKernel<4, 16, 1>), grid(16), dim3(16 * kWave), 0, s, QA, sa,
                           QWt, sw, C, acc, m, n, k);
    } else if (M <= 32) {
      hipLaunchKernelGGL((GemmI8SkinnyKernel<2, 4, 1>), grid(16), dim3(4 * kWave), 0, s, QA, sa, QWt,
                         sw, C, acc, m, n, k);
    } else {
      hipLaunchKernelGGL((GemmI8SkinnyKernel<4, 4, 1>), grid(16), dim3(4 * kWave), 0, s, QA, sa, QWt,
                         sw, C, acc, m, n, k);
    }
    return hipGetLastError();
  }
  if (vec_ok) {
    // Tile geometry (TilePolicy): from M, N >= w8a8_large_min the policy's
    // large kernel -- by default the direct-to-LDS 256 x 256 when K is a
    // multiple of its 64-byte stage -- else 128 x 128 (four waves).
    const bool big = M >= policy.w8a8_large_min && N >= policy.w8a8_large_min;
    const int pick = !big ? 3 : policy.w8a8_large_kernel;
    const bool dma_ok = K >= kDmaBK && K % kDmaBK == 0 && K * 256 < (1ull << 31);
    if (pick == 1 && dma_ok) {
      const unsigned tiles = static_cast<unsigned>(((M + 255) / 256) * ((N + 255) / 256));
      hipLaunchKernelGGL((GemmI8DmaKernel<4, 2, 4>), dim3(tiles), dim3(512), 0, s, QA, sa, QWt, sw, C,
                         acc, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K));
    } else if (pick <= 2) {
      const unsigned tiles = static_cast<unsigned>(((M + 255) / 256) * ((N + 255) / 256));
      hipLaunchKernelGGL((GemmI8TileKernel<256, 256, 128, 4, 4>), dim3(tiles), dim3(1024), 0, s, QA,
                         sa, QWt, sw, C, acc, static_cast<int>(M), static_cast<int>(N),
                         static_cast<int>(K));
    } else {
      const unsigned tiles = static_cast<unsigned>(((M + 127) / 128) * ((N + 127) / 128));
      hipLaunchKernelGGL((GemmI8TileKernel<128, 128, 128, 2, 2>), dim3(tiles), dim3(256), 0, s, QA,
                         sa, QWt, sw, C, acc, static_cast<int>(M), static_cast<int>(N),
                         static_cast<int>(K));
    }
    return hipGetLastError();
  }
  hipLaunchKernelGGL(GemmI8NaiveKernel, dim3(GridFor(M * N, kThreads, 1u << 30)), dim3(kThreads), 0,
                     s, QA, sa, QWt, sw, C, acc, M, N, K);
  return hipGetLastError();
}

}  // namespace seeai
