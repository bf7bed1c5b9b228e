// k_gemm_bf16.hip -- the relaxed family's frozen-weight products on bf16
// MFMA (kFlagRelaxed on kGemmNN / kGemmNT with f32 weights and on kGemmNNQ8
// / kGemmNTQ8 with int8 levels, source/plan/instruction.h:356-384: the
// activations rounded to bf16 once at the GEMM input, the weight in reduced
// precision, f32 accumulation).  int8 levels are exact in bf16, so a q8
// product's only rounding is the activation's: the per-tensor scale and the
// NT k-scale multiply A before it rounds (gemm.cc:626-674), the NN column
// scale multiplies the finished dot.
//
// A 128 x 128 tile of C per 256-lane workgroup: four waves in 2 x 2, each a
// 64 x 64 block of 2 x 2 v_mfma_f32_32x32x16_bf16 tiles.  K walks in steps
// of 64; each step's A rows and B columns are converted to bf16 as they are
// staged and stored k-contiguous in LDS (As[m][k], Bs[n][k], rows padded to
// 72 elements = 144 bytes), so one 16-byte read gives a lane its 8-element
// MFMA fragment.  LDS is double buffered: the next step's f32 operands load
// into registers while the current step multiplies, and one barrier
// separates steps.  NN's B is [K, N] in memory: a lane loads a 4 x 4 block
// (four k rows, four n) and transposes it in registers.  The epilogue is the
// exact family's (column scale, alpha, addend, accumulate, bias,
// activation) on four consecutive columns of a row per lane, stored as one
// 16-byte write.
#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 ToBf16(float4 v) {
  return bf16x4{static_cast<__bf16>(v.x), static_cast<__bf16>(v.y), static_cast<__bf16>(v.z),
                static_cast<__bf16>(v.w)};
}

__device__ __forceinline__ __bf16 Level(uint32_t w, int c) {
  return static_cast<__bf16>(static_cast<float>(static_cast<int8_t>(w >> (8 * c))));
}

// kLayout 0 = NN (B[K, N]), 1 = NT (B[N, K]); kBKind 0 = f32 weights, 1 =
// int8 levels.  Requires K % 4 == 0, and for NN N % 4 == 0, with 16-byte
// aligned A and f32 B, 4-byte aligned int8 B (checked by the launcher).
template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) GemmBf16Kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) __bf16 As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[2][BN * LDK];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = (wave / 2) * 64, wn = (wave % 2) * 64;
  const size_t M = g.M, N = g.N, K = g.K;
  // Tiles in column-major order of the tile grid: consecutive workgroups
  // share one B panel (the weight), which then stays in L2.
  const size_t tiles_m = (M + BM - 1) / BM;
  const size_t m0 = (blockIdx.x % tiles_m) * BM, n0 = (blockIdx.x / tiles_m) * BN;
  const float* __restrict__ A = g.A;
  const float* __restrict__ B = static_cast<const float*>(g.B);
  const int8_t* __restrict__ Bq = static_cast<const int8_t*>(g.B);
  const float alpha = g.alpha_a;

  // Staging: a row-major operand (A, or NT's B) moves as 16 lanes x 4 k per
  // row, 16 rows per pass, 8 passes; NN's B as 4 x 4 blocks (16 k-quads x
  // 32 n-quads = 512 blocks, 2 per lane), consecutive lanes on consecutive
  // k-quads so the transposed LDS writes of a wave fill whole rows.
  float4 ra[8], rb[8];
  uint32_t rq[8];  // int8 weights: four levels per register
  auto load_rows = [&](const float* src, size_t rows, size_t r0, size_t k0, float4* dst,
                       bool scale_a) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int r = p * 16 + tid / 16, k4 = (tid % 16) * 4;
      const size_t row = r0 + r, k = k0 + k4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < rows && k < K) {
        v = *reinterpret_cast<const float4*>(src + row * K + k);
        if (scale_a) {
          if (g.a_k_scale) {
            v.x *= g.a_k_scale[k];
            v.y *= g.a_k_scale[k + 1];
            v.z *= g.a_k_scale[k + 2];
            v.w *= g.a_k_scale[k + 3];
          }
          if (alpha != 1.0f) {
            v.x *= alpha;
            v.y *= alpha;
            v.z *= alpha;
            v.w *= alpha;
          }
        }
      }
      dst[p] = v;
    }
  };
  auto load_nn_b = [&](size_t k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int blk = tid + h * kThreads, kq = blk % 16, nq = blk / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t k = k0 + kq * 4 + r, n = n0 + nq * 4;
        rb[h * 4 + r] = (k < K && n < N) ? *reinterpret_cast<const float4*>(B + k * N + n)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto load_q8 = [&](size_t k0) {
    if constexpr (kLayout == 1) {  // rows n of [N, K], four k per lane
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int r = p * 16 + tid / 16, k4 = (tid % 16) * 4;
        const size_t row = n0 + r, k = k0 + k4;
        rq[p] = (row < N && k < K) ? *reinterpret_cast<const uint32_t*>(Bq + row * K + k) : 0u;
      }
    } else {  // 4 x 4 blocks of [K, N]: four k rows of four n
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = tid + h * kThreads, kq = blk % 16, nq = blk / 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t k = k0 + kq * 4 + r, n = n0 + nq * 4;
          rq[h * 4 + r] = (k < K && n < N) ? *reinterpret_cast<const uint32_t*>(Bq + k * N + n) : 0u;
        }
      }
    }
  };
  auto load = [&](size_t k0) {
    load_rows(A, M, m0, k0, ra, true);
    if constexpr (kBKind == 1)
      load_q8(k0);
    else if constexpr (kLayout == 1)
      load_rows(B, N, n0, k0, rb, false);
    else
      load_nn_b(k0);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int r = p * 16 + tid / 16, k4 = (tid % 16) * 4;
      *reinterpret_cast<bf16x4*>(&As[buf][r * LDK + k4]) = ToBf16(ra[p]);
    }
    if constexpr (kBKind == 1 && kLayout == 1) {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int r = p * 16 + tid / 16, k4 = (tid % 16) * 4;
        *reinterpret_cast<bf16x4*>(&Bs[buf][r * LDK + k4]) =
            bf16x4{Level(rq[p], 0), Level(rq[p], 1), Level(rq[p], 2), Level(rq[p], 3)};
      }
    } else if constexpr (kBKind == 1) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = tid + h * kThreads, kq = blk % 16, nq = blk / 16;
#pragma unroll
        for (int c = 0; c < 4; ++c)  // rq[h*4 + r] byte c: k row r, n col c
          *reinterpret_cast<bf16x4*>(&Bs[buf][(nq * 4 + c) * LDK + kq * 4]) =
              bf16x4{Level(rq[h * 4], c), Level(rq[h * 4 + 1], c), Level(rq[h * 4 + 2], c),
                     Level(rq[h * 4 + 3], c)};
      }
    } else if constexpr (kLayout == 1) {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int r = p * 16 + tid / 16, k4 = (tid % 16) * 4;
        *reinterpret_cast<bf16x4*>(&Bs[buf][r * LDK + k4]) = ToBf16(rb[p]);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = tid + h * kThreads, kq = blk % 16, nq = blk / 16;
        const float* f = reinterpret_cast<const float*>(&rb[h * 4]);  // f[4 r + c]: k row r, n col c
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<bf16x4*>(&Bs[buf][(nq * 4 + c) * LDK + kq * 4]) =
              bf16x4{static_cast<__bf16>(f[c]), static_cast<__bf16>(f[4 + c]),
                     static_cast<__bf16>(f[8 + c]), static_cast<__bf16>(f[12 + c])};
      }
    }
  };

  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

  const int c32 = lane % 32, g8 = (lane / 32) * 8;
  const size_t steps = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  for (size_t s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) load((s + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][(wm + i * 32 + c32) * LDK + kk + g8]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(wn + j * 32 + c32) * LDK + kk + g8]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: with the B fragment as the MFMA's first operand, acc[i][j]
  // element 4q + e is C row wm + 32i + lane%32, column wn + 32j + 8q +
  // 4(lane/32) + e: four consecutive columns of one row per (i, j, q).
  const bool vec = N % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(g.C) | reinterpret_cast<uintptr_t>(g.addend)) & 15) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const size_t m = m0 + wm + i * 32 + c32;
        const size_t n = n0 + wn + j * 32 + 8 * q + 4 * (lane / 32);
        if (m >= M || n >= N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[i][j][4 * q + e];
          if (n + e >= N) continue;
          if (kBKind == 1 && g.b_col_scale) v[e] = v[e] * g.b_col_scale[n + e];
          if (g.alpha_dot != 1.0f) v[e] = g.alpha_dot * v[e];
        }
        const size_t o = m * N + n;
        if (vec) {
          if (g.addend) {
            const float4 a4 = *reinterpret_cast<const float4*>(g.addend + o);
            v[0] = a4.x + v[0], v[1] = a4.y + v[1], v[2] = a4.z + v[2], v[3] = a4.w + v[3];
          }
          if (g.accumulate) {
            const float4 c4 = *reinterpret_cast<const float4*>(g.C + o);
            v[0] = c4.x + v[0], v[1] = c4.y + v[1], v[2] = c4.z + v[2], v[3] = c4.w + v[3];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (g.bias) v[e] = v[e] + g.bias[n + e];
            if (g.act) v[e] = ActExpr(g.act, v[e]);
          }
          *reinterpret_cast<float4*>(g.C + o) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e >= N) continue;
            float x = v[e];
            if (g.addend) x = g.addend[o + e] + x;
            if (g.accumulate) x = g.C[o + e] + x;
            if (g.bias) x = x + g.bias[n + e];
            if (g.act) x = ActExpr(g.act, x);
            g.C[o + e] = x;
          }
        }
      }
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool GemmBf16Fits(const GemmArgs& a) {
  if (a.b_kind > 1 || a.layout > 1 || a.M < 64 || a.N < 64 || a.K < 64) return false;
  if (a.K % 4 != 0 || (a.layout == 0 && a.N % 4 != 0)) return false;
  if (!Aligned16(a.A)) return false;
  if (a.b_kind == 0 ? !Aligned16(a.B) : (reinterpret_cast<uintptr_t>(a.B) & 3) != 0) return false;
  const size_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  return tiles < (size_t{1} << 31);
}

hipError_t LaunchGemmBf16(const GemmArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN)));
  switch (a.layout * 2 + a.b_kind) {
    case 0: hipLaunchKernelGGL((GemmBf16Kernel<0, 0>), grid, dim3(kThreads), 0, s, a); break;
    case 1: hipLaunchKernelGGL((GemmBf16Kernel<0, 1>), grid, dim3(kThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((GemmBf16Kernel<1, 0>), grid, dim3(kThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((GemmBf16Kernel<1, 1>), grid, dim3(kThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace seeai
