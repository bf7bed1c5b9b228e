// k_gemm_f32.hip -- the plan's f32-output GEMM family on CDNA4 MFMA
// (runtime/executor/gemm.cc:582-699): kGemmNN / NT / TN / AccNN, the int8-
// weight kGemmNNQ8 / NTQ8 (per-tensor or per-column scales) and the bf16-
// weight kGemmNNBF16 / NTBF16, with the fused epilogues (bias + activation,
// addend, alpha).
//
// One kernel template covers them all.  A BM x BN tile of C per 256-lane
// workgroup (four waves in 2 x 2, each a (BM/2) x (BN/2) block of 16 x 16
// v_mfma_f32_16x16x4_f32 tiles); K walks in steps of 16 through LDS, the
// next step's operands prefetched into registers while the current one
// multiplies.  Operands are staged k-major in LDS (As[k][m], Bs[k][n]), so
// the MFMA operand reads are unit-stride across lanes for every layout.
//
// Where each scale lands is the reference's (instruction.h:396-404,
// gemm.cc:626-674): the NN / TN alpha and the per-tensor q8 scale multiply
// A's elements as they are staged (one rounding each, as the CPU's
// `alpha * a`); a per-column q8 scale multiplies the widened weight; a q8
// k-scale multiplies A's elements; the NT alpha multiplies the finished dot.
// Then C = [D +] dot, and act(C + bias).  The products are exact and the
// MFMA sums them in f32 in its own order, so results agree with the
// reference to rounding (max-rel 1e-5).  This serves the relaxed family
// (kFlagRelaxed) where the bf16 MFMA kernel (k_gemm_bf16.hip: f32 weights,
// tiles of 64 and more) does not; the exact family runs the reference's
// order in k_gemm_exact.hip.
#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;

template <int kLayout, int kBKind>
__device__ __forceinline__ float LoadB(const void* B, size_t N, size_t K, size_t n, size_t k,
                                       const float* col_scale) {
  size_t idx = kLayout == 1 ? n * K + k : k * N + n;
  if constexpr (kBKind == 0) {
    return static_cast<const float*>(B)[idx];
  } else if constexpr (kBKind == 1) {
    const float w = static_cast<float>(static_cast<const int8_t*>(B)[idx]);
    return col_scale ? w * col_scale[n] : w;
  } else {
    return Bf16ToF32(static_cast<const uint16_t*>(B)[idx]);
  }
}

template <int BM, int BN, int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads)
GemmKernel(GemmArgs a) {
  constexpr int WM = BM / 2, WN = BN / 2;       // per-wave block
  constexpr int TM = WM / 16, TN = WN / 16;     // 16x16 MFMA tiles per wave
  constexpr int kAElems = BM * kBK / kThreads;  // staged per lane
  constexpr int kBElems = BN * kBK / kThreads;
  __shared__ float As[kBK][BM + 4];
  __shared__ float Bs[kBK][BN + 4];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int wm = (wave / 2) * WM, wn = (wave % 2) * WN;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * BM;
  const size_t n0 = static_cast<size_t>(blockIdx.x) * BN;
  const size_t M = a.M, N = a.N, K = a.K;
  const float* __restrict__ A = a.A;

  v4f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  float ra[kAElems], rb[kBElems];
  // Element e of this lane's share: A as (m, k) in the tile, B as (k, n).
  auto a_coord = [&](int e, int& mi, int& ki) {
    const int idx = tid + e * kThreads;
    if constexpr (kLayout == 2) {  // A[K, M]: consecutive lanes walk m
      mi = idx % BM;
      ki = idx / BM;
    } else {  // A[M, K]: consecutive lanes walk k
      ki = idx % kBK;
      mi = idx / kBK;
    }
  };
  auto b_coord = [&](int e, int& ki, int& ni) {
    const int idx = tid + e * kThreads;
    if constexpr (kLayout == 1) {  // B[N, K]
      ki = idx % kBK;
      ni = idx / kBK;
    } else {  // B[K, N]
      ni = idx % BN;
      ki = idx / BN;
    }
  };
  auto load = [&](size_t k0) {
#pragma unroll
    for (int e = 0; e < kAElems; ++e) {
      int mi, ki;
      a_coord(e, mi, ki);
      const size_t m = m0 + mi, k = k0 + ki;
      float v = 0.0f;
      if (m < M && k < K) {
        v = kLayout == 2 ? A[k * M + m] : A[m * K + k];
        if (a.a_k_scale) v = v * a.a_k_scale[k];
        v = a.alpha_a * v;
      }
      ra[e] = v;
    }
#pragma unroll
    for (int e = 0; e < kBElems; ++e) {
      int ki, ni;
      b_coord(e, ki, ni);
      const size_t n = n0 + ni, k = k0 + ki;
      rb[e] = (n < N && k < K) ? LoadB<kLayout, kBKind>(a.B, N, K, n, k, a.b_col_scale) : 0.0f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < kAElems; ++e) {
      int mi, ki;
      a_coord(e, mi, ki);
      As[ki][mi] = ra[e];
    }
#pragma unroll
    for (int e = 0; e < kBElems; ++e) {
      int ki, ni;
      b_coord(e, ki, ni);
      Bs[ki][ni] = rb[e];
    }
  };

  load(0);
  for (size_t k0 = 0; k0 < K; k0 += kBK) {
    __syncthreads();
    store();
    __syncthreads();
    if (k0 + kBK < K) load(k0 + kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 4) {
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[kk + lane / 16][wm + i * 16 + lane % 16];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[kk + lane / 16][wn + j * 16 + lane % 16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: lane holds C[4*(lane/16) + r][lane % 16] of each 16x16 tile.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t m = m0 + wm + i * 16 + (lane / 16) * 4 + r;
        const size_t n = n0 + wn + j * 16 + lane % 16;
        if (m >= M || n >= N) continue;
        float v = acc[i][j][r];
        if (a.alpha_dot != 1.0f) v = a.alpha_dot * v;
        const size_t o = m * N + n;
        if (a.addend) v = a.addend[o] + v;
        if (a.accumulate) v = a.C[o] + v;
        if (a.bias) v = v + a.bias[n];
        if (a.act) v = ActExpr(a.act, v);
        a.C[o] = v;
      }
}

template <int BM, int BN, int kLayout, int kBKind>
hipError_t Run(const GemmArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.N + BN - 1) / BN),
                  static_cast<unsigned>((a.M + BM - 1) / BM));
  hipLaunchKernelGGL((GemmKernel<BM, BN, kLayout, kBKind>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

template <int kLayout, int kBKind>
hipError_t Dispatch(const GemmArgs& a, hipStream_t s) {
  // Tile by shape: 128 x 128 once both sides fill it, 32-row tiles for the
  // skinny LoRA products (M or N at the adapter rank).
  if (a.M >= 128 && a.N >= 128) return Run<128, 128, kLayout, kBKind>(a, s);
  if (a.M >= 64 && a.N >= 64) return Run<64, 64, kLayout, kBKind>(a, s);
  return Run<32, 32, kLayout, kBKind>(a, s);
}

}  // namespace

hipError_t LaunchGemm(const GemmArgs& a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  // The extra outputs of the direct-to-LDS kernel's epilogue exist there only.
  if (a.lr_out || a.lr_sink || a.row_max_part) return hipErrorInvalidValue;
  // The exact family keeps the reference's reduction order (bit-exact,
  // k_gemm_exact.hip); MFMA's own summation order is the relaxed family's.
  if (!a.relaxed) return LaunchGemmExact(a, s);
  if (GemmBf16Fits(a)) return LaunchGemmBf16(a, s);
  switch (a.layout * 3 + a.b_kind) {
    case 0: return Dispatch<0, 0>(a, s);
    case 1: return Dispatch<0, 1>(a, s);
    case 2: return Dispatch<0, 2>(a, s);
    case 3: return Dispatch<1, 0>(a, s);
    case 4: return Dispatch<1, 1>(a, s);
    case 5: return Dispatch<1, 2>(a, s);
    case 6: return Dispatch<2, 0>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace seeai
