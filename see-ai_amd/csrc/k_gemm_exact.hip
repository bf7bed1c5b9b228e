// k_gemm_exact.hip -- the exact family's f32-output GEMMs in the
// reference's own reduction order, so every output element is the CPU
// executor's bits (runtime/executor/gemm.cc:73-187, 304-527, 536-699):
//
//   NN / TN / AccNN: C starts at 0 (AccNN: at C); for each k-quad from
//     k = 0,  c += ((a0*b0 + a1*b1) + a2*b2) + a3*b3  with a = alpha*A
//     rounded as staged; then the K % 4 tail, c += a*b one term at a time
//     (gemm.cc:118-182: the quads align to k = 0 because every K tile is a
//     multiple of 4);
//   NT: lane l = k mod 8 accumulates a*b in k order, the eight lanes add
//     in lane order, then alpha multiplies the dot (gemm.cc:341-424);
//   then C = D + C (addend) and C = act(C + bias) (gemm.cc:536-578).
//
// B widens as the reference widens it: int8 exactly, times the column
// scale in one rounding for NN (gemm.cc:96-103); bf16 exactly.  A q8
// k-scale multiplies A as it is staged (gemm.cc:646-674).  Products and
// sums are separate IEEE operations (no contraction: -ffp-contract=off and
// __fmul_rn / __fadd_rn).
//
// Three shapes of kernel share these chains: short K (the whole panel in
// LDS, one output per lane), long K over few outputs (quads formed in
// parallel, folded in order), and the general tiled kernel.
//
// Tiled: a BM x BN tile of C per 256-lane workgroup, each lane a TM x TN
// register block, K walked in steps of 16 through LDS (k-major: As[k][m],
// Bs[k][n]); the next step's operands are loaded into registers while the
// current one accumulates.  Every output has one writer.  The chains are
// VALU multiply-adds (two operations per product), which bounds the kernel
// at half the non-packed f32 VALU rate.
#include "common.h"

namespace seeai {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;

__device__ __forceinline__ float Mul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float Add(float a, float b) { return __fadd_rn(a, b); }

template <int kLayout, int kBKind>
__device__ __forceinline__ float LoadB(const void* B, size_t N, size_t K, size_t n, size_t k,
                                       const float* col_scale) {
  const size_t idx = kLayout == 1 ? n * K + k : k * N + n;
  if constexpr (kBKind == 0) {
    return static_cast<const float*>(B)[idx];
  } else if constexpr (kBKind == 1) {
    const float w = static_cast<float>(static_cast<const int8_t*>(B)[idx]);
    return col_scale ? Mul(w, col_scale[n]) : w;
  } else {
    return Bf16ToF32(static_cast<const uint16_t*>(B)[idx]);
  }
}

// kLayout: 0 NN, 1 NT, 2 TN.  TM x TN outputs per lane; 16 x 16 lanes.
template <int kLayout, int kBKind, int TM, int TN>
__global__ void __launch_bounds__(kThreads) GemmExactKernel(GemmArgs g) {
  constexpr int BM = 16 * TM, BN = 16 * TN;
  constexpr bool kNT = kLayout == 1;
  constexpr int kLanes = kNT ? 8 : 1;  // per-output accumulators
  __shared__ float As[kBK][BM + 4];
  __shared__ float Bs[kBK][BN + 4];
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * BM;
  const size_t n0 = static_cast<size_t>(blockIdx.x) * BN;
  const size_t M = g.M, N = g.N, K = g.K;
  const float* __restrict__ A = g.A;

  float acc[TM][TN][kLanes];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int l = 0; l < kLanes; ++l) acc[i][j][l] = 0.0f;
  if (g.accumulate) {  // GemmAccNN: the chains start at C
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const size_t m = m0 + ty * TM + i, n = n0 + tx * TN + j;
        if (m < M && n < N) acc[i][j][0] = g.C[m * N + n];
      }
  }

  // Staging: each lane loads BM*16/256 A and 16*BN/256 B elements per step.
  constexpr int kAPer = BM * kBK / kThreads, kBPer = BN * kBK / kThreads;
  float ra[kAPer], rb[kBPer];
  auto load = [&](size_t k0) {
#pragma unroll
    for (int e = 0; e < kAPer; ++e) {
      const int idx = tid + e * kThreads;
      int mm, kk;
      if constexpr (kLayout == 2) {  // A[K, M]: m fastest
        mm = idx % BM;
        kk = idx / BM;
      } else {  // A[M, K]: k fastest
        kk = idx % kBK;
        mm = idx / kBK;
      }
      const size_t m = m0 + mm, k = k0 + kk;
      float v = 0.0f;
      if (m < M && k < K) {
        v = kLayout == 2 ? A[k * M + m] : A[m * K + k];
        if (g.a_k_scale) v = Mul(v, g.a_k_scale[k]);
        if (g.alpha_a != 1.0f) v = Mul(g.alpha_a, v);
      }
      ra[e] = v;
    }
#pragma unroll
    for (int e = 0; e < kBPer; ++e) {
      const int idx = tid + e * kThreads;
      int nn, kk;
      if constexpr (kNT) {  // B[N, K]: k fastest
        kk = idx % kBK;
        nn = idx / kBK;
      } else {  // B[K, N]: n fastest
        nn = idx % BN;
        kk = idx / BN;
      }
      const size_t n = n0 + nn, k = k0 + kk;
      rb[e] = (n < N && k < K) ? LoadB<kLayout, kBKind>(g.B, N, K, n, k, g.b_col_scale) : 0.0f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < kAPer; ++e) {
      const int idx = tid + e * kThreads;
      if constexpr (kLayout == 2)
        As[idx / BM][idx % BM] = ra[e];
      else
        As[idx % kBK][idx / kBK] = ra[e];
    }
#pragma unroll
    for (int e = 0; e < kBPer; ++e) {
      const int idx = tid + e * kThreads;
      if constexpr (kNT)
        Bs[idx % kBK][idx / kBK] = rb[e];
      else
        Bs[idx / BN][idx % BN] = rb[e];
    }
  };
  auto frag = [&](int k, float* a, float* b) {
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = As[k][ty * TM + i];
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = Bs[k][tx * TN + j];
  };

  load(0);
  for (size_t k0 = 0; k0 < K; k0 += kBK) {
    __syncthreads();  // the previous step's reads are done
    store();
    __syncthreads();
    if (k0 + kBK < K) load(k0 + kBK);
    const int kn = K - k0 < static_cast<size_t>(kBK) ? static_cast<int>(K - k0) : kBK;
    if constexpr (kNT) {
      // Lane (k mod 8): k0 is a multiple of 16, so the lane is kk % 8.
      if (kn == kBK) {
#pragma unroll
        for (int kk = 0; kk < kBK; ++kk) {
          float a[TM], b[TN];
          frag(kk, a, b);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j][kk % 8] = Add(acc[i][j][kk % 8], Mul(a[i], b[j]));
        }
      } else {
        for (int kk = 0; kk < kn; ++kk) {
          float a[TM], b[TN];
          frag(kk, a, b);
#pragma unroll
          for (int l = 0; l < 8; ++l)
            if ((kk & 7) == l)
#pragma unroll
              for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j][l] = Add(acc[i][j][l], Mul(a[i], b[j]));
        }
      }
    } else {
      const int kq = kn & ~3;  // full quads of this step
#pragma unroll 4
      for (int kk = 0; kk < kq; kk += 4) {
        float a0[TM], a1[TM], a2[TM], a3[TM], b0[TN], b1[TN], b2[TN], b3[TN];
        frag(kk + 0, a0, b0);
        frag(kk + 1, a1, b1);
        frag(kk + 2, a2, b2);
        frag(kk + 3, a3, b3);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const float q = Add(Add(Add(Mul(a0[i], b0[j]), Mul(a1[i], b1[j])), Mul(a2[i], b2[j])),
                                Mul(a3[i], b3[j]));
            acc[i][j][0] = Add(acc[i][j][0], q);
          }
      }
      for (int kk = kq; kk < kn; ++kk) {  // the K % 4 tail, one term at a time
        float a[TM], b[TN];
        frag(kk, a, b);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j][0] = Add(acc[i][j][0], Mul(a[i], b[j]));
      }
    }
  }

  // Epilogue: NT folds its lanes and applies alpha; then addend, bias, act.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const size_t m = m0 + ty * TM + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const size_t n = n0 + tx * TN + j;
      if (n >= N) continue;
      float c = acc[i][j][0];
      if constexpr (kNT) {
#pragma unroll
        for (int l = 1; l < 8; ++l) c = Add(c, acc[i][j][l]);
        c = Mul(g.alpha_dot, c);
      }
      if (g.addend) c = Add(g.addend[m * N + n], c);
      if (g.bias) c = Add(c, g.bias[n]);
      if (g.act) c = ActExpr(g.act, c);
      g.C[m * N + n] = c;
    }
  }
}

// Staged A element (m, k): the q8 k-scale and the NN / TN alpha applied as
// the reference applies them, one rounding each.
template <int kLayout>
__device__ __forceinline__ float LoadA(const GemmArgs& g, size_t m, size_t k) {
  float v = kLayout == 2 ? g.A[k * g.M + m] : g.A[m * g.K + k];
  if (g.a_k_scale) v = Mul(v, g.a_k_scale[k]);
  if (g.alpha_a != 1.0f) v = Mul(g.alpha_a, v);
  return v;
}

// The finished dot of output (m, n) through the epilogue.
__device__ __forceinline__ float Epilogue(const GemmArgs& g, size_t m, size_t n, float c) {
  if (g.addend) c = Add(g.addend[m * g.N + n], c);
  if (g.bias) c = Add(c, g.bias[n]);
  if (g.act) c = ActExpr(g.act, c);
  return c;
}

// ---------------------------------------------------------------------------
// Short reductions (K <= kPanelK): a 16 x 16 block of C per workgroup, one
// output per lane.  Both operand panels -- 16 rows of A and 16 columns of B
// over the whole K -- are loaded into LDS at once (one round trip to
// memory), k-major (As[k][m], Bs[k][n]) so a wave's reads of one k are
// consecutive words; then every lane runs its output's chain.
// ---------------------------------------------------------------------------
constexpr int kPanelK = 512;  // 2 x 16 x 512 floats = the 64 KiB of LDS

template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) GemmPanelKernel(GemmArgs g) {
  constexpr bool kNT = kLayout == 1;
  extern __shared__ float panel[];
  const int K = static_cast<int>(g.K);
  float* As = panel;           // [K][16]
  float* Bs = panel + 16 * K;  // [K][16]
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * 16, n0 = static_cast<size_t>(blockIdx.x) * 16;
  for (int e = tid; e < 16 * K; e += kThreads) {
    int r, k;
    if (kLayout == 2) {  // A[K, M]: m fastest
      r = e % 16;
      k = e / 16;
    } else {             // A[M, K]: k fastest
      r = e / K;
      k = e % K;
    }
    const size_t m = m0 + r;
    As[k * 16 + r] = m < g.M ? LoadA<kLayout>(g, m, k) : 0.0f;
  }
  for (int e = tid; e < 16 * K; e += kThreads) {
    int c, k;
    if (kNT) {  // B[N, K]: k fastest
      c = e / K;
      k = e % K;
    } else {    // B[K, N]: n fastest
      c = e % 16;
      k = e / 16;
    }
    const size_t n = n0 + c;
    Bs[k * 16 + c] = n < g.N ? LoadB<kLayout, kBKind>(g.B, g.N, g.K, n, k, g.b_col_scale) : 0.0f;
  }
  __syncthreads();
  const size_t m = m0 + ty, n = n0 + tx;
  if (m >= g.M || n >= g.N) return;
  auto a = [&](int k) { return As[k * 16 + ty]; };
  auto b = [&](int k) { return Bs[k * 16 + tx]; };
  float c;
  if constexpr (kNT) {
    float lane[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int k = 0;
    for (; k + 8 <= K; k += 8)
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = Add(lane[l], Mul(a(k + l), b(k + l)));
#pragma unroll
    for (int l = 0; l < 8; ++l)
      if (k + l < K) lane[l] = Add(lane[l], Mul(a(k + l), b(k + l)));
    c = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) c = Add(c, lane[l]);
    c = Mul(g.alpha_dot, c);
  } else {
    c = g.accumulate ? g.C[m * g.N + n] : 0.0f;
    int k = 0;
    for (; k + 4 <= K; k += 4)
      c = Add(c, Add(Add(Add(Mul(a(k), b(k)), Mul(a(k + 1), b(k + 1))), Mul(a(k + 2), b(k + 2))),
                     Mul(a(k + 3), b(k + 3))));
    for (; k < K; ++k) c = Add(c, Mul(a(k), b(k)));
  }
  g.C[m * g.N + n] = Epilogue(g, m, n, c);
}

// ---------------------------------------------------------------------------
// Long reductions over few outputs (NN / TN, M*N small, K large: the LoRA
// dA / dB over every token).  A workgroup owns 64 outputs.  K goes by in
// chunks of kChunkQ quads: waves 1-3 form the chunk's quad sums into LDS
// (lane = output, each wave every third quad) while wave 0 adds the
// previous chunk's quads onto each output's chain in k order (double
// buffered).  The quads and their order are the reference's, so the
// result is too.
// ---------------------------------------------------------------------------
constexpr int kChunkQ = 96;

template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) GemmLongKKernel(GemmArgs g) {
  __shared__ float Q[2][kChunkQ][64];
  const int tid = threadIdx.x;
  const size_t total = g.M * g.N;
  const int oi = tid % 64, wave = tid / 64;
  const size_t o = static_cast<size_t>(blockIdx.x) * 64 + oi;
  const bool live = o < total;
  const size_t m = live ? o / g.N : 0, n = live ? o % g.N : 0;
  const size_t quads = g.K / 4;
  const size_t chunks = (quads + kChunkQ - 1) / kChunkQ;
  auto count = [&](size_t ch) {
    const size_t q0 = ch * kChunkQ;
    return static_cast<int>(quads - q0 < static_cast<size_t>(kChunkQ) ? quads - q0 : kChunkQ);
  };
  float c = (g.accumulate && live) ? g.C[m * g.N + n] : 0.0f;
  for (size_t ch = 0; ch <= chunks; ++ch) {
    const int buf = ch & 1;
    if (wave > 0 && ch < chunks) {
      const int nq = count(ch);
      for (int i = wave - 1; i < nq; i += 3) {
        float q = 0.0f;
        if (live) {
          const size_t k = (ch * kChunkQ + i) * 4;
          float p[4];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            p[t] = Mul(LoadA<kLayout>(g, m, k + t), LoadB<kLayout, kBKind>(g.B, g.N, g.K, n, k + t, g.b_col_scale));
          q = Add(Add(Add(p[0], p[1]), p[2]), p[3]);
        }
        Q[buf][i][oi] = q;
      }
    }
    if (wave == 0 && ch > 0) {
      const int nq = count(ch - 1);
      for (int i = 0; i < nq; ++i) c = Add(c, Q[buf ^ 1][i][oi]);
    }
    __syncthreads();
  }
  if (!live || wave != 0) return;
  for (size_t k = quads * 4; k < g.K; ++k)  // the K % 4 tail
    c = Add(c, Mul(LoadA<kLayout>(g, m, k), LoadB<kLayout, kBKind>(g.B, g.N, g.K, n, k, g.b_col_scale)));
  g.C[m * g.N + n] = Epilogue(g, m, n, c);
}

template <int kLayout, int kBKind>
hipError_t Run(const GemmArgs& a, hipStream_t s) {
  if (a.K <= static_cast<size_t>(kPanelK) && a.K > 0 && (a.M + 15) / 16 <= 65535) {
    const dim3 grid(static_cast<unsigned>((a.N + 15) / 16), static_cast<unsigned>((a.M + 15) / 16));
    const size_t lds = 2 * 16 * a.K * sizeof(float);
    hipLaunchKernelGGL((GemmPanelKernel<kLayout, kBKind>), grid, dim3(kThreads), lds, s, a);
    return hipGetLastError();
  }
  if constexpr (kLayout != 1) {
    if (a.M * a.N <= 16384 && a.K >= 1024) {
      const dim3 grid(static_cast<unsigned>((a.M * a.N + 63) / 64));
      hipLaunchKernelGGL((GemmLongKKernel<kLayout, kBKind>), grid, dim3(kThreads), 0, s, a);
      return hipGetLastError();
    }
  }
  constexpr int TM = kLayout == 1 ? 2 : 4, TN = 4;
  if ((a.M + 16 * TM - 1) / (16 * TM) > 65535) return hipErrorInvalidValue;  // grid.y
  const dim3 grid(static_cast<unsigned>((a.N + 16 * TN - 1) / (16 * TN)),
                  static_cast<unsigned>((a.M + 16 * TM - 1) / (16 * TM)));
  hipLaunchKernelGGL((GemmExactKernel<kLayout, kBKind, TM, TN>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t LaunchGemmExact(const GemmArgs& a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  switch (a.layout * 3 + a.b_kind) {
    case 0: return Run<0, 0>(a, s);
    case 1: return Run<0, 1>(a, s);
    case 2: return Run<0, 2>(a, s);
    case 3: return Run<1, 0>(a, s);
    case 4: return Run<1, 1>(a, s);
    case 5: return Run<1, 2>(a, s);
    case 6: return Run<2, 0>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace seeai
