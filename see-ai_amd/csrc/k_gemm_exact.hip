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
#include <cstdlib>

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
// NT over few outputs (the small-batch plans' dX and dt products): the
// reference's eight chains per output (lane l adds the products of k = l
// mod 8 in k order) each get a lane of their own, 32 outputs per workgroup,
// reading A's and B's rows straight from memory (the eight lanes of an
// output read eight consecutive words); the eight chains then add in lane
// order, alpha multiplies, the epilogue follows -- the panel kernel's
// expression, spread over 8 x more lanes.
// ---------------------------------------------------------------------------
template <int kBKind>
__global__ void __launch_bounds__(kThreads) GemmNTLanesKernel(GemmArgs g) {
  __shared__ float part[kThreads];
  const int tid = threadIdx.x, l = tid % 8;
  const size_t o = static_cast<size_t>(blockIdx.x) * (kThreads / 8) + tid / 8;
  const size_t MN = g.M * g.N;
  const bool live = o < MN;
  const size_t m = live ? o / g.N : 0, n = live ? o % g.N : 0;
  float chain = 0.0f;
  if (live)
    for (size_t k = l; k < g.K; k += 8)
      chain = Add(chain, Mul(LoadA<1>(g, m, k), LoadB<1, kBKind>(g.B, g.N, g.K, n, k, g.b_col_scale)));
  part[tid] = chain;
  __syncthreads();
  if (!live || l != 0) return;
  float c = part[tid];
#pragma unroll
  for (int j = 1; j < 8; ++j) c = Add(c, part[tid + j]);
  c = Mul(g.alpha_dot, c);
  g.C[m * g.N + n] = Epilogue(g, m, n, c);
}

// ---------------------------------------------------------------------------
// Rank-r products (K <= 32, f32 B, N % 4 == 0: the LoRA site's s (t B) + C
// and dt A^T + dX, wide outputs over a tiny reduction).  The output and the
// addend are the traffic, so a lane owns four consecutive outputs of one
// row and moves them as 16-byte loads and stores; a workgroup covers 4 rows
// x 256 columns.  A's row (K values, alpha applied as staged) is common to
// the row's 64 lanes; B is small enough to stay in cache.  The chains are
// the reference's: NN / TN / AccNN quads from k = 0 then the tail; NT eight
// lanes by k mod 8, added in lane order, then alpha.
// ---------------------------------------------------------------------------
constexpr int kRankK = 32, kRankRows = 32;

template <int kLayout>
__global__ void __launch_bounds__(kThreads) GemmRankKernel(GemmArgs g) {
  constexpr bool kNT = kLayout == 1;
  __shared__ __attribute__((aligned(16))) float Bt[kRankK][256 + 4];  // B tile as [k][n]
  __shared__ float At[kRankRows][kRankK + 1];                          // A rows, alpha applied
  const size_t M = g.M, N = g.N;
  const int K = static_cast<int>(g.K);
  const int tid = threadIdx.x, tx = tid % 64, ty = tid / 64;
  const size_t n0 = static_cast<size_t>(blockIdx.x) * 256;
  const size_t mb = static_cast<size_t>(blockIdx.y) * kRankRows;
  const float* __restrict__ B = static_cast<const float*>(g.B);
  for (int e = tid; e < kRankRows * K; e += kThreads) {
    const int r = e / K, k = e % K;
    At[r][k] = mb + r < M ? LoadA<kLayout>(g, mb + r, k) : 0.0f;
  }
  for (int e = tid; e < K * 256; e += kThreads) {  // coalesced along B's contiguous index
    int k, nn;
    if constexpr (kNT) {  // B[N, K]
      nn = e / K;
      k = e % K;
    } else {              // B[K, N]
      k = e / 256;
      nn = e % 256;
    }
    const size_t n = n0 + nn;
    Bt[k][nn] = n < N ? (kNT ? B[n * K + k] : B[static_cast<size_t>(k) * N + n]) : 0.0f;
  }
  __syncthreads();
  const size_t n = n0 + tx * 4;
  if (n >= N) return;
  for (int r = 0; r < kRankRows / 4; ++r) {
    const int rr = r * 4 + ty;
    const size_t m = mb + rr;
    if (m >= M) return;
    float c[4];
    if constexpr (kNT) {
      float lane[4][8];
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane[e][l] = 0.0f;
#pragma unroll
      for (int k = 0; k < kRankK; ++k) {
        if (k < K) {
          const float a = At[rr][k];
          const float4 b = *reinterpret_cast<const float4*>(&Bt[k][tx * 4]);
          lane[0][k % 8] = Add(lane[0][k % 8], Mul(a, b.x));
          lane[1][k % 8] = Add(lane[1][k % 8], Mul(a, b.y));
          lane[2][k % 8] = Add(lane[2][k % 8], Mul(a, b.z));
          lane[3][k % 8] = Add(lane[3][k % 8], Mul(a, b.w));
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = lane[e][0];
#pragma unroll
        for (int l = 1; l < 8; ++l) v = Add(v, lane[e][l]);
        c[e] = Mul(g.alpha_dot, v);
      }
    } else {
      if (g.accumulate) {
        const float4 c0 = *reinterpret_cast<const float4*>(g.C + m * N + n);
        c[0] = c0.x, c[1] = c0.y, c[2] = c0.z, c[3] = c0.w;
      } else {
        c[0] = c[1] = c[2] = c[3] = 0.0f;
      }
      const int kq = K & ~3;
#pragma unroll
      for (int k = 0; k < kRankK; k += 4) {
        if (k < kq) {
          float a[4];
          float4 b[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            a[t] = At[rr][k + t];
            b[t] = *reinterpret_cast<const float4*>(&Bt[k + t][tx * 4]);
          }
          c[0] = Add(c[0], Add(Add(Add(Mul(a[0], b[0].x), Mul(a[1], b[1].x)), Mul(a[2], b[2].x)), Mul(a[3], b[3].x)));
          c[1] = Add(c[1], Add(Add(Add(Mul(a[0], b[0].y), Mul(a[1], b[1].y)), Mul(a[2], b[2].y)), Mul(a[3], b[3].y)));
          c[2] = Add(c[2], Add(Add(Add(Mul(a[0], b[0].z), Mul(a[1], b[1].z)), Mul(a[2], b[2].z)), Mul(a[3], b[3].z)));
          c[3] = Add(c[3], Add(Add(Add(Mul(a[0], b[0].w), Mul(a[1], b[1].w)), Mul(a[2], b[2].w)), Mul(a[3], b[3].w)));
        }
      }
#pragma unroll
      for (int k = 0; k < kRankK; ++k) {
        if (k >= kq && k < K) {  // the K % 4 tail
          const float a = At[rr][k];
          const float4 b = *reinterpret_cast<const float4*>(&Bt[k][tx * 4]);
          c[0] = Add(c[0], Mul(a, b.x));
          c[1] = Add(c[1], Mul(a, b.y));
          c[2] = Add(c[2], Mul(a, b.z));
          c[3] = Add(c[3], Mul(a, b.w));
        }
      }
    }
    const size_t o = m * N + n;
    float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g.addend) d = *reinterpret_cast<const float4*>(g.addend + o);
    const float dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = c[e];
      if (g.addend) x = Add(dv[e], x);
      if (g.bias) x = Add(x, g.bias[n + e]);
      if (g.act) x = ActExpr(g.act, x);
      c[e] = x;
    }
    *reinterpret_cast<float4*>(g.C + o) = make_float4(c[0], c[1], c[2], c[3]);
  }
}

bool RankFits(const GemmArgs& a) {
  const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return a.b_kind == 0 && a.K > 0 && a.K <= static_cast<size_t>(kRankK) && a.N % 4 == 0 &&
         a.M >= 64 && a.N >= 256 && al(a.C) && (!a.addend || al(a.addend)) &&
         (a.M + kRankRows - 1) / kRankRows <= 65535;
}

// ---------------------------------------------------------------------------
// Long reductions over few outputs (NN / TN, M*N small, K large: the LoRA
// dA / dB over every token).  A workgroup owns a BMo x BNo block of C (32
// outputs; BNo the largest power of two <= min(N, 32), so slice indices
// are shifts) and walks K in chunks of 128.  Each chunk's
// slices of A (128 x BMo) and B (128 x BNo) are staged through LDS, the next
// chunk's loads in flight while the current one computes; 256 lanes form
// the chunk's 32 quads for each of the 32 outputs, then 32 lanes add them
// onto their output's chain in k order (double-buffered quad store).  The
// quads and their order are the reference's, so the result is too.
// ---------------------------------------------------------------------------
constexpr int kLongOut = 32, kChunkK = 128, kChunkQ = kChunkK / 4;
constexpr int kLongLoads = kChunkK * kLongOut / kThreads;  // 16 per lane, per operand

template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) GemmLongKKernel(GemmArgs g, int lb) {
  __shared__ float As[kChunkK][kLongOut];
  __shared__ float Bs[kChunkK][kLongOut + 1];
  __shared__ float Q[2][kChunkQ][kLongOut + 1];
  const int BNo = 1 << lb, lbm = 5 - lb, BMo = 1 << lbm;  // 32 = 2^5 outputs
  const int tid = threadIdx.x;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * BMo, n0 = static_cast<size_t>(blockIdx.x) * BNo;
  const size_t K = g.K;
  float ra[kLongLoads], rb[kLongLoads];
  // Element e of a staged slice: A as (kk, mm), B as (kk, nn).
  auto a_of = [&](int e, int& kk, int& mm) {
    if (kLayout == 2) {  // A[K, M]: the slice's rows are short, k outer
      kk = e >> lbm;
      mm = e & (BMo - 1);
    } else {             // A[M, K]: k inner
      mm = e / kChunkK;
      kk = e % kChunkK;
    }
  };
  auto load = [&](size_t k0) {
#pragma unroll
    for (int r = 0; r < kLongLoads; ++r) {
      const int e = tid + r * kThreads;
      float va = 0.0f, vb = 0.0f;
      if (e < kChunkK * BMo) {
        int kk, mm;
        a_of(e, kk, mm);
        const size_t k = k0 + kk, m = m0 + mm;
        if (k < K && m < g.M) va = LoadA<kLayout>(g, m, k);
      }
      if (e < kChunkK * BNo) {
        const int kk = e >> lb, nn = e & (BNo - 1);
        const size_t k = k0 + kk, n = n0 + nn;
        if (k < K && n < g.N) vb = LoadB<kLayout, kBKind>(g.B, g.N, K, n, k, g.b_col_scale);
      }
      ra[r] = va;
      rb[r] = vb;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int r = 0; r < kLongLoads; ++r) {
      const int e = tid + r * kThreads;
      if (e < kChunkK * BMo) {
        int kk, mm;
        a_of(e, kk, mm);
        As[kk][mm] = ra[r];
      }
      if (e < kChunkK * BNo) Bs[e >> lb][e & (BNo - 1)] = rb[r];
    }
  };
  // This lane's quads: output i (mm = i / BNo, nn = i % BNo), quads j, j+8, ...
  const int i = tid % kLongOut, j0 = tid / kLongOut;
  const int mm = i >> lb, nn = i & (BNo - 1);
  const size_t quads = K / 4;
  const size_t chunks = (quads + kChunkQ - 1) / kChunkQ;
  const size_t mf = m0 + (tid >> lb), nf = n0 + (tid & (BNo - 1));  // the folding lane's output
  const bool folds = tid < kLongOut && mf < g.M && nf < g.N;
  float c = (folds && g.accumulate) ? g.C[mf * g.N + nf] : 0.0f;
  load(0);
  for (size_t ch = 0; ch <= chunks; ++ch) {
    const int buf = ch & 1;
    if (ch < chunks) {
      __syncthreads();  // the previous chunk's As / Bs reads are done
      store();
      __syncthreads();
      if (ch + 1 < chunks) load((ch + 1) * kChunkK);
      const size_t q0 = ch * kChunkQ;
      const int nq = static_cast<int>(quads - q0 < static_cast<size_t>(kChunkQ) ? quads - q0 : kChunkQ);
      for (int j = j0; j < nq; j += kThreads / kLongOut) {
        const int k = 4 * j;
        const float p0 = Mul(As[k][mm], Bs[k][nn]), p1 = Mul(As[k + 1][mm], Bs[k + 1][nn]);
        const float p2 = Mul(As[k + 2][mm], Bs[k + 2][nn]), p3 = Mul(As[k + 3][mm], Bs[k + 3][nn]);
        Q[buf][j][i] = Add(Add(Add(p0, p1), p2), p3);
      }
    }
    if (ch > 0 && folds) {  // the previous chunk, in k order
      const size_t q0 = (ch - 1) * kChunkQ;
      const int nq = static_cast<int>(quads - q0 < static_cast<size_t>(kChunkQ) ? quads - q0 : kChunkQ);
      for (int j = 0; j < nq; ++j) c = Add(c, Q[buf ^ 1][j][tid]);
    }
  }
  if (!folds) return;
  for (size_t k = quads * 4; k < K; ++k)  // the K % 4 tail
    c = Add(c, Mul(LoadA<kLayout>(g, mf, k), LoadB<kLayout, kBKind>(g.B, g.N, K, nf, k, g.b_col_scale)));
  g.C[mf * g.N + nf] = Epilogue(g, mf, nf, c);
}

// ---------------------------------------------------------------------------
// Long reductions with a workspace: the same chains in two passes.  Pass 1
// forms every quad sum, fully parallel (lane = output, four consecutive
// quads per lane), into Q[o][j] (output-major); pass 2 gives each output one
// lane that adds its quads in k order, reading them sixteen bytes at a time.
// ---------------------------------------------------------------------------
template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) LongKQuadsKernel(GemmArgs g, unsigned quads4) {
  const unsigned MN = static_cast<unsigned>(g.M * g.N), N = static_cast<unsigned>(g.N);
  const unsigned o = blockIdx.x * kThreads + threadIdx.x;
  if (o >= MN) return;
  const size_t m = o / N, n = o % N, Q = g.K / 4;
  for (unsigned jq = blockIdx.y; jq < quads4; jq += gridDim.y) {
    float q[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const size_t j = static_cast<size_t>(jq) * 4 + t;
      float v = 0.0f;
      if (j < Q) {
        const size_t k = j * 4;
        float p[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          p[u] = Mul(LoadA<kLayout>(g, m, k + u), LoadB<kLayout, kBKind>(g.B, g.N, g.K, n, k + u, g.b_col_scale));
        v = Add(Add(Add(p[0], p[1]), p[2]), p[3]);
      }
      q[t] = v;
    }
    *reinterpret_cast<float4*>(g.scratch + static_cast<size_t>(o) * quads4 * 4 + static_cast<size_t>(jq) * 4) =
        make_float4(q[0], q[1], q[2], q[3]);
  }
}

template <int kLayout, int kBKind>
__global__ void __launch_bounds__(kThreads) LongKFoldKernel(GemmArgs g, unsigned quads4) {
  const unsigned MN = static_cast<unsigned>(g.M * g.N);
  const unsigned o = blockIdx.x * kThreads + threadIdx.x;
  if (o >= MN) return;
  const size_t m = o / g.N, n = o % g.N, Q = g.K / 4;
  float c = g.accumulate ? g.C[o] : 0.0f;
  const float4* qs = reinterpret_cast<const float4*>(g.scratch + static_cast<size_t>(o) * quads4 * 4);
  const size_t full = Q / 4;
#pragma unroll 8
  for (size_t jq = 0; jq < full; ++jq) {
    const float4 v = qs[jq];
    c = Add(Add(Add(Add(c, v.x), v.y), v.z), v.w);
  }
  for (size_t j = full * 4; j < Q; ++j) c = Add(c, g.scratch[static_cast<size_t>(o) * quads4 * 4 + j]);
  for (size_t k = Q * 4; k < g.K; ++k)  // the K % 4 tail
    c = Add(c, Mul(LoadA<kLayout>(g, m, k), LoadB<kLayout, kBKind>(g.B, g.N, g.K, n, k, g.b_col_scale)));
  g.C[o] = Epilogue(g, m, n, c);
}

// ---------------------------------------------------------------------------
// Long reductions over a few hundred thousand outputs or fewer (the LoRA
// products t = X A, dt = dC B^T and the adapter gradients dA = X^T dt,
// dB = t^T dC): one output per lane, BM x BN = 256 outputs per workgroup,
// so the grid has M N / 256 workgroups where the tiled kernel would have
// M N / 4096.  K walks in chunks of kChainK through two LDS buffers, stored
// k-contiguous per row (As[m][k], Bs[n][k]) so a lane reads a quad of A and
// of B as one 16-byte read each.  With one output per lane there are few
// waves to hide memory latency, so the loads run kChainDepth chunks ahead
// of the chunk being reduced (a chunk of 256 holds more arithmetic than
// one load round trip), in a ring of registers; one barrier per
// chunk.  The chains are the tiled kernel's: quads from k = 0 then the
// K % 4 tail (NN / TN / AccNN), or eight lanes by k mod 8 added in lane
// order then alpha (NT).
// ---------------------------------------------------------------------------
constexpr int kChainK = 128, kChainLd = kChainK + 4, kChainDepth = 2;

// s_waitcnt vmcnt(0), the other counters untouched (gfx9 encoding).
__device__ __forceinline__ void WaitVmAll() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

template <int kLayout, int kBKind, int BM, int BN>
__global__ void __launch_bounds__(kThreads) GemmChainKernel(GemmArgs g) {
  static_assert(BM * BN == kThreads, "one output per lane");
  constexpr bool kNT = kLayout == 1;
  constexpr int kAPer = BM * kChainK / kThreads, kBPer = BN * kChainK / kThreads;
  __shared__ __attribute__((aligned(16))) float As[2][BM][kChainLd];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN][kChainLd];
  const int tid = threadIdx.x;
  const int mi = tid / BN, ni = tid % BN;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * BM, n0 = static_cast<size_t>(blockIdx.x) * BN;
  const size_t M = g.M, N = g.N, K = g.K;
  // Element e of a chunk: A's (mm, kk) with the contiguous index fastest.
  auto a_of = [&](int e, int& mm, int& kk) {
    if constexpr (kLayout == 2) {  // A[K, M]
      kk = e / BM;
      mm = e % BM;
    } else {                       // A[M, K]
      mm = e / kChainK;
      kk = e % kChainK;
    }
  };
  auto b_of = [&](int e, int& nn, int& kk) {
    if constexpr (kNT) {           // B[N, K]
      nn = e / kChainK;
      kk = e % kChainK;
    } else {                       // B[K, N]
      kk = e / BN;
      nn = e % BN;
    }
  };
  // The ring holds the operands as loaded (A as floats, B as raw bits):
  // a value the lane does not touch until it is stored needs no wait for
  // its load.  Loads are branch-free (indices clamped into the operand; a
  // branch around a load makes the compiler wait for every load at the
  // join); out-of-range elements become zero at the store, where the scales
  // (alpha, the q8 k- and column scales) and the widening also apply, in
  // the order LoadA / LoadB apply them.
  constexpr bool kKScale = kLayout == 1 && kBKind == 1;  // NT q8: k-scale on A
  constexpr bool kColScale = kLayout != 1 && kBKind == 1;  // NN q8: column scale on B
  float ra[kChainDepth][kAPer];
  uint32_t rb[kChainDepth][kBPer];
  auto load = [&](size_t k0, float* dra, uint32_t* drb) {
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      int mm, kk;
      a_of(tid + r * kThreads, mm, kk);
      const size_t m = min(m0 + mm, M - 1), k = min(k0 + kk, K - 1);
      dra[r] = kLayout == 2 ? g.A[k * M + m] : g.A[m * K + k];
    }
#pragma unroll
    for (int r = 0; r < kBPer; ++r) {
      int nn, kk;
      b_of(tid + r * kThreads, nn, kk);
      const size_t n = min(n0 + nn, N - 1), k = min(k0 + kk, K - 1);
      const size_t idx = kNT ? n * K + k : k * N + n;
      if constexpr (kBKind == 0)
        drb[r] = __float_as_uint(static_cast<const float*>(g.B)[idx]);
      else if constexpr (kBKind == 1)
        drb[r] = static_cast<uint32_t>(static_cast<int32_t>(static_cast<const int8_t*>(g.B)[idx]));
      else
        drb[r] = static_cast<const uint16_t*>(g.B)[idx];
    }
  };
  auto store = [&](int buf, size_t k0, const float* sra, const uint32_t* srb) {
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      int mm, kk;
      a_of(tid + r * kThreads, mm, kk);
      const size_t k = k0 + kk;
      float v = sra[r];
      if constexpr (kKScale)
        if (g.a_k_scale) v = Mul(v, g.a_k_scale[min(k, K - 1)]);
      if (g.alpha_a != 1.0f) v = Mul(g.alpha_a, v);
      As[buf][mm][kk] = (m0 + mm < M && k < K) ? v : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < kBPer; ++r) {
      int nn, kk;
      b_of(tid + r * kThreads, nn, kk);
      const size_t n = n0 + nn, k = k0 + kk;
      float v;
      if constexpr (kBKind == 0) {
        v = __uint_as_float(srb[r]);
      } else if constexpr (kBKind == 1) {
        v = static_cast<float>(static_cast<int32_t>(srb[r]));
        if constexpr (kColScale)
          if (g.b_col_scale) v = Mul(v, g.b_col_scale[min(n, N - 1)]);
      } else {
        v = Bf16ToF32(static_cast<uint16_t>(srb[r]));
      }
      Bs[buf][nn][kk] = (n < N && k < K) ? v : 0.0f;
    }
  };
  const size_t m = m0 + mi, n = n0 + ni;
  const bool live = m < M && n < N;
  float c = (live && g.accumulate) ? g.C[m * N + n] : 0.0f;
  float lane[kNT ? 8 : 1];
#pragma unroll
  for (int l = 0; l < (kNT ? 8 : 1); ++l) lane[l] = 0.0f;
  auto reduce = [&](int buf, int kn) {
    const float* ar = As[buf][mi];
    const float* br = Bs[buf][ni];
    if constexpr (kNT) {
      if (kn == kChainK) {
#pragma unroll 8
        for (int kk = 0; kk < kChainK; kk += 4) {  // k0 is a multiple of 8: lane = kk % 8 + t
          const float4 a = *reinterpret_cast<const float4*>(ar + kk);
          const float4 b = *reinterpret_cast<const float4*>(br + kk);
          const int l = kk % 8;
          lane[l] = Add(lane[l], Mul(a.x, b.x));
          lane[l + 1] = Add(lane[l + 1], Mul(a.y, b.y));
          lane[l + 2] = Add(lane[l + 2], Mul(a.z, b.z));
          lane[l + 3] = Add(lane[l + 3], Mul(a.w, b.w));
        }
      } else {
        for (int kk = 0; kk < kn; ++kk)
#pragma unroll
          for (int l = 0; l < 8; ++l)
            if ((kk & 7) == l) lane[l] = Add(lane[l], Mul(ar[kk], br[kk]));
      }
    } else {
      // One loop for full and partial chunks.  (A copy of this loop
      // unrolled for full chunks, next to it for a partial last chunk,
      // gave wrong sums when the last chunk held whole quads -- K = 520,
      // 600 -- while each form alone was exact for every K tried; kept to
      // the single loop.)
      const int kq = kn & ~3;
      for (int kk = 0; kk < kq; kk += 4) {
        const float4 a = *reinterpret_cast<const float4*>(ar + kk);
        const float4 b = *reinterpret_cast<const float4*>(br + kk);
        c = Add(c, Add(Add(Add(Mul(a.x, b.x), Mul(a.y, b.y)), Mul(a.z, b.z)), Mul(a.w, b.w)));
      }
      for (int kk = kq; kk < kn; ++kk) c = Add(c, Mul(ar[kk], br[kk]));  // the K % 4 tail
    }
  };
  const size_t chunks = (K + kChainK - 1) / kChainK;
  // The compiler places each store's wait by counting the loads issued
  // after the ring slot's own: kChainDepth - 1 chunks of them in the steady
  // state.  Near the end fewer follow (no chunk to load), so there the
  // store waits for every load itself.  (Loads past the end are not issued
  // instead: registers of a load nothing reads are taken as free while the
  // load is still in flight.)
  // Prologue: chunks 0 .. depth-1 in flight, chunk 0 stored.
#pragma unroll
  for (int u = 0; u < kChainDepth; ++u)
    if (static_cast<size_t>(u) < chunks) load(static_cast<size_t>(u) * kChainK, ra[u], rb[u]);
  WaitVmAll();
  store(0, 0, ra[0], rb[0]);
  if (static_cast<size_t>(kChainDepth) < chunks)
    load(static_cast<size_t>(kChainDepth) * kChainK, ra[0], rb[0]);
  __syncthreads();
  // Chunk i sits in LDS buffer i & 1 and came from ring slot i % depth; the
  // ring slot of chunk i + 1 is stored after chunk i is reduced and then
  // refilled with chunk i + 1 + depth.  The loop is unrolled by the ring
  // depth so every slot index is a constant.
  for (size_t i0 = 0; i0 < chunks; i0 += kChainDepth) {
#pragma unroll
    for (int u = 0; u < kChainDepth; ++u) {
      const size_t i = i0 + u;
      if (i < chunks) {
        const size_t k0 = i * kChainK;
        const int kn = K - k0 < static_cast<size_t>(kChainK) ? static_cast<int>(K - k0) : kChainK;
        reduce(static_cast<int>(i & 1), kn);
        const int nx = (u + 1) % kChainDepth;  // a constant once unrolled
        if (i + 1 < chunks) {
          if (i + kChainDepth >= chunks) WaitVmAll();  // fewer loads follow this slot's
          store(static_cast<int>((i + 1) & 1), (i + 1) * kChainK, ra[nx], rb[nx]);
          if (i + 1 + kChainDepth < chunks) load((i + 1 + kChainDepth) * kChainK, ra[nx], rb[nx]);
        }
        __syncthreads();
      }
    }
  }
  if (!live) return;
  if constexpr (kNT) {
    c = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) c = Add(c, lane[l]);
    c = Mul(g.alpha_dot, c);
  }
  g.C[m * N + n] = Epilogue(g, m, n, c);
}

// ---------------------------------------------------------------------------
// NT over N <= 16 outputs per row and a long K (the LoRA dt = dC B^T): the
// reference's eight chains of an output (lane l takes every k = l mod 8, in
// k order) sit in eight GPU lanes, each lane running its chain for eight
// outputs of kRL rows at once, so one read of A[m][k] feeds eight products
// and one read of B's eight values (a row of a k-major tile that every lane
// of the same l reads together) feeds 8 kRL.  A wave holds 8 kRL rows x 8
// chains for one group of eight outputs; a workgroup 32 kRL / kNG rows x kNG
// groups.  A is staged row-major and B transposed (Bs[k][n]) through two LDS
// buffers, chunk by chunk, the next chunk's loads in flight while one is
// reduced.  At the end each
// output's eight chain values are added in lane order (lane 0 first) and
// multiplied by alpha, then the epilogue: the chain kernel's bits.
// ---------------------------------------------------------------------------
template <int kNG, int kRL, int kKLChunk>
__global__ void __launch_bounds__(kThreads) GemmNTKLaneKernel(GemmArgs g) {
  // kRL rows per lane: lane (r8, l) of a wave runs rows r8 + 8 r (r < kRL).
  constexpr int kRows = 32 * kRL / kNG, kN = 8 * kNG, kKLLdA = kKLChunk + 8;
  constexpr int kAPer = kRows * kKLChunk / 4 / kThreads;  // float4 of A per thread and chunk
  static_assert(kAPer * 4 * kThreads == kRows * kKLChunk, "A loads cover the chunk");
  static_assert(kKLChunk <= kThreads, "one k per thread for B");
  __shared__ __attribute__((aligned(16))) float As[2][kRows][kKLLdA];
  __shared__ __attribute__((aligned(16))) float Bs[2][kKLChunk][kN];
  __shared__ __attribute__((aligned(16))) float Red[kRows][kN][8];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int l = lane % 8, ng = wave % kNG, rbase = (wave / kNG) * 8 * kRL + lane / 8;
  const size_t M = g.M, N = g.N, K = g.K;
  const size_t m0 = static_cast<size_t>(blockIdx.x) * kRows;
  const float* __restrict__ A = g.A;
  const float* __restrict__ B = static_cast<const float*>(g.B);
  float4 ra[kAPer];
  float rb[kN];
  auto load = [&](size_t k0) {
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      const int f = tid + r * kThreads, row = f / (kKLChunk / 4), c4 = f % (kKLChunk / 4);
      const size_t m = min(m0 + row, M - 1), k = min(k0 + 4 * c4, K - 4);
      ra[r] = *reinterpret_cast<const float4*>(A + m * K + k);
    }
    if (tid < kKLChunk) {
      const size_t k = min(k0 + tid, K - 1);
#pragma unroll
      for (int n = 0; n < kN; ++n) rb[n] = B[min(static_cast<size_t>(n), N - 1) * K + k];
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      const int f = tid + r * kThreads, row = f / (kKLChunk / 4), c4 = f % (kKLChunk / 4);
      float4 v = ra[r];
      if (g.alpha_a != 1.0f)
        v = make_float4(Mul(g.alpha_a, v.x), Mul(g.alpha_a, v.y), Mul(g.alpha_a, v.z),
                        Mul(g.alpha_a, v.w));
      *reinterpret_cast<float4*>(&As[buf][row][4 * c4]) = v;
    }
    if (tid < kKLChunk) {
#pragma unroll
      for (int n4 = 0; n4 < kN / 4; ++n4) {
        float4 v = make_float4(rb[4 * n4], rb[4 * n4 + 1], rb[4 * n4 + 2], rb[4 * n4 + 3]);
        if (static_cast<size_t>(4 * n4 + 3) >= N) {  // outputs past N: zeros
          if (static_cast<size_t>(4 * n4) >= N) v.x = 0.0f;
          if (static_cast<size_t>(4 * n4 + 1) >= N) v.y = 0.0f;
          if (static_cast<size_t>(4 * n4 + 2) >= N) v.z = 0.0f;
          v.w = 0.0f;
        }
        *reinterpret_cast<float4*>(&Bs[buf][tid][4 * n4]) = v;
      }
    }
  };
  float acc[kRL][8];
#pragma unroll
  for (int r = 0; r < kRL; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[r][j] = 0.0f;
  auto step = [&](int buf, int k) {
    const float4 b0 = *reinterpret_cast<const float4*>(&Bs[buf][k][8 * ng]);
    const float4 b1 = *reinterpret_cast<const float4*>(&Bs[buf][k][8 * ng + 4]);
    const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int r = 0; r < kRL; ++r) {
      const float a = As[buf][rbase + 8 * r][k];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r][j] = Add(acc[r][j], Mul(a, b[j]));
    }
  };
  const size_t chunks = (K + kKLChunk - 1) / kKLChunk;
  load(0);
  store(0);
  if (chunks > 1) load(kKLChunk);
  __syncthreads();
  for (size_t i = 0; i < chunks; ++i) {
    const int buf = static_cast<int>(i & 1);
    const size_t k0 = i * kKLChunk;
    const int kn = K - k0 < static_cast<size_t>(kKLChunk) ? static_cast<int>(K - k0) : kKLChunk;
    if (kn == kKLChunk) {
#pragma unroll 4
      for (int k = l; k < kKLChunk; k += 8) step(buf, k);
    } else {
      for (int k = l; k < kn; k += 8) step(buf, k);
    }
    if (i + 1 < chunks) {
      store(buf ^ 1);
      if (i + 2 < chunks) load(k0 + 2 * kKLChunk);
    }
    __syncthreads();
  }
  // Each output's chains in lane order: lane l of a row adds output 8 ng + l.
#pragma unroll
  for (int r = 0; r < kRL; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) Red[rbase + 8 * r][8 * ng + j][l] = acc[r][j];
  __builtin_amdgcn_wave_barrier();
  const size_t n = static_cast<size_t>(8 * ng + l);
#pragma unroll
  for (int r = 0; r < kRL; ++r) {
    const int mi = rbase + 8 * r;
    const size_t m = m0 + mi;
    const float4 c0 = *reinterpret_cast<const float4*>(&Red[mi][n][0]);
    const float4 c1 = *reinterpret_cast<const float4*>(&Red[mi][n][4]);
    float c = c0.x;
    c = Add(c, c0.y), c = Add(c, c0.z), c = Add(c, c0.w);
    c = Add(c, c1.x), c = Add(c, c1.y), c = Add(c, c1.z), c = Add(c, c1.w);
    c = Mul(g.alpha_dot, c);
    if (m < M && n < N) g.C[m * N + n] = Epilogue(g, m, n, c);
  }
}

// ---------------------------------------------------------------------------
// Long reductions over few outputs, NN / TN (the adapter gradients
// dA = X^T dt and dB = s t^T dC over every token): the quads of a chunk are
// independent, only their sum into the output is a chain.  A workgroup owns
// 64 outputs (BMo x BNo) and walks K in chunks of kFoldK: four lanes per
// output form the chunk's quads ((a0 b0 + a1 b1) + a2 b2) + a3 b3 into LDS,
// then one lane per output adds them onto its output in k order -- the
// reference's chain, with four times the lanes of one output per lane.  The
// operands are staged k-contiguous per row (a quad is one 16-byte read of
// A and of B); the next chunk's raw loads are in flight while the current
// one is reduced, its scales applied at the store.
// ---------------------------------------------------------------------------
constexpr int kFoldK = 512, kFoldQ = kFoldK / 4, kFoldOut = 64, kFoldLd = kFoldK + 4;

template <int kLayout, int BNo>
__global__ void __launch_bounds__(kThreads) GemmFoldKernel(GemmArgs g) {
  static_assert(kLayout != 1, "NT keeps its eight k-lanes");
  constexpr int BMo = kFoldOut / BNo;
  constexpr int kAPer = BMo * kFoldK / kThreads, kBPer = BNo * kFoldK / kThreads;
  static_assert(kAPer * kThreads == BMo * kFoldK && kBPer * kThreads == BNo * kFoldK,
                "every chunk element has a lane");
  __shared__ __attribute__((aligned(16))) float As[BMo][kFoldLd];
  __shared__ __attribute__((aligned(16))) float Bs[BNo][kFoldLd];
  __shared__ float Q[kFoldQ][kFoldOut + 1];
  const int tid = threadIdx.x;
  const size_t M = g.M, N = g.N, K = g.K;
  // Workgroup b runs on XCD b % 8, each XCD with its own L2.  A workgroup
  // reads BMo- and BNo-wide strips of rows far longer than a cache line, so
  // the strips of neighbouring workgroups share lines: each XCD takes a
  // contiguous run of blocks, and a line leaves HBM once instead of once
  // per XCD.
  const unsigned total = gridDim.x * gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
  const unsigned t = total % 8 == 0 ? (lin % 8) * (total / 8) + lin / 8 : lin;
  const size_t m0 = static_cast<size_t>(t / gridDim.x) * BMo, n0 = static_cast<size_t>(t % gridDim.x) * BNo;
  const float* __restrict__ B = static_cast<const float*>(g.B);
  // Chunk element e: A's (mm, kk), B's (nn, kk), the contiguous index fastest.
  auto a_of = [&](int e, int& mm, int& kk) {
    if constexpr (kLayout == 2) {  // A[K, M]
      kk = e / BMo;
      mm = e % BMo;
    } else {                       // A[M, K]
      mm = e / kFoldK;
      kk = e % kFoldK;
    }
  };
  auto b_of = [&](int e, int& nn, int& kk) {  // B[K, N]
    kk = e / BNo;
    nn = e % BNo;
  };
  float ra[kAPer], rb[kBPer];
  auto load = [&](size_t k0) {  // raw and branch-free: indices clamped into the operand
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      int mm, kk;
      a_of(tid + r * kThreads, mm, kk);
      const size_t m = min(m0 + mm, M - 1), k = min(k0 + kk, K - 1);
      ra[r] = kLayout == 2 ? g.A[k * M + m] : g.A[m * K + k];
    }
#pragma unroll
    for (int r = 0; r < kBPer; ++r) {
      int nn, kk;
      b_of(tid + r * kThreads, nn, kk);
      const size_t n = min(n0 + nn, N - 1), k = min(k0 + kk, K - 1);
      rb[r] = B[k * N + n];
    }
  };
  auto store = [&](size_t k0) {
#pragma unroll
    for (int r = 0; r < kAPer; ++r) {
      int mm, kk;
      a_of(tid + r * kThreads, mm, kk);
      float v = ra[r];
      if (g.alpha_a != 1.0f) v = Mul(g.alpha_a, v);
      As[mm][kk] = (m0 + mm < M && k0 + kk < K) ? v : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < kBPer; ++r) {
      int nn, kk;
      b_of(tid + r * kThreads, nn, kk);
      Bs[nn][kk] = (n0 + nn < N && k0 + kk < K) ? rb[r] : 0.0f;
    }
  };
  const int o = tid % kFoldOut, slot = tid / kFoldOut;  // this lane's output and quad slot
  const int mo = o / BNo, no = o % BNo;
  const size_t mf = m0 + mo, nf = n0 + no;
  const bool folds = tid < kFoldOut && mf < M && nf < N;
  float c = (folds && g.accumulate) ? g.C[mf * N + nf] : 0.0f;
  const size_t quads = K / 4;
  const size_t chunks = (quads + kFoldQ - 1) / kFoldQ;
  load(0);
  for (size_t ch = 0; ch < chunks; ++ch) {
    const size_t k0 = ch * kFoldK;
    __syncthreads();  // the previous chunk's As / Bs / Q reads are done
    if (ch + 1 == chunks) WaitVmAll();  // no loads follow this chunk's (see GemmChainKernel)
    store(k0);
    __syncthreads();
    if (ch + 1 < chunks) load(k0 + kFoldK);
    const int nq = static_cast<int>(quads - ch * kFoldQ < static_cast<size_t>(kFoldQ) ? quads - ch * kFoldQ : kFoldQ);
    for (int j = slot; j < nq; j += kThreads / kFoldOut) {
      const float4 a = *reinterpret_cast<const float4*>(&As[mo][4 * j]);
      const float4 b = *reinterpret_cast<const float4*>(&Bs[no][4 * j]);
      Q[j][o] = Add(Add(Add(Mul(a.x, b.x), Mul(a.y, b.y)), Mul(a.z, b.z)), Mul(a.w, b.w));
    }
    __syncthreads();
    if (folds)
      for (int j = 0; j < nq; ++j) c = Add(c, Q[j][o]);
  }
  if (!folds) return;
  for (size_t k = quads * 4; k < K; ++k)  // the K % 4 tail, one term at a time
    c = Add(c, Mul(LoadA<kLayout>(g, mf, k), B[k * N + nf]));
  g.C[mf * N + nf] = Epilogue(g, mf, nf, c);
}

// The fold kernel with its waves split by role (TN or NN, f32 operands
// 16-byte aligned, M % BMo == N % BNo == 0, K * M and K * N below 2^31, NN
// with K % 4 == 0, no q8 k-scale): the chain of each output is a strict
// sequence of adds, so one
// wave does nothing but fold -- kF outputs per lane, their chains
// interleaved -- while the other kW - 1 waves load, stage and form the
// quads.  Operands and quads are double-buffered, one barrier per interval:
// in interval i the producers form chunk i's quads (QM x QN output blocks
// per task, written k-contiguous per output, Q[o][j]) and stage chunk i + 1
// from a ring of kD register slots that runs kD chunks ahead, while the
// folder adds chunk i - 1's quads, reading four of them per 16-byte read.
// A and B are staged in rounds of their own (whole wave-uniform loads, the
// last round's spare lanes re-reading the last element), and the steady
// state issues its loads unconditionally -- with the folder's loop apart
// from the producers' there is no join in it, so each store waits for its
// own slot's loads and no more; the last intervals wait for every load.
// Rows past K are clamped reads: they meet only quads past K / 4, which are
// never folded.  The sums are GemmFoldKernel's, operation for operation.
//
// A is staged k-contiguous per output row: TN's A [K, M] transposed on the
// way in, NN's A [M, K] as it lies (16-byte row segments).
//
// LDS layout (64 banks of 4 bytes): a wave's transposed stores put lanes f
// at (row 4 (f % W) + t, column f / W), W = BMo / 4 or BNo / 4, so the row
// stride is padded to 8 (mod 16) floats for W = 2 and 4 (mod 16) otherwise,
// which spreads the W row groups over disjoint banks; a producer task takes
// the quad index fastest, so a wave's quad writes and operand reads walk
// consecutive columns of one block (conflict-free whatever the strides).
//
// The body takes its block of the product's grid (gx blocks across N, block
// `lin` of `total`) as arguments, so one launch can run two products.
template <int kLayout, int BMo, int BNo, int kKc, int kD, int QM, int QN, int kW, int kF>
__device__ __forceinline__ void FoldSplitBody(const GemmArgs& g, unsigned gx, unsigned lin,
                                              unsigned total) {
  static_assert(kLayout == 0 || kLayout == 2, "NN or TN");
  constexpr bool kTN = kLayout == 2;
  constexpr int kOut = BMo * BNo, kQc = kKc / 4, kQLd = kQc + 4;
  constexpr int kLdA = kKc + (kTN && BMo / 4 == 2 ? 8 : 4), kLdB = kKc + (BNo / 4 == 2 ? 8 : 4);
  static_assert(kOut == 64 * kF || (kF == 1 && kOut < 64), "kF outputs per folder lane");
  constexpr int kP = 64 * (kW - 1);  // producer lanes
  constexpr int kAf = kKc * BMo / 4, kBf = kKc * BNo / 4;  // float4 per chunk
  constexpr int kRA = (kAf + kP - 1) / kP, kRB = (kBf + kP - 1) / kP;
  constexpr int kBlkN = BNo / QN, kBlk = (BMo / QM) * kBlkN, kTasks = kBlk * kQc;
  constexpr int kT = (kTasks + kP - 1) / kP;
  static_assert(BMo % QM == 0 && BNo % QN == 0 && QM % 4 == 0 && QN % 4 == 0, "whole blocks");
  __shared__ __attribute__((aligned(16))) float As[2][BMo][kLdA];
  __shared__ __attribute__((aligned(16))) float Bs[2][BNo][kLdB];
  __shared__ __attribute__((aligned(16))) float Q[2][kOut][kQLd];
  const int tid = threadIdx.x;
  const int p = tid - 64;
  const unsigned M = static_cast<unsigned>(g.M), N = static_cast<unsigned>(g.N),
                 K = static_cast<unsigned>(g.K);
  const unsigned t = total % 8 == 0 ? (lin % 8) * (total / 8) + lin / 8 : lin;
  const unsigned m0 = (t / gx) * BMo, n0 = (t % gx) * BNo;
  const float* __restrict__ A = g.A;
  const float* __restrict__ B = static_cast<const float*>(g.B);
  float4 ra[kD][kRA], rb[kD][kRB];
  auto load = [&](int s, unsigned k0) {
#pragma unroll
    for (int r = 0; r < kRA; ++r) {
      const int f = min(p + r * kP, kAf - 1);
      if constexpr (kTN) {  // A [K, M]: four consecutive m at one k
        const int kk = f / (BMo / 4), c4 = f % (BMo / 4);
        ra[s][r] = *reinterpret_cast<const float4*>(A + min(k0 + kk, K - 1) * M + m0 + 4 * c4);
      } else {              // A [M, K]: four consecutive k of one row
        const int mm = f / (kKc / 4), c4 = f % (kKc / 4);
        ra[s][r] = *reinterpret_cast<const float4*>(A + static_cast<size_t>(m0 + mm) * K +
                                                    min(k0 + 4 * c4, K - 4));
      }
    }
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      const int f = min(p + r * kP, kBf - 1), kk = f / (BNo / 4), c4 = f % (BNo / 4);
      rb[s][r] = *reinterpret_cast<const float4*>(B + min(k0 + kk, K - 1) * N + n0 + 4 * c4);
    }
  };
  // Transposed into k-contiguous rows, alpha applied; the spare lanes of a
  // last round (their loads re-read the last element) store nothing, so no
  // two lanes of a store meet at one address.
  auto store = [&](int s, int buf) {
#pragma unroll
    for (int r = 0; r < kRA; ++r) {
      if (kRA * kP > kAf && p + r * kP >= kAf) continue;
      const int f = min(p + r * kP, kAf - 1);
      float4 v = ra[s][r];
      if (g.alpha_a != 1.0f)
        v = make_float4(Mul(g.alpha_a, v.x), Mul(g.alpha_a, v.y), Mul(g.alpha_a, v.z),
                        Mul(g.alpha_a, v.w));
      if constexpr (kTN) {
        const int kk = f / (BMo / 4), c4 = f % (BMo / 4);
        As[buf][4 * c4 + 0][kk] = v.x;
        As[buf][4 * c4 + 1][kk] = v.y;
        As[buf][4 * c4 + 2][kk] = v.z;
        As[buf][4 * c4 + 3][kk] = v.w;
      } else {
        const int mm = f / (kKc / 4), c4 = f % (kKc / 4);
        *reinterpret_cast<float4*>(&As[buf][mm][4 * c4]) = v;
      }
    }
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      if (kRB * kP > kBf && p + r * kP >= kBf) continue;
      const int f = min(p + r * kP, kBf - 1), kk = f / (BNo / 4), c4 = f % (BNo / 4);
      const float4 v = rb[s][r];
      Bs[buf][4 * c4 + 0][kk] = v.x;
      Bs[buf][4 * c4 + 1][kk] = v.y;
      Bs[buf][4 * c4 + 2][kk] = v.z;
      Bs[buf][4 * c4 + 3][kk] = v.w;
    }
  };
  auto quads_of = [&](int buf, int nq) {
#pragma unroll
    for (int r = 0; r < kT; ++r) {
      const int task = p + r * kP;
      if (task >= kTasks) continue;
      const int j = task % kQc, qb = task / kQc;
      if (j >= nq) continue;
      const int bm = qb / kBlkN, bn = qb % kBlkN;
      float4 a[QM], b[QN];
#pragma unroll
      for (int u = 0; u < QM; ++u) a[u] = *reinterpret_cast<const float4*>(&As[buf][QM * bm + u][4 * j]);
#pragma unroll
      for (int v = 0; v < QN; ++v) b[v] = *reinterpret_cast<const float4*>(&Bs[buf][QN * bn + v][4 * j]);
#pragma unroll
      for (int u = 0; u < QM; ++u)
#pragma unroll
        for (int v = 0; v < QN; ++v)
          Q[buf][(QM * bm + u) * BNo + QN * bn + v][j] =
              Add(Add(Add(Mul(a[u].x, b[v].x), Mul(a[u].y, b[v].y)), Mul(a[u].z, b[v].z)),
                  Mul(a[u].w, b[v].w));
    }
  };
  const unsigned quads = K / 4;
  const unsigned chunks = (quads + kQc - 1) / kQc;
  auto nq_of = [&](unsigned i) { return static_cast<int>(min(quads - i * kQc, static_cast<unsigned>(kQc))); };
  const int fo = min(tid, kOut - 1);  // a folder lane's first output (lanes past kOut idle)
  float c[kF];
#pragma unroll
  for (int e = 0; e < kF; ++e) {
    const int o = min(fo + 64 * e, kOut - 1);
    c[e] = (tid < kOut && g.accumulate) ? g.C[static_cast<size_t>(m0 + o / BNo) * N + n0 + o % BNo] : 0.0f;
  }
  auto fold = [&](int buf, int nq) {
    if (nq == kQc) {
      constexpr int kH = kF == 1 ? kQc / 4 : kQc / 8;  // 16-byte reads per batch per output
      static_assert((kQc / 4) % kH == 0, "whole batches");
#pragma unroll
      for (int h = 0; h < kQc / 4; h += kH) {
        float4 q[kF][kH];
#pragma unroll
        for (int e = 0; e < kF; ++e)
#pragma unroll
          for (int i = 0; i < kH; ++i) q[e][i] = *reinterpret_cast<const float4*>(&Q[buf][fo + 64 * e][4 * (h + i)]);
        __builtin_amdgcn_sched_barrier(0);  // every read of the batch in flight before the adds
#pragma unroll
        for (int i = 0; i < kH; ++i)
#pragma unroll
          for (int e = 0; e < kF; ++e) {
            c[e] = Add(c[e], q[e][i].x);
            c[e] = Add(c[e], q[e][i].y);
            c[e] = Add(c[e], q[e][i].z);
            c[e] = Add(c[e], q[e][i].w);
          }
      }
    } else {
      for (int j = 0; j < nq; ++j)
#pragma unroll
        for (int e = 0; e < kF; ++e) c[e] = Add(c[e], Q[buf][fo + 64 * e][j]);
    }
  };
  if (chunks <= static_cast<unsigned>(kD) + 1) {  // a few chunks: one at a time
    for (unsigned i = 0; i < chunks; ++i) {
      if (tid >= 64) {
        load(0, i * kKc);
        WaitVmAll();
        store(0, 0);
      }
      __syncthreads();
      if (tid >= 64) quads_of(0, nq_of(i));
      __syncthreads();
      if (tid < 64) fold(0, nq_of(i));
      __syncthreads();
    }
  } else if (tid < 64) {
    __syncthreads();
    for (unsigned i = 0; i <= chunks; ++i) {
      if (i >= 1) fold((i - 1) & 1, nq_of(i - 1));
      __syncthreads();
    }
  } else {
#pragma unroll
    for (int s = 0; s < kD; ++s) load(s, s * kKc);
    WaitVmAll();
    store(0, 0);
    load(0, kD * kKc);
    __syncthreads();
    // Interval i: chunk i's quads; chunk i + 1 stored from ring slot
    // (i + 1) % kD, which then takes chunk i + 1 + kD.
    const unsigned nmain = (chunks - kD - 1) / kD * kD;
    for (unsigned i0 = 0; i0 < nmain; i0 += kD) {
#pragma unroll
      for (int u = 0; u < kD; ++u) {
        const unsigned i = i0 + u;
        quads_of(i & 1, kQc);
        const int nx = (u + 1) % kD;
        store(nx, (i + 1) & 1);
        load(nx, (i + 1 + kD) * kKc);
        __syncthreads();
      }
    }
    for (unsigned i = nmain; i <= chunks; ++i) {
      if (i < chunks) quads_of(i & 1, nq_of(i));
      if (i + 1 < chunks) {
        WaitVmAll();
        const unsigned slot = (i + 1) % kD;
#pragma unroll
        for (int u = 0; u < kD; ++u)
          if (slot == static_cast<unsigned>(u)) {
            store(u, (i + 1) & 1);
            if (i + 1 + kD < chunks) load(u, (i + 1 + kD) * kKc);
          }
      }
      __syncthreads();
    }
  }
  if (tid >= kOut || tid >= 64) return;
#pragma unroll
  for (int e = 0; e < kF; ++e) {
    const int o = tid + 64 * e;
    const unsigned mf = m0 + o / BNo, nf = n0 + o % BNo;
    float v = c[e];
    for (unsigned k = quads * 4; k < K; ++k)  // the K % 4 tail, one term at a time
      v = Add(v, Mul(LoadA<2>(g, mf, k), B[static_cast<size_t>(k) * N + nf]));
    g.C[static_cast<size_t>(mf) * N + nf] = Epilogue(g, mf, nf, v);
  }
}

template <int kLayout, int BMo, int BNo, int kKc, int kD, int QM, int QN, int kW, int kF>
__global__ void __launch_bounds__(64 * kW) GemmFoldSplitKernel(GemmArgs g) {
  FoldSplitBody<kLayout, BMo, BNo, kKc, kD, QM, QN, kW, kF>(
      g, gridDim.x, blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
}

// Two independent products of one fold geometry in one launch: blocks
// 0 .. n0 - 1 run g0's grid (gx0 across), the rest g1's.  Products that
// each leave CUs idle (C4's adapter gradients: 192 blocks each) then run
// side by side.
template <int kLayout, int BMo, int BNo, int kKc, int kD, int QM, int QN, int kW, int kF>
__global__ void __launch_bounds__(64 * kW)
GemmFoldSplitPairKernel(GemmArgs g0, GemmArgs g1, unsigned n0, unsigned gx0, unsigned gx1) {
  const unsigned b = blockIdx.x;
  if (b < n0)
    FoldSplitBody<kLayout, BMo, BNo, kKc, kD, QM, QN, kW, kF>(g0, gx0, b, n0);
  else
    FoldSplitBody<kLayout, BMo, BNo, kKc, kD, QM, QN, kW, kF>(g1, gx1, b - n0, gridDim.x - n0);
}

// The fold kernel for TN with f32 B over K >= 1024 when the outputs fill at
// most a few thousand workgroups (NN over these shapes measured faster on
// the chain kernel).
// TN from K = 1024 (the adapter gradients); NN from K = 1024 past the
// two-pass form's output count (the LoRA products t = X A; C5's
// 8192 x 16 x 2048: 49.2 -> 44.2 us against the chain kernel, while C4's
// 8192 x 8 x 768 measured 19.6 on the chain kernel against 31.2 here): up to
// 2^18 outputs, each one reduction chain.
bool Fold(const GemmArgs& a) {
  if (a.b_kind != 0 || a.M * a.N > (size_t{1} << 18) || a.K < 1024) return false;
  return a.layout == 2 || (a.layout == 0 && a.M * a.N > 16384);
}

// NN with a narrow f32 B -- the LoRA products t = X A, N = 8 or 16 -- over
// many rows and K past the panel kernel's: role-split folds of 32 x 8 or
// 16 x 16 output blocks, four outputs per folder lane, 128-deep chunks (two
// workgroups' LDS per CU).  C4's 8192 x 8 x 768: 17.8 us on the chain
// kernel -> 8.0; C5's 8192 x 16 x 2048: 37.9 on the 8 x 16 fold -> 29-30
// (one box, bitwise the same sums).
bool FoldNarrowNN(const GemmArgs& a) {
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return a.layout == 0 && a.b_kind == 0 && (a.N == 8 || a.N == 16) &&
         a.K > static_cast<size_t>(kPanelK) && a.K % 4 == 0 && a.M % 32 == 0 && a.M >= 4096 &&
         a.M / 16 <= 65535 && a.K * a.M < (size_t{1} << 31) && al16(a.A) && al16(a.B) &&
         !a.a_k_scale;
}

hipError_t LaunchFoldNarrowNN(const GemmArgs& a, hipStream_t s) {
  if (a.N == 8) {
    hipLaunchKernelGGL((GemmFoldSplitKernel<0, 32, 8, 128, 2, 4, 4, 9, 4>),
                       dim3(1, static_cast<unsigned>(a.M / 32)), dim3(576), 0, s, a);
  } else {
    hipLaunchKernelGGL((GemmFoldSplitKernel<0, 16, 16, 128, 2, 4, 4, 9, 4>),
                       dim3(1, static_cast<unsigned>(a.M / 16)), dim3(576), 0, s, a);
  }
  return hipGetLastError();
}

template <int kLayout>
hipError_t LaunchFold(const GemmArgs& a, hipStream_t s) {
  // BNo: N rounded up to a power of two in [2, 16] (a chunk of B then spans
  // whole lanes: BNo * kFoldK >= 256).
  int bno = 2;
  while (bno < 16 && static_cast<size_t>(bno) < a.N) bno *= 2;
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.M % 4 == 0 && a.N % 8 == 0 && a.K * a.M < (size_t{1} << 31) &&
      a.K * a.N < (size_t{1} << 31) && al16(a.A) && al16(a.B) && !a.a_k_scale &&
      (kLayout == 2 || a.K % 4 == 0)) {
    // Role-split folds: 8 x 16 blocks (two outputs per folder lane, eight
    // producer waves: the 512 tasks of a chunk in one round; seven took two
    // rounds, the second 1/7 busy -- C5's 2048 x 16 and 16 x 2048 gradients
    // 38.0 / 35.1 -> 35.6 / 32.8 us, its 8192 x 16 x 2048 t 44.2 -> 39.1) where
    // they still fill the machine, else 4 x 8 with four producer waves (C4's
    // 768 x 8 and 8 x 768 20 us against 33 on the one-pass fold).
    if (a.M % 8 == 0 && a.N % 16 == 0 && (a.M / 8) * (a.N / 16) >= 256) {
      const dim3 grid(static_cast<unsigned>(a.N / 16), static_cast<unsigned>(a.M / 8));
      if (grid.y > 65535) return hipErrorInvalidValue;
      hipLaunchKernelGGL((GemmFoldSplitKernel<kLayout, 8, 16, 256, 2, 4, 4, 9, 2>), grid, dim3(576),
                         0, s, a);
      return hipGetLastError();
    }
    const dim3 grid(static_cast<unsigned>(a.N / 8), static_cast<unsigned>(a.M / 4));
    if (grid.y > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL((GemmFoldSplitKernel<kLayout, 4, 8, 512, 2, 4, 4, 5, 1>), grid, dim3(320), 0,
                       s, a);
    return hipGetLastError();
  }
  const size_t bmo = kFoldOut / bno;
  const size_t gx = (a.N + bno - 1) / bno, gy = (a.M + bmo - 1) / bmo;
  if (gy > 65535) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  switch (bno) {
    case 2: hipLaunchKernelGGL((GemmFoldKernel<kLayout, 2>), grid, dim3(kThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((GemmFoldKernel<kLayout, 4>), grid, dim3(kThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((GemmFoldKernel<kLayout, 8>), grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((GemmFoldKernel<kLayout, 16>), grid, dim3(kThreads), 0, s, a); break;
  }
  return hipGetLastError();
}

// The chain kernel where the tiled kernel's grid would be small for the
// reduction it carries: under 512 tiles of 64 x 64 and K above the panel.
bool Chain(const GemmArgs& a) {
  const size_t tiles = ((a.M + 63) / 64) * ((a.N + 63) / 64);
  return a.K > static_cast<size_t>(kPanelK) && tiles < 512;
}

template <int kLayout, int kBKind, int BM, int BN>
hipError_t LaunchChain(const GemmArgs& a, hipStream_t s) {
  const size_t gy = (a.M + BM - 1) / BM, gx = (a.N + BN - 1) / BN;
  if (gy > 65535 || gx > (size_t{1} << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((GemmChainKernel<kLayout, kBKind, BM, BN>),
                     dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)), dim3(kThreads), 0,
                     s, a);
  return hipGetLastError();
}

bool LongK(const GemmArgs& a) { return a.layout != 1 && a.M * a.N <= 16384 && a.K >= 1024; }

// NT over at most 16 outputs per row, enough rows to fill the machine and a
// long K, with 16-byte rows of A: the k-lane kernel.
bool KLane(const GemmArgs& a) {
  return a.layout == 1 && a.b_kind == 0 && !a.a_k_scale && a.N <= 16 && a.M >= 2048 &&
         a.K >= 256 && a.K % 4 == 0 && (reinterpret_cast<uintptr_t>(a.A) & 15) == 0 &&
         a.M * a.K < (size_t{1} << 40);
}

// Short reductions over few outputs (the small-batch plans' products, e.g.
// 32 x 8 over K = 512): the panel kernel would give the whole GEMM a handful
// of workgroups, each lane running its output's chain alone; the two-pass
// workspace form spreads the quads over the machine and folds them in k
// order -- the same quads, the same order, the same bits.
bool ShortKQuads(const GemmArgs& a) {
  if (a.layout == 1 || a.K < 128 || a.K > static_cast<size_t>(kPanelK) || a.M * a.N > 16384)
    return false;
  return ((a.M + 15) / 16) * ((a.N + 15) / 16) < 128;
}

// NT over few outputs and a short K: one lane per chain (GemmNTLanesKernel)
// where the panel kernel would leave most CUs idle.
bool NTLanes(const GemmArgs& a) {
  if (a.layout != 1 || a.K < 64 || a.K > static_cast<size_t>(kPanelK) || a.M * a.N > 16384)
    return false;
  return ((a.M + 15) / 16) * ((a.N + 15) / 16) < 128;
}

// Where both apply, the two-pass workspace form runs before the chain
// kernel unless the tile policy puts the chain kernel first.
bool LongKFirst(const GemmArgs& a) { return !a.policy || a.policy->exact_longk_first != 2; }

// The two-pass workspace form: every quad sum in parallel, then each
// output's quads added in k order.
template <int kLayout, int kBKind>
hipError_t LaunchQuadsFold(const GemmArgs& a, hipStream_t s) {
  const unsigned quads4 = static_cast<unsigned>((a.K / 4 + 3) / 4);
  const unsigned ob = static_cast<unsigned>((a.M * a.N + kThreads - 1) / kThreads);
  const dim3 g1(ob, quads4 < 1024 ? quads4 : 1024);
  hipLaunchKernelGGL((LongKQuadsKernel<kLayout, kBKind>), g1, dim3(kThreads), 0, s, a, quads4);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL((LongKFoldKernel<kLayout, kBKind>), dim3(ob), dim3(kThreads), 0, s, a, quads4);
  return hipGetLastError();
}

template <int kLayout, int kBKind>
hipError_t Run(const GemmArgs& a, hipStream_t s) {
  if (kBKind == 0 && RankFits(a)) {
    const dim3 grid(static_cast<unsigned>((a.N + 255) / 256),
                    static_cast<unsigned>((a.M + kRankRows - 1) / kRankRows));
    hipLaunchKernelGGL((GemmRankKernel<kLayout>), grid, dim3(kThreads), 0, s, a);
    return hipGetLastError();
  }
  if constexpr (kLayout != 1) {
    if (ShortKQuads(a) && a.scratch) return LaunchQuadsFold<kLayout, kBKind>(a, s);
  } else {
    if (NTLanes(a)) {
      const unsigned grid = static_cast<unsigned>((a.M * a.N + kThreads / 8 - 1) / (kThreads / 8));
      hipLaunchKernelGGL((GemmNTLanesKernel<kBKind>), dim3(grid), dim3(kThreads), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.K <= static_cast<size_t>(kPanelK) && a.K > 0 && (a.M + 15) / 16 <= 65535) {
    const dim3 grid(static_cast<unsigned>((a.N + 15) / 16), static_cast<unsigned>((a.M + 15) / 16));
    const size_t lds = 2 * 16 * a.K * sizeof(float);
    hipLaunchKernelGGL((GemmPanelKernel<kLayout, kBKind>), grid, dim3(kThreads), lds, s, a);
    return hipGetLastError();
  }
  if constexpr (kLayout == 0 && kBKind == 0)
    if (FoldNarrowNN(a)) return LaunchFoldNarrowNN(a, s);
  if constexpr (kLayout != 1 && kBKind == 0)
    if (Fold(a)) return LaunchFold<kLayout>(a, s);
  if constexpr (kLayout == 1 && kBKind == 0)
    if (KLane(a)) {
      if (a.N <= 8) {
        hipLaunchKernelGGL((GemmNTKLaneKernel<1, 1, 128>),
                           dim3(static_cast<unsigned>((a.M + 31) / 32)), dim3(kThreads), 0, s, a);
      } else {  // 256-deep chunks (two rows per lane, one wave per SIMD: slower)
        hipLaunchKernelGGL((GemmNTKLaneKernel<2, 1, 256>),
                           dim3(static_cast<unsigned>((a.M + 15) / 16)), dim3(kThreads), 0, s, a);
      }
      return hipGetLastError();
    }
  if (Chain(a) && !(kLayout != 1 && LongK(a) && a.scratch && LongKFirst(a))) {
    if (a.N <= 8) return LaunchChain<kLayout, kBKind, 32, 8>(a, s);
    if (a.M <= 8) return LaunchChain<kLayout, kBKind, 8, 32>(a, s);
    return LaunchChain<kLayout, kBKind, 16, 16>(a, s);
  }
  if constexpr (kLayout != 1) {
    if (LongK(a) && a.scratch) return LaunchQuadsFold<kLayout, kBKind>(a, s);
    if (LongK(a)) {
      int lb = 0;
      while (lb < 5 && (size_t{2} << lb) <= a.N) ++lb;  // BNo = 2^lb <= min(N, 32)
      const size_t bno = size_t{1} << lb, bmo = kLongOut / bno;
      const dim3 grid(static_cast<unsigned>((a.N + bno - 1) / bno),
                      static_cast<unsigned>((a.M + bmo - 1) / bmo));
      if (grid.y > 65535) return hipErrorInvalidValue;
      hipLaunchKernelGGL((GemmLongKKernel<kLayout, kBKind>), grid, dim3(kThreads), 0, s, a, lb);
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

// Two TN products that each take the fold kernel (K >= 1024, f32 B) and
// between them fill at most one block per CU on 8 x 8 output blocks: one
// launch, the blocks side by side (C4's adapter gradients dB 8 x 768 and
// dA 768 x 8 over 8192 tokens: 40.9 us as two launches, 21.9 as one; the
// same sums, bit for bit).
bool GemmExactPairFits(const GemmArgs& a, const GemmArgs& b) {
  const auto fits = [](const GemmArgs& g) {
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return g.layout == 2 && g.b_kind == 0 && Fold(g) && g.M % 8 == 0 && g.N % 8 == 0 &&
           g.K * g.M < (size_t{1} << 31) && g.K * g.N < (size_t{1} << 31) && al16(g.A) &&
           al16(g.B) && !g.a_k_scale;
  };
  const size_t blocks = (a.M / 8) * (a.N / 8) + (b.M / 8) * (b.N / 8);
  return fits(a) && fits(b) && blocks <= static_cast<size_t>(DeviceCUs());
}

hipError_t LaunchGemmExactPair(const GemmArgs& a, const GemmArgs& b, hipStream_t s) {
  if (!GemmExactPairFits(a, b)) return hipErrorInvalidValue;
  const unsigned gxa = static_cast<unsigned>(a.N / 8), na = gxa * static_cast<unsigned>(a.M / 8);
  const unsigned gxb = static_cast<unsigned>(b.N / 8), nb = gxb * static_cast<unsigned>(b.M / 8);
  hipLaunchKernelGGL((GemmFoldSplitPairKernel<2, 8, 8, 256, 2, 4, 4, 5, 1>), dim3(na + nb),
                     dim3(320), 0, s, a, b, na, gxa, gxb);
  return hipGetLastError();
}

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

size_t GemmExactScratchBytes(const GemmArgs& a) {
  if (!LongK(a) && !ShortKQuads(a)) return 0;
  return a.M * a.N * ((a.K / 4 + 3) / 4) * 4 * sizeof(float);
}

}  // namespace seeai
