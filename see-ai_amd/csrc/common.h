// common.h -- shared device helpers and the internal launcher interface of
// the SeeAI gfx950 executor.  Every kernel family (.hip file) exposes its
// launchers through the declarations at the bottom; capi.cpp (the C-ABI and
// the instruction dispatcher) is the only caller.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <initializer_list>

namespace seeai {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// A wave-uniform value held in a vector register, as a scalar.
__device__ __forceinline__ int Uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// The fused-epilogue activations (instruction.h:384-396, the expressions of
// kernel_policy.h:122-136).  Built with -ffp-contract=off, so every product
// and sum rounds where the reference's x86-64 build rounds it.
__device__ __forceinline__ float SigmoidExpr(float x) {
  return 1.0f / (1.0f + expf(-x));
}
__device__ __forceinline__ float ReluExpr(float x) { return x > 0.0f ? x : 0.0f; }
__device__ __forceinline__ float GeluExpr(float x) {
  const float kC = 0.7978845608028654f, kA = 0.044715f;
  const float t = tanhf(kC * (x + kA * x * x * x));
  return 0.5f * x * (1.0f + t);
}
__device__ __forceinline__ float SiluExpr(float x) { return x * SigmoidExpr(x); }
// SiluBwd (activation.cc:62-75): dy * (s (1 + x (1 - s))), s = sigmoid(x).
__device__ __forceinline__ float SiluBwdExpr(float dy, float x) {
  const float sg = SigmoidExpr(x);
  return dy * (sg * (1.0f + x * (1.0f - sg)));
}
__device__ __forceinline__ float ActExpr(int act, float v) {
  switch (act) {
    case 1: return ReluExpr(v);
    case 2: return GeluExpr(v);
    case 3: return SiluExpr(v);
    default: return v;
  }
}

// Wave-wide butterfly sums: a fixed pairing of lanes, so the result is a
// pure function of the 64 inputs (bitwise reproducible run to run).
__device__ __forceinline__ double WaveSumD(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float WaveMaxF(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum of one double per thread through LDS, combined in wave
// order: fixed association for a fixed block size.
template <int kThreads>
__device__ __forceinline__ double BlockSumD(double v, double* lds) {
  v = WaveSumD(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  if (l == 0) lds[w] = v;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < kThreads / kWave; ++i) s += lds[i];
    lds[0] = s;
  }
  __syncthreads();
  s = lds[0];
  __syncthreads();
  return s;
}
template <int kThreads>
__device__ __forceinline__ float BlockMaxF(float v, float* lds) {
  v = WaveMaxF(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  if (l == 0) lds[w] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = lds[0];
    for (int i = 1; i < kThreads / kWave; ++i) s = fmaxf(s, lds[i]);
    lds[0] = s;
  }
  __syncthreads();
  const float r = lds[0];
  __syncthreads();
  return r;
}
template <int kThreads>
__device__ __forceinline__ float BlockSumF(float v, float* lds) {
  v = WaveSumF(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  if (l == 0) lds[w] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int i = 0; i < kThreads / kWave; ++i) s += lds[i];
    lds[0] = s;
  }
  __syncthreads();
  const float r = lds[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float Bf16ToF32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round-to-nearest-even narrowing (source/plan/bf16.h:18-24).
__device__ __forceinline__ uint16_t F32ToBf16(float f) {
  const uint32_t bits = __float_as_uint(f);
  if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  const uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>((bits + bias) >> 16);
}

inline unsigned GridFor(size_t n, unsigned threads, unsigned cap = 65536u) {
  size_t g = (n + threads - 1) / threads;
  if (g == 0) g = 1;
  return static_cast<unsigned>(g < cap ? g : cap);
}

// ---------------------------------------------------------------------------
// Launchers (host side).  All take the stream last; all return hipError_t.
// Pointers are device pointers.  The workspace (`ws`) pointers are scratch
// device memory the caller owns; each launcher documents the bytes it needs.
// ---------------------------------------------------------------------------

// A producer's output as the next relaxed GEMM would round it into its
// bf16 workspace (ConvertFlatKernel's expression: RNE(alpha * (v * ks[k])),
// k = flat index mod K, K a multiple of 32, ks 16-byte aligned), written by
// the producer itself so the GEMM skips its conversion pass; store_f32 = 0
// drops the f32 output where nothing else reads it.  out null: no copy.
struct Bf16Sink {
  uint16_t* out = nullptr;
  const float* ks = nullptr;
  float alpha = 1.0f;
  uint32_t K = 0;
  int store_f32 = 1;
};
// Elements i .. i + 3 (i a multiple of 4) of a sink.
__device__ __forceinline__ void SinkStore4(const Bf16Sink& s, size_t i, float4 v) {
  float x[4] = {v.x, v.y, v.z, v.w};
  if (s.ks) {
    const float4 sc = *reinterpret_cast<const float4*>(s.ks + i % s.K);
    x[0] = x[0] * sc.x, x[1] = x[1] * sc.y, x[2] = x[2] * sc.z, x[3] = x[3] * sc.w;
  }
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = static_cast<__bf16>(s.alpha != 1.0f ? s.alpha * x[e] : x[e]);
  *reinterpret_cast<bf16x4_t*>(s.out + i) = o;
}
// Four floats rounded to bf16 (nearest even) in one 8-byte store.
__device__ __forceinline__ void StoreBf16x4(uint16_t* dst, const float v[4]) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const bf16x4_t o = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]),
                      static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
  *reinterpret_cast<bf16x4_t*>(dst) = o;
}

// Elementwise family (k_elementwise.hip).
hipError_t LaunchAddEW(const float* x, const float* y, float* out, size_t n, hipStream_t s,
                       const Bf16Sink& sink = Bf16Sink{});
// Whether rows of `cols` floats (a multiple of 4; the non-null operands
// 16-byte aligned) go out as float4 stores and so can feed a sink: the
// normalisations' rows, and the residual add as one row of n.
bool NormSinkFits(size_t cols, std::initializer_list<const void*> ptrs);
hipError_t LaunchMulEW(const float* x, const float* y, float* out, size_t n, hipStream_t s);
hipError_t LaunchAddBias(const float* x, const float* b, float* out, size_t rows, size_t cols,
                         hipStream_t s);
// A sink (GELU only: kind 2) takes the output's bf16 copy.
hipError_t LaunchUnary(int kind, const float* x, float* out, size_t n, float alpha, hipStream_t s,
                       const Bf16Sink& sink = Bf16Sink{});
hipError_t LaunchBinaryBwd(int kind, const float* dy, const float* x, float* dx, size_t n,
                           hipStream_t s, const Bf16Sink& sink = Bf16Sink{});
// Whether LaunchUnary / LaunchBinaryBwd can feed a sink for this call.
bool ElementwiseSinkFits(int kind, size_t n, const void* a, const void* b, const void* out);
hipError_t LaunchReduceRows(const float* dy, float* db, size_t rows, size_t cols, hipStream_t s);
hipError_t LaunchFill(float* dst, float value, size_t n, hipStream_t s);
hipError_t LaunchCopy(const float* src, float* dst, size_t n, hipStream_t s);
hipError_t LaunchAccumulate(float* dst, const float* src, size_t n, hipStream_t s);
hipError_t LaunchEmbed(const int32_t* tokens, const float* table, float* out, size_t rows,
                       size_t dim, hipStream_t s);
hipError_t LaunchFusedMap(const float* x, const float* o1, const float* o2, float* out, size_t n,
                          uint64_t stages, float imm0, float imm1, hipStream_t s);
hipError_t LaunchLayerNormFwd(const float* x, const float* g, const float* b, float* y,
                              float* mean, float* rstd, size_t rows, size_t cols, float eps,
                              hipStream_t s, const Bf16Sink& sink = Bf16Sink{});
// With res, dx = res + the normalisation's gradient (a residual add fused
// behind it; dx may be res itself).
hipError_t LaunchLayerNormBwd(const float* dy, const float* x, const float* g,
                              const float* mean, const float* rstd, float* dx, size_t rows,
                              size_t cols, hipStream_t s, const Bf16Sink& sink = Bf16Sink{},
                              const float* res = nullptr);
hipError_t LaunchRmsNormFwd(const float* x, const float* g, float* y, float* rstd, size_t rows,
                            size_t cols, float eps, hipStream_t s,
                            const Bf16Sink& sink = Bf16Sink{});
hipError_t LaunchRmsNormBwd(const float* dy, const float* x, const float* g, const float* rstd,
                            float* dx, size_t rows, size_t cols, hipStream_t s,
                            const Bf16Sink& sink = Bf16Sink{}, const float* res = nullptr);
// sink: also a bf16 copy of y (with the sink's scales; the attention's copy
// is plain round to nearest even), on the row kernel only (RopeRowsFits).
bool RopeRowsFits(const float* x, const float* y, size_t B, size_t S, size_t H, size_t d,
                  const float* table);
hipError_t LaunchRope(const float* x, float* y, size_t B, size_t S, size_t H, size_t d,
                      float step, const float* table, int backward, hipStream_t s,
                      const Bf16Sink& sink = Bf16Sink{});
hipError_t LaunchRopeTable(float* table, size_t S, size_t d, float step, hipStream_t s);
hipError_t LaunchSegmentStarts(const int32_t* tokens, int32_t* starts, size_t B, size_t S,
                               int32_t eos, hipStream_t s);
hipError_t LaunchArgmaxRows(const float* probs, size_t rows, size_t cols, int32_t* out,
                            hipStream_t s);
// counts[0] = rows whose label (not -1) is their argmax, counts[1] = rows
// with a label; both zeroed first on the stream.
hipError_t LaunchArgmaxTally(const float* probs, const int32_t* labels, size_t rows, size_t cols,
                             uint64_t* counts, hipStream_t s);

// Loss family (k_loss.hip).  ws: XEntFwdScratchBytes(rows) for the forward,
// 64 bytes for the backward.
size_t XEntFwdScratchBytes(size_t rows);
hipError_t LaunchXEntFwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                         size_t N, size_t C, int masked, void* ws, hipStream_t s);
hipError_t LaunchXEntBwd(const float* probs, const int32_t* labels, const float* seed,
                         float* dlogits, size_t N, size_t C, int masked, void* ws,
                         hipStream_t s, const Bf16Sink& sink = Bf16Sink{});
// The forward, the fill of the backward's seed (fill_n floats of fill_v at
// fill_dst) and the backward as one: probabilities (stored where probs is
// given) and their gradients in one pass (scale from seed as the backward
// forms it); rows 16-byte aligned.  A few rows run in one workgroup.
bool XEntFusedFits(const float* logits, const float* probs, const float* dlogits, size_t C);
hipError_t LaunchXEntFwdBwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                            float* fill_dst, uint64_t fill_n, float fill_v, const float* seed,
                            float* dlogits, size_t N, size_t C, int masked, void* ws,
                            hipStream_t s, const Bf16Sink& sink = Bf16Sink{},
                            const float* max_parts = nullptr);
// Whether the fused loss turn of N rows of C runs in one workgroup (no row
// max pass).
bool XEntOneWorkgroup(size_t N, size_t C);
// max_parts: the logits' partial row maxima [N, ceil(C / 64)] a GEMM
// epilogue left (GemmArgs::row_max_part); the row max is formed from them.
// Whether the backward's row kernel can feed a sink (float4 rows).
bool XEntBwdSinkFits(const float* probs, const float* dlogits, size_t C);

// Optimizer family (k_optim.hip).  `flag` is the device refusal word that
// every parameter-writing kernel honours; `scale` a device float slot.
// ws for the norm: 8 * 1024 bytes.
hipError_t LaunchClipFactor(const float* g, size_t n, float max_norm, float* scale, int* flag,
                            void* ws, hipStream_t s);
hipError_t LaunchSqNormAccum(const float* g, size_t n, float* acc, void* ws, hipStream_t s);
hipError_t LaunchGlobalClipFactor(const float* acc, float max_norm, float* scale, int* flag,
                                  hipStream_t s);
hipError_t LaunchScaleByFactor(float* g, size_t n, const float* scale, const int* flag,
                               hipStream_t s);
// hyper: null, or device memory holding {lr, inv_bc1, inv_bc2} that take the
// place of the arguments (a replayed graph reads each step's values there).
hipError_t LaunchAdamW(float* p, const float* g, float* m, float* v, size_t n, float lr,
                       float beta1, float beta2, float eps, float wd, float inv_bc1,
                       float inv_bc2, const float* scale, const int* flag, hipStream_t s,
                       const float* hyper = nullptr);
hipError_t LaunchSgd(float* p, const float* g, size_t n, float lr, float wd, const float* scale,
                     const int* flag, hipStream_t s, const float* hyper = nullptr);
// Up to kAdamWMulti tensors' AdamW steps (no clip) in one launch, each
// element's update AdamWKernel's.
constexpr int kAdamWMulti = 16;
struct AdamWTensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  size_t n;
};
struct AdamWTable {
  AdamWTensor t[kAdamWMulti];
  int first[kAdamWMulti + 1];  // first workgroup of each tensor (set by the launcher)
  int count;
};
hipError_t LaunchAdamWMulti(const AdamWTable& tab, float lr, float beta1, float beta2, float eps,
                            float wd, float inv_bc1, float inv_bc2, const int* flag, hipStream_t s,
                            const float* hyper = nullptr);

// fp32-output GEMM family on MFMA (k_gemm_f32.hip).
// Kernel-geometry choices (the C ABI's seeai_tile_policy): each field picks
// among kernels that give identical bits, so a policy changes time, never
// results.  A default-constructed policy is the built-in choice.
struct TilePolicy {
  int w8a8_large_kernel = 1;           // 1 direct-to-LDS 256 x 256, 2 register-staged 256 x 256,
                                       // 3 register-staged 128 x 128
  size_t w8a8_large_min = 4096;        // M and N from which w8a8_large_kernel applies
  int quantize_waves_per_cu = 32;      // waves per CU walking the quantizer's rows of at most
                                       // 1024 or more than 8192 floats (rows in between take
                                       // a workgroup of four waves each)
  size_t relaxed_min_tiles_256 = 256;  // relaxed bf16 GEMM: 256 x 256 tiles from this many
  int relaxed_min_fill_256 = 0;        // ... and when their last round of tiles over
                                       // the CUs is at least this percent full
  size_t relaxed_nt_dma_min_k = 768;   // relaxed NT: the direct-to-LDS kernel from this K
                                       // (below it the register-staged bf16 kernel)
  int convert_wgs_per_cu = 8;          // workgroups per CU of the activation conversion
  int exact_longk_first = 1;           // exact skinny long-K GEMM: 1 the two-pass workspace
                                       // form before the chain kernel, 2 the chain kernel first
  int relaxed_tile_192 = 2;            // relaxed bf16 GEMM below 256 x 256: 1 128 x 192 tiles
                                       // when they take fewer CU rounds per unit of work,
                                       // 2 never (default: measured slower on the decoder's
                                       // 8192 x 768 products), 3 always (N >= 192)
};

struct GemmArgs {
  int layout;          // 0 NN (A[M,K], B[K,N]), 1 NT (B[N,K]), 2 TN (A[K,M])
  int b_kind;          // 0 f32, 1 int8, 2 bf16
  const float* A;
  const void* B;
  float* C;
  size_t M, N, K;
  float alpha_a;       // multiplies A's elements as they enter (NN / TN alpha, q8 scale)
  float alpha_dot;     // multiplies the finished dot (NT alpha, NT q8 scale)
  const float* b_col_scale;  // NN q8: widened weight * scale[n]
  const float* a_k_scale;    // NT q8: A[m,k] * scale[k]
  const float* addend;       // C = D + dot
  const float* bias;         // epilogue bias [N]
  int act;                   // epilogue activation
  int accumulate;            // C += (GemmAccNN)
  int relaxed;               // kFlagRelaxed taken: MFMA summation order
  float* scratch;            // device workspace (GemmExactScratchBytes), or null
  const TilePolicy* policy;  // kernel geometry (null: the defaults)
  // Low-rank epilogue (the relaxed direct-to-LDS kernel): the next
  // instruction of a LoRA site, lr_out = C + rank-r product with C as its
  // addend, joins this product's epilogue.  C's value is formed as without
  // it (and stored when lr_store_c); the rank-r dot follows that
  // instruction's exact chain -- NN: quads of (lr_alpha * t) * b from k = 0,
  // then the tail; NT: eight lanes by k mod 8 added in order, times
  // lr_alpha -- and the addend comes first: lr_out = C + dot.
  const float* lr_t;   // [M, lr_k]
  const float* lr_b;   // NN: [lr_k, N]; NT: [N, lr_k]
  float* lr_out;       // [M, N]; null: no low-rank epilogue
  int lr_layout;       // 0 NN, 1 NT
  int lr_k;            // 1..kLowRankMaxK
  int lr_store_c;      // also store C
  float lr_alpha;
  // A residual add behind the site (NT sites): lr_out = lr_res + (C + dot),
  // the add's operand order immaterial (IEEE addition commutes); null: none.
  const float* lr_res;
  // lr_out's bf16 copy (round to nearest even, same [M, N] layout) for the
  // attention that reads it next -- C's, on the kernel without a low-rank
  // term; null: none.
  uint16_t* lr_sink;
  // The relaxed direct-to-LDS kernel without a low-rank term: C's row maxima
  // over each group of 64 columns, [M, ceil(N / 64)] (fmax: NaN ignored, a
  // group of NaN gives NaN), for the loss turn that reads C next; null: none.
  float* row_max_part;
};
constexpr int kLowRankMaxK = 16;
// Relaxed -> MFMA (k_gemm_f32.hip); otherwise the reference's order.
hipError_t LaunchGemm(const GemmArgs& a, hipStream_t s);
hipError_t LaunchGemmExact(const GemmArgs& a, hipStream_t s);
// Two independent exact TN products in one launch, where both take the
// fold kernel and their blocks fit the CUs side by side.
bool GemmExactPairFits(const GemmArgs& a, const GemmArgs& b);
hipError_t LaunchGemmExactPair(const GemmArgs& a, const GemmArgs& b, hipStream_t s);
// Workspace the exact kernels can use for this GEMM (0: none).
size_t GemmExactScratchBytes(const GemmArgs& a);
// Relaxed NN / NT on bf16 operands staged by direct-to-LDS loads
// (k_gemm_bf16dma.hip): A converted into a bf16 workspace [M, Kp] with its
// scales, the weight's bf16 shadow [N, Kp] made once; Kp = K rounded up to 32.
size_t Bf16DmaKp(size_t K);
bool Bf16DmaFits(const GemmArgs& a);
// Whether the low-rank epilogue can join this product (N % 4 == 0, rank
// operands 16-byte aligned, 1 <= lr_k <= kLowRankMaxK).
bool Bf16DmaRowMaxFits(const GemmArgs& a);
bool Bf16DmaLowRankFits(const GemmArgs& a);
hipError_t LaunchConvertRowsBf16(const float* A, size_t M, size_t K, float alpha,
                                 const float* kscale, void* out, int wgs_per_cu, hipStream_t s);
hipError_t LaunchWeightShadow(const GemmArgs& a, void* out, hipStream_t s);
hipError_t LaunchGemmBf16Dma(const void* A, const void* W, const GemmArgs& a, hipStream_t s);
// Relaxed NN / NT with f32 or int8 weights on bf16 MFMA (k_gemm_bf16.hip),
// when it fits.
bool GemmBf16Fits(const GemmArgs& a);
hipError_t LaunchGemmBf16(const GemmArgs& a, hipStream_t s);

// Compute units of the current device (cached per device).
int DeviceCUs();

// SwiGLU's elementwise chains as one pass each (range fusion of adjacent
// instructions over the same n; every output disjoint from every other
// operand).  Forward: y = SiLU(x), h = y * u.  Backward: o1 = a1 * b1,
// o2 = a2 * b2, dx = SiluBwd(o1, x), o1 not stored when null (a dead store).
// The standalone kernels' expressions.
// A sink takes h's (forward) or dx's (backward) bf16 copy; the float4
// kernels only (n % 4 == 0, 16-byte aligned operands: SwigluFits).
hipError_t LaunchSiluMul(const float* x, const float* u, float* y, float* h, size_t n,
                         hipStream_t s, const Bf16Sink& sink = Bf16Sink{});
hipError_t LaunchSwigluBwd(const float* a1, const float* b1, float* o1, const float* a2,
                           const float* b2, float* o2, const float* x, float* dx, size_t n,
                           hipStream_t s, const Bf16Sink& sink = Bf16Sink{},
                           const Bf16Sink& sink2 = Bf16Sink{}, bool silu_b2 = false);
bool SwigluFits(size_t n, std::initializer_list<const void*> ptrs);

// W8A8 (k_gemm_i8.hip).
hipError_t LaunchQuantizeRows(const float* X, int8_t* Q, float* scale, size_t rows, size_t cols,
                              int waves_per_cu, hipStream_t s);
hipError_t LaunchPackWeightsI8(const float* W, int8_t* Qt, float* scale, size_t K, size_t N,
                               hipStream_t s);
hipError_t LaunchGemmW8A8(const int8_t* QA, const float* sa, const int8_t* QWt, const float* sw,
                          float* C, int32_t* acc, size_t M, size_t N, size_t K,
                          const TilePolicy& policy, hipStream_t s);

// Attention (k_attention.hip).  dtype 0 = f32 exact family, 1 = bf16 MFMA.
hipError_t LaunchAttnFwdTiled(int dtype, const float* q, const float* k, const float* v, float* o,
                              float* stats, size_t B, size_t S, size_t H, size_t d,
                              const int32_t* starts, hipStream_t s);
hipError_t LaunchAttnDQTiled(int dtype, const float* q, const float* k, const float* v,
                             const float* dout, float* stats, float* dq, size_t B, size_t S,
                             size_t H, size_t d, hipStream_t s);
hipError_t LaunchAttnDKTiled(int dtype, const float* q, const float* k, const float* v,
                             const float* dout, const float* stats, float* dk, size_t B,
                             size_t S, size_t H, size_t d, hipStream_t s);
hipError_t LaunchAttnDVTiled(int dtype, const float* q, const float* k, const float* dout,
                             const float* stats, float* dv, size_t B, size_t S, size_t H,
                             size_t d, hipStream_t s);
// The exact family on f32 operands for head widths 64 and 128, staged
// through LDS (k_attn32.hip).  In LaunchAttn32DKDV one or both of dk, dv are
// non-null; each output has the same bits either way.
bool Attn32Fits(size_t B, size_t S, size_t H, size_t d, std::initializer_list<const void*> ptrs);
hipError_t LaunchAttn32Fwd(const float* q, const float* k, const float* v, float* o, float* stats,
                           size_t B, size_t S, size_t H, size_t d, const int32_t* starts,
                           hipStream_t s);
hipError_t LaunchAttn32DQ(const float* q, const float* k, const float* v, const float* dout,
                          float* stats, float* dq, size_t B, size_t S, size_t H, size_t d,
                          hipStream_t s);
hipError_t LaunchAttn32DKDV(const float* q, const float* k, const float* v, const float* dout,
                            const float* stats, float* dk, float* dv, size_t B, size_t S, size_t H,
                            size_t d, hipStream_t s);
// dK and dV of the exact family in one pass (k_attention.hip): Fusable says
// whether the pass takes the shape; otherwise Launch returns
// hipErrorNotSupported and launches nothing.
bool AttnDKDVExactFusable(const float* q, const float* k, const float* v, const float* dout,
                          const float* stats, const float* dk, const float* dv, size_t B, size_t S,
                          size_t H, size_t d);
hipError_t LaunchAttnDKDVExact(const float* q, const float* k, const float* v, const float* dout,
                               const float* stats, float* dk, float* dv, size_t B, size_t S,
                               size_t H, size_t d, hipStream_t s);
// dK and dV in one pass (relaxed family; k_attention.hip).  Fusable says
// whether the fused launch takes the shape; otherwise it returns
// hipErrorNotSupported and launches nothing.
bool AttnDKDVFusable(const float* q, const float* k, const float* v, const float* dout,
                     const float* dk, const float* dv, size_t B, size_t S, size_t H, size_t d);
hipError_t LaunchAttnDKDVFused(const float* q, const float* k, const float* v, const float* dout,
                               const float* stats, float* dk, float* dv, size_t B, size_t S,
                               size_t H, size_t d, hipStream_t s);
// Relaxed tiled attention on bf16 MFMA (k_flash.hip), d in {64, 128}.  In
// LaunchFlashDKDV one or both of dk, dv are non-null; both only where
// FlashFusedDKDV(d).
bool FlashFits(size_t B, size_t S, size_t H, size_t d);
// Head width 64 on bf16 operands in HBM (k_attn16.hip).
bool Attn16Fits(size_t B, size_t S, size_t H, size_t d);
// sink: the output's bf16 copy for the relaxed product after it (the
// attention output o is [B·S, H·64], the product's A).
hipError_t LaunchAttn16Fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* o,
                           float* stats, size_t B, size_t S, size_t H, const int32_t* starts,
                           hipStream_t s, const Bf16Sink& sink = Bf16Sink{});
hipError_t LaunchAttn16DQ(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const uint16_t* dout, float* stats, float* dq, size_t B, size_t S,
                          size_t H, hipStream_t s);
hipError_t LaunchAttn16DKDV(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* dout, const float* stats, float* dk, float* dv,
                            size_t B, size_t S, size_t H, hipStream_t s,
                            const Bf16Sink& sink_v = Bf16Sink{});
bool FlashFusedDKDV(size_t d);
hipError_t LaunchFlashFwd(const float* q, const float* k, const float* v, float* o, float* stats,
                          size_t B, size_t S, size_t H, size_t d, const int32_t* starts,
                          hipStream_t s);
hipError_t LaunchFlashDQ(const float* q, const float* k, const float* v, const float* dout,
                         float* stats, float* dq, size_t B, size_t S, size_t H, size_t d,
                         int one_pass, hipStream_t s);
hipError_t LaunchFlashDKDV(const float* q, const float* k, const float* v, const float* dout,
                           const float* stats, float* dk, float* dv, size_t B, size_t S, size_t H,
                           size_t d, hipStream_t s);
hipError_t LaunchAttnFwdCached(const float* q, const float* k, const float* v, float* o,
                               float* probs, size_t B, size_t S, size_t H, size_t d,
                               const int32_t* starts, hipStream_t s);
hipError_t LaunchAttnDP(const float* dout, const float* v, float* dp, size_t B, size_t S,
                        size_t H, size_t d, hipStream_t s);
hipError_t LaunchAttnDV(const float* probs, const float* dout, float* dv, size_t B, size_t S,
                        size_t H, size_t d, hipStream_t s);
hipError_t LaunchSoftmaxRowsBwd(const float* probs, const float* dp, float* ds, size_t rows,
                                size_t cols, hipStream_t s);
hipError_t LaunchAttnDQ(const float* ds, const float* k, float* dq, size_t B, size_t S, size_t H,
                        size_t d, hipStream_t s);
hipError_t LaunchAttnDK(const float* ds, const float* q, float* dk, size_t B, size_t S, size_t H,
                        size_t d, hipStream_t s);

}  // namespace seeai
