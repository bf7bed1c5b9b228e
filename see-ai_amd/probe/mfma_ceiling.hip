// mfma_ceiling.hip -- a measurement probe, not part of the executor: the
// int8 and bf16 MFMA issue rates on gfx950 with operands held in registers,
// for the roofline discussion of the W8A8 and relaxed bf16 GEMMs.  Each lane keeps eight A and eight B
// fragments (v4i) and issues eight independent v_mfma_i32_32x32x32_i8 per
// loop trip; nothing else runs.  Three operand sets:
//   0  constant bytes (the same fragment every MFMA),
//   1  uniformly random bytes (levels -128..127),
//   2  random levels with |q| <= 31 (the W8A8 bench's typical magnitudes).
// Built into its own library (libseeai_probe.so); bench.py --mfma-ceiling
// loads it.
#include <hip/hip_runtime.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ int Level(unsigned& x, int mode) {
  x = x * 1664525u + 1013904223u;
  const int b = static_cast<int>(x >> 24);  // 0..255
  return mode == 1 ? (b - 128) & 0xff : ((b % 63) - 31) & 0xff;
}

__global__ void __launch_bounds__(256) MfmaI8Probe(int* out, int iters, int mode) {
  v4i a[8], b[8];
  unsigned x = 2654435761u * (blockIdx.x * 256 + threadIdx.x) + 12345u;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 4; ++e) {
      int va = 0x01010101, vb = 0x01010101;
      if (mode != 0) {
        va = vb = 0;
        for (int k = 0; k < 4; ++k) {
          va |= Level(x, mode) << (8 * k);
          vb |= Level(x, mode) << (8 * k);
        }
      }
      a[i][e] = va;
      b[i][e] = vb;
    }
  v16i acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = v16i{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[(3 * i + 1) % 8], acc[i], 0, 0, 0);
  }
  int t = 0;
  for (int i = 0; i < 8; ++i)
    for (int r = 0; r < 16; ++r) t ^= acc[i][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// bf16 operands: mode 0 the constant 1.0, mode 1 values of roughly unit
// magnitude with random signs and mantissas (what a normalized activation
// times a weight gives the GEMM).
__device__ __bf16 Bf16Value(unsigned& x, int mode) {
  if (mode == 0) return static_cast<__bf16>(1.0f);
  x = x * 1664525u + 1013904223u;
  const float u = static_cast<float>(x >> 8) * (1.0f / 16777216.0f);  // [0, 1)
  return static_cast<__bf16>((u - 0.5f) * 4.0f);
}

__global__ void __launch_bounds__(256) MfmaBf16Probe(float* out, int iters, int mode) {
  bf16x8 a[8], b[8];
  unsigned x = 2654435761u * (blockIdx.x * 256 + threadIdx.x) + 777u;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 8; ++e) {
      a[i][e] = Bf16Value(x, mode);
      b[i][e] = Bf16Value(x, mode);
    }
  v16f acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = v16f{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[(3 * i + 1) % 8], acc[i], 0, 0, 0);
  }
  float t = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int r = 0; r < 16; ++r) t += acc[i][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

typedef float v4f __attribute__((ext_vector_type(4)));

// The same on v_mfma_f32_16x16x32_bf16 (16 x 16 tiles, K = 32 per issue).
__global__ void __launch_bounds__(256) MfmaBf16Probe16(float* out, int iters, int mode) {
  bf16x8 a[8], b[8];
  unsigned x = 2654435761u * (blockIdx.x * 256 + threadIdx.x) + 777u;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 8; ++e) {
      a[i][e] = Bf16Value(x, mode);
      b[i][e] = Bf16Value(x, mode);
    }
  v4f acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = v4f{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[(3 * i + 1) % 8], acc[i], 0, 0, 0);
  }
  float t = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int r = 0; r < 4; ++r) t += acc[i][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// v_mfma_f32_32x32x16_f16 on the same operand pattern.
__global__ void __launch_bounds__(256) MfmaF16Probe(float* out, int iters, int mode) {
  f16x8 a[8], b[8];
  unsigned x = 2654435761u * (blockIdx.x * 256 + threadIdx.x) + 777u;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 8; ++e) {
      a[i][e] = static_cast<_Float16>(static_cast<float>(Bf16Value(x, mode)));
      b[i][e] = static_cast<_Float16>(static_cast<float>(Bf16Value(x, mode)));
    }
  v16f acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = v16f{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[(3 * i + 1) % 8], acc[i], 0, 0, 0);
  }
  float t = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int r = 0; r < 16; ++r) t += acc[i][r];
  out[blockIdx.x * 256 + threadIdx.x] = t;
}

}  // namespace

// shape 32: v_mfma_f32_32x32x16_bf16, 16: v_mfma_f32_16x16x32_bf16,
// 33: v_mfma_f32_32x32x16_f16.
extern "C" float seeai_probe_mfma_bf16_shape(int shape, int workgroups, int iters, int mode,
                                             float* out) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
  auto k = shape == 16 ? MfmaBf16Probe16 : shape == 33 ? MfmaF16Probe : MfmaBf16Probe;
  hipLaunchKernelGGL(k, dim3(workgroups), dim3(256), 0, 0, out, 16, mode);  // warm-up
  hipEventRecord(e0, 0);
  hipLaunchKernelGGL(k, dim3(workgroups), dim3(256), 0, 0, out, iters, mode);
  hipEventRecord(e1, 0);
  float ms = -1.0f;
  if (hipEventSynchronize(e1) == hipSuccess && hipGetLastError() == hipSuccess)
    hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  return ms;
}

extern "C" float seeai_probe_mfma_bf16(int workgroups, int iters, int mode, float* out) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
  hipLaunchKernelGGL(MfmaBf16Probe, dim3(workgroups), dim3(256), 0, 0, out, 16, mode);  // warm-up
  hipEventRecord(e0, 0);
  hipLaunchKernelGGL(MfmaBf16Probe, dim3(workgroups), dim3(256), 0, 0, out, iters, mode);
  hipEventRecord(e1, 0);
  float ms = -1.0f;
  if (hipEventSynchronize(e1) == hipSuccess && hipGetLastError() == hipSuccess)
    hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  return ms;
}

// Runs the probe with `workgroups` x 256 lanes (workgroups / 256 waves per
// SIMD on 256 CUs), `iters` loop trips, operand set `mode`; returns the
// kernel time in milliseconds (HIP events), or a negative value on error.
// `out` receives workgroups * 256 ints.
extern "C" float seeai_probe_mfma_i8(int workgroups, int iters, int mode, int* out) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
  hipLaunchKernelGGL(MfmaI8Probe, dim3(workgroups), dim3(256), 0, 0, out, 16, mode);  // warm-up
  hipEventRecord(e0, 0);
  hipLaunchKernelGGL(MfmaI8Probe, dim3(workgroups), dim3(256), 0, 0, out, iters, mode);
  hipEventRecord(e1, 0);
  float ms = -1.0f;
  if (hipEventSynchronize(e1) == hipSuccess && hipGetLastError() == hipSuccess)
    hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  return ms;
}
