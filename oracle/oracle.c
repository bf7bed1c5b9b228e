/*
 * oracle.c -- CPU restatement of the SeeAI executor kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of it.
 * Built with gcc -O2 -ffp-contract=off so that each expression rounds the
 * way the reference's x86-64 build rounds it (no FMA contraction).  Every
 * function names the reference lines it restates; the reductions follow
 * the reference's order exactly (k-quads for the NN core, 8 k-lanes for the
 * NT core, double accumulators where the reference uses double, ParallelFor
 * chunk partials combined in chunk order).
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Shared helpers                                                           */
/* ------------------------------------------------------------------------ */

enum { kMaxChunks = 256 };             /* parallel_for.h:53 */
static const size_t kGrainCheap = 32768; /* kernel_policy.h:39 */
static const size_t kGrainMath = 4096;   /* kernel_policy.h:40 */

/* parallel_for.h:55-67 */
size_t orc_chunk_grain(size_t n, size_t grain) {
  if (grain == 0) grain = 1;
  size_t cap = (n + kMaxChunks - 1) / kMaxChunks;
  return grain < cap ? cap : grain;
}
size_t orc_chunk_count(size_t n, size_t grain) {
  if (n == 0) return 0;
  size_t g = orc_chunk_grain(n, grain);
  return (n + g - 1) / g;
}
/* kernel_policy.h:43-45 */
static size_t row_grain(size_t per_row, size_t budget) {
  return per_row == 0 ? budget : (budget / per_row > 0 ? budget / per_row : 1);
}

/* Threads.  Work is cut into the reference's ParallelFor chunks
 * (parallel_for.h:50-67: chunk = max(grain, ceil(n / 256))) and the chunks
 * are handed to the threads in any order; every chunk writes only its own
 * outputs (and its own partial, combined afterwards in chunk order), so the
 * bits are those of one thread at every thread count, as the reference's
 * "same bits, any thread count" rule requires.  The count is
 * orc_set_threads(), else SEEAI_ORACLE_THREADS, else 1. */
typedef void (*orc_chunk_fn)(void* ctx, size_t begin, size_t end, size_t chunk);
static int g_threads = 0;

void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int orc_threads(void) {
  if (g_threads <= 0) {
    const char* e = getenv("SEEAI_ORACLE_THREADS");
    const int n = e ? atoi(e) : 1;
    g_threads = n > 0 ? n : 1;
  }
  return g_threads;
}

typedef struct {
  orc_chunk_fn fn;
  void* ctx;
  size_t n, grain, count;
  size_t next;   /* the next chunk to take */
} OrcWork;

static void orc_run_chunks(OrcWork* w) {
  for (;;) {
    const size_t c = __atomic_fetch_add(&w->next, 1, __ATOMIC_RELAXED);
    if (c >= w->count) break;
    const size_t b = c * w->grain;
    const size_t e = b + w->grain < w->n ? b + w->grain : w->n;
    w->fn(w->ctx, b, e, c);
  }
}

/* A persistent pool (the reference keeps one too, parallel_for.h): worker i
 * sleeps until its own generation word moves, so a job wakes exactly the
 * workers it seats (seats < workers leaves the rest asleep); the caller works
 * beside them and waits on `done` until every seated worker has left the
 * job. */
enum { kMaxWorkers = 255 };
static struct {
  pthread_mutex_t mu;
  pthread_cond_t done;
  pthread_cond_t go[kMaxWorkers];
  unsigned long gen[kMaxWorkers]; /* worker i's job generation */
  int workers;
  OrcWork* job;
  int busy; /* seated workers still inside the current job */
  int quit; /* set by orc_pool_stop: the next wake ends the worker */
} g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .done = PTHREAD_COND_INITIALIZER};

/* Worker i starts at generation 0 (its creator zeroed gen[i] and seats it
 * in the job being published, which moves gen[i] to 1). */
static void* orc_pool_worker(void* arg) {
  const int i = (int)(uintptr_t)arg;
  unsigned long seen = 0;
  pthread_mutex_lock(&g_pool.mu);
  for (;;) {
    while (g_pool.gen[i] == seen) pthread_cond_wait(&g_pool.go[i], &g_pool.mu);
    seen = g_pool.gen[i];
    if (g_pool.quit) {
      if (--g_pool.busy == 0) pthread_cond_signal(&g_pool.done);
      pthread_mutex_unlock(&g_pool.mu);
      return NULL;
    }
    OrcWork* w = g_pool.job;
    pthread_mutex_unlock(&g_pool.mu);
    orc_run_chunks(w);
    pthread_mutex_lock(&g_pool.mu);
    if (--g_pool.busy == 0) pthread_cond_signal(&g_pool.done);
  }
  return NULL;
}

/* Runs fn over [0, n) in chunks of orc_chunk_grain(n, grain) on the caller
 * and up to orc_threads() - 1 pool workers; returns the chunk count.  Not
 * reentrant: one job at a time (the oracle runs one instruction at a time).
 * `unit_cost` (operations per unit, 0 = unknown) caps the threads at one
 * per kThreadWork operations, so a small job stays on the calling thread as
 * the reference's small tensors do (kernel_policy.h:36-40: grains chosen so
 * small tensors never leave the calling thread); the chunks, and so the
 * bits, do not depend on it. */
enum { kThreadWork = 1 << 22 };
static size_t orc_parallel_cost(size_t n, size_t grain, size_t unit_cost, orc_chunk_fn fn,
                                void* ctx) {
  if (n == 0) return 0;
  OrcWork w = {fn, ctx, n, orc_chunk_grain(n, grain), 0, 0};
  w.count = (n + w.grain - 1) / w.grain;
  int t = orc_threads();
  if ((size_t)t > w.count) t = (int)w.count;
  if (unit_cost > 0) {
    const double work = (double)n * (double)unit_cost;
    const double cap = work / kThreadWork;
    if (cap < (double)t) t = cap < 1.0 ? 1 : (int)cap;
  }
  if (t <= 1) {
    orc_run_chunks(&w);
    return w.count;
  }
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.workers < t - 1 && g_pool.workers < kMaxWorkers) {
    const int i = g_pool.workers;
    pthread_cond_init(&g_pool.go[i], NULL);
    g_pool.gen[i] = 0;
    pthread_t id;
    if (pthread_create(&id, NULL, orc_pool_worker, (void*)(uintptr_t)i) != 0) break;
    pthread_detach(id);
    ++g_pool.workers;
  }
  const int seats = t - 1 < g_pool.workers ? t - 1 : g_pool.workers;
  g_pool.job = &w;
  g_pool.busy = seats;
  for (int i = 0; i < seats; ++i) {
    ++g_pool.gen[i];
    pthread_cond_signal(&g_pool.go[i]);
  }
  pthread_mutex_unlock(&g_pool.mu);
  orc_run_chunks(&w);
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.busy > 0) pthread_cond_wait(&g_pool.done, &g_pool.mu);
  pthread_mutex_unlock(&g_pool.mu);
  return w.count;
}
static size_t orc_parallel(size_t n, size_t grain, orc_chunk_fn fn, void* ctx) {
  return orc_parallel_cost(n, grain, 0, fn, ctx);
}

/* Ends every pool worker and waits until each has left its loop; the next
 * orc_parallel starts a fresh pool. */
void orc_pool_stop(void) {
  pthread_mutex_lock(&g_pool.mu);
  if (g_pool.workers > 0) {
    g_pool.quit = 1;
    g_pool.busy = g_pool.workers;
    for (int i = 0; i < g_pool.workers; ++i) {
      ++g_pool.gen[i];
      pthread_cond_signal(&g_pool.go[i]);
    }
    while (g_pool.busy > 0) pthread_cond_wait(&g_pool.done, &g_pool.mu);
    for (int i = 0; i < g_pool.workers; ++i) pthread_cond_destroy(&g_pool.go[i]);
    g_pool.workers = 0;
    g_pool.quit = 0;
  }
  pthread_mutex_unlock(&g_pool.mu);
}
/* kernel_policy.h:122-136: the shared activation expressions. */
static const float kGeluC = 0.7978845608028654f;
static const float kGeluA = 0.044715f;
static float sigmoid_expr(float x) { return 1.0f / (1.0f + expf(-x)); }
static float relu_expr(float x) { return x > 0.0f ? x : 0.0f; }
static float gelu_expr(float x) {
  const float t = tanhf(kGeluC * (x + kGeluA * x * x * x));
  return 0.5f * x * (1.0f + t);
}
static float silu_expr(float x) { return x * sigmoid_expr(x); }
static float act_expr(int act, float v) {
  switch (act) {
    case 1: return relu_expr(v);
    case 2: return gelu_expr(v);
    case 3: return silu_expr(v);
    default: return v;
  }
}

/* source/plan/bf16.h:28-30: exact widening. */
static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ------------------------------------------------------------------------ */
/* GEMM family                                                              */
/* ------------------------------------------------------------------------ */

/* The NN/TN core's per-element reduction (gemm.cc:36-43, 73-187; the
 * reference test's ReferenceNN, kernels_test.cc:1733-1757):
 *   c += a0*b0 + a1*b1 + a2*b2 + a3*b3   over k-quads aligned to k = 0,
 *   then one term per k for the K % 4 tail; a_i = alpha * A (one rounding).
 * B element kinds: 0 f32, 1 int8 (widened), 2 bf16 (widened); with a
 * column scale the widened int8 is multiplied by cs[n] (gemm.cc:98-104).
 * `accumulate` keeps C's prior contents (GemmAccNN, gemm.cc:617-624). */
typedef struct {
  const float* A;
  const float* B; /* widened to f32 (int8 times its column scale, bf16) */
  float* C;
  size_t M, N, K;
  float alpha;
  int a_transposed, accumulate;
} NnArgs;
/* One output row at a time: the row's N sums advance together quad by quad,
 * each element through exactly the chain above (its order of operations is
 * unchanged; only independent elements sit side by side in vector lanes). */
__attribute__((target_clones("avx2", "default")))
static void nn_rows(void* ctx, size_t m0, size_t m1, size_t chunk) {
  (void)chunk;
  const NnArgs* g = (const NnArgs*)ctx;
  const float* A = g->A;
  const float* B = g->B;
  const size_t M = g->M, N = g->N, K = g->K;
  const float alpha = g->alpha;
  for (size_t m = m0; m < m1; ++m) {
    float* restrict c = g->C + m * N;
    if (!g->accumulate)
      for (size_t n = 0; n < N; ++n) c[n] = 0.0f;
#define ORC_A(kk) (g->a_transposed ? A[(kk) * M + m] : A[m * K + (kk)])
    size_t k = 0;
    for (; k + 4 <= K; k += 4) {
      const float a0 = alpha * ORC_A(k + 0);
      const float a1 = alpha * ORC_A(k + 1);
      const float a2 = alpha * ORC_A(k + 2);
      const float a3 = alpha * ORC_A(k + 3);
      const float* restrict b0 = B + (k + 0) * N;
      const float* restrict b1 = B + (k + 1) * N;
      const float* restrict b2 = B + (k + 2) * N;
      const float* restrict b3 = B + (k + 3) * N;
      for (size_t n = 0; n < N; ++n) c[n] += a0 * b0[n] + a1 * b1[n] + a2 * b2[n] + a3 * b3[n];
    }
    for (; k < K; ++k) {
      const float a = alpha * ORC_A(k);
      const float* restrict bk = B + k * N;
      for (size_t n = 0; n < N; ++n) c[n] += a * bk[n];
    }
#undef ORC_A
  }
}
/* B's elements as the core reads them: f32 as is; int8 widened, times the
 * column scale where there is one (gemm.cc:98-104); bf16 widened.  Returns
 * B itself for f32, else a buffer the caller frees. */
static const float* widen(const void* B, int b_kind, const float* col_scale, size_t rows,
                          size_t cols, int scale_by_col) {
  if (b_kind == 0) return (const float*)B;
  const size_t count = rows * cols;
  float* w = (float*)malloc((count ? count : 1) * sizeof(float));
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < cols; ++c) {
      const size_t i = r * cols + c;
      if (b_kind == 1)
        w[i] = scale_by_col && col_scale ? (float)((const int8_t*)B)[i] * col_scale[c]
                                         : (float)((const int8_t*)B)[i];
      else
        w[i] = bf16_to_f32(((const uint16_t*)B)[i]);
    }
  return w;
}
static void nn_core(const float* A, const void* B, int b_kind,
                    const float* col_scale, float* C, size_t M, size_t N,
                    size_t K, float alpha, int a_transposed, int accumulate) {
  const float* Bf = widen(B, b_kind, col_scale, K, N, 1);
  NnArgs g = {A, Bf, C, M, N, K, alpha, a_transposed, accumulate};
  orc_parallel_cost(M, 1, N * K, nn_rows, &g);
  if (Bf != B) free((void*)Bf);
}

/* The NT core (gemm.cc:304-527; ReferenceNT, kernels_test.cc:1759-1775):
 * lane l accumulates every k = l (mod 8) in k order, the lanes combine in
 * lane order, and alpha multiplies the finished dot.  The eight lanes are
 * one 8-wide vector; each lane's chain is the reference's. */
typedef struct {
  const float* A;
  const float* B; /* [N, K], widened to f32 */
  float* C;
  size_t N, K;
  float alpha;
} NtArgs;
__attribute__((target_clones("avx2", "default")))
static void nt_rows(void* ctx, size_t m0, size_t m1, size_t chunk) {
  (void)chunk;
  const NtArgs* g = (const NtArgs*)ctx;
  const size_t N = g->N, K = g->K;
  for (size_t m = m0; m < m1; ++m) {
    const float* restrict a = g->A + m * K;
    for (size_t n = 0; n < N; ++n) {
      const float* restrict b = g->B + n * K;
      float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      size_t k = 0;
      for (; k + 8 <= K; k += 8)
        for (int l = 0; l < 8; ++l) lane[l] += a[k + l] * b[k + l];
      for (; k < K; ++k) lane[k % 8] += a[k] * b[k];
      float s = lane[0];
      for (int l = 1; l < 8; ++l) s += lane[l];
      g->C[m * N + n] = g->alpha * s;
    }
  }
}
static void nt_core(const float* A, const void* B, int b_kind, float* C,
                    size_t M, size_t N, size_t K, float alpha) {
  const float* Bf = widen(B, b_kind, NULL, N, K, 0);
  NtArgs g = {A, Bf, C, N, K, alpha};
  orc_parallel_cost(M, 1, N * K, nt_rows, &g);
  if (Bf != B) free((void*)Bf);
}

/* gemm.cc:562-578: addend C = D + s, then the bias/act epilogue
 * C = act(C + bias[n]) (gemm.cc:536-560). */
static void addend_rows(float* C, const float* D, size_t M, size_t N) {
  for (size_t i = 0; i < M * N; ++i) C[i] = D[i] + C[i];
}
static void epilogue_rows(float* C, const float* bias, int act, size_t M,
                          size_t N) {
  if (!bias && act == 0) return;
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      const float v = bias ? C[m * N + n] + bias[n] : C[m * N + n];
      C[m * N + n] = act_expr(act, v);
    }
}

/* gemm.cc:582-593 */
void orc_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act, const float* addend,
                 float alpha) {
  nn_core(A, B, 0, NULL, C, M, N, K, alpha, 0, 0);
  if (addend) addend_rows(C, addend, M, N);
  epilogue_rows(C, bias, act, M, N);
}
/* gemm.cc:595-603 */
void orc_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha) {
  nt_core(A, B, 0, C, M, N, K, alpha);
  if (addend) addend_rows(C, addend, M, N);
}
/* gemm.cc:605-615 */
void orc_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha) {
  nn_core(A, B, 0, NULL, C, M, N, K, alpha, 1, 0);
  if (addend) addend_rows(C, addend, M, N);
}
/* gemm.cc:617-624 */
void orc_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha) {
  nn_core(A, B, 0, NULL, C, M, N, K, alpha, 0, 1);
}
/* gemm.cc:626-638: per-tensor scale folds into A as alpha; a column scale
 * joins B's widening. */
void orc_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act,
                    const float* col_scale) {
  nn_core(A, B, 1, col_scale, C, M, N, K, col_scale ? 1.0f : scale, 0, 0);
  epilogue_rows(C, NULL, act, M, N);
}
/* gemm.cc:646-674: per-tensor scale multiplies the finished dot (NT alpha);
 * a k-scale pre-multiplies A's elements, then the NT core runs with 1. */
void orc_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, const float* k_scale) {
  if (!k_scale) {
    nt_core(A, B, 1, C, M, N, K, scale);
    return;
  }
  float* scaled = (float*)malloc((M * K > 0 ? M * K : 1) * sizeof(float));
  for (size_t m = 0; m < M; ++m)
    for (size_t k = 0; k < K; ++k) scaled[m * K + k] = A[m * K + k] * k_scale[k];
  nt_core(scaled, B, 1, C, M, N, K, 1.0f);
  free(scaled);
}
/* gemm.cc:679-699 */
void orc_gemm_nn_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K, const float* bias, int act) {
  nn_core(A, B, 2, NULL, C, M, N, K, 1.0f, 0, 0);
  epilogue_rows(C, bias, act, M, N);
}
void orc_gemm_nt_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K) {
  nt_core(A, B, 2, C, M, N, K, 1.0f);
}

/* ------------------------------------------------------------------------ */
/* W8A8 -- no reference counterpart.                                        */
/* ------------------------------------------------------------------------ */

/* The scale rule of the reference's column-scale packer
 * (compiler/backend/allocation/arena_binder.cc:129-154): max|x| / 127, an
 * all-zero vector takes 1, a subnormal quotient takes FLT_MIN.  The level
 * rule (arena_binder.cc:170-177): divide (never a hoisted reciprocal),
 * round half away from zero, clamp to [-127, 127]. */
static float quant_scale(float max_abs) {
  if (max_abs == 0.0f) return 1.0f;
  const float s = max_abs / 127.0f;
  return s > FLT_MIN ? s : FLT_MIN;
}
static int8_t quant_level(float x, float scale) {
  float r = roundf(x / scale);
  if (r < -127.0f) r = -127.0f;
  if (r > 127.0f) r = 127.0f;
  return (int8_t)r;
}
void orc_quantize_rows(const float* X, int8_t* Q, float* scale, size_t rows,
                       size_t cols) {
  for (size_t r = 0; r < rows; ++r) {
    float mx = 0.0f;
    for (size_t c = 0; c < cols; ++c) mx = fmaxf(mx, fabsf(X[r * cols + c]));
    const float s = quant_scale(mx);
    scale[r] = s;
    for (size_t c = 0; c < cols; ++c) Q[r * cols + c] = quant_level(X[r * cols + c], s);
  }
}
void orc_quantize_cols(const float* W, int8_t* Q, float* scale, size_t K,
                       size_t N) {
  for (size_t n = 0; n < N; ++n) {
    float mx = 0.0f;
    for (size_t k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(W[k * N + n]));
    scale[n] = quant_scale(mx);
  }
  for (size_t k = 0; k < K; ++k)
    for (size_t n = 0; n < N; ++n) Q[k * N + n] = quant_level(W[k * N + n], scale[n]);
}
typedef struct {
  const int8_t *QA, *QW;
  const float *sa, *sw;
  int32_t* acc;
  float* C;
  size_t N, K;
} W8Args;
static void w8a8_rows(void* ctx, size_t m0, size_t m1, size_t chunk) {
  (void)chunk;
  const W8Args* g = (const W8Args*)ctx;
  const int8_t *QA = g->QA, *QW = g->QW;
  const float *sa = g->sa, *sw = g->sw;
  int32_t* acc = g->acc;
  float* C = g->C;
  const size_t N = g->N, K = g->K;
  int32_t* row = (int32_t*)malloc((N ? N : 1) * sizeof(int32_t));
  for (size_t m = m0; m < m1; ++m) {
    memset(row, 0, N * sizeof(int32_t));
    for (size_t k = 0; k < K; ++k) {
      const int32_t a = QA[m * K + k];
      const int8_t* w = QW + k * N;
      for (size_t n = 0; n < N; ++n) row[n] += a * (int32_t)w[n];
    }
    for (size_t n = 0; n < N; ++n) {
      if (acc) acc[m * N + n] = row[n];
      C[m * N + n] = ((float)row[n] * sa[m]) * sw[n];
    }
  }
  free(row);
}
void orc_gemm_w8a8(const int8_t* QA, const float* sa, const int8_t* QW,
                   const float* sw, int32_t* acc, float* C, size_t M,
                   size_t N, size_t K) {
  W8Args g = {QA, QW, sa, sw, acc, C, N, K};
  orc_parallel(M, 1, w8a8_rows, &g);
}

/* ------------------------------------------------------------------------ */
/* Elementwise / activation / normalization                                 */
/* ------------------------------------------------------------------------ */

/* elementwise.cc:16-27 */
void orc_add_ew(const float* x, const float* y, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] + y[i];
}
void orc_mul_ew(const float* x, const float* y, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * y[i];
}
/* elementwise.cc:29-36 */
void orc_add_bias(const float* x, const float* b, float* out, size_t rows,
                  size_t cols) {
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < cols; ++c) out[r * cols + c] = x[r * cols + c] + b[c];
}
/* activation.cc:22-75 */
void orc_relu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = relu_expr(x[i]);
}
void orc_relu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  for (size_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? dy[i] : 0.0f;
}
void orc_gelu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = gelu_expr(x[i]);
}
void orc_gelu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float u = kGeluC * (v + kGeluA * v * v * v);
    const float t = tanhf(u);
    const float one_minus_t2 = 1.0f - t * t;
    const float tail =
        one_minus_t2 == 0.0f
            ? 0.0f
            : 0.5f * v * one_minus_t2 * (kGeluC * (1.0f + 3.0f * kGeluA * v * v));
    dx[i] = dy[i] * (0.5f * (1.0f + t) + tail);
  }
}
void orc_silu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = silu_expr(x[i]);
}
void orc_silu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float s = sigmoid_expr(x[i]);
    dx[i] = dy[i] * (s * (1.0f + x[i] * (1.0f - s)));
  }
}
/* elementwise.cc:44-48 */
void orc_scale(const float* x, float* out, float alpha, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = alpha * x[i];
}
/* elementwise.cc:160-187: per-column sums in row order. */
void orc_reduce_rows(const float* dy, float* db, size_t rows, size_t cols) {
  for (size_t c = 0; c < cols; ++c) {
    float acc = 0.0f;
    for (size_t r = 0; r < rows; ++r) acc += dy[r * cols + c];
    db[c] = acc;
  }
}
/* elementwise.cc:189-199 */
void orc_fill(float* dst, float value, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = value;
}
void orc_copy(const float* src, float* dst, size_t n) {
  memcpy(dst, src, n * sizeof(float));
}
/* elementwise.cc:38-42 */
void orc_accumulate(float* dst, const float* src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] += src[i];
}
/* elementwise.cc:151-158 */
void orc_embed_fwd(const int32_t* tokens, const float* table, float* out,
                   size_t rows, size_t dim) {
  for (size_t r = 0; r < rows; ++r)
    memcpy(out + r * dim, table + (size_t)tokens[r] * dim, dim * sizeof(float));
}
/* elementwise.cc:56-149 and instruction.h:270-297: each stage evaluates
 * its standalone kernel's expression on the running value. */
void orc_fused_map(const float* x, const float* other1, const float* other2,
                   float* out, size_t n, uint64_t stages, float imm0,
                   float imm1) {
  uint8_t prog[4];
  size_t count = 0;
  for (; count < 4; ++count) {
    prog[count] = (uint8_t)(stages >> (8 * count));
    if ((prog[count] & 0x0F) == 0) break;
  }
  if (count == 0) return;
  for (size_t i = 0; i < n; ++i) {
    float run = x[i];
    for (size_t s = 0; s < count; ++s) {
      const uint8_t st = prog[s];
      const int arg = (st >> 4) & 0x03;
      const int right = (st & 0x80) != 0;
      const float* other = arg == 1 ? other1 : other2;
      switch (st & 0x0F) {
        case 1: run = right ? other[i] + run : run + other[i]; break;
        case 2: run = right ? other[i] * run : run * other[i]; break;
        case 3: run = (arg == 0 ? imm0 : imm1) * run; break;
        case 4: run = relu_expr(run); break;
        case 5: run = gelu_expr(run); break;
        case 6: run = silu_expr(run); break;
        default: break;
      }
    }
    out[i] = run;
  }
}
/* normalization.cc:17-45 */
void orc_layernorm_fwd(const float* x, const float* gamma, const float* beta,
                       float* y, float* mean, float* rstd, size_t rows,
                       size_t cols, float eps) {
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double sum = 0.0;
    for (size_t c = 0; c < cols; ++c) sum += xr[c];
    const float mu = (float)(sum / (double)cols);
    double var = 0.0;
    for (size_t c = 0; c < cols; ++c) {
      const double d = (double)xr[c] - mu;
      var += d * d;
    }
    const float rs = 1.0f / sqrtf((float)(var / (double)cols) + eps);
    mean[r] = mu;
    rstd[r] = rs;
    for (size_t c = 0; c < cols; ++c)
      y[r * cols + c] = (xr[c] - mu) * rs * gamma[c] + beta[c];
  }
}
/* normalization.cc:47-78 */
void orc_layernorm_bwd(const float* dy, const float* x, const float* gamma,
                       const float* mean, const float* rstd, float* dx,
                       size_t rows, size_t cols) {
  const float inv_d = 1.0f / (float)cols;
  for (size_t r = 0; r < rows; ++r) {
    const float* dyr = dy + r * cols;
    const float* xr = x + r * cols;
    const float mu = mean[r], rs = rstd[r];
    double sum_g = 0.0, sum_gx = 0.0;
    for (size_t c = 0; c < cols; ++c) {
      const float xhat = (xr[c] - mu) * rs;
      const float g = dyr[c] * gamma[c];
      sum_g += g;
      sum_gx += (double)g * xhat;
    }
    const float mg = (float)sum_g * inv_d;
    const float mgx = (float)sum_gx * inv_d;
    for (size_t c = 0; c < cols; ++c) {
      const float xhat = (xr[c] - mu) * rs;
      const float g = dyr[c] * gamma[c];
      dx[r * cols + c] = rs * (g - mg - xhat * mgx);
    }
  }
}
/* normalization.cc:80-95 */
void orc_rmsnorm_fwd(const float* x, const float* gamma, float* y, float* rstd,
                     size_t rows, size_t cols, float eps) {
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double ss = 0.0;
    for (size_t c = 0; c < cols; ++c) ss += (double)xr[c] * xr[c];
    const float rs = 1.0f / sqrtf((float)(ss / (double)cols) + eps);
    rstd[r] = rs;
    for (size_t c = 0; c < cols; ++c) y[r * cols + c] = xr[c] * rs * gamma[c];
  }
}
/* normalization.cc:97-113 */
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* gamma,
                     const float* rstd, float* dx, size_t rows, size_t cols) {
  const float inv_d = 1.0f / (float)cols;
  for (size_t r = 0; r < rows; ++r) {
    const float* dyr = dy + r * cols;
    const float* xr = x + r * cols;
    const float rs = rstd[r];
    double sum_gx = 0.0;
    for (size_t c = 0; c < cols; ++c) sum_gx += (double)(dyr[c] * gamma[c]) * xr[c];
    const float mgx = (float)sum_gx * inv_d;
    for (size_t c = 0; c < cols; ++c)
      dx[r * cols + c] = rs * (dyr[c] * gamma[c] - xr[c] * rs * rs * mgx);
  }
}
/* attention.cc:103-174: rotation by s * base^(-2c/d) through the
 * multiplicative frequency recurrence (or the table). */
void orc_rope(const float* x, float* y, size_t B, size_t S, size_t H,
              size_t d, float base, const float* table, int backward) {
  const size_t D = H * d, half = d / 2;
  const float step = powf(base, -2.0f / (float)d);
  for (size_t u = 0; u < B * S * H; ++u) {
    const size_t s = (u / H) % S;
    const float* xr = x + (u / H) * D + (u % H) * d;
    float* yr = y + (u / H) * D + (u % H) * d;
    const float* row = table ? table + s * half * 2 : NULL;
    float freq = 1.0f;
    for (size_t c = 0; c + 1 < d; c += 2) {
      float cs, sn;
      if (row) {
        cs = row[c];
        sn = row[c + 1];
      } else {
        const float theta = (float)s * freq;
        cs = cosf(theta);
        sn = sinf(theta);
        freq *= step;
      }
      const float a = xr[c], b2 = xr[c + 1];
      if (backward) {
        yr[c] = a * cs + b2 * sn;
        yr[c + 1] = -a * sn + b2 * cs;
      } else {
        yr[c] = a * cs - b2 * sn;
        yr[c + 1] = a * sn + b2 * cs;
      }
    }
  }
}
void orc_rope_table(float* table, size_t S, size_t d, float base) {
  const size_t half = d / 2;
  const float step = powf(base, -2.0f / (float)d);
  for (size_t s = 0; s < S; ++s) {
    float* row = table + s * half * 2;
    float freq = 1.0f;
    for (size_t c = 0; c < half; ++c) {
      const float theta = (float)s * freq;
      row[2 * c] = cosf(theta);
      row[2 * c + 1] = sinf(theta);
      freq *= step;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

/* attention.cc:176-185 */
void orc_segment_starts(const int32_t* tokens, int32_t* starts, size_t B,
                        size_t S, int32_t eos) {
  for (size_t b = 0; b < B; ++b) {
    int32_t start = 0;
    for (size_t t = 0; t < S; ++t) {
      starts[b * S + t] = start;
      if (tokens[b * S + t] == eos) start = (int32_t)(t + 1);
    }
  }
}

/* A double-accumulated dot of two f32 rows in c order (attention.cc:39-59,
 * 396-437): the product of two floats is exact in double. */
static double dot_d(const float* a, const float* b, size_t d) {
  double acc = 0.0;
  for (size_t c = 0; c < d; ++c) acc += (double)a[c] * (double)b[c];
  return acc;
}
static size_t clamp_start(const int32_t* starts, size_t b, size_t S, size_t i) {
  if (!starts) return 0;
  const int32_t s0 = starts[b * S + i];
  return s0 <= 0 ? 0 : ((size_t)s0 < i ? (size_t)s0 : i);
}
/* instruction.h:246-250 */
static size_t stats_start(float stored, size_t i) {
  if (!(stored > 0.0f)) return 0;
  const float cap = (float)i;
  return stored >= cap ? i : (size_t)stored;
}

/* attention.cc:187-241 */
void orc_attn_fwd(const float* q, const float* k, const float* v, float* o,
                  float* probs, size_t B, size_t S, size_t H, size_t d,
                  const int32_t* starts) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* qi = q + (b * S + i) * D + h * d;
    float* prow = probs + u * S;
    const size_t j0 = clamp_start(starts, b, S, i);
    for (size_t j = 0; j < j0; ++j) prow[j] = 0.0f;
    float row_max = -INFINITY;
    for (size_t j = j0; j <= i; ++j) {
      const float s = (float)dot_d(qi, k + (b * S + j) * D + h * d, d) * inv_sqrt_d;
      prow[j] = s;
      if (s > row_max) row_max = s;
    }
    double denom = 0.0;
    for (size_t j = j0; j <= i; ++j) {
      const float e = expf(prow[j] - row_max);
      prow[j] = e;
      denom += e;
    }
    const float inv_denom = 1.0f / (float)denom;
    for (size_t j = j0; j <= i; ++j) prow[j] *= inv_denom;
    for (size_t j = i + 1; j < S; ++j) prow[j] = 0.0f;
    float* oi = o + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) oi[c] = 0.0f;
    for (size_t j = j0; j <= i; ++j) {
      const float p = prow[j];
      const float* vj = v + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) oi[c] += p * vj[c];
    }
  }
}
/* attention.cc:243-265 */
void orc_attn_dp(const float* dout, const float* v, float* dp, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* doi = dout + (b * S + i) * D + h * d;
    float* dprow = dp + u * S;
    for (size_t j = 0; j <= i; ++j)
      dprow[j] = (float)dot_d(doi, v + (b * S + j) * D + h * d, d);
    for (size_t j = i + 1; j < S; ++j) dprow[j] = 0.0f;
  }
}
/* attention.cc:267-284 */
void orc_attn_dv(const float* probs, const float* dout, float* dv, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    float* dvj = dv + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dvj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float p = probs[((b * H + h) * S + i) * S + j];
      const float* doi = dout + (b * S + i) * D + h * d;
      for (size_t c = 0; c < d; ++c) dvj[c] += p * doi[c];
    }
  }
}
/* attention.cc:286-302 */
void orc_softmax_rows_bwd(const float* probs, const float* dp, float* ds,
                          size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; ++r) {
    const float* pr = probs + r * cols;
    const float* dpr = dp + r * cols;
    double dot = 0.0;
    for (size_t c = 0; c < cols; ++c) dot += (double)dpr[c] * pr[c];
    const float sum = (float)dot;
    for (size_t c = 0; c < cols; ++c) ds[r * cols + c] = pr[c] * (dpr[c] - sum);
  }
}
/* attention.cc:304-322 */
void orc_attn_dq(const float* ds, const float* k, float* dq, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* dsrow = ds + u * S;
    float* dqi = dq + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) dqi[c] = 0.0f;
    for (size_t j = 0; j <= i; ++j) {
      const float g = dsrow[j] * inv_sqrt_d;
      const float* kj = k + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) dqi[c] += g * kj[c];
    }
  }
}
/* attention.cc:324-343 */
void orc_attn_dk(const float* ds, const float* q, float* dk, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    float* dkj = dk + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dkj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float g = ds[((b * H + h) * S + i) * S + j] * inv_sqrt_d;
      const float* qi = q + (b * S + i) * D + h * d;
      for (size_t c = 0; c < d; ++c) dkj[c] += g * qi[c];
    }
  }
}

/* p(i, j) from the stored (m, 1/l): attention.cc:405-431. */
static float prob_of(const float* qi, const float* kj, size_t d,
                     float inv_sqrt_d, float m, float inv_denom) {
  const float s = (float)dot_d(qi, kj, d) * inv_sqrt_d;
  const float e = expf(s - m);
  return e * inv_denom;
}

/* attention.cc:448-493 */
/* The tiled family's arguments; each unit u = (b, h, row) is independent. */
typedef struct {
  const float *q, *k, *v, *dout;
  float *o, *stats, *out;
  const int32_t* starts;
  size_t B, S, H, d;
} AttnArgs;

static void attn_fwd_units(void* ctx, size_t u0, size_t u1, size_t chunk) {
  (void)chunk;
  const AttnArgs* a = (const AttnArgs*)ctx;
  const float *q = a->q, *k = a->k, *v = a->v;
  float *o = a->o, *stats = a->stats;
  const int32_t* starts = a->starts;
  const size_t S = a->S, H = a->H, d = a->d;
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  float* prow = (float*)malloc((S ? S : 1) * sizeof(float));
  for (size_t u = u0; u < u1; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* qi = q + (b * S + i) * D + h * d;
    const size_t j0 = clamp_start(starts, b, S, i);
    float row_max = -INFINITY;
    for (size_t j = j0; j <= i; ++j) {
      const float s = (float)dot_d(qi, k + (b * S + j) * D + h * d, d) * inv_sqrt_d;
      prow[j] = s;
      if (s > row_max) row_max = s;
    }
    double denom = 0.0;
    for (size_t j = j0; j <= i; ++j) {
      const float e = expf(prow[j] - row_max);
      prow[j] = e;
      denom += e;
    }
    const float inv_denom = 1.0f / (float)denom;
    for (size_t j = j0; j <= i; ++j) prow[j] *= inv_denom;
    float* oi = o + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) oi[c] = 0.0f;
    for (size_t j = j0; j <= i; ++j) {
      const float p = prow[j];
      const float* vj = v + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) oi[c] += p * vj[c];
    }
    float* st = stats + u * 4;
    st[0] = row_max;
    st[1] = inv_denom;
    st[2] = 0.0f;
    st[3] = (float)j0;
  }
  free(prow);
}
void orc_attn_fwd_tiled(const float* q, const float* k, const float* v,
                        float* o, float* stats, size_t B, size_t S, size_t H,
                        size_t d, const int32_t* starts) {
  AttnArgs a = {q, k, v, NULL, o, stats, NULL, starts, B, S, H, d};
  orc_parallel_cost(B * H * S, 1, S * d, attn_fwd_units, &a);
}
/* attention.cc:495-535 */
static void attn_dq_units(void* ctx, size_t u0, size_t u1, size_t chunk) {
  (void)chunk;
  const AttnArgs* a = (const AttnArgs*)ctx;
  const float *q = a->q, *k = a->k, *v = a->v, *dout = a->dout;
  float *stats = a->stats, *dq = a->out;
  const size_t S = a->S, H = a->H, d = a->d;
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  float* prow = (float*)malloc((S ? 2 * S : 2) * sizeof(float));
  float* dprow = prow + S;
  for (size_t u = u0; u < u1; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* qi = q + (b * S + i) * D + h * d;
    const float* doi = dout + (b * S + i) * D + h * d;
    float* st = stats + u * 4;
    const size_t j0 = stats_start(st[3], i);
    for (size_t j = j0; j <= i; ++j)
      prow[j] = prob_of(qi, k + (b * S + j) * D + h * d, d, inv_sqrt_d, st[0], st[1]);
    double dot = 0.0;
    for (size_t j = j0; j <= i; ++j) {
      dprow[j] = (float)dot_d(doi, v + (b * S + j) * D + h * d, d);
      dot += (double)dprow[j] * prow[j];
    }
    const float delta = (float)dot;
    st[2] = delta;
    float* dqi = dq + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) dqi[c] = 0.0f;
    for (size_t j = j0; j <= i; ++j) {
      const float ds = prow[j] * (dprow[j] - delta);
      const float g = ds * inv_sqrt_d;
      const float* kj = k + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) dqi[c] += g * kj[c];
    }
  }
  free(prow);
}
void orc_attn_dq_tiled(const float* q, const float* k, const float* v,
                       const float* dout, float* stats, float* dq, size_t B,
                       size_t S, size_t H, size_t d) {
  AttnArgs a = {q, k, v, dout, NULL, stats, dq, NULL, B, S, H, d};
  orc_parallel_cost(B * H * S, 1, S * d, attn_dq_units, &a);
}
/* attention.cc:537-563 */
static void attn_dk_units(void* ctx, size_t u0, size_t u1, size_t chunk) {
  (void)chunk;
  const AttnArgs* a = (const AttnArgs*)ctx;
  const float *q = a->q, *k = a->k, *v = a->v, *dout = a->dout, *stats = a->stats;
  float* dk = a->out;
  const size_t S = a->S, H = a->H, d = a->d;
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = u0; u < u1; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    const float* kj = k + (b * S + j) * D + h * d;
    const float* vj = v + (b * S + j) * D + h * d;
    float* dkj = dk + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dkj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float* qi = q + (b * S + i) * D + h * d;
      const float* doi = dout + (b * S + i) * D + h * d;
      const float* st = stats + ((b * H + h) * S + i) * 4;
      if (j < stats_start(st[3], i)) continue;
      const float p = prob_of(qi, kj, d, inv_sqrt_d, st[0], st[1]);
      const float ds = p * ((float)dot_d(doi, vj, d) - st[2]);
      const float g = ds * inv_sqrt_d;
      for (size_t c = 0; c < d; ++c) dkj[c] += g * qi[c];
    }
  }
}
void orc_attn_dk_tiled(const float* q, const float* k, const float* v,
                       const float* dout, const float* stats, float* dk,
                       size_t B, size_t S, size_t H, size_t d) {
  AttnArgs a = {q, k, v, dout, NULL, (float*)stats, dk, NULL, B, S, H, d};
  orc_parallel_cost(B * H * S, 1, S * d, attn_dk_units, &a);
}
/* attention.cc:565-590 */
static void attn_dv_units(void* ctx, size_t u0, size_t u1, size_t chunk) {
  (void)chunk;
  const AttnArgs* a = (const AttnArgs*)ctx;
  const float *q = a->q, *k = a->k, *dout = a->dout, *stats = a->stats;
  float* dv = a->out;
  const size_t S = a->S, H = a->H, d = a->d;
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = u0; u < u1; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    const float* kj = k + (b * S + j) * D + h * d;
    float* dvj = dv + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dvj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float* qi = q + (b * S + i) * D + h * d;
      const float* doi = dout + (b * S + i) * D + h * d;
      const float* st = stats + ((b * H + h) * S + i) * 4;
      if (j < stats_start(st[3], i)) continue;
      const float p = prob_of(qi, kj, d, inv_sqrt_d, st[0], st[1]);
      for (size_t c = 0; c < d; ++c) dvj[c] += p * doi[c];
    }
  }
}
void orc_attn_dv_tiled(const float* q, const float* k, const float* dout,
                       const float* stats, float* dv, size_t B, size_t S,
                       size_t H, size_t d) {
  AttnArgs a = {q, k, NULL, dout, NULL, (float*)stats, dv, NULL, B, S, H, d};
  orc_parallel_cost(B * H * S, 1, S * d, attn_dv_units, &a);
}

/* ------------------------------------------------------------------------ */
/* Losses                                                                   */
/* ------------------------------------------------------------------------ */

/* loss.cc:21-32 (inv_T = 1: logits * 1.0f is exact). */
static void row_softmax(const float* logits, float* probs, size_t C) {
  float max_v = logits[0];
  for (size_t c = 1; c < C; ++c) max_v = fmaxf(max_v, logits[c]);
  float sum = 0.0f;
  for (size_t c = 0; c < C; ++c) {
    probs[c] = expf(logits[c] - max_v);
    sum += probs[c];
  }
  const float inv_sum = 1.0f / sum;
  for (size_t c = 0; c < C; ++c) probs[c] *= inv_sum;
}
/* loss.cc:45-51: NaN propagates, the clamp rescues underflow only. */
static double safe_log_term(float p) {
  const double safe = isnan(p) ? (double)p : (double)fmaxf(p, 1e-12f);
  return log(safe);
}
/* loss.cc:35-59: one double partial per ParallelFor chunk, in chunk order. */
typedef struct {
  const float* logits;
  const int32_t* labels;
  float* probs;
  size_t C;
  int masked;
  double part[kMaxChunks];
  uint64_t targets[kMaxChunks];
} XentArgs;
static void xent_chunk(void* ctx, size_t r0, size_t r1, size_t chunk) {
  XentArgs* a = (XentArgs*)ctx;
  const size_t C = a->C;
  double part = 0.0;
  uint64_t t = 0;
  for (size_t n = r0; n < r1; ++n) {
    row_softmax(a->logits + n * C, a->probs + n * C, C);
    if (a->masked && a->labels[n] < 0) continue;
    part -= safe_log_term(a->probs[n * C + (size_t)a->labels[n]]);
    ++t;
  }
  a->part[chunk] = part;
  a->targets[chunk] = t;
}
void orc_xent_fwd(const float* logits, const int32_t* labels, float* loss,
                  float* probs, size_t N, size_t C) {
  XentArgs* a = (XentArgs*)calloc(1, sizeof(XentArgs));
  a->logits = logits, a->labels = labels, a->probs = probs, a->C = C, a->masked = 0;
  const size_t chunks = orc_parallel_cost(N, row_grain(C, kGrainMath), 8 * C, xent_chunk, a);
  double total = 0.0;
  for (size_t c = 0; c < chunks; ++c) total += a->part[c];  /* chunk order */
  free(a);
  *loss = (float)(total / (double)N);
}
/* loss.cc:61-72 */
void orc_xent_bwd(const float* probs, const int32_t* labels, const float* seed,
                  float* dlogits, size_t N, size_t C) {
  const float scale = *seed / (float)N;
  for (size_t n = 0; n < N; ++n) {
    for (size_t c = 0; c < C; ++c) dlogits[n * C + c] = scale * probs[n * C + c];
    dlogits[n * C + (size_t)labels[n]] -= scale;
  }
}
/* loss.cc:74-105 */
void orc_xent_masked_fwd(const float* logits, const int32_t* labels,
                         float* loss, float* probs, size_t N, size_t C) {
  XentArgs* a = (XentArgs*)calloc(1, sizeof(XentArgs));
  a->logits = logits, a->labels = labels, a->probs = probs, a->C = C, a->masked = 1;
  const size_t chunks = orc_parallel_cost(N, row_grain(C, kGrainMath), 8 * C, xent_chunk, a);
  double total = 0.0;
  uint64_t T = 0;
  for (size_t c = 0; c < chunks; ++c) {  /* chunk order */
    total += a->part[c];
    T += a->targets[c];
  }
  free(a);
  *loss = T ? (float)(total / (double)T) : 0.0f;
}
/* loss.cc:107-126 */
void orc_xent_masked_bwd(const float* probs, const int32_t* labels,
                         const float* seed, float* dlogits, size_t N,
                         size_t C) {
  uint64_t T = 0;
  for (size_t n = 0; n < N; ++n) T += labels[n] >= 0;
  const float scale = T ? *seed / (float)T : 0.0f;
  for (size_t n = 0; n < N; ++n) {
    if (labels[n] < 0) {
      for (size_t c = 0; c < C; ++c) dlogits[n * C + c] = 0.0f;
      continue;
    }
    for (size_t c = 0; c < C; ++c) dlogits[n * C + c] = scale * probs[n * C + c];
    dlogits[n * C + (size_t)labels[n]] -= scale;
  }
}

/* ------------------------------------------------------------------------ */
/* Optimizer                                                                */
/* ------------------------------------------------------------------------ */

/* optimizer.cc:19-35: ||g||^2 with one double partial per chunk of
 * kGrainCheap (raised to n/256), combined in chunk order. */
static double l2_squared(const float* g, size_t n) {
  const size_t grain = orc_chunk_grain(n, kGrainCheap);
  double sq = 0.0;
  for (size_t b = 0; b < n; b += grain) {
    const size_t e = b + grain < n ? b + grain : n;
    double part = 0.0;
    for (size_t i = b; i < e; ++i) part += (double)g[i] * (double)g[i];
    sq += part;
  }
  return sq;
}
/* optimizer.cc:40-50 */
static int clip_scale(const float* g, size_t n, float max_norm, float* scale) {
  *scale = 1.0f;
  if (!(max_norm > 0.0f)) return 1;
  const double norm = sqrt(l2_squared(g, n));
  if (!isfinite(norm)) return 0;
  if (norm <= (double)max_norm || norm == 0.0) return 1;
  *scale = (float)((double)max_norm / norm);
  return 1;
}
/* optimizer.cc:54-68 */
int orc_clip_norm(float* g, size_t n, float max_norm) {
  if (!isfinite(max_norm) || !(max_norm > 0.0f)) return 0;
  const double norm = sqrt(l2_squared(g, n));
  if (!isfinite(norm)) return 0;
  if (norm <= (double)max_norm || norm == 0.0) return 1;
  const float s = (float)((double)max_norm / norm);
  for (size_t i = 0; i < n; ++i) g[i] *= s;
  return 1;
}
/* optimizer.cc:70-72 */
void orc_sqnorm_accum(const float* g, size_t n, float* acc) {
  acc[0] = (float)((double)acc[0] + l2_squared(g, n));
}
/* optimizer.cc:74-85 */
int orc_clip_global(float* g, size_t n, const float* acc, float max_norm) {
  if (!isfinite(max_norm) || !(max_norm > 0.0f)) return 0;
  const double norm = sqrt((double)acc[0]);
  if (!isfinite(norm)) return 0;
  if (norm <= (double)max_norm || norm == 0.0) return 1;
  const float s = (float)((double)max_norm / norm);
  for (size_t i = 0; i < n; ++i) g[i] *= s;
  return 1;
}
/* optimizer.cc:91-102 */
int orc_sgd_step(float* p, const float* g, size_t n, float lr, float wd,
                 float clip_norm) {
  float s = 1.0f;
  if (!clip_scale(g, n, clip_norm, &s)) return 0;
  for (size_t i = 0; i < n; ++i) {
    const float gi = g[i] * s;
    p[i] -= lr * (gi + wd * p[i]);
  }
  return 1;
}
/* optimizer.cc:115-118 */
void orc_adamw_bias_corrections(float beta1, float beta2, uint64_t step,
                                float* inv_bc1, float* inv_bc2) {
  *inv_bc1 = 1.0f / (1.0f - powf(beta1, (float)step));
  *inv_bc2 = 1.0f / (1.0f - powf(beta2, (float)step));
}
/* optimizer.cc:104-132 */
int orc_adamw_step(float* p, const float* g, float* m, float* v, size_t n,
                   float lr, float beta1, float beta2, float eps, float wd,
                   uint64_t step, float clip_norm) {
  float s = 1.0f;
  if (!clip_scale(g, n, clip_norm, &s)) return 0;
  float inv_bc1, inv_bc2;
  orc_adamw_bias_corrections(beta1, beta2, step, &inv_bc1, &inv_bc2);
  const float om_b1 = 1.0f - beta1;
  const float om_b2 = 1.0f - beta2;
  for (size_t i = 0; i < n; ++i) {
    const float gi = g[i] * s;
    const float mi = beta1 * m[i] + om_b1 * gi;
    const float vi = beta2 * v[i] + om_b2 * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float m_hat = mi * inv_bc1;
    const float v_hat = vi * inv_bc2;
    p[i] -= lr * (m_hat / (sqrtf(v_hat) + eps) + wd * p[i]);
  }
  return 1;
}

/* ------------------------------------------------------------------------ */
/* Eval argmax                                                              */
/* ------------------------------------------------------------------------ */

/* update_engine.cc:552-560: first maximum wins (strict >). */
void orc_argmax_rows(const float* probs, size_t rows, size_t cols,
                     int32_t* out) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = probs + r * cols;
    uint64_t am = 0;
    for (uint64_t c = 1; c < cols; ++c)
      if (row[c] > row[am]) am = c;
    out[r] = (int32_t)am;
  }
}
void orc_argmax_tally(const float* probs, const int32_t* labels, size_t rows,
                      size_t cols, uint64_t* hits, uint64_t* judged) {
  uint64_t h = 0, j = 0;
  for (size_t r = 0; r < rows; ++r) {
    if (labels[r] < 0) continue;
    ++j;
    const float* row = probs + r * cols;
    uint64_t am = 0;
    for (uint64_t c = 1; c < cols; ++c)
      if (row[c] > row[am]) am = c;
    if ((uint64_t)labels[r] == am) ++h;
  }
  *hits = h;
  *judged = j;
}

/* ------------------------------------------------------------------------ */
/* Instruction interpreter: runtime/executor/cpu_backend.cc:260-646.        */
/* ------------------------------------------------------------------------ */

typedef struct {
  uint16_t opcode, flags;
  uint32_t imm;
  uint64_t in[4];
  uint64_t out[3];
} OrcIns; /* instruction.h:438-447, 64 bytes packed */

static const uint64_t kRodataBit = 1ULL << 63;
static const uint64_t kSourceBit = 1ULL << 62;
static const uint64_t kNullRef = ~0ULL;

static float bits_f32(uint64_t w) {
  uint32_t u = (uint32_t)w;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
/* cpu_backend.cc:221-240 (ReadPtr): bit 63 names rodata, bit 62 alone the
 * source model file's image, neither the arena. */
static void* ref_ptr(uint64_t ref, uint8_t* arena, const uint8_t* rodata,
                     const uint8_t* source) {
  const uint64_t off = ref & ~(kRodataBit | kSourceBit);
  if (ref & kRodataBit) return (void*)(rodata + off);
  if (ref & kSourceBit) return (void*)(source + off);
  return arena + off;
}

int orc_execute(const void* instruction, uint8_t* arena, const uint8_t* rodata,
                const OrcStepParams* P) {
  return orc_execute_src(instruction, arena, rodata, NULL, P);
}

int orc_execute_src(const void* instruction, uint8_t* arena, const uint8_t* rodata,
                    const uint8_t* source, const OrcStepParams* P) {
  OrcIns ins;
  memcpy(&ins, instruction, sizeof ins);
  /* A source ref with no source image bound: refused before any read.  Only
   * the in[] slots carry operand refs a source image may back. */
  for (int i = 0; i < 4; ++i)
    if (!source && ins.in[i] != kNullRef &&
        (ins.in[i] & (kRodataBit | kSourceBit)) == kSourceBit)
      return 3;
#define RP(r) ((float*)ref_ptr((r), arena, rodata, source))
#define IP(r) ((int32_t*)ref_ptr((r), arena, rodata, source))
  const int act = (ins.flags >> 1) & 3;
  const float alpha = ins.imm == 0 ? 1.0f : bits_f32(ins.imm);
  const float norm_eps = ins.imm == 0 ? 1e-5f : bits_f32(ins.imm);
  switch (ins.opcode) {
    case 0: break;
    case 1:
      orc_gemm_nn(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0],
                  ins.out[1], ins.out[2], (ins.flags & 1) ? RP(ins.in[3]) : NULL,
                  act, (ins.flags & 8) ? RP(ins.in[3]) : NULL, alpha);
      break;
    case 2:
      orc_gemm_nt(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0],
                  ins.out[1], ins.out[2], (ins.flags & 8) ? RP(ins.in[3]) : NULL,
                  alpha);
      break;
    case 3:
      orc_gemm_tn(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0],
                  ins.out[1], ins.out[2], (ins.flags & 8) ? RP(ins.in[3]) : NULL,
                  alpha);
      break;
    case 4:
      orc_gemm_acc_nn(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0],
                      ins.out[1], ins.out[2], bits_f32(ins.in[3]));
      break;
    case 29: {
      const int cs = (ins.flags & 16) != 0;
      orc_gemm_nn_q8(RP(ins.in[0]), (const int8_t*)ref_ptr(ins.in[1], arena, rodata, source),
                     RP(ins.in[2]), ins.out[0], ins.out[1], ins.out[2],
                     cs ? 1.0f : bits_f32(ins.in[3]), act, cs ? RP(ins.in[3]) : NULL);
      break;
    }
    case 30: {
      const int cs = (ins.flags & 16) != 0;
      orc_gemm_nt_q8(RP(ins.in[0]), (const int8_t*)ref_ptr(ins.in[1], arena, rodata, source),
                     RP(ins.in[2]), ins.out[0], ins.out[1], ins.out[2],
                     cs ? 1.0f : bits_f32(ins.in[3]), cs ? RP(ins.in[3]) : NULL);
      break;
    }
    case 43:
      orc_gemm_nn_bf16(RP(ins.in[0]), (const uint16_t*)ref_ptr(ins.in[1], arena, rodata, source),
                       RP(ins.in[2]), ins.out[0], ins.out[1], ins.out[2],
                       (ins.flags & 1) ? RP(ins.in[3]) : NULL, act);
      break;
    case 44:
      orc_gemm_nt_bf16(RP(ins.in[0]), (const uint16_t*)ref_ptr(ins.in[1], arena, rodata, source),
                       RP(ins.in[2]), ins.out[0], ins.out[1], ins.out[2]);
      break;
    case 5: orc_add_ew(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0]); break;
    case 21: orc_mul_ew(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0]); break;
    case 6:
      orc_add_bias(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0], ins.out[1]);
      break;
    case 7: orc_relu_fwd(RP(ins.in[0]), RP(ins.in[1]), ins.out[0]); break;
    case 8: orc_relu_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0]); break;
    case 22: orc_gelu_fwd(RP(ins.in[0]), RP(ins.in[1]), ins.out[0]); break;
    case 23: orc_gelu_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0]); break;
    case 24: orc_silu_fwd(RP(ins.in[0]), RP(ins.in[1]), ins.out[0]); break;
    case 25: orc_silu_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0]); break;
    case 9: orc_scale(RP(ins.in[0]), RP(ins.in[1]), bits_f32(ins.in[2]), ins.out[0]); break;
    case 10: orc_reduce_rows(RP(ins.in[0]), RP(ins.in[1]), ins.out[0], ins.out[1]); break;
    case 11:
      orc_xent_fwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                   ins.out[0], ins.out[1]);
      break;
    case 12:
      orc_xent_bwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                   ins.out[0], ins.out[1]);
      break;
    case 51:
      orc_xent_masked_fwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]),
                          RP(ins.in[3]), ins.out[0], ins.out[1]);
      break;
    case 52:
      orc_xent_masked_bwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]),
                          RP(ins.in[3]), ins.out[0], ins.out[1]);
      break;
    case 17:
      if (!orc_sgd_step(RP(ins.in[0]), RP(ins.in[1]), ins.out[0], P->lr,
                        P->weight_decay, bits_f32(ins.out[1])))
        return 1;
      break;
    case 18:
      if (!orc_adamw_step(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                          RP(ins.in[3]), ins.out[0], P->lr, P->beta1, P->beta2,
                          P->eps, P->weight_decay, P->step, bits_f32(ins.out[1])))
        return 1;
      break;
    case 28: {
      const float cap = bits_f32(ins.in[1]);
      if (!isfinite(cap) || !(cap > 0.0f)) return 4;
      if (!orc_clip_norm(RP(ins.in[0]), ins.out[0], cap)) return 1;
      break;
    }
    case 53: orc_sqnorm_accum(RP(ins.in[0]), ins.out[0], RP(ins.in[1])); break;
    case 54: {
      const float cap = bits_f32(ins.in[2]);
      if (!isfinite(cap) || !(cap > 0.0f)) return 4;
      if (!orc_clip_global(RP(ins.in[0]), ins.out[0], RP(ins.in[1]), cap)) return 1;
      break;
    }
    case 19: orc_fill(RP(ins.in[0]), bits_f32(ins.in[1]), ins.out[0]); break;
    case 20: orc_copy(RP(ins.in[0]), RP(ins.in[1]), ins.out[0]); break;
    case 42: orc_accumulate(RP(ins.in[0]), RP(ins.in[1]), ins.out[0]); break;
    case 26:
      orc_layernorm_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                        RP(ins.out[1]), RP(ins.out[2]), ins.out[0] >> 32,
                        ins.out[0] & 0xFFFFFFFFu, norm_eps);
      break;
    case 27:
      orc_layernorm_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.out[0]),
                        RP(ins.out[1]), RP(ins.in[3]), ins.out[2] >> 32,
                        ins.out[2] & 0xFFFFFFFFu);
      break;
    case 31:
      orc_rmsnorm_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                      ins.out[0] >> 32, ins.out[0] & 0xFFFFFFFFu, norm_eps);
      break;
    case 32:
      orc_rmsnorm_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.out[0]),
                      RP(ins.in[3]), ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu);
      break;
    case 33:
    case 34:
      orc_rope(RP(ins.in[0]), RP(ins.in[1]), ins.out[0] >> 32, ins.out[0] & 0xFFFFFFFFu,
               ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu, bits_f32(ins.out[2]),
               ins.in[2] == kNullRef ? NULL : RP(ins.in[2]), ins.opcode == 34);
      break;
    case 45:
      orc_rope_table(RP(ins.in[0]), ins.out[0] >> 32, ins.out[0] & 0xFFFFFFFFu,
                     bits_f32(ins.out[1]));
      break;
    case 46:
      orc_fused_map(RP(ins.in[0]), ins.in[1] == kNullRef ? NULL : RP(ins.in[1]),
                    ins.in[2] == kNullRef ? NULL : RP(ins.in[2]), RP(ins.in[3]),
                    ins.out[0], ins.out[1], bits_f32(ins.out[2]),
                    bits_f32(ins.out[2] >> 32));
      break;
    case 35:
      orc_attn_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                   RP(ins.out[0]), ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu,
                   ins.out[2] >> 32, ins.out[2] & 0xFFFFFFFFu, NULL);
      break;
    case 56: {
      const uint64_t g = ins.out[1];
      orc_attn_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                   RP(ins.out[0]), g >> 48, (g >> 32) & 0xFFFF, (g >> 16) & 0xFFFF,
                   g & 0xFFFF, IP(ins.out[2]));
      break;
    }
    case 55:
      orc_segment_starts(IP(ins.in[0]), IP(ins.in[1]), ins.out[0] >> 32,
                         ins.out[0] & 0xFFFFFFFFu, (int32_t)ins.out[1]);
      break;
    case 36:
      orc_attn_dp(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0] >> 32,
                  ins.out[0] & 0xFFFFFFFFu, ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu);
      break;
    case 37:
      orc_attn_dv(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0] >> 32,
                  ins.out[0] & 0xFFFFFFFFu, ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu);
      break;
    case 38:
      orc_softmax_rows_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                           ins.out[0] >> 32, ins.out[0] & 0xFFFFFFFFu);
      break;
    case 39:
      orc_attn_dq(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0] >> 32,
                  ins.out[0] & 0xFFFFFFFFu, ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu);
      break;
    case 40:
      orc_attn_dk(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0] >> 32,
                  ins.out[0] & 0xFFFFFFFFu, ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu);
      break;
    case 47:
      orc_attn_fwd_tiled(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                         RP(ins.out[0]), ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu,
                         ins.out[2] >> 32, ins.out[2] & 0xFFFFFFFFu, NULL);
      break;
    case 57: {
      const uint64_t g = ins.out[1];
      orc_attn_fwd_tiled(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                         RP(ins.out[0]), g >> 48, (g >> 32) & 0xFFFF,
                         (g >> 16) & 0xFFFF, g & 0xFFFF, IP(ins.out[2]));
      break;
    }
    case 48:
    case 49:
    case 50: {
      const uint64_t g = ins.out[2];
      const size_t B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF,
                   d = g & 0xFFFF;
      if (ins.opcode == 48)
        orc_attn_dq_tiled(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                          RP(ins.out[0]), RP(ins.out[1]), B, S, H, d);
      else if (ins.opcode == 49)
        orc_attn_dk_tiled(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.in[3]),
                          RP(ins.out[0]), RP(ins.out[1]), B, S, H, d);
      else
        orc_attn_dv_tiled(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[3]), RP(ins.out[0]),
                          RP(ins.out[1]), B, S, H, d);
      break;
    }
    case 41:
      orc_embed_fwd(IP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), ins.out[0],
                    ins.out[1] & 0xFFFFFFFFu);
      break;
    default:
      return 2; /* MSE / KL: outside the hot path */
  }
#undef RP
#undef IP
  return 0;
}

/* --- plan self-hash (source/identity/hash.h:31-158) --------------------- */
static const uint64_t kFnvBasis = 0xcbf29ce484222325ULL;
static const uint64_t kFnvPrime = 0x100000001b3ULL;

/* hash.h:71-78: a 64-bit word folded low byte first. */
static uint64_t fnv_word(uint64_t h, uint64_t w) {
  for (int b = 0; b < 8; ++b) {
    h ^= (w >> (8 * b)) & 0xffu;
    h *= kFnvPrime;
  }
  return h;
}

/* hash.h:82-100, with the byte at `zero_at` (if inside) read as zero. */
static uint64_t striped(const uint8_t* p, size_t n, size_t base, size_t zero_lo, size_t zero_hi) {
  uint64_t lane[8];
  for (size_t l = 0; l < 8; ++l) lane[l] = kFnvBasis ^ (0x9E3779B97F4A7C15ULL * (l + 1));
  for (size_t i = 0; i < n; ++i) {
    const size_t at = base + i;
    const uint8_t byte = (at >= zero_lo && at < zero_hi) ? 0 : p[i];
    lane[i % 8] ^= byte;
    lane[i % 8] *= kFnvPrime;
  }
  uint64_t h = kFnvBasis;
  for (size_t l = 0; l < 8; ++l) h = fnv_word(h, lane[l]);
  return fnv_word(h, (uint64_t)n);
}

uint64_t orc_plan_self_hash(const uint8_t* plan, size_t size, size_t hash_offset) {
  const size_t grain = orc_chunk_grain(size, (size_t)1 << 20); /* hash.h:63 */
  const size_t chunks = orc_chunk_count(size, (size_t)1 << 20);
  uint64_t h = kFnvBasis;
  if (chunks == 0) {
    h = fnv_word(h, striped(plan, 0, 0, hash_offset, hash_offset + 8));
  } else {
    for (size_t c = 0; c < chunks; ++c) {
      const size_t b = c * grain, e = (b + grain < size) ? b + grain : size;
      h = fnv_word(h, striped(plan + b, e - b, b, hash_offset, hash_offset + 8));
    }
  }
  return fnv_word(h, (uint64_t)size);
}
