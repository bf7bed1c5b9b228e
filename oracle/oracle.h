/*
 * oracle.h -- CPU restatement of the SeeAI executor's kernel library.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * C++ backend, the Python host mirror) links, loads or calls this code; it
 * is the checker that the parity tests, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the GPU path against.
 *
 * Every function restates one reference kernel, in the reference's own
 * per-element expression and reduction order, so that on an x86-64 host
 * (no FMA contraction: built with -ffp-contract=off) it reproduces the
 * reference's bits.  Each definition in oracle.c cites the reference
 * file:line it follows.  The W8A8 pair (orc_quantize_rows, orc_gemm_w8a8)
 * has no reference counterpart: the quantizer restates the reference's
 * int8 weight packer rule and the GEMM is exact integer arithmetic.
 *
 * Pinning (how each function is checked, see tests/):
 *   - every kernel here is compared bit-for-bit with the reference kernel
 *     library compiled from /root/reference (oracle/_ref) on ragged
 *     shapes, and against golden vectors that library wrote
 *     (tests/golden/);
 *   - closed forms and invariants of the reference's own known-answer
 *     tests (hand GEMM, uniform-logit xent = log C, AdamW step 1,
 *     single-token attention = V, RoPE golden angles, FD gradients);
 *   - the W8A8 GEMM against an int64 brute force and the quantizer against
 *     its definition on hand-built rows (ties, zero rows, clamps).
 */
#ifndef SEEAI_ORACLE_H_
#define SEEAI_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ParallelFor chunk geometry (source/parallel/parallel_for.h:55-67). */
size_t orc_chunk_grain(size_t n, size_t grain);
size_t orc_chunk_count(size_t n, size_t grain);

/* --- GEMM family (runtime/executor/gemm.cc) ------------------------------ */
/* act: 0 none, 1 relu, 2 gelu, 3 silu.  bias / addend may be NULL. */
void orc_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act, const float* addend,
                 float alpha);
void orc_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha);
void orc_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha);
void orc_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha);
void orc_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act,
                    const float* col_scale);
void orc_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, const float* k_scale);
void orc_gemm_nn_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K, const float* bias, int act);
void orc_gemm_nt_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K);

/* --- W8A8 (no reference counterpart) ------------------------------------- */
/* Per-row symmetric int8: scale[r] = max|x_r|/127 (0 -> 1, subnormal ->
 * FLT_MIN), q = clamp(round(x / scale), -127, 127). */
void orc_quantize_rows(const float* X, int8_t* Q, float* scale, size_t rows,
                       size_t cols);
/* Per-output-column quantization of W [K, N] (the packer's column rule). */
void orc_quantize_cols(const float* W, int8_t* Q, float* scale, size_t K,
                       size_t N);
/* acc[m,n] = sum_k qa[m,k] * qw[k,n] in int32 (exact);
 * C[m,n] = ((float)acc * sa[m]) * sw[n].  acc may be NULL. */
void orc_gemm_w8a8(const int8_t* QA, const float* sa, const int8_t* QW,
                   const float* sw, int32_t* acc, float* C, size_t M,
                   size_t N, size_t K);

/* --- Elementwise / activation / normalization ---------------------------- */
void orc_add_ew(const float* x, const float* y, float* out, size_t n);
void orc_mul_ew(const float* x, const float* y, float* out, size_t n);
void orc_add_bias(const float* x, const float* b, float* out, size_t rows,
                  size_t cols);
void orc_relu_fwd(const float* x, float* out, size_t n);
void orc_relu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_gelu_fwd(const float* x, float* out, size_t n);
void orc_gelu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_silu_fwd(const float* x, float* out, size_t n);
void orc_silu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_scale(const float* x, float* out, float alpha, size_t n);
void orc_reduce_rows(const float* dy, float* db, size_t rows, size_t cols);
void orc_fill(float* dst, float value, size_t n);
void orc_copy(const float* src, float* dst, size_t n);
void orc_accumulate(float* dst, const float* src, size_t n);
void orc_embed_fwd(const int32_t* tokens, const float* table, float* out,
                   size_t rows, size_t dim);
void orc_fused_map(const float* x, const float* other1, const float* other2,
                   float* out, size_t n, uint64_t stages, float imm0,
                   float imm1);
void orc_layernorm_fwd(const float* x, const float* gamma, const float* beta,
                       float* y, float* mean, float* rstd, size_t rows,
                       size_t cols, float eps);
void orc_layernorm_bwd(const float* dy, const float* x, const float* gamma,
                       const float* mean, const float* rstd, float* dx,
                       size_t rows, size_t cols);
void orc_rmsnorm_fwd(const float* x, const float* gamma, float* y, float* rstd,
                     size_t rows, size_t cols, float eps);
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* gamma,
                     const float* rstd, float* dx, size_t rows, size_t cols);
void orc_rope(const float* x, float* y, size_t B, size_t S, size_t H,
              size_t d, float base, const float* table, int backward);
void orc_rope_table(float* table, size_t S, size_t d, float base);

/* --- Attention (runtime/executor/attention.cc) --------------------------- */
void orc_segment_starts(const int32_t* tokens, int32_t* starts, size_t B,
                        size_t S, int32_t eos);
void orc_attn_fwd(const float* q, const float* k, const float* v, float* o,
                  float* probs, size_t B, size_t S, size_t H, size_t d,
                  const int32_t* starts);
void orc_attn_dp(const float* dout, const float* v, float* dp, size_t B,
                 size_t S, size_t H, size_t d);
void orc_attn_dv(const float* probs, const float* dout, float* dv, size_t B,
                 size_t S, size_t H, size_t d);
void orc_softmax_rows_bwd(const float* probs, const float* dp, float* ds,
                          size_t rows, size_t cols);
void orc_attn_dq(const float* ds, const float* k, float* dq, size_t B,
                 size_t S, size_t H, size_t d);
void orc_attn_dk(const float* ds, const float* q, float* dk, size_t B,
                 size_t S, size_t H, size_t d);
void orc_attn_fwd_tiled(const float* q, const float* k, const float* v,
                        float* o, float* stats, size_t B, size_t S, size_t H,
                        size_t d, const int32_t* starts);
void orc_attn_dq_tiled(const float* q, const float* k, const float* v,
                       const float* dout, float* stats, float* dq, size_t B,
                       size_t S, size_t H, size_t d);
void orc_attn_dk_tiled(const float* q, const float* k, const float* v,
                       const float* dout, const float* stats, float* dk,
                       size_t B, size_t S, size_t H, size_t d);
void orc_attn_dv_tiled(const float* q, const float* k, const float* dout,
                       const float* stats, float* dv, size_t B, size_t S,
                       size_t H, size_t d);

/* --- Losses (runtime/executor/loss.cc) ----------------------------------- */
void orc_xent_fwd(const float* logits, const int32_t* labels, float* loss,
                  float* probs, size_t N, size_t C);
void orc_xent_bwd(const float* probs, const int32_t* labels, const float* seed,
                  float* dlogits, size_t N, size_t C);
void orc_xent_masked_fwd(const float* logits, const int32_t* labels,
                         float* loss, float* probs, size_t N, size_t C);
void orc_xent_masked_bwd(const float* probs, const int32_t* labels,
                         const float* seed, float* dlogits, size_t N,
                         size_t C);

/* --- Optimizer (runtime/executor/optimizer.cc) --------------------------- */
/* Return 1 on success, 0 on refusal (non-finite norm / bad cap). */
int orc_clip_norm(float* g, size_t n, float max_norm);
void orc_sqnorm_accum(const float* g, size_t n, float* acc);
int orc_clip_global(float* g, size_t n, const float* acc, float max_norm);
int orc_sgd_step(float* p, const float* g, size_t n, float lr, float wd,
                 float clip_norm);
int orc_adamw_step(float* p, const float* g, float* m, float* v, size_t n,
                   float lr, float beta1, float beta2, float eps, float wd,
                   uint64_t step, float clip_norm);
/* The two bias-correction reciprocals AdamW hoists (optimizer.cc:115-118). */
void orc_adamw_bias_corrections(float beta1, float beta2, uint64_t step,
                                float* inv_bc1, float* inv_bc2);

/* --- Eval argmax (runtime/dispatcher/update_engine.cc:537-565) ----------- */
/* hits / judged rows over `rows` rows; a label < 0 is not judged. */
void orc_argmax_tally(const float* probs, const int32_t* labels, size_t rows,
                      size_t cols, uint64_t* hits, uint64_t* judged);
void orc_argmax_rows(const float* probs, size_t rows, size_t cols,
                     int32_t* out);

/* PlanSelfHash (source/identity/hash.h:136-158): 8 interleaved FNV-1a
 * chains per chunk (hash.h:82-100), chunk digests folded in chunk order,
 * then the size; the 8 bytes at hash_offset read as zero. */
uint64_t orc_plan_self_hash(const uint8_t* plan, size_t size, size_t hash_offset);

/* --- Threads: every function gives the same bits at every count -------- */
/* Work runs in the reference's ParallelFor chunks (parallel_for.h:50-67)
 * spread over n threads; 0 or less means 1.  The default is
 * SEEAI_ORACLE_THREADS, else 1. */
void orc_set_threads(int n);
/* Ends the worker pool's threads (a later threaded call starts new ones). */
void orc_pool_stop(void);
int orc_threads(void);

/* --- Instruction interpreter (runtime/executor/cpu_backend.cc:260-646) --- */
/* Runs one 64-byte UpdateInstruction against an arena / rodata pair.
 * Returns 0 ok, 1 refusal (non-finite norm), 4 clip-threshold refusal,
 * 2 unsupported opcode. */
typedef struct OrcStepParams {
  float lr, beta1, beta2, eps, weight_decay;
  uint32_t pad;
  uint64_t step;
} OrcStepParams;
int orc_execute(const void* instruction, uint8_t* arena, const uint8_t* rodata,
                const OrcStepParams* params);
/* The same with the source model file's image bound (source refs, bit 62,
 * read from it: cpu_backend.cc:221-240).  orc_execute binds none: an
 * instruction naming a source ref there returns 3. */
int orc_execute_src(const void* instruction, uint8_t* arena, const uint8_t* rodata,
                    const uint8_t* source, const OrcStepParams* params);

#ifdef __cplusplus
}
#endif

#endif /* SEEAI_ORACLE_H_ */
