/*
 * seeai_hip.h -- the C ABI of the SeeAI gfx950 executor (libseeai_hip.so).
 *
 * The reference executor has no C ABI: its seam is the C++ class
 * ExecutorBackend (runtime/executor/backend.h:82-166) with the CPU backend
 * (runtime/executor/cpu_backend.cc) and a Metal backend behind it.  This
 * header is the thin C layer a HIP ExecutorBackend sits on: plain pointers
 * and sizes, no C++ or torch types, one status code per call.
 *
 *   status  0 ok
 *           1 refused: a non-finite gradient norm (kNonFiniteNormRefusal) or
 *             a clip threshold that is not a finite positive float
 *             (kClipThresholdRefusal); seeai_last_error() holds the
 *             reference's exact words (runtime/executor/backend.h:65-80)
 *           2 invalid argument (unknown opcode, shape the kernel refuses)
 *           3 HIP runtime error
 *
 * Threading: a context is single-threaded; all its work is enqueued on one
 * HIP stream in call order (the reference's one-engine-thread contract,
 * backend.h:82-166 and update_engine.cc:325-364).
 *
 * Pointers named `d_*` are device pointers; the others are host pointers.
 */
#ifndef SEEAI_HIP_H_
#define SEEAI_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SEEAI_OK 0
#define SEEAI_REFUSED 1
#define SEEAI_INVALID 2
#define SEEAI_HIP_ERROR 3

typedef struct seeai_ctx seeai_ctx;

/* Per-range optimizer scalars: StepParams (runtime/executor/backend.h:56-63). */
typedef struct seeai_step_params {
  float lr;
  float beta1;
  float beta2;
  float eps;
  float weight_decay;
  uint32_t reserved;
  uint64_t step; /* 1-indexed AdamW timestep */
} seeai_step_params;

/* --- Context: the backend object (CreateBackend, backend.cc:26-60) ------- */
int seeai_create(int device, seeai_ctx** out);
void seeai_destroy(seeai_ctx* ctx);
/* The message of the last non-zero status (never NULL). */
const char* seeai_last_error(const seeai_ctx* ctx);
/* Enqueue on `hip_stream` (a hipStream_t at default priority; NULL is the
 * null stream) instead of the context's own stream, which seeai_get_stream
 * returns right after seeai_create. */
int seeai_set_stream(seeai_ctx* ctx, void* hip_stream);
void* seeai_get_stream(seeai_ctx* ctx);
/* Whether kFlagRelaxed (instruction.h:356-390) is taken as a permission
 * (default 1): relaxed frozen-weight GEMMs run on bf16 MFMA (bf16-rounded
 * activations against the stored weight, f32 accumulation). */
int seeai_set_relaxed(seeai_ctx* ctx, int allow);
/* Relaxed tiled attention (kAttnFwdTiled .. kAttnDVTiled with kFlagRelaxed)
 * grants f32 products with reordered sums (instruction.h:384-390), which the
 * f32 MFMA family provides: the default (0).  With 1 it runs on bf16 MFMA
 * instead -- Q, K, V, dO, P and dS rounded to bf16, f32 accumulation and
 * softmax -- for models trained in bf16 activations (BASELINE configs[2]
 * bf16, [3], [4]); each such run counts as a relaxed execution.  The
 * environment variable SEEAI_ATTENTION_BF16=1 sets it at seeai_create. */
int seeai_set_attention_bf16(seeai_ctx* ctx, int on);
/* ExecutorBackend::relaxed_executions (backend.h:149-162). */
uint64_t seeai_relaxed_executions(const seeai_ctx* ctx);

/* --- Binding: ExecutorBackend::Bind / BindSource (backend.h:99-109) ------ */
/* Allocates the device arena (zeroed, arena_bytes rounded up to 16 KiB,
 * kArenaAlignment backend.h:51) and uploads the rodata image.  A failed
 * bind keeps the previous binding. */
int seeai_bind(seeai_ctx* ctx, uint64_t arena_bytes, const void* rodata,
               uint64_t rodata_bytes);
int seeai_bind_source(seeai_ctx* ctx, const void* data, uint64_t bytes);
/* Host <-> arena copies for the engine's host-sync points: the I/O slots
 * and the loss slot (update_engine.cc:853-856), eval probabilities (:535),
 * the persistent segment (:763) and merge deltas (:1051-1060).
 * Stream-ordered; seeai_download returns with the bytes on the host. */
int seeai_upload(seeai_ctx* ctx, uint64_t arena_offset, const void* src,
                 uint64_t bytes);
int seeai_download(seeai_ctx* ctx, uint64_t arena_offset, void* dst,
                   uint64_t bytes);
/* The device side of the feeder (BatchPipeline, runtime/pipeline/
 * batch_pipeline.h:13-57): a batch is staged while the current step runs --
 * copied into pinned host memory and uploaded on the feeder's own stream
 * (default priority) into device staging -- and seeai_feeder_next moves the
 * oldest staged batch into the arena's I/O slots on the context's stream,
 * ordered after its upload by an event (update_engine.cc:853-856).  At most
 * two batches are staged ahead (status 2 on a third).  seeai_feeder_stage
 * touches only the feeder's own stream and buffers, so the engine's feeder
 * thread may call it while the context's thread enqueues steps;
 * seeai_feeder_next belongs to the context's thread.  Staging buffers are
 * reused only after the arena copy that read them has run on the device. */
typedef struct seeai_feeder seeai_feeder;
int seeai_feeder_create(seeai_ctx* ctx, uint64_t input_bytes, uint64_t label_bytes,
                        seeai_feeder** out);
void seeai_feeder_destroy(seeai_feeder* feeder);
const char* seeai_feeder_last_error(const seeai_feeder* feeder);
int seeai_feeder_stage(seeai_feeder* feeder, const void* input, const void* labels);
int seeai_feeder_next(seeai_feeder* feeder, uint64_t input_offset, uint64_t label_offset);
/* The device arena's base (for callers that place tensors themselves). */
void* seeai_arena(seeai_ctx* ctx);
uint64_t seeai_arena_bytes(const seeai_ctx* ctx);

/* --- Execution: ExecutorBackend::Execute / Flush (backend.h:122-147) ----- */
/* Enqueues one validated 64-byte UpdateInstruction (instruction.h:438-447)
 * against the bound arena / rodata / source. */
int seeai_execute(seeai_ctx* ctx, const void* instruction,
                  const seeai_step_params* params);
/* Runs `count` consecutive instructions (ExecuteRange's loop,
 * update_engine.cc:345-351); stops at the first non-zero status and
 * reports its index in *failed_at. */
int seeai_execute_range(seeai_ctx* ctx, const void* instructions,
                        uint64_t count, const seeai_step_params* params,
                        uint64_t* failed_at);
/* ExecutorBackend::BeginRange / EndRange (backend.h:139-142): the whole
 * program of the range about to run, `count` 64-byte words of which
 * [begin, end) execute.  The caller keeps `program` alive until
 * seeai_end_range and passes seeai_execute pointers into it; two adjacent
 * instructions may then run as one dispatch (relaxed kAttnDKTiled +
 * kAttnDVTiled of one attention), the second returning at once.  Without a
 * range every instruction runs alone. */
int seeai_begin_range(seeai_ctx* ctx, const void* program, uint64_t count,
                      uint64_t begin, uint64_t end);
int seeai_end_range(seeai_ctx* ctx);
/* A whole range, as seeai_begin_range + seeai_execute of each of
 * [begin, end) + seeai_end_range would run it (the engine's ExecuteRange,
 * update_engine.cc:345-351), with the same bits.  No counterpart in the
 * reference (its CPU executor runs each instruction): for callers that run
 * the same range step after step.  The first run of a range runs
 * instruction by instruction (it sizes the workspaces and makes the weight
 * shadows); the second is captured as a HIP graph and the graph launched;
 * later runs launch the graph again, one launch per range, the step's
 * optimizer values (lr and the bias corrections of `params`) copied to the
 * device ahead of it.  Any bind, setting, policy or workspace change drops
 * the captured graphs; a range whose capture fails runs instruction by
 * instruction from then on.  The program's bytes must not change while a
 * graph of it is kept (they are hashed at every call).  A failure reports
 * the failing instruction's index in *failed_at. */
int seeai_run_range(seeai_ctx* ctx, const void* program, uint64_t count, uint64_t begin,
                    uint64_t end, const seeai_step_params* params, uint64_t* failed_at);
/* Graph replay in seeai_run_range (default 0: every range runs instruction
 * by instruction; SEEAI_GRAPHS=1 in the environment starts a context with
 * it on).  Measured on MI355X, replay runs the decoder and MLP ranges no
 * faster: the GPU's per-dispatch cost, not the host's launches, sets their
 * pace. */
int seeai_set_graph_replay(seeai_ctx* ctx, int on);
/* Ranges seeai_run_range has run as one graph launch so far. */
uint64_t seeai_graph_launches(const seeai_ctx* ctx);
/* Whether adjacent instructions may fuse (default 1), and how many fused
 * dispatches ran (ExecutorBackend::fused_dispatches, backend.h:165). */
int seeai_set_fusion(seeai_ctx* ctx, int allow);
uint64_t seeai_fused_dispatches(const seeai_ctx* ctx);
/* How many stores fused passes skipped as dead: a value the program, run
 * again from its start, overwrites before any read or never touches again
 * (the rule metal_backend.mm:1281-1313 applies to a LoRA site's base
 * value): the base value, the SwiGLU backward's dh*up product, a
 * producer's f32 output whose only reader converts it to bf16, the output
 * of a producer whose residual add ran inside it, unread probabilities.
 * Such a slot keeps its old bytes; a caller that downloads intermediates
 * sets SEEAI_KEEP_DEAD_STORES=1 at seeai_create to keep every store. */
uint64_t seeai_dropped_stores(const seeai_ctx* ctx);
/* How many relaxed products' bf16 activation copies their producers wrote
 * as they stored (within a range, with fusion on: the SwiGLU passes, GELU
 * forward / backward, the softmax-xent backward, LayerNorm / RMSNorm
 * forward and backward and the residual adds, when the next instruction is
 * a relaxed frozen-weight product on the direct-to-LDS path reading their
 * output; the product then skips its conversion pass, and the producer
 * skips its f32 store where nothing else reads it). */
uint64_t seeai_fused_conversions(const seeai_ctx* ctx);
/* Waits for the stream; reports a refusal raised on the device since the
 * last flush (non-finite clip norm: nothing it guarded was written). */
int seeai_flush(seeai_ctx* ctx);
/* seeai_flush with `bytes` of the arena at `arena_offset` read back into
 * `dst` in the same drain (one stream synchronisation for the step's
 * refusal check and its loss).  No counterpart in the reference: its
 * engine flushes and then syncs the loss to the host
 * (update_engine.cc:345-360); this is both for a caller that runs a step
 * per batch. */
int seeai_flush_download(seeai_ctx* ctx, uint64_t arena_offset, void* dst, uint64_t bytes);

/* --- Kernel geometry: ExecutorBackend::Configure (backend.h:117) -------- */
/* The gfx950 member of the reference's schema-1 kernel-policy table
 * (compiler/backend/architecture/kernel_policy_table.cc:294-404 reads
 * hosts.<key>.cpu; this backend's table reader takes hosts.<key>.gfx950
 * beside it).  Every field chooses among kernels that give identical bits,
 * so a policy changes time, never results; 0 keeps the built-in default. */
typedef struct seeai_tile_policy {
  uint32_t w8a8_large_kernel;     /* 1 direct-to-LDS 256x256 (default), 2 register-staged 256x256,
                                     3 register-staged 128x128 */
  uint32_t w8a8_large_min;        /* M and N from which it applies (default 4096) */
  uint32_t quantize_waves_per_cu; /* waves per CU walking the quantizer's rows of at most 1024
                                     or more than 8192 floats (default 32, <= 32); rows in
                                     between take a workgroup of four waves each */
  uint32_t relaxed_min_tiles_256; /* relaxed bf16 GEMM: 256x256 tiles from this many (default 256) */
  uint32_t relaxed_min_fill_256;  /* ... and when their last round over the CUs is at least
                                     this percent full (<= 100) */
  uint32_t relaxed_nt_dma_min_k;  /* relaxed NT on rodata weights: the direct-to-LDS kernel from
                                     this K, the register-staged one below (default 768) */
  uint32_t convert_wgs_per_cu;    /* workgroups per CU of the relaxed GEMMs' activation
                                     conversion (default 8, <= 64) */
  uint32_t exact_longk_first;     /* exact skinny long-K GEMM: 1 the two-pass form before the
                                     chain kernel (default), 2 the chain kernel first */
  uint32_t relaxed_tile_192;      /* relaxed bf16 GEMM below the 256x256 threshold: 1 128x192
                                     tiles where they take fewer CU rounds per unit of work than
                                     128x128, 2 never (default), 3 always (N >= 192) */
} seeai_tile_policy;
/* NULL restores the defaults; an out-of-range field is status 2 and leaves
 * the policy in force unchanged. */
int seeai_configure(seeai_ctx* ctx, const seeai_tile_policy* policy);
/* The policy in force, defaults filled in. */
int seeai_policy(const seeai_ctx* ctx, seeai_tile_policy* out);
/* The device's table key, the GPU counterpart of HostKey
 * (compiler/backend/architecture/host_arch.h:41-50): one line,
 * "<gfx arch>;<device name>;cus=<n>;lds=<bytes per CU>;l2=<bytes>;wave=<lanes>". */
int seeai_device_key(int device, char* buf, uint64_t bytes);

/* --- Op-family entry points on caller-owned device memory --------------- */
/* GemmNN / NT / TN / AccNN (runtime/executor/gemm.cc:582-624).
 * layout 0 NN (A[M,K], B[K,N]), 1 NT (B[N,K]), 2 TN (A[K,M]);
 * act 0 none 1 relu 2 gelu 3 silu; d_bias [N] or NULL; d_addend [M,N] or
 * NULL; accumulate = 1 is GemmAccNN (C += alpha A@B). */
int seeai_gemm_f32(seeai_ctx* ctx, int layout, const float* d_A,
                   const float* d_B, float* d_C, uint64_t M, uint64_t N,
                   uint64_t K, const float* d_bias, int act,
                   const float* d_addend, float alpha, int accumulate);
/* GemmNNQ8 / GemmNTQ8 (gemm.cc:626-674): nt 0 -> B int8 [K,N], 1 -> [N,K];
 * d_col_scale (kFlagQ8ColScale): NN per output column [N], NT per
 * reduction index [K]; NULL uses the per-tensor `scale`. */
int seeai_gemm_q8(seeai_ctx* ctx, int nt, const float* d_A,
                  const int8_t* d_B, float* d_C, uint64_t M, uint64_t N,
                  uint64_t K, float scale, const float* d_col_scale, int act);
/* GemmNNBF16 / GemmNTBF16 (gemm.cc:676-699). */
int seeai_gemm_bf16w(seeai_ctx* ctx, int nt, const float* d_A,
                     const uint16_t* d_B, float* d_C, uint64_t M, uint64_t N,
                     uint64_t K, const float* d_bias, int act);

/* W8A8 -- no reference counterpart (the reference's int8 GEMMs widen int8
 * weights into f32 arithmetic); the quantizer rule is the reference's int8
 * packer's (compiler/backend/allocation/arena_binder.cc:129-177). */
/* Per-row symmetric int8 of X [rows, cols]: d_scale[rows], d_Q [rows, cols]. */
int seeai_w8a8_quantize_rows(seeai_ctx* ctx, const float* d_X, int8_t* d_Q,
                             float* d_scale, uint64_t rows, uint64_t cols);
/* Per-output-column int8 of W [K, N], packed K-contiguous: d_Qt [N, K]. */
int seeai_w8a8_pack_weights(seeai_ctx* ctx, const float* d_W, int8_t* d_Qt,
                            float* d_scale, uint64_t K, uint64_t N);
/* C[m,n] = (f32(sum_k QA[m,k] QWt[n,k]) * sa[m]) * sw[n]; the int32
 * accumulators also land in d_acc [M,N] when it is not NULL. */
int seeai_w8a8_gemm(seeai_ctx* ctx, const int8_t* d_QA, const float* d_sa,
                    const int8_t* d_QWt, const float* d_sw, float* d_C,
                    int32_t* d_acc, uint64_t M, uint64_t N, uint64_t K);

/* Tiled attention (kAttnFwdTiled..kAttnDVTiled, attention.cc:448-590):
 * q, k, v, o, dout [B*S, H*d]; stats [B*H*S, 4]; d_starts [B*S] or NULL.
 * dtype 0 = f32 (exact family), 1 = bf16 MFMA (relaxed family). */
int seeai_attn_fwd(seeai_ctx* ctx, int dtype, const float* d_q,
                   const float* d_k, const float* d_v, float* d_o,
                   float* d_stats, uint64_t B, uint64_t S, uint64_t H,
                   uint64_t d, const int32_t* d_starts);
/* The tiled forward on bf16 operands held in HBM as bf16 ([B*S, H*64],
 * head width 64): O (f32) and the stats row as seeai_attn_fwd.  Staged
 * straight into LDS, 32 queries per wave; results within the bf16 bar of
 * the exact family on the same (bf16-valued) inputs. */
int seeai_attn_fwd_bf16(seeai_ctx* ctx, const uint16_t* d_q, const uint16_t* d_k,
                        const uint16_t* d_v, float* d_o, float* d_stats, uint64_t B,
                        uint64_t S, uint64_t H, uint64_t d, const int32_t* d_starts);
/* dQ and the stats row's delta, then dK and dV, on the same bf16 operands
 * (dout bf16 too) and the forward's stats rows: AttnDQTiled and the fused
 * AttnDKTiled + AttnDVTiled pair (attention.cc:494-590) with bf16 in HBM.
 * dQ, dK, dV are f32 [B*S, H*64]; in seeai_attn_dkdv_bf16 one of d_dk, d_dv
 * may be NULL. */
int seeai_attn_dq_bf16(seeai_ctx* ctx, const uint16_t* d_q, const uint16_t* d_k,
                       const uint16_t* d_v, const uint16_t* d_dout, float* d_stats,
                       float* d_dq, uint64_t B, uint64_t S, uint64_t H, uint64_t d);
int seeai_attn_dkdv_bf16(seeai_ctx* ctx, const uint16_t* d_q, const uint16_t* d_k,
                         const uint16_t* d_v, const uint16_t* d_dout, const float* d_stats,
                         float* d_dk, float* d_dv, uint64_t B, uint64_t S, uint64_t H,
                         uint64_t d);
int seeai_attn_dq(seeai_ctx* ctx, int dtype, const float* d_q,
                  const float* d_k, const float* d_v, const float* d_dout,
                  float* d_stats, float* d_dq, uint64_t B, uint64_t S,
                  uint64_t H, uint64_t d);
int seeai_attn_dk(seeai_ctx* ctx, int dtype, const float* d_q,
                  const float* d_k, const float* d_v, const float* d_dout,
                  const float* d_stats, float* d_dk, uint64_t B, uint64_t S,
                  uint64_t H, uint64_t d);
int seeai_attn_dv(seeai_ctx* ctx, int dtype, const float* d_q,
                  const float* d_k, const float* d_dout, const float* d_stats,
                  float* d_dv, uint64_t B, uint64_t S, uint64_t H,
                  uint64_t d);
/* AttnDKTiled + AttnDVTiled (attention.cc:537-590) in one relaxed pass
 * (bf16 MFMA): what a fused pair of the two instructions runs.  d = 64,
 * 16-byte aligned operands; status 2 otherwise. */
int seeai_attn_dkdv(seeai_ctx* ctx, const float* d_q, const float* d_k,
                    const float* d_v, const float* d_dout,
                    const float* d_stats, float* d_dk, float* d_dv,
                    uint64_t B, uint64_t S, uint64_t H, uint64_t d);
/* AttnDKTiled + AttnDVTiled (attention.cc:537-590) in one exact-family pass
 * (f32 MFMA): what an adjacent exact pair runs in a range, each output the
 * bits of its own pass (seeai_attn_dk / seeai_attn_dv).  d = 64 or 128,
 * 16-byte aligned operands, both outputs; status 2 otherwise. */
int seeai_attn_dkdv_f32(seeai_ctx* ctx, const float* d_q, const float* d_k,
                        const float* d_v, const float* d_dout,
                        const float* d_stats, float* d_dk, float* d_dv,
                        uint64_t B, uint64_t S, uint64_t H, uint64_t d);

/* SoftmaxXEntFwd / Bwd and the masked pair (loss.cc:35-126). */
int seeai_xent_fwd(seeai_ctx* ctx, const float* d_logits,
                   const int32_t* d_labels, float* d_loss, float* d_probs,
                   uint64_t N, uint64_t C, int masked);
/* seeai_xent_fwd that allocates nothing -- no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels and bits as seeai_xent_fwd; its per-row partials live in a 2 MiB
 * device array the library holds on each GPU until the process ends, so N
 * is at most SEEAI_XENT_NOALLOC_MAX_ROWS (status 2 beyond).  Every call on
 * one GPU shares that array: calls that overlap on one GPU (several
 * contexts or streams at once) race. */
#define SEEAI_XENT_NOALLOC_MAX_ROWS 131056u
int seeai_xent_fwd_noalloc(seeai_ctx* ctx, const float* d_logits,
                           const int32_t* d_labels, float* d_loss, float* d_probs,
                           uint64_t N, uint64_t C, int masked);
int seeai_xent_bwd(seeai_ctx* ctx, const float* d_probs,
                   const int32_t* d_labels, const float* d_seed,
                   float* d_dlogits, uint64_t N, uint64_t C, int masked);
/* AdamWStep with the fused clip (optimizer.cc:104-132); a refused step is
 * reported by the next seeai_flush. */
int seeai_adamw_step(seeai_ctx* ctx, float* d_p, const float* d_g,
                     float* d_m, float* d_v, uint64_t n,
                     const seeai_step_params* params, float clip_norm);
/* The eval argmax, first maximum wins (update_engine.cc:537-565). */
int seeai_argmax_rows(seeai_ctx* ctx, const float* d_probs, uint64_t rows,
                      uint64_t cols, int32_t* d_out);
/* The eval accuracy tally (update_engine.cc:537-565): over the rows whose
 * label is not -1, *hits counts those whose label is the row's argmax (first
 * maximum wins) and *judged those counted.  Device probabilities and i32
 * labels in, host counts out; waits for the stream. */
int seeai_argmax_tally(seeai_ctx* ctx, const float* d_probs, const int32_t* d_labels,
                       uint64_t rows, uint64_t cols, uint64_t* hits, uint64_t* judged);

#ifdef __cplusplus
}
#endif

#endif /* SEEAI_HIP_H_ */
