/*
 * seeai_engine.h -- the C ABI of the plan engine above the executor
 * (libseeai_hip.so, see-ai_amd/host/).  The reference loads a .seeu plan
 * and steps it in C++ (runtime/loader/plan_loader.cc, runtime/dispatcher/
 * update_engine.cc); these entry points expose the same load / train /
 * evaluate / merge verbs over the gfx950 HipBackend to callers that are not
 * C++ (the Python tests and bench).  Status codes are seeai_hip.h's.
 */
#ifndef SEEAI_ENGINE_H_
#define SEEAI_ENGINE_H_

#include <stddef.h>
#include <stdint.h>

#include "seeai_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct seeai_engine seeai_engine;

/* PlanSelfHash (source/identity/hash.h:136-158) of a plan blob with the
 * 8-byte field at `hash_offset` (216 for the PlanHeader) read as zero. */
uint64_t seeai_plan_self_hash(const void* blob, uint64_t bytes, uint64_t hash_offset);
/* DecodePlan's header contract (plan_loader.cc:19-49, plan_contract.h:
 * 35-180) and the executor contract (VerifyExecutorContract,
 * runtime/loader/contract.cc:51-244: every operand of every program in
 * bounds, unaliased where written, the flag bits each opcode takes, the
 * feeder-bounded label / token operands, emit entries in the arena) without
 * a device: 0 if the plan is loadable, else SEEAI_INVALID and the refusal in
 * `msg` (NUL-terminated, truncated to msg_bytes). */
int seeai_plan_check(const void* blob, uint64_t bytes, char* msg, uint64_t msg_bytes);

/* Load a plan onto `device` (DecodePlan + AllocateArena + Bind).  On
 * failure *out is NULL and the reason is in `msg`. */
int seeai_engine_create(int device, const void* blob, uint64_t bytes, seeai_engine** out,
                        char* msg, uint64_t msg_bytes);
void seeai_engine_destroy(seeai_engine* engine);
const char* seeai_engine_last_error(const seeai_engine* engine);
/* The decoded PlanHeader (320 bytes). */
int seeai_engine_header(const seeai_engine* engine, void* out);

/* One optimizer step (update_engine.cc:840-870): max(1, grad_accum_steps)
 * batches of input_floats floats and label_bytes label bytes, consecutive. */
int seeai_engine_train_step(seeai_engine* engine, const float* inputs, const void* labels,
                            float* loss);
/* The train program again on the batch already staged, no host-to-device
 * copy: the device-resident step. */
int seeai_engine_train_resident(seeai_engine* engine, float* loss);
/* Optimizer steps over `batches` consecutive batches (max(1,
 * grad_accum_steps) per step) with the reference's BatchPipeline overlap
 * (runtime/pipeline/batch_pipeline.h:13-57): a feeder thread checks and
 * uploads the next batch while the current step runs.  Bit-identical to
 * seeai_engine_train_step once per step; one loss per step in `losses`. */
int seeai_engine_train_steps(seeai_engine* engine, const float* inputs, const void* labels,
                             uint64_t batches, float* losses);
int seeai_engine_evaluate(seeai_engine* engine, const float* input, const void* labels,
                          float* loss);
/* The eval program with its accuracy tally (update_engine.cc:437-565): the
 * loss, the rows whose argmax (first maximum wins) is their label, and the
 * rows judged (label not -1).  *judged is 0 where the plan tracks no
 * accuracy (no class labels, or no eval softmax covering the batch). */
int seeai_engine_evaluate_metrics(seeai_engine* engine, const float* input, const void* labels,
                                  float* loss, uint64_t* hits, uint64_t* judged);
int seeai_engine_merge(seeai_engine* engine);
/* UpdateEngine::BindSourceModel (update_engine.cc:82): the source model
 * file's image, read by source refs (bit 62).  Refused when smaller than the
 * extent the plan's programs read; until one is bound, a plan that reads it
 * refuses to run. */
int seeai_engine_bind_source(seeai_engine* engine, const void* data, uint64_t bytes);
/* Arena bytes through the host mirror. */
int seeai_engine_read(seeai_engine* engine, uint64_t offset, void* dst, uint64_t bytes);
int seeai_engine_write(seeai_engine* engine, uint64_t offset, const void* src, uint64_t bytes);

uint64_t seeai_engine_step(const seeai_engine* engine);
void seeai_engine_set_step(seeai_engine* engine, uint64_t step);
void seeai_engine_set_horizon(seeai_engine* engine, uint64_t steps);
/* EffectiveLr at the current step (update_engine.cc:370-391). */
float seeai_engine_lr(const seeai_engine* engine);
uint64_t seeai_engine_relaxed_executions(const seeai_engine* engine);
/* The executor context underneath (its stream, relaxed switch). */
seeai_ctx* seeai_engine_context(seeai_engine* engine);

#ifdef __cplusplus
}
#endif

#endif /* SEEAI_ENGINE_H_ */
