// capi_engine.cc -- the plan engine's C ABI (include/seeai_engine.h).
#include <cstring>
#include <memory>
#include <string>

#include "engine.h"
#include "seeai_engine.h"

using seeai::host::PlanEngine;

struct seeai_engine {
  std::unique_ptr<PlanEngine> engine;
  std::string error;
};

namespace {

void CopyMessage(const std::string& text, char* msg, uint64_t msg_bytes) {
  if (!msg || msg_bytes == 0) return;
  const size_t n = text.size() < msg_bytes - 1 ? text.size() : msg_bytes - 1;
  std::memcpy(msg, text.data(), n);
  msg[n] = '\0';
}

// Refusals of a step keep their status: the executor's kNonFiniteNormRefusal
// and kClipThresholdRefusal (backend.h:65-80) arrive inside the engine's
// "failed at instruction" / "failed to complete" wrappers.
int StatusOf(const std::string& message) {
  if (message.find("gradient norm is not finite") != std::string::npos ||
      message.find("clip threshold is not a finite positive float") != std::string::npos)
    return SEEAI_REFUSED;
  if (message.find("hip:") != std::string::npos) return SEEAI_HIP_ERROR;
  return SEEAI_INVALID;
}

template <class R>
int Report(seeai_engine* e, const R& r) {
  if (r) return SEEAI_OK;
  e->error = r.error();
  return StatusOf(e->error);
}

}  // namespace

extern "C" {

uint64_t seeai_plan_self_hash(const void* blob, uint64_t bytes, uint64_t hash_offset) {
  return seeai::host::PlanSelfHash(static_cast<const uint8_t*>(blob), bytes, hash_offset);
}

int seeai_plan_check(const void* blob, uint64_t bytes, char* msg, uint64_t msg_bytes) {
  if (!blob && bytes) return SEEAI_INVALID;
  auto plan = seeai::host::ReadPlan({static_cast<const uint8_t*>(blob), bytes});
  if (!plan) {
    CopyMessage(plan.error(), msg, msg_bytes);
    return SEEAI_INVALID;
  }
  uint64_t source = 0;
  if (auto ok = seeai::host::VerifyPrograms(*plan, &source); !ok) {
    CopyMessage(ok.error(), msg, msg_bytes);
    return SEEAI_INVALID;
  }
  CopyMessage("", msg, msg_bytes);
  return SEEAI_OK;
}

int seeai_engine_create(int device, const void* blob, uint64_t bytes, seeai_engine** out,
                        char* msg, uint64_t msg_bytes) {
  if (!out) return SEEAI_INVALID;
  *out = nullptr;
  if (!blob && bytes) return SEEAI_INVALID;
  auto engine = PlanEngine::Load({static_cast<const uint8_t*>(blob), bytes}, device);
  if (!engine) {
    CopyMessage(engine.error(), msg, msg_bytes);
    return StatusOf(engine.error());
  }
  *out = new seeai_engine{std::move(*engine), {}};
  CopyMessage("", msg, msg_bytes);
  return SEEAI_OK;
}

void seeai_engine_destroy(seeai_engine* e) { delete e; }

const char* seeai_engine_last_error(const seeai_engine* e) { return e ? e->error.c_str() : ""; }

int seeai_engine_header(const seeai_engine* e, void* out) {
  if (!e || !out) return SEEAI_INVALID;
  std::memcpy(out, &e->engine->header(), sizeof(seeai::host::PlanHeader));
  return SEEAI_OK;
}

int seeai_engine_train_step(seeai_engine* e, const float* inputs, const void* labels, float* loss) {
  if (!e || !inputs) return SEEAI_INVALID;
  auto r = e->engine->TrainStep(inputs, labels);
  if (r && loss) *loss = *r;
  return Report(e, r);
}

int seeai_engine_train_steps(seeai_engine* e, const float* inputs, const void* labels,
                             uint64_t batches, float* losses) {
  if (!e || !inputs || !losses) return SEEAI_INVALID;
  return Report(e, e->engine->TrainSteps(inputs, labels, batches, losses));
}

int seeai_engine_train_resident(seeai_engine* e, float* loss) {
  if (!e) return SEEAI_INVALID;
  auto r = e->engine->TrainStepResident();
  if (r && loss) *loss = *r;
  return Report(e, r);
}

int seeai_engine_evaluate(seeai_engine* e, const float* input, const void* labels, float* loss) {
  if (!e || !input) return SEEAI_INVALID;
  auto r = e->engine->Evaluate(input, labels);
  if (r && loss) *loss = *r;
  return Report(e, r);
}

int seeai_engine_evaluate_metrics(seeai_engine* e, const float* input, const void* labels,
                                  float* loss, uint64_t* hits, uint64_t* judged) {
  if (!e || !input) return SEEAI_INVALID;
  auto r = e->engine->EvaluateMetrics(input, labels);
  if (r) {
    if (loss) *loss = r->loss;
    if (hits) *hits = r->hits;
    if (judged) *judged = r->judged;
  }
  return Report(e, r);
}

int seeai_engine_merge(seeai_engine* e) {
  if (!e) return SEEAI_INVALID;
  return Report(e, e->engine->Merge());
}

int seeai_engine_bind_source(seeai_engine* e, const void* data, uint64_t bytes) {
  if (!e || (!data && bytes)) return SEEAI_INVALID;
  return Report(e, e->engine->BindSource(static_cast<const uint8_t*>(data), bytes));
}

int seeai_engine_read(seeai_engine* e, uint64_t offset, void* dst, uint64_t bytes) {
  if (!e || (!dst && bytes)) return SEEAI_INVALID;
  return Report(e, e->engine->Read(offset, dst, bytes));
}

int seeai_engine_write(seeai_engine* e, uint64_t offset, const void* src, uint64_t bytes) {
  if (!e || (!src && bytes)) return SEEAI_INVALID;
  return Report(e, e->engine->Write(offset, src, bytes));
}

uint64_t seeai_engine_step(const seeai_engine* e) { return e ? e->engine->step() : 0; }
void seeai_engine_set_step(seeai_engine* e, uint64_t step) {
  if (e) e->engine->set_step(step);
}
void seeai_engine_set_horizon(seeai_engine* e, uint64_t steps) {
  if (e) e->engine->set_horizon(steps);
}
float seeai_engine_lr(const seeai_engine* e) { return e ? e->engine->EffectiveLr() : 0.0f; }
uint64_t seeai_engine_relaxed_executions(const seeai_engine* e) {
  return e ? e->engine->backend().relaxed_executions() : 0;
}
seeai_ctx* seeai_engine_context(seeai_engine* e) { return e ? e->engine->backend().context() : nullptr; }

}  // extern "C"
