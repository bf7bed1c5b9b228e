// engine.cc -- the plan engine's step loop (see engine.h).
#include "engine.h"

#include <sys/mman.h>

#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>

#include "seeai_hip.h"

namespace seeai::host {
namespace {

constexpr uint16_t kOpSoftmaxXEntFwd = 11, kOpSoftmaxXEntBwd = 12;              // instruction.h:63-64
constexpr uint16_t kOpSoftmaxXEntMaskedFwd = 51, kOpSoftmaxXEntMaskedBwd = 52;  // v22 masked pair
constexpr uint16_t kOpEmbedFwd = 41;                                            // instruction.h:141

bool IsXent(uint16_t op) {
  return op == kOpSoftmaxXEntFwd || op == kOpSoftmaxXEntBwd || op == kOpSoftmaxXEntMaskedFwd ||
         op == kOpSoftmaxXEntMaskedBwd;
}

}  // namespace

Result<std::unique_ptr<PlanEngine>> PlanEngine::Load(std::span<const uint8_t> blob, int device) {
  std::unique_ptr<PlanEngine> e(new PlanEngine());
  e->blob_.assign(blob.begin(), blob.end());
  auto plan = ReadPlan(e->blob_);
  if (!plan) return Fail(plan.error());
  e->plan_ = std::move(*plan);
  const PlanHeader& h = e->plan_.header;
  if (auto ok = VerifyPrograms(e->plan_, &e->source_required_); !ok) return Fail(ok.error());

  // plan_loader.cc:151-166: the narrowest softmax width anywhere bounds the
  // class labels the feeder may stage.
  for (const auto* program : {&e->plan_.train, &e->plan_.merge, &e->plan_.eval, &e->plan_.step})
    for (const Instruction& ins : *program) {
      if (IsXent(ins.opcode) && ins.out[1] != 0 &&
          (e->num_classes_ == 0 || ins.out[1] < e->num_classes_))
        e->num_classes_ = ins.out[1];
      if (ins.opcode == kOpSoftmaxXEntMaskedFwd || ins.opcode == kOpSoftmaxXEntMaskedBwd)
        e->masked_labels_ = true;
      // plan_loader.cc:196-204: the narrowest embedding bounds token ids.
      if (ins.opcode == kOpEmbedFwd) {
        const uint64_t vocab = ins.out[1] >> 32;
        if (vocab != 0 && (e->vocab_bound_ == 0 || vocab < e->vocab_bound_)) e->vocab_bound_ = vocab;
      }
    }
  // update_engine.cc:474-478: accuracy is read from the eval program's
  // softmax probabilities.
  for (const Instruction& ins : e->plan_.eval)
    if (ins.opcode == kOpSoftmaxXEntFwd || ins.opcode == kOpSoftmaxXEntMaskedFwd) {
      e->eval_probs_ = IsArenaRef(ins.in[3]);
      e->eval_probs_off_ = RefOffset(ins.in[3]);
      e->eval_rows_ = ins.out[0];
      e->eval_cols_ = ins.out[1];
    }
  if (h.input_kind > 1) return Fail("unknown plan input kind " + std::to_string(h.input_kind));
  if (h.input_kind == 1) {
    if (e->vocab_bound_ == 0)
      return Fail("token plan carries no embedding \xe2\x80\x94 its token ids could never be validated");
    if (h.seq_len == 0 || h.batch % h.seq_len != 0)
      return Fail("token plan sequence length must be nonzero and divide the batch");
  }
  if (h.label_kind == 1 && e->num_classes_ == 0)
    return Fail("class-label plan carries no softmax cross-entropy \xe2\x80\x94 its labels could "
                "never be validated");

  // plan_loader.cc:251-288: one zeroed, 16 KiB-aligned allocation holding
  // the persistent image at offset 0.  Anonymous pages read as zero until
  // written, so the arena past the image costs no host memory or time (the
  // mapping is over-sized by one alignment unit and the arena starts at its
  // first 16 KiB boundary).
  e->arena_bytes_ = (h.arena_size + (kArenaAlignment - 1)) & ~(kArenaAlignment - 1);
  if (e->arena_bytes_ == 0) e->arena_bytes_ = kArenaAlignment;
  e->map_bytes_ = e->arena_bytes_ + kArenaAlignment;
  void* map = mmap(nullptr, e->map_bytes_, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS,
                   -1, 0);
  if (map == MAP_FAILED) return Fail("arena allocation failed");
  e->map_ = map;
  e->arena_ = reinterpret_cast<uint8_t*>(
      (reinterpret_cast<uintptr_t>(map) + (kArenaAlignment - 1)) & ~uintptr_t{kArenaAlignment - 1});
  if (!e->plan_.persist_init.empty())
    std::memcpy(e->arena_, e->plan_.persist_init.data(), e->plan_.persist_init.size());

  auto backend = HipBackend::Create(device);
  if (!backend) return Fail(backend.error());
  e->backend_ = std::move(*backend);
  if (auto r = e->backend_->Bind(e->arena_, e->arena_bytes_, e->plan_.rodata.data(),
                                 e->plan_.rodata.size(), e->plan_.rodata.size());
      !r)
    return Fail(r.error());
  if (auto r = e->backend_->Configure(); !r) return Fail(r.error());
  return e;
}

PlanEngine::~PlanEngine() {
  seeai_feeder_destroy(feeder_);  // before the context it copies into
  backend_.reset();  // the backend's views die before the memory they view
  if (map_) munmap(map_, map_bytes_);
}

float PlanEngine::EffectiveLr() const {
  const PlanHeader& h = plan_.header;
  const float base = h.lr;
  if (static_cast<LrSchedule>(h.lr_schedule) != LrSchedule::kCosineWithWarmup) return base;
  if (h.warmup_steps > 0 && step_ <= h.warmup_steps)
    return base * static_cast<float>(step_) / static_cast<float>(h.warmup_steps);
  const uint64_t run = horizon();
  const uint64_t span = run > h.warmup_steps ? run - h.warmup_steps : 0;
  const float floor = base * h.min_lr_factor;
  if (span == 0 || step_ - h.warmup_steps >= span) return floor;
  const float t = static_cast<float>(step_ - h.warmup_steps) / static_cast<float>(span);
  constexpr float kPi = 3.14159265358979323846f;
  return floor + (base - floor) * 0.5f * (1.0f + std::cos(kPi * t));
}

Result<void> PlanEngine::CheckBatch(const float* input, const void* labels) const {
  const PlanHeader& h = plan_.header;
  if (h.input_kind == 1) {
    // The feeder's token contract: every id indexes an embedding row.
    const auto* tok = reinterpret_cast<const int32_t*>(input);
    for (uint64_t i = 0; i < h.input_floats; ++i)
      if (tok[i] < 0 || static_cast<uint64_t>(tok[i]) >= vocab_bound_)
        return Fail("token " + std::to_string(tok[i]) + " at position " + std::to_string(i) +
                    " is outside the plan's " + std::to_string(vocab_bound_) + "-token vocabulary");
  }
  if (h.label_kind == 0) return {};
  if (!labels) return Fail("this plan trains on labels: none were staged");
  if (h.label_kind == 1) {
    // The feeder's value contract: every class index below the plan's
    // narrowest softmax width (-1, an ignored position, only where the
    // plan's masked loss expects it).
    const bool masked = masked_labels_;
    const auto* lab = static_cast<const int32_t*>(labels);
    for (uint64_t i = 0; i < h.label_bytes / sizeof(int32_t); ++i)
      if (lab[i] >= static_cast<int64_t>(num_classes_) || lab[i] < (masked ? -1 : 0))
        return Fail("label " + std::to_string(lab[i]) + " at position " + std::to_string(i) +
                    " is outside the plan's " + std::to_string(num_classes_) + " classes");
  }
  return {};
}

Result<void> PlanEngine::Stage(const float* input, const void* labels) {
  const PlanHeader& h = plan_.header;
  if (auto r = CheckBatch(input, labels); !r) return r;
  const uint64_t in_off = RefOffset(h.input_ref), in_bytes = h.input_floats * sizeof(float);
  std::memcpy(arena_ + in_off, input, in_bytes);
  if (auto r = backend_->SyncToDevice(in_off, in_bytes); !r) return r;
  if (h.label_kind == 0) return {};
  const uint64_t lab_off = RefOffset(h.label_ref);
  std::memcpy(arena_ + lab_off, labels, h.label_bytes);
  return backend_->SyncToDevice(lab_off, h.label_bytes);
}

Result<void> PlanEngine::ExecuteRange(const std::vector<Instruction>& program, size_t begin,
                                      size_t end, float* loss_after) {
  const PlanHeader& h = plan_.header;
  if (source_required_ > source_bytes_)
    return Fail("this plan reads the source model: bind it with BindSource before running");
  const StepParams params{EffectiveLr(), h.beta1, h.beta2, h.eps, h.weight_decay, step_};
  // BeginRange, Execute of each instruction, EndRange -- replayed as one
  // graph launch once the range has run before (HipBackend::RunRange).
  size_t idx = begin;
  if (auto r = backend_->RunRange(std::span<const Instruction>(program), begin, end, params, &idx);
      !r)
    return Fail(std::string("backend '") + backend_->name() + "' failed at instruction " +
                std::to_string(idx) + ": " + r.error());
  if (loss_after) {  // the loss synced to the host in the flush's own drain
    const uint64_t off = RefOffset(plan_.header.loss_ref);
    if (auto flushed = backend_->FlushSyncToHost(off, sizeof(float)); !flushed)
      return Fail(std::string("backend '") + backend_->name() + "' failed to complete: " +
                  flushed.error());
    std::memcpy(loss_after, arena_ + off, sizeof(float));
    return {};
  }
  auto flushed = backend_->Flush();
  if (!flushed)
    return Fail(std::string("backend '") + backend_->name() + "' failed to complete: " +
                flushed.error());
  return {};
}

Result<void> PlanEngine::BindSource(const uint8_t* data, uint64_t bytes) {
  // update_engine.cc:82: the source model's image; every source operand
  // the programs name must lie inside it.
  if (bytes < source_required_)
    return Fail("source model is " + std::to_string(bytes) + " bytes; the plan reads " +
                std::to_string(source_required_));
  if (auto r = backend_->BindSource(data, bytes); !r) return r;
  source_bytes_ = bytes;
  return {};
}

Result<float> PlanEngine::Loss() {
  const uint64_t off = RefOffset(plan_.header.loss_ref);
  if (auto r = backend_->SyncToHost(off, sizeof(float)); !r) return Fail(r.error());
  float loss;
  std::memcpy(&loss, arena_ + off, sizeof(loss));
  return loss;
}

Result<float> PlanEngine::TrainStep(const float* inputs, const void* labels) {
  const PlanHeader& h = plan_.header;
  const uint64_t micro = h.grad_accum_steps > 1 ? h.grad_accum_steps : 1;
  // A refused batch refuses the step before it runs: no timestep is spent.
  for (uint64_t g = 0; g < micro; ++g) {
    const auto* lab = labels ? static_cast<const uint8_t*>(labels) + g * h.label_bytes : nullptr;
    if (auto r = CheckBatch(inputs + g * h.input_floats, lab); !r) return Fail(r.error());
  }
  ++step_;  // the 1-indexed timestep of this optimizer step
  double loss_sum = 0.0;
  for (uint64_t g = 0; g < micro; ++g) {
    const auto* lab = labels ? static_cast<const uint8_t*>(labels) + g * h.label_bytes : nullptr;
    if (auto r = Stage(inputs + g * h.input_floats, lab); !r) return Fail(r.error());
    float loss = 0.0f;
    if (auto r = ExecuteRange(plan_.train, 0, plan_.train.size(), &loss); !r) return Fail(r.error());
    loss_sum += loss;
  }
  if (!plan_.step.empty())
    if (auto r = ExecuteRange(plan_.step, 0, plan_.step.size()); !r) return Fail(r.error());
  return static_cast<float>(loss_sum / static_cast<double>(micro));
}

Result<void> PlanEngine::TrainSteps(const float* inputs, const void* labels, uint64_t batches,
                                    float* losses) {
  const PlanHeader& h = plan_.header;
  const uint64_t micro = h.grad_accum_steps > 1 ? h.grad_accum_steps : 1;
  if (!inputs || !losses || batches == 0 || batches % micro != 0)
    return Fail("train_steps takes a whole number of optimizer steps' batches (" +
                std::to_string(micro) + " per step)");
  if (h.label_kind != 0 && !labels) return Fail("this plan trains on labels: none were staged");
  const uint64_t in_bytes = h.input_floats * sizeof(float);
  const uint64_t lab_bytes = h.label_kind != 0 ? h.label_bytes : 0;
  const uint64_t in_off = RefOffset(h.input_ref), lab_off = lab_bytes ? RefOffset(h.label_ref) : 0;
  seeai_ctx* ctx = backend_->context();
  if (!feeder_ && seeai_feeder_create(ctx, in_bytes, lab_bytes, &feeder_) != SEEAI_OK)
    return Fail(std::string("backend 'hip' failed to create the feeder: ") + seeai_last_error(ctx));

  // The feeder thread stays at most two batches ahead of the steps (the
  // device feeder's two slots); `taken` counts batches moved into the slots.
  std::mutex mu;
  std::condition_variable cv;
  uint64_t staged = 0, taken = 0;
  bool stop = false;
  std::string feeder_error;
  std::thread feeder([&] {
    for (uint64_t b = 0; b < batches; ++b) {
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return stop || staged - taken < 2; });
        if (stop) return;
      }
      const float* in = inputs + b * h.input_floats;
      const void* lab = lab_bytes ? static_cast<const uint8_t*>(labels) + b * h.label_bytes : nullptr;
      std::string err;
      if (seeai_feeder_stage(feeder_, in, lab) != SEEAI_OK) err = seeai_feeder_last_error(feeder_);
      std::lock_guard<std::mutex> lk(mu);
      if (!err.empty()) {
        feeder_error = "batch " + std::to_string(b) + ": " + err;
        stop = true;
        cv.notify_all();
        return;
      }
      ++staged;
      cv.notify_all();
    }
  });
  // Every exit joins the feeder (batch_pipeline.h's destructor contract).
  auto finish = [&](Result<void> r) -> Result<void> {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    cv.notify_all();
    feeder.join();
    return r;
  };
  for (uint64_t s = 0; s < batches / micro; ++s) {
    // As TrainStep: every micro-batch of the step is checked before the
    // step's timestep is spent, so a refusal leaves the engine where the
    // previous step left it (the feeder only stages).
    for (uint64_t g = 0; g < micro; ++g) {
      const uint64_t b = s * micro + g;
      const void* lab = lab_bytes ? static_cast<const uint8_t*>(labels) + b * h.label_bytes : nullptr;
      if (auto r = CheckBatch(inputs + b * h.input_floats, lab); !r)
        return finish(Fail("batch " + std::to_string(b) + ": " + r.error()));
    }
    double loss_sum = 0.0;
    for (uint64_t g = 0; g < micro; ++g) {
      bool starved;
      std::string why;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return stop || staged > taken; });
        starved = staged == taken;
        why = feeder_error;
      }
      if (starved) return finish(Fail(why));  // finish takes the lock itself
      if (g == 0) ++step_;  // the 1-indexed timestep of this optimizer step
      if (seeai_feeder_next(feeder_, in_off, lab_off) != SEEAI_OK)
        return finish(Fail(std::string("backend 'hip' failed to feed the batch: ") +
                           seeai_last_error(ctx)));
      {
        std::lock_guard<std::mutex> lk(mu);
        ++taken;
      }
      cv.notify_all();
      float loss = 0.0f;
      if (auto r = ExecuteRange(plan_.train, 0, plan_.train.size(), &loss); !r)
        return finish(Fail(r.error()));
      loss_sum += loss;
    }
    if (!plan_.step.empty())
      if (auto r = ExecuteRange(plan_.step, 0, plan_.step.size()); !r) return finish(Fail(r.error()));
    losses[s] = static_cast<float>(loss_sum / static_cast<double>(micro));
  }
  return finish({});
}

Result<float> PlanEngine::TrainStepResident() {
  if (plan_.header.grad_accum_steps > 1)
    return Fail("a resident step replays one staged batch; this plan accumulates micro-batches");
  ++step_;
  float loss = 0.0f;
  if (auto r = ExecuteRange(plan_.train, 0, plan_.train.size(), &loss); !r) return Fail(r.error());
  return loss;
}

Result<PlanEngine::EvalMetrics> PlanEngine::EvaluateMetrics(const float* input,
                                                             const void* labels) {
  if (plan_.eval.empty()) return Fail("plan carries no eval program");
  if (auto r = Stage(input, labels); !r) return Fail(r.error());
  if (auto r = ExecuteRange(plan_.eval, 0, plan_.eval.size()); !r) return Fail(r.error());
  auto loss = Loss();
  if (!loss) return Fail(loss.error());
  EvalMetrics m;
  m.loss = *loss;
  const PlanHeader& h = plan_.header;
  // update_engine.cc:467-470: class labels staged, and a softmax whose rows
  // cover the batch.
  if (h.label_kind == 1 && eval_probs_ && eval_cols_ > 0 && eval_rows_ >= h.batch) {
    uint8_t* dev = static_cast<uint8_t*>(seeai_arena(backend_->context()));
    const auto* probs = reinterpret_cast<const float*>(dev + eval_probs_off_);
    const auto* lab = reinterpret_cast<const int32_t*>(dev + RefOffset(h.label_ref));
    if (seeai_argmax_tally(backend_->context(), probs, lab, h.batch, eval_cols_, &m.hits,
                           &m.judged) != SEEAI_OK)
      return Fail(std::string("backend 'hip' failed to tally the eval accuracy: ") +
                  seeai_last_error(backend_->context()));
    m.tracked = true;
  }
  return m;
}

Result<float> PlanEngine::Evaluate(const float* input, const void* labels) {
  auto m = EvaluateMetrics(input, labels);
  if (!m) return Fail(m.error());
  return m->loss;
}

Result<void> PlanEngine::Merge() {
  if (auto r = ExecuteRange(plan_.merge, 0, plan_.merge.size()); !r) return r;
  for (const EmitEntry& e : plan_.emit)
    if (auto r = backend_->SyncToHost(e.arena_offset, e.byte_size); !r) return r;
  return {};
}

Result<void> PlanEngine::Read(uint64_t offset, void* dst, uint64_t bytes) {
  if (auto r = backend_->SyncToHost(offset, bytes); !r) return r;
  std::memcpy(dst, arena_ + offset, bytes);
  return {};
}

Result<void> PlanEngine::Write(uint64_t offset, const void* src, uint64_t bytes) {
  if (offset > arena_bytes_ || bytes > arena_bytes_ - offset)
    return Fail("arena write outside the arena");
  std::memcpy(arena_ + offset, src, bytes);
  return backend_->SyncToDevice(offset, bytes);
}

}  // namespace seeai::host
