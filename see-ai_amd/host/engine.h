// engine.h -- the step loop of the reference's UpdateEngine
// (runtime/dispatcher/update_engine.cc) over the gfx950 HipBackend: load a
// plan, keep the host arena as the mirror of the device arena, and run the
// train / eval / merge programs one range at a time with the reference's
// step and learning-rate discipline.  The feeder, checkpointing, gating and
// reporting around that loop stay with the reference's dispatcher.
#pragma once

#include <cstdint>
#include <memory>
#include <span>
#include <vector>

#include "hip_backend.h"
#include "plan.h"
#include "result.h"

struct seeai_feeder;

namespace seeai::host {

class PlanEngine {
 public:
  // DecodePlan + AllocateArena + Bind (plan_loader.cc:19-288,
  // update_engine.cc:234-263).  The blob is copied; rodata is uploaded.
  static Result<std::unique_ptr<PlanEngine>> Load(std::span<const uint8_t> blob, int device);
  ~PlanEngine();

  const PlanHeader& header() const { return plan_.header; }
  const Plan& plan() const { return plan_; }
  HipBackend& backend() { return *backend_; }

  // update_engine.cc:370-391: constant, or linear warmup then cosine decay
  // to lr * min_lr_factor over the run's horizon (the plan's default_steps
  // unless set).
  float EffectiveLr() const;
  uint64_t step() const { return step_; }
  void set_step(uint64_t step) { step_ = step; }
  void set_horizon(uint64_t steps) { horizon_ = steps; }
  uint64_t horizon() const { return horizon_ ? horizon_ : plan_.header.default_steps; }

  // One optimizer step (update_engine.cc:840-870): the step counter moves
  // to the next 1-indexed timestep; each of the max(1, grad_accum_steps)
  // micro-batches is staged into the I/O slots and the train program runs;
  // the step program follows when the plan accumulates.  `inputs` holds
  // that many batches of input_floats floats, `labels` as many batches of
  // label_bytes.  Returns the micro-batches' mean loss.
  Result<float> TrainStep(const float* inputs, const void* labels);
  // Optimizer steps over `batches` consecutive batches (each step takes
  // max(1, grad_accum_steps) of them), fed as the reference's BatchPipeline
  // feeds them (runtime/pipeline/batch_pipeline.h:13-57): a feeder thread
  // checks and stages batch b + 1 -- pinned copy, upload on the feeder's
  // own stream -- while the step on batch b runs, and each step begins by
  // moving its staged batch into the I/O slots behind the upload's event.
  // The batches and their order are TrainStep's, so the results are bit
  // for bit those of calling TrainStep once per step.  One loss per step
  // lands in `losses`.  The host mirror's I/O slots are not refreshed.
  Result<void> TrainSteps(const float* inputs, const void* labels, uint64_t batches,
                          float* losses);
  // Runs the train program again on the batch already staged (the bench's
  // device-resident step: no host-to-device copy inside the step).
  Result<float> TrainStepResident();
  // The eval program on one staged batch (update_engine.cc:437-565): the
  // loss, and -- where the plan trains on class labels and its eval program
  // ends in a softmax over at least the batch's rows -- the accuracy tally:
  // rows whose argmax (first maximum wins) is their label, over the rows
  // whose label is not -1 (:537-565).  judged = 0 where accuracy is not
  // tracked.
  struct EvalMetrics {
    float loss = 0.0f;
    uint64_t hits = 0;
    uint64_t judged = 0;
    bool tracked = false;
  };
  Result<EvalMetrics> EvaluateMetrics(const float* input, const void* labels);
  Result<float> Evaluate(const float* input, const void* labels);
  // The merge program, then the emit entries' deltas copied to the host
  // mirror (update_engine.cc:1028-1063).
  Result<void> Merge();

  // update_engine.cc:82 (BindSourceModel): the source model file's image,
  // which source refs (bit 62) read; refused when smaller than what the
  // programs read.
  Result<void> BindSource(const uint8_t* data, uint64_t bytes);

  // Arena access through the host mirror (checkpoint / parity reads).
  Result<void> Read(uint64_t offset, void* dst, uint64_t bytes);
  Result<void> Write(uint64_t offset, const void* src, uint64_t bytes);

 private:
  PlanEngine() = default;
  Result<void> Stage(const float* input, const void* labels);
  // The feeder's token and label contracts on one batch.
  Result<void> CheckBatch(const float* input, const void* labels) const;
  // Runs [begin, end) of a program and drains the stream; with loss_after,
  // the plan's loss is read back in the same drain.
  Result<void> ExecuteRange(const std::vector<Instruction>& program, size_t begin, size_t end,
                            float* loss_after = nullptr);
  Result<float> Loss();

  std::vector<uint8_t> blob_;
  Plan plan_;
  std::unique_ptr<HipBackend> backend_;
  uint8_t* arena_ = nullptr;  // 16 KiB-aligned, inside the anonymous mapping map_
  uint64_t arena_bytes_ = 0;
  void* map_ = nullptr;
  uint64_t map_bytes_ = 0;
  uint64_t step_ = 0;
  uint64_t horizon_ = 0;
  uint64_t num_classes_ = 0;
  bool masked_labels_ = false;  // the plan's loss ignores positions labelled -1
  uint64_t vocab_bound_ = 0;     // token plans: the narrowest embedding's rows
  uint64_t source_required_ = 0;  // bytes of the source model the programs read
  // The eval program's last softmax (update_engine.cc:474-478): its
  // probabilities' arena offset, rows and width.
  uint64_t eval_probs_off_ = 0, eval_rows_ = 0, eval_cols_ = 0;
  bool eval_probs_ = false;
  uint64_t source_bytes_ = 0;     // bytes of the bound source model
  seeai_feeder* feeder_ = nullptr;  // TrainSteps' device staging, made on first use
};

}  // namespace seeai::host
