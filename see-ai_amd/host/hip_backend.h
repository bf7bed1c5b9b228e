// hip_backend.h -- the executor seam (runtime/executor/backend.h:82-166,
// class ExecutorBackend) implemented over this repository's C ABI
// (include/seeai_hip.h).  The reference's engine calls exactly these
// methods: Bind (+ Configure) at load, BeginRange / Execute* / Flush /
// EndRange per range, relaxed_executions() for reporting.  A discrete GPU
// also needs the two host-sync verbs the seam lacks (the reference's Metal
// arena is zero-copy shared memory): SyncToDevice for the feeder's I/O
// slots before a range, SyncToHost for what the engine reads after Flush.
#pragma once

#include <cstdint>
#include <memory>
#include <span>
#include <string>

#include "plan.h"
#include "result.h"

struct seeai_ctx;
struct seeai_tile_policy;

namespace seeai::host {

// backend.h:56-63: the per-range scalars the optimizer instructions read.
struct StepParams {
  float lr = 0.0f;
  float beta1 = 0.0f;
  float beta2 = 0.0f;
  float eps = 0.0f;
  float weight_decay = 0.0f;
  uint64_t step = 0;
};

class HipBackend {
 public:
  // The device is opened here: no GPU, or no library, is a failure value.
  static Result<std::unique_ptr<HipBackend>> Create(int device);
  ~HipBackend();
  HipBackend(const HipBackend&) = delete;
  HipBackend& operator=(const HipBackend&) = delete;

  const char* name() const { return "hip"; }
  std::string device() const;

  // backend.h:89-101: the engine's host arena stays the host mirror; the
  // device arena is allocated at the same size and initialised from it;
  // rodata is uploaded once.  A refused Bind leaves the previous binding
  // executable.
  Result<void> Bind(uint8_t* arena, uint64_t arena_bytes, const uint8_t* rodata,
                    uint64_t rodata_bytes, uint64_t rodata_mapped_bytes);
  Result<void> BindSource(const uint8_t* data, uint64_t bytes);
  // backend.h:117: the kernel geometry, called after every successful Bind.
  // The plan header's CPU tile words do not apply to the gfx950 kernels; the
  // policy is the gfx950 member of the kernel-policy table (null: the
  // built-in geometry).  Every choice gives the same bits.
  Result<void> Configure(const seeai_tile_policy* policy = nullptr);
  Result<void> Execute(const Instruction& ins, const StepParams& params);
  // backend.h:139-142: whole-program visibility around a range.
  // The backend keeps the span until EndRange: Execute is then called with
  // references into it, and adjacent relaxed dK / dV instructions of one
  // attention run as one dispatch.
  void BeginRange(std::span<const Instruction> program, size_t begin, size_t end);
  void EndRange();
  // The range [begin, end) as BeginRange + Execute each + EndRange, replayed
  // from a captured HIP graph from its second run (seeai_run_range); on
  // failure *failed_at names the instruction.
  Result<void> RunRange(std::span<const Instruction> program, size_t begin, size_t end,
                        const StepParams& params, size_t* failed_at);
  // backend.h:147: drains the stream; reports a refused optimizer step.
  Result<void> Flush();
  // Flush with `bytes` of the arena at `offset` synced to the host in the
  // same drain (seeai_flush_download).
  Result<void> FlushSyncToHost(uint64_t offset, uint64_t bytes);
  uint64_t relaxed_executions() const;
  uint64_t fused_dispatches() const;
  void SetRelaxed(bool allow);
  // Relaxed tiled attention on bf16 operands (true) or f32 products (false,
  // the default): seeai_set_attention_bf16.
  void SetAttentionBf16(bool on);

  Result<void> SyncToDevice(uint64_t offset, uint64_t bytes);
  Result<void> SyncToHost(uint64_t offset, uint64_t bytes);

  seeai_ctx* context() const { return ctx_; }

 private:
  // Uploads the blocks of `arena` holding a nonzero byte into the device
  // arena seeai_bind zeroed.
  Result<void> UploadNonZero(const uint8_t* arena, uint64_t bytes);
  explicit HipBackend(seeai_ctx* ctx) : ctx_(ctx) {}
  Result<void> Check(int status) const;

  seeai_ctx* ctx_;
  uint8_t* host_ = nullptr;
  uint64_t host_bytes_ = 0;
};

}  // namespace seeai::host
