// plan.h -- the .seeu plan as the gfx950 executor's host side reads it:
// the 320-byte PlanHeader, the 64-byte instruction word and the 24-byte
// emit entry (layouts fixed by source/plan/schema.h:296-412 and
// instruction.h:438-449, little-endian, packed), the plan's self-hash
// (source/identity/hash.h:34-158) and the header contract the loader
// enforces before any section is decoded (runtime/loader/plan_loader.cc:
// 19-49, source/contract/plan_contract.h:35-180).
//
// VerifyPrograms (verify.cc) is the per-instruction operand proof the
// reference's loader runs before anything executes (VerifyExecutorContract,
// runtime/loader/contract.cc:51-244): after it, the backend dispatches the
// programs blindly, as the reference's does.
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>
#include <string>
#include <vector>

#include "result.h"

namespace seeai::host {

inline constexpr uint32_t kSeeuMagic = 0x55454553;    // "SEEU", schema.h:18
inline constexpr uint32_t kSeeuVersion = 26;          // schema.h:165
inline constexpr uint32_t kSeeuOldestReadable = 4;    // schema.h:286
inline constexpr uint32_t kSeeuGemmTilesVersion = 11; // plan_contract.h:72
inline constexpr uint32_t kSeeuGradAccumVersion = 9;  // plan_contract.h:88
inline constexpr uint64_t kRodataAlignment = 16;      // plan_contract.h:54
inline constexpr uint64_t kArenaAlignment = 16384;    // plan_loader.cc:268
inline constexpr uint64_t kNullRef = ~uint64_t{0};
inline constexpr uint64_t kRodataBit = uint64_t{1} << 63;
inline constexpr uint64_t kSourceBit = uint64_t{1} << 62;

inline constexpr uint64_t RefOffset(uint64_t ref) { return ref & ~(kRodataBit | kSourceBit); }
inline constexpr bool IsRodataRef(uint64_t ref) { return ref != kNullRef && (ref & kRodataBit); }
inline constexpr bool IsArenaRef(uint64_t ref) {
  return ref != kNullRef && (ref & (kRodataBit | kSourceBit)) == 0;
}
inline constexpr bool IsSourceRef(uint64_t ref) {
  return ref != kNullRef && (ref & (kRodataBit | kSourceBit)) == kSourceBit;
}

enum class LrSchedule : uint32_t { kConstant = 0, kCosineWithWarmup = 1 };  // config.h:31

#pragma pack(push, 1)
struct PlanHeader {
  uint32_t magic = kSeeuMagic;
  uint32_t version = kSeeuVersion;
  uint64_t arena_size = 0;
  uint64_t persistent_size = 0;
  uint64_t input_ref = kNullRef;
  uint64_t input_floats = 0;
  uint64_t label_ref = kNullRef;
  uint64_t label_bytes = 0;
  uint32_t label_kind = 0;  // 0 none, 1 class indices (i32), 2 dense f32
  uint32_t optimizer_kind = 1;
  uint64_t loss_ref = kNullRef;
  uint64_t train_instr_offset = 0;
  uint64_t train_instr_count = 0;
  uint64_t merge_instr_offset = 0;
  uint64_t merge_instr_count = 0;
  uint64_t rodata_offset = 0;
  uint64_t rodata_size = 0;
  uint64_t persist_init_offset = 0;
  uint64_t persist_init_size = 0;
  uint64_t emit_table_offset = 0;
  uint64_t emit_count = 0;
  float lr = 1e-3f;
  float beta1 = 0.9f;
  float beta2 = 0.999f;
  float eps = 1e-8f;
  float weight_decay = 0.01f;
  uint32_t gemm_tile_k = 0;
  uint64_t batch = 0;
  uint64_t default_steps = 0;
  uint64_t eval_instr_offset = 0;
  uint64_t eval_instr_count = 0;
  uint64_t source_model_hash = 0;
  uint64_t plan_hash = 0;
  uint32_t lr_schedule = 0;
  uint32_t gemm_tile_n = 0;
  uint64_t warmup_steps = 0;
  float min_lr_factor = 0.0f;
  float clip_norm = 0.0f;
  uint32_t input_kind = 0;
  uint32_t grad_accum_steps = 0;
  uint64_t seq_len = 0;
  uint64_t step_instr_offset = 0;
  uint64_t step_instr_count = 0;
  uint64_t tokenizer_hash = 0;
  uint64_t corpus_hash = 0;
  uint64_t split_seed = 0;
  uint64_t val_split_hash = 0;
  uint32_t val_frac_bits = 0;
  uint32_t data_flags = 0;
};

struct EmitEntry {
  uint64_t smf_data_offset = 0;
  uint64_t byte_size = 0;
  uint64_t arena_offset = 0;
};

struct Instruction {
  uint16_t opcode = 0;
  uint16_t flags = 0;
  uint32_t imm = 0;
  uint64_t in[4] = {kNullRef, kNullRef, kNullRef, kNullRef};
  uint64_t out[3] = {0, 0, 0};
};
#pragma pack(pop)

static_assert(sizeof(PlanHeader) == 320, "PlanHeader layout is the .seeu ABI");
static_assert(sizeof(EmitEntry) == 24, "EmitEntry layout is the .seeu ABI");
static_assert(sizeof(Instruction) == 64, "the instruction word is 64 bytes");
inline constexpr size_t kPlanHashOffset = offsetof(PlanHeader, plan_hash);  // 216

// hash.h:136-158: ContentHash64's chunked 8-lane FNV-1a fold with the 8-byte
// hash field read as zero.  Chunks are 1 MiB, raised so there are at most
// 256 (parallel_for.h:55-67); folded in chunk order, then the size.
uint64_t PlanSelfHash(const uint8_t* plan, size_t size, size_t hash_offset = kPlanHashOffset);

// A decoded plan: the header and copies of its instruction and emit
// sections; rodata and the persistent image are views into the blob.
struct Plan {
  PlanHeader header{};
  std::vector<Instruction> train, eval, merge, step;
  std::vector<EmitEntry> emit;
  std::span<const uint8_t> rodata;
  std::span<const uint8_t> persist_init;
};

// DecodePlan's header stage (plan_loader.cc:19-49 with plan_contract.h:
// 35-180): size, magic, version window, self-hash, then the section and
// slot bounds, the hyperparameter ranges and the step-program rule; the
// refusal strings are the reference's.  Sections are then decoded.
Result<Plan> ReadPlan(std::span<const uint8_t> blob);

// The executor contract (contract.cc:51-244 over plan_validator.cc:160-745):
// every operand of every program non-null, aligned, in bounds of the space
// its ref names, never a write into rodata or the source model, no written
// operand overlapping another of the same instruction; only the flag bits
// each opcode takes; the label, token and segment-start operands the
// feeder's bounds cover; finite positive scales and clip thresholds; emit
// entries inside the arena.  *source_extent receives the bytes of the
// source model the programs read (0: none), checked when one is bound.
Result<void> VerifyPrograms(const Plan& plan, uint64_t* source_extent);

}  // namespace seeai::host
