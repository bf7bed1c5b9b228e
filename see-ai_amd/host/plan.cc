// plan.cc -- reading a .seeu plan (see plan.h).
#include "plan.h"

#include <cmath>
#include <cstring>

namespace seeai::host {
namespace {

constexpr uint64_t kFnvOffsetBasis = 0xcbf29ce484222325ULL;  // hash.h:31-32
constexpr uint64_t kFnvPrime = 0x100000001b3ULL;
constexpr size_t kLanes = 8;                 // hash.h:62
constexpr size_t kChunk = size_t{1} << 20;   // hash.h:63
constexpr size_t kMaxChunks = 256;           // parallel_for.h:50

uint64_t MixWord(uint64_t state, uint64_t word) {
  for (int b = 0; b < 8; ++b) {
    state ^= (word >> (8 * b)) & 0xff;
    state *= kFnvPrime;
  }
  return state;
}

// Eight FNV-1a chains, byte i feeding chain i % 8, each chain seeded
// distinctly; the chains and then the length are folded into one state.
uint64_t Striped(const uint8_t* data, size_t size) {
  uint64_t lane[kLanes];
  for (size_t l = 0; l < kLanes; ++l) lane[l] = kFnvOffsetBasis ^ (0x9E3779B97F4A7C15ULL * (l + 1));
  size_t i = 0;
  for (; i + kLanes <= size; i += kLanes)
    for (size_t l = 0; l < kLanes; ++l) {
      lane[l] ^= data[i + l];
      lane[l] *= kFnvPrime;
    }
  for (size_t l = 0; i < size; ++i, ++l) {
    lane[l] ^= data[i];
    lane[l] *= kFnvPrime;
  }
  uint64_t h = kFnvOffsetBasis;
  for (size_t l = 0; l < kLanes; ++l) h = MixWord(h, lane[l]);
  return MixWord(h, size);
}

bool MulOk(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  *out = a * b;
  return true;
}
bool RangeOk(uint64_t off, uint64_t bytes, uint64_t size) { return off <= size && bytes <= size - off; }

// plan_contract.h:35-180, the rules this reader needs to address the
// sections and the I/O slots safely.
const char* HeaderViolation(const PlanHeader& h, uint64_t plan_size, std::string* detail) {
  uint64_t train = 0, merge = 0, eval = 0, step = 0, emit = 0;
  if (!MulOk(h.train_instr_count, sizeof(Instruction), &train) ||
      !MulOk(h.merge_instr_count, sizeof(Instruction), &merge) ||
      !MulOk(h.eval_instr_count, sizeof(Instruction), &eval) ||
      !MulOk(h.step_instr_count, sizeof(Instruction), &step) ||
      !MulOk(h.emit_count, sizeof(EmitEntry), &emit))
    return "plan section size overflows";
  if (h.rodata_size != 0 && h.rodata_offset % kRodataAlignment != 0) {
    *detail = "rodata section is not " + std::to_string(kRodataAlignment) + "-byte aligned";
    return nullptr;
  }
  if (!RangeOk(h.train_instr_offset, train, plan_size) ||
      !RangeOk(h.merge_instr_offset, merge, plan_size) ||
      !RangeOk(h.eval_instr_offset, eval, plan_size) ||
      !RangeOk(h.step_instr_offset, step, plan_size) ||
      !RangeOk(h.rodata_offset, h.rodata_size, plan_size) ||
      !RangeOk(h.persist_init_offset, h.persist_init_size, plan_size) ||
      !RangeOk(h.emit_table_offset, emit, plan_size))
    return "plan section out of bounds";
  if (h.version < kSeeuGemmTilesVersion && (h.gemm_tile_k != 0 || h.gemm_tile_n != 0)) {
    *detail = "plan carries GEMM tile fields below v" + std::to_string(kSeeuGemmTilesVersion);
    return nullptr;
  }
  if (h.gemm_tile_k % 4 != 0) {
    *detail = "plan gemm_tile_k " + std::to_string(h.gemm_tile_k) +
              " is not a multiple of the kernel's 4-wide unroll";
    return nullptr;
  }
  if ((h.grad_accum_steps > 1) != (h.step_instr_count > 0))
    return "plan step program presence disagrees with grad_accum_steps";
  if (h.version < kSeeuGradAccumVersion && (h.grad_accum_steps > 1 || h.step_instr_count > 0)) {
    *detail = "pre-v" + std::to_string(kSeeuGradAccumVersion) +
              " plan carries gradient-accumulation fields";
    return nullptr;
  }
  if (h.batch == 0) return "plan batch size is zero";
  if (h.input_floats == 0) return "plan input width is zero";
  if (h.arena_size > UINT64_MAX - 63) return "arena size overflows";
  if (h.persist_init_size > h.arena_size || h.persistent_size > h.arena_size)
    return "persistent segment exceeds arena";
  const struct {
    const char* name;
    float value;
    bool in_range;
  } rules[] = {
      {"lr", h.lr, h.lr > 0.0f},
      {"beta1", h.beta1, h.beta1 >= 0.0f && h.beta1 < 1.0f},
      {"beta2", h.beta2, h.beta2 >= 0.0f && h.beta2 < 1.0f},
      {"eps", h.eps, h.eps > 0.0f},
      {"weight_decay", h.weight_decay, h.weight_decay >= 0.0f},
      {"clip_norm", h.clip_norm, h.clip_norm >= 0.0f},
      {"min_lr_factor", h.min_lr_factor, h.min_lr_factor >= 0.0f && h.min_lr_factor <= 1.0f},
  };
  for (const auto& r : rules)
    if (!std::isfinite(r.value) || !r.in_range) {
      *detail = std::string("plan header ") + r.name + " is not a finite value in its range";
      return nullptr;
    }
  uint64_t input_bytes = 0;
  if (IsRodataRef(h.input_ref) || IsSourceRef(h.input_ref) || RefOffset(h.input_ref) % 4 != 0 ||
      !MulOk(h.input_floats, 4, &input_bytes) ||
      !RangeOk(RefOffset(h.input_ref), input_bytes, h.arena_size))
    return "plan input slot out of bounds";
  if (h.label_kind != 0 &&
      (IsRodataRef(h.label_ref) || IsSourceRef(h.label_ref) || RefOffset(h.label_ref) % 4 != 0 ||
       !RangeOk(RefOffset(h.label_ref), h.label_bytes, h.arena_size)))
    return "plan label slot out of bounds";
  if (IsRodataRef(h.loss_ref) || IsSourceRef(h.loss_ref) || RefOffset(h.loss_ref) % 4 != 0 ||
      !RangeOk(RefOffset(h.loss_ref), 4, h.arena_size))
    return "plan loss slot out of bounds";
  return "";
}

template <class T>
std::vector<T> Section(std::span<const uint8_t> blob, uint64_t offset, uint64_t count) {
  std::vector<T> out(count);
  if (count) std::memcpy(out.data(), blob.data() + offset, count * sizeof(T));
  return out;
}

}  // namespace

uint64_t PlanSelfHash(const uint8_t* plan, size_t size, size_t hash_offset) {
  size_t grain = kChunk;
  const size_t cap = (size + kMaxChunks - 1) / kMaxChunks;
  if (grain < cap) grain = cap;
  const size_t chunks = size == 0 ? 0 : (size + grain - 1) / grain;
  uint64_t h = kFnvOffsetBasis;
  std::vector<uint8_t> patched;
  for (size_t c = 0; c < (chunks ? chunks : 1); ++c) {
    const size_t begin = c * grain, end = size < begin + grain ? size : begin + grain;
    uint64_t digest;
    if (hash_offset >= end || hash_offset + 8 <= begin) {
      digest = Striped(plan + begin, end - begin);
    } else {  // the chunk holding the hash field hashes it as zero
      patched.assign(plan + begin, plan + end);
      for (size_t i = 0; i < 8; ++i)
        if (hash_offset + i >= begin && hash_offset + i < end) patched[hash_offset + i - begin] = 0;
      digest = Striped(patched.data(), patched.size());
    }
    h = MixWord(h, digest);
  }
  return MixWord(h, size);
}

Result<Plan> ReadPlan(std::span<const uint8_t> blob) {
  Plan plan;
  PlanHeader& h = plan.header;
  if (blob.size() < sizeof(h)) return Fail("plan smaller than its header");
  std::memcpy(&h, blob.data(), sizeof(h));
  if (h.magic != kSeeuMagic) return Fail("bad plan magic");
  if (h.version < kSeeuOldestReadable || h.version > kSeeuVersion)
    return Fail("unsupported plan version " + std::to_string(h.version) + " (this runtime reads v" +
                std::to_string(kSeeuOldestReadable) + "..v" + std::to_string(kSeeuVersion) + ")");
  if (PlanSelfHash(blob.data(), blob.size()) != h.plan_hash)
    return Fail("plan hash mismatch \xe2\x80\x94 the .seeu blob is corrupt");
  std::string detail;
  if (const char* why = HeaderViolation(h, blob.size(), &detail); why == nullptr || *why)
    return Fail(why ? std::string(why) : detail);
  plan.train = Section<Instruction>(blob, h.train_instr_offset, h.train_instr_count);
  plan.merge = Section<Instruction>(blob, h.merge_instr_offset, h.merge_instr_count);
  plan.eval = Section<Instruction>(blob, h.eval_instr_offset, h.eval_instr_count);
  plan.step = Section<Instruction>(blob, h.step_instr_offset, h.step_instr_count);
  plan.emit = Section<EmitEntry>(blob, h.emit_table_offset, h.emit_count);
  plan.rodata = blob.subspan(h.rodata_offset, h.rodata_size);
  plan.persist_init = blob.subspan(h.persist_init_offset, h.persist_init_size);
  return plan;
}

}  // namespace seeai::host
