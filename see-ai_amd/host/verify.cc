// verify.cc -- the executor contract a plan must meet before any of its
// programs reaches the device (see plan.h, VerifyPrograms).
//
// The backend dispatches instructions blindly (backend.h:119-121): every
// pointer a kernel forms is base + ref offset, so every operand of every
// program is proven here against the address space it names, as the
// reference's loader proves it before Execute (plan_loader.cc:90-99 calling
// VerifyExecutorContract, runtime/loader/contract.cc:51-244, over the
// validator's per-opcode extents, runtime/verifier/plan_validator.cc:
// 160-745).  The extents come from operands.h, the table the executor's
// dead-store scan also reads.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../csrc/operands.h"
#include "plan.h"

namespace seeai::host {
namespace {

constexpr uint16_t kFlagBias = 1u << 0, kFlagActMask = 3u << 1, kFlagAddend = 1u << 3,
                   kFlagColScale = 1u << 4, kFlagRelaxed = 1u << 5;
constexpr uint16_t kKnownFlags = kFlagBias | kFlagActMask | kFlagAddend | kFlagColScale | kFlagRelaxed;
constexpr uint32_t kDataFlagMaskedLoss = 1u << 0;  // schema.h:173
constexpr uint32_t kSourceWeightsVersion = 21;     // schema.h:188

float F32(uint64_t word) {
  const uint32_t u = static_cast<uint32_t>(word);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// A float carried as bits in a word's low half: finite and positive, the
// high half zero (plan_validator.cc's clip and dequant-scale rules).
bool PositiveFloatWord(uint64_t word) {
  const float f = F32(word);
  return (word >> 32) == 0 && std::isfinite(f) && f > 0.0f;
}

bool IsGemm(uint16_t op) {
  return (op >= 1 && op <= 4) || op == 29 || op == 30 || op == 43 || op == 44;
}
bool TakesRelaxed(uint16_t op) {  // instruction.h:356-390: frozen-weight GEMMs, tiled attention
  return op == 1 || op == 2 || op == 29 || op == 30 || op == 43 || op == 44 ||
         (op >= 47 && op <= 50) || op == 57;
}

// instruction.h:298-404: which flag bits an opcode may carry.
const char* FlagViolation(const Instruction& ins) {
  const uint16_t f = ins.flags, op = ins.opcode;
  if (f & ~kKnownFlags) return "instruction carries unknown flag bits";
  if ((f & kFlagBias) && op != 1 && op != 43) return "epilogue bias on an opcode that takes none";
  if ((f & kFlagActMask) && op != 1 && op != 43 && op != 29)
    return "epilogue activation on an opcode that takes none";
  if ((f & kFlagAddend) && (op < 1 || op > 3)) return "GEMM addend on an opcode that takes none";
  if ((f & kFlagAddend) && (f & (kFlagBias | kFlagActMask)))
    return "GEMM addend beside an epilogue";
  if ((f & kFlagColScale) && op != 29 && op != 30) return "column scales on a non-int8 opcode";
  if ((f & kFlagRelaxed) && !TakesRelaxed(op)) return "relaxed bit on an opcode that takes none";
  if (op >= 1 && op <= 3 && ins.imm != 0) {
    const float alpha = F32(ins.imm);
    if (!std::isfinite(alpha) || alpha == 0.0f) return "GEMM alpha must be a finite nonzero float";
    if (f & kFlagRelaxed) return "GEMM alpha on a relaxed instruction";
  }
  return nullptr;
}

std::string At(const char* program, size_t idx, const Instruction& ins, const std::string& what) {
  return std::string(what) + " (" + program + " program, instruction " + std::to_string(idx) +
         ", opcode " + std::to_string(ins.opcode) + ")";
}

struct Range {
  uint64_t off, bytes;
  int space;  // 0 arena, 1 rodata, 2 source
  bool write;
};

}  // namespace

Result<void> VerifyPrograms(const Plan& plan, uint64_t* source_extent) {
  const PlanHeader& h = plan.header;
  uint64_t source_end = 0;
  bool saw_masked = false;
  const bool masked_plan = (h.data_flags & kDataFlagMaskedLoss) != 0;
  struct Named {
    const char* name;
    const std::vector<Instruction>* program;
  };
  const Named programs[] = {{"train", &plan.train}, {"merge", &plan.merge}, {"eval", &plan.eval},
                            {"step", &plan.step}};
  for (const Named& p : programs) {
    // Segment starts written by kSegmentStarts of this program and not
    // written over since: the only starts a segmented attention may read
    // (contract.cc:178-202), since the kernels use them as loop bounds.
    std::vector<Range> starts_live;
    const bool eval_or_merge = p.program == &plan.eval || p.program == &plan.merge;
    const bool source_ok = p.program == &plan.eval || h.version >= kSourceWeightsVersion;
    for (size_t idx = 0; idx < p.program->size(); ++idx) {
      const Instruction& ins = (*p.program)[idx];
      if (const char* why = FlagViolation(ins)) return Fail(At(p.name, idx, ins, why));
      if ((ins.flags & kFlagRelaxed) && eval_or_merge)
        return Fail(At(p.name, idx, ins, "a relaxed instruction outside the train / step programs"));
      OperandRef ops[kMaxOperands];
      const int n = DescribeOperands(ins, ops);
      if (n == kOperandsUnknownOpcode) return Fail(At(p.name, idx, ins, "unknown opcode"));
      if (n == kOperandsUnsupported)
        return Fail(At(p.name, idx, ins, "opcode not supported by the gfx950 executor"));
      if (n < 0) return Fail(At(p.name, idx, ins, "instruction geometry is zero or overflows"));
      Range r[kMaxOperands];
      for (int i = 0; i < n; ++i) {
        const OperandRef& o = ops[i];
        uint64_t bytes = 0;
        const int space = IsRodataRef(o.ref) ? 1 : IsSourceRef(o.ref) ? 2 : 0;
        const uint64_t off = RefOffset(o.ref);
        const bool bad = o.ref == kNullRef || o.elems == 0 ||
                         (o.elems > UINT64_MAX / o.elem_bytes) || off % o.elem_bytes != 0 ||
                         (o.write && space != 0) || (space == 2 && !source_ok);
        if (!bad) bytes = o.elems * o.elem_bytes;
        const uint64_t limit = space == 0 ? h.arena_size : space == 1 ? h.rodata_size : UINT64_MAX;
        if (bad || off > limit || bytes > limit - off)
          return Fail(At(p.name, idx, ins, "instruction operand out of bounds"));
        if (space == 2 && off + bytes > source_end) source_end = off + bytes;
        r[i] = {off, bytes, space, o.write};
      }
      // Restrict-qualified kernels: a written range may not overlap any
      // other operand in the same space (plan_validator.cc:164-224).
      for (int i = 0; i < n; ++i)
        for (int j = i + 1; j < n; ++j)
          if ((r[i].write || r[j].write) && r[i].space == r[j].space &&
              r[i].off < r[j].off + r[j].bytes && r[j].off < r[i].off + r[i].bytes)
            return Fail(At(p.name, idx, ins, "instruction operands alias a written range"));
      // Narrow weights, column scales and embedding tables are the
      // compiler's packing: rodata (or, for a table, the source model).
      const uint16_t op = ins.opcode;
      if ((op == 29 || op == 30 || op == 43 || op == 44) && !IsRodataRef(ins.in[1]))
        return Fail(At(p.name, idx, ins, "narrow-weight GEMM operand outside rodata"));
      if ((op == 29 || op == 30) && (ins.flags & kFlagColScale)) {
        if (!IsRodataRef(ins.in[3]))
          return Fail(At(p.name, idx, ins, "column scales outside rodata"));
        const uint64_t count = op == 30 ? ins.out[2] : ins.out[1];
        const uint8_t* s = plan.rodata.data() + RefOffset(ins.in[3]);
        for (uint64_t i = 0; i < count; ++i) {
          float v;
          std::memcpy(&v, s + 4 * i, 4);
          if (!std::isfinite(v) || v <= 0.0f)
            return Fail(At(p.name, idx, ins,
                           "quantized GEMM column scale " + std::to_string(i) +
                               " is not a finite positive float"));
        }
      } else if ((op == 29 || op == 30) && !PositiveFloatWord(ins.in[3])) {
        return Fail(At(p.name, idx, ins, "quantized GEMM dequant scale must be a finite positive float"));
      }
      if (op == 41 && !IsRodataRef(ins.in[1]) && !(IsSourceRef(ins.in[1]) && source_ok))
        return Fail(At(p.name, idx, ins, "embedding table outside rodata and the source model"));
      if (op == 28 && !PositiveFloatWord(ins.in[1]))
        return Fail(At(p.name, idx, ins, "clip_norm threshold must be a finite positive float"));
      if (op == 54 && !PositiveFloatWord(ins.in[2]))
        return Fail(At(p.name, idx, ins, "global clip threshold must be a finite positive float"));
      if ((op == 17 || op == 18) && ins.out[1] != 0 && !PositiveFloatWord(ins.out[1]))
        return Fail(At(p.name, idx, ins, "optimizer step clip threshold must be a finite positive float"));
      // The feeder's slots: no program writes them (contract.cc:97-124).
      for (int i = 0; i < n; ++i) {
        if (!r[i].write || r[i].space != 0) continue;
        const auto hits = [&](uint64_t ref, uint64_t bytes) {
          const uint64_t s = RefOffset(ref);
          return ref != kNullRef && bytes && r[i].off < s + bytes && s < r[i].off + r[i].bytes;
        };
        if (hits(h.input_ref, h.input_floats * 4))
          return Fail(At(p.name, idx, ins, "an instruction writes the staged input slot"));
        if (h.label_kind != 0 && hits(h.label_ref, h.label_bytes))
          return Fail(At(p.name, idx, ins, "an instruction writes the staged label slot"));
      }
      // Data-dependent indexing (contract.cc:131-176): class labels and
      // token ids are bounded by the feeder only in the staged slots, for
      // the staged batch.
      const bool masked_op = op == 51 || op == 52;
      if (masked_op && !masked_plan)
        return Fail(At(p.name, idx, ins, "masked cross-entropy in a plan without the masked-loss flag"));
      if ((op == 11 || op == 12) && masked_plan)
        return Fail(At(p.name, idx, ins, "plain cross-entropy in a plan that carries the masked-loss flag"));
      saw_masked |= masked_op;
      if (op == 11 || op == 12 || masked_op) {
        if (h.label_kind != 1)
          return Fail(At(p.name, idx, ins, "softmax cross-entropy in a plan without class labels"));
        if (ins.in[1] != h.label_ref)
          return Fail(At(p.name, idx, ins, "softmax labels are not the plan's staged label slot"));
        if (ins.out[0] != h.batch)
          return Fail(At(p.name, idx, ins, "softmax row count disagrees with the plan batch"));
      }
      if (op == 41) {
        if (h.input_kind != 1)
          return Fail(At(p.name, idx, ins, "embedding gather in a plan without token input"));
        if (ins.in[0] != h.input_ref)
          return Fail(At(p.name, idx, ins, "embedding tokens are not the plan's staged input slot"));
        if (ins.out[0] != h.batch)
          return Fail(At(p.name, idx, ins, "embedding row count disagrees with the plan batch"));
      }
      if (op == 56 || op == 57) {
        const uint64_t starts = RefOffset(ins.out[2]);
        bool live = false;
        for (const Range& s : starts_live) live |= s.off == starts;
        if (!live)
          return Fail(At(p.name, idx, ins,
                         "segment-masked attention reads starts no segment_starts of the same "
                         "program wrote"));
      }
      for (int i = 0; i < n; ++i) {
        if (!r[i].write || r[i].space != 0) continue;
        std::vector<Range> keep;
        for (const Range& s : starts_live)
          if (!(r[i].off < s.off + s.bytes && s.off < r[i].off + r[i].bytes)) keep.push_back(s);
        starts_live.swap(keep);
      }
      if (op == 55) starts_live.push_back(r[1]);
    }
  }
  if (masked_plan && !saw_masked)
    return Fail("plan carries the masked-loss flag but no masked cross-entropy");
  // contract.cc:228-236: the merge's deltas are read back through float*.
  for (const EmitEntry& e : plan.emit) {
    if (e.arena_offset > h.arena_size || e.byte_size > h.arena_size - e.arena_offset)
      return Fail("emit entry outside the arena");
    if (e.arena_offset % 4 != 0 || e.byte_size % 4 != 0) return Fail("emit entry misaligned");
  }
  if (source_extent) *source_extent = source_end;
  return {};
}

}  // namespace seeai::host
