// operands.h -- every operand an instruction names: which ref, how many
// elements of how many bytes, and whether the instruction writes it.
//
// One table serves two callers: the plan engine's load-time proof that every
// operand of every program lies inside its address space (the reference's
// VerifyExecutorContract over DescribeInstruction,
// runtime/loader/contract.cc:51-244, runtime/verifier/plan_validator.cc:
// 160-745), and the executor's dead-store scan, which needs each operand's
// byte extent.  Roles and element counts are the validator's; a
// read-modify-write operand (AdamW's p, GemmAccNN's C) is one written
// operand, as there.  Header-only, no device code: it is compiled into the
// host layer and into the C ABI.
#pragma once

#include <cstdint>
#include <cstring>

namespace seeai {

struct OperandRef {
  uint64_t ref;        // the instruction's word: bit 63 rodata, bit 62 source
  uint64_t elems;      // element count
  uint32_t elem_bytes;
  bool write;
};

inline constexpr int kMaxOperands = 8;
inline constexpr int kOperandsUnknownOpcode = -1;  // no such opcode
inline constexpr int kOperandsBadGeometry = -2;    // zero or overflowing dimensions
inline constexpr int kOperandsUnsupported = -3;    // a real opcode this executor does not run

namespace operands_detail {

inline bool Mul(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > ~uint64_t{0} / a) return false;
  *out = a * b;
  return true;
}

// [B*S, H*d] activations and the [B*H*S, S] probability matrix, from the
// two-word form (B<<32|S, H<<32|d).
inline bool AttnSizes(uint64_t B, uint64_t S, uint64_t H, uint64_t d, uint64_t* td,
                      uint64_t* pn, uint64_t* bhs) {
  uint64_t t, hd, bh;
  if (!B || !S || !H || !d) return false;
  return Mul(B, S, &t) && Mul(H, d, &hd) && Mul(t, hd, td) && Mul(t, H, &bh) && Mul(bh, S, pn) &&
         Mul(t, H, bhs);
}

}  // namespace operands_detail

// Fills `out` (at most kMaxOperands) and returns the operand count, or one of
// the negative codes above.  W is any 64-byte instruction word type with
// opcode, flags, imm, in[4], out[3].
template <class W>
int DescribeOperands(const W& ins, OperandRef* out) {
  using operands_detail::AttnSizes;
  using operands_detail::Mul;
  constexpr uint64_t kNull = ~uint64_t{0};
  int k = 0;
  const auto add = [&](uint64_t ref, uint64_t elems, bool write, uint32_t bytes = 4) {
    out[k++] = OperandRef{ref, elems, bytes, write};
  };
  const uint64_t d0 = ins.out[0], d1 = ins.out[1], d2 = ins.out[2];
  const auto hi = [](uint64_t w) { return w >> 32; };
  const auto lo = [](uint64_t w) { return w & 0xFFFFFFFFu; };
  uint64_t a = 0, b = 0, c = 0;
  switch (ins.opcode) {
    case 0:  // kNop
      return 0;
    case 1: case 2: case 3: case 4: case 29: case 30: case 43: case 44: {
      // GEMMs: d0 = M, d1 = N, d2 = K.  A [M*K] and C [M*N] f32; B [K*N] in
      // the weight's storage width; in[3] by flag: bias [N], addend [M*N],
      // column scales (N for NN, K for NT); else a scalar's bits.
      const bool q8 = ins.opcode == 29 || ins.opcode == 30;
      const bool bf16 = ins.opcode == 43 || ins.opcode == 44;
      if (!Mul(d0, d2, &a) || !Mul(d2, d1, &b) || !Mul(d0, d1, &c)) return kOperandsBadGeometry;
      add(ins.in[0], a, false);
      add(ins.in[1], b, false, q8 ? 1 : bf16 ? 2 : 4);
      add(ins.in[2], c, true);
      if (ins.flags & (1u << 0)) add(ins.in[3], d1, false);
      else if (ins.flags & (1u << 3)) add(ins.in[3], c, false);
      else if (q8 && (ins.flags & (1u << 4))) add(ins.in[3], ins.opcode == 30 ? d2 : d1, false);
      return k;
    }
    case 5: case 21: case 8: case 23: case 25:  // AddEW, MulEW, activation backward
      add(ins.in[0], d0, false), add(ins.in[1], d0, false), add(ins.in[2], d0, true);
      return k;
    case 6:  // AddBias
      if (!Mul(d0, d1, &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], d1, false), add(ins.in[2], c, true);
      return k;
    case 7: case 22: case 24: case 9: case 20:  // activation forward, Scale, Copy
      add(ins.in[0], d0, false), add(ins.in[1], d0, true);
      return k;
    case 10:  // ReduceRows
      if (!Mul(d0, d1, &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], d1, true);
      return k;
    case 11: case 51:  // SoftmaxXEnt forward: logits, labels (i32), loss, probabilities
      if (!Mul(d0, d1, &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], d0, false), add(ins.in[2], 1, true),
          add(ins.in[3], c, true);
      return k;
    case 12: case 52:  // SoftmaxXEnt backward: probabilities, labels, seed, dlogits
      if (!Mul(d0, d1, &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], d0, false), add(ins.in[2], 1, false),
          add(ins.in[3], c, true);
      return k;
    case 13: case 14: case 15: case 16:  // MSE and KL distillation
      return kOperandsUnsupported;
    case 17:  // SgdStep
    case 42:  // Accumulate: dst read and written, src
      add(ins.in[0], d0, true), add(ins.in[1], d0, false);
      return k;
    case 18:  // AdamWStep: p, g, m, v
      add(ins.in[0], d0, true), add(ins.in[1], d0, false), add(ins.in[2], d0, true),
          add(ins.in[3], d0, true);
      return k;
    case 19:  // Fill
    case 28:  // ClipNorm (threshold bits in in[1])
      add(ins.in[0], d0, true);
      return k;
    case 53:  // SqNormAccum: reads g, adds into its slot
      add(ins.in[0], d0, false), add(ins.in[1], 1, true);
      return k;
    case 54:  // ClipGlobal: scales g by the slot's factor
      add(ins.in[0], d0, true), add(ins.in[1], 1, false);
      return k;
    case 26:  // LayerNormFwd: x, gamma, beta -> y; mean, rstd in out[1], out[2]
      if (!lo(d0) || !Mul(hi(d0), lo(d0), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], lo(d0), false), add(ins.in[2], lo(d0), false),
          add(ins.in[3], c, true), add(ins.out[1], hi(d0), true), add(ins.out[2], hi(d0), true);
      return k;
    case 27:  // LayerNormBwd: dy, x, gamma, mean (out[0]), rstd (out[1]) -> dx (in[3])
      if (!lo(d2) || !Mul(hi(d2), lo(d2), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], c, false), add(ins.in[2], lo(d2), false),
          add(ins.in[3], c, true), add(ins.out[0], hi(d2), false), add(ins.out[1], hi(d2), false);
      return k;
    case 31:  // RmsNormFwd: x, g -> y, rstd
      if (!lo(d0) || !Mul(hi(d0), lo(d0), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], lo(d0), false), add(ins.in[2], c, true),
          add(ins.in[3], hi(d0), true);
      return k;
    case 32:  // RmsNormBwd: dy, x, g, rstd (out[0]) -> dx (in[3])
      if (!lo(d1) || !Mul(hi(d1), lo(d1), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], c, false), add(ins.in[2], lo(d1), false),
          add(ins.in[3], c, true), add(ins.out[0], hi(d1), false);
      return k;
    case 33: case 34: {  // RoPE: x -> y, optional [S, d] angle table in in[2]
      uint64_t td, pn, bhs;
      if (!AttnSizes(hi(d0), lo(d0), hi(d1), lo(d1), &td, &pn, &bhs) || lo(d1) % 2)
        return kOperandsBadGeometry;
      add(ins.in[0], td, false), add(ins.in[1], td, true);
      if (ins.in[2] != kNull) {
        if (!Mul(lo(d0), lo(d1), &c)) return kOperandsBadGeometry;
        add(ins.in[2], c, false);
      }
      return k;
    }
    case 45:  // RopeTable: [S, d] angles
      if (!hi(d0) || !lo(d0) || lo(d0) % 2 || !Mul(hi(d0), lo(d0), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, true);
      return k;
    case 46:  // FusedMap: x, optional a, optional b -> y
      add(ins.in[0], d0, false);
      if (ins.in[1] != kNull) add(ins.in[1], d0, false);
      if (ins.in[2] != kNull) add(ins.in[2], d0, false);
      add(ins.in[3], d0, true);
      return k;
    case 41:  // EmbedFwd: i32 tokens [d0], [V, D] table -> [d0, D]
      if (!Mul(hi(d1), lo(d1), &b) || !Mul(d0, lo(d1), &c)) return kOperandsBadGeometry;
      add(ins.in[0], d0, false), add(ins.in[1], b, false), add(ins.in[2], c, true);
      return k;
    case 55:  // SegmentStarts: i32 tokens [B*S] -> i32 starts [B*S]
      if (!hi(d0) || !lo(d0) || !Mul(hi(d0), lo(d0), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], c, true);
      return k;
    case 35: case 56: case 47: case 57: {  // attention forward: q, k, v -> o (+ cache / stats)
      uint64_t B, S, H, d;
      if (ins.opcode == 35 || ins.opcode == 47)
        B = hi(d1), S = lo(d1), H = hi(d2), d = lo(d2);
      else
        B = d1 >> 48, S = (d1 >> 32) & 0xFFFF, H = (d1 >> 16) & 0xFFFF, d = d1 & 0xFFFF;
      uint64_t td, pn, bhs, st;
      if (!AttnSizes(B, S, H, d, &td, &pn, &bhs) || !Mul(bhs, 4, &st)) return kOperandsBadGeometry;
      add(ins.in[0], td, false), add(ins.in[1], td, false), add(ins.in[2], td, false),
          add(ins.in[3], td, true);
      add(ins.out[0], ins.opcode == 35 || ins.opcode == 56 ? pn : st, true);
      if (ins.opcode == 56 || ins.opcode == 57) add(d2, B * S, false);  // i32 segment starts
      return k;
    }
    case 36: case 37: case 39: case 40: {  // cached backward: DP, DV, DQ, DK
      uint64_t td, pn, bhs;
      if (!AttnSizes(hi(d0), lo(d0), hi(d1), lo(d1), &td, &pn, &bhs)) return kOperandsBadGeometry;
      if (ins.opcode == 36)
        add(ins.in[0], td, false), add(ins.in[1], td, false), add(ins.in[2], pn, true);
      else
        add(ins.in[0], pn, false), add(ins.in[1], td, false), add(ins.in[2], td, true);
      return k;
    }
    case 38:  // SoftmaxRowsBwd
      if (!Mul(hi(d0), lo(d0), &c)) return kOperandsBadGeometry;
      add(ins.in[0], c, false), add(ins.in[1], c, false), add(ins.in[2], c, true);
      return k;
    case 48: case 49: case 50: {  // tiled dQ / dK / dV; dQ also writes the stats' delta
      const uint64_t B = d2 >> 48, S = (d2 >> 32) & 0xFFFF, H = (d2 >> 16) & 0xFFFF, d = d2 & 0xFFFF;
      uint64_t td, pn, bhs, st;
      if (!AttnSizes(B, S, H, d, &td, &pn, &bhs) || !Mul(bhs, 4, &st)) return kOperandsBadGeometry;
      for (int i = 0; i < 4; ++i) add(ins.in[i], td, false);
      add(ins.out[0], st, ins.opcode == 48), add(ins.out[1], td, true);
      return k;
    }
    default:
      return kOperandsUnknownOpcode;
  }
}

}  // namespace seeai
