"""CPU: the executor contract a plan must meet before it reaches the device
(VerifyExecutorContract, runtime/loader/contract.cc:51-244, over the
validator's operand extents, runtime/verifier/plan_validator.cc:160-745).

Each case takes the config-1 plan (or a tiny decoder plan), changes one word
the way a corrupt or crafted .seeu would, re-seals the self-hash so the
header contract passes, and checks that seeai_plan_check -- the same
VerifyPrograms the engine runs at load -- refuses it with the reason."""
from __future__ import annotations

import importlib
import struct

import pytest

pw = importlib.import_module("see-ai_amd.planwriter")

RODATA, SOURCE, NULL = 1 << 63, 1 << 62, (1 << 64) - 1
WORD = struct.Struct("<HHI4Q3Q")


@pytest.fixture(scope="module")
def c1(hip):
    return pw.mlp_lora(hip.plan_self_hash)


def words(blob, program):
    h = pw.parse_header(blob)
    off, n = h[program + "_instr_offset"], h[program + "_instr_count"]
    return [list(WORD.unpack_from(blob, off + 64 * i)) for i in range(n)]


def reseal(hip, blob: bytearray) -> bytes:
    blob[216:224] = b"\0" * 8
    blob[216:224] = struct.pack("<Q", hip.plan_self_hash(bytes(blob)))
    return bytes(blob)


def patched(hip, blob, program, idx, edit):
    """The plan with instruction `idx` of `program` replaced by edit(fields);
    fields = [opcode, flags, imm, in0..in3, out0..out2]."""
    h = pw.parse_header(blob)
    out = bytearray(blob)
    off = h[program + "_instr_offset"] + 64 * idx
    f = list(WORD.unpack_from(out, off))
    edit(f)
    WORD.pack_into(out, off, *f)
    return reseal(hip, out)


def find(blob, program, opcode):
    for i, w in enumerate(words(blob, program)):
        if w[0] == opcode:
            return i, w
    raise AssertionError(f"no opcode {opcode} in {program}")


def test_writer_plans_meet_the_contract(hip, c1):
    assert hip.plan_check(c1.blob) == ""
    tiny = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2)
    for relaxed in (True, False):
        assert hip.plan_check(pw.decoder_lora(hip.plan_self_hash, relaxed=relaxed, **tiny).blob) == ""
        q8 = pw.decoder_q8_lora(hip.plan_self_hash, relaxed=relaxed, rank=16,
                                **dict(tiny, ffn=352))
        assert hip.plan_check(q8.blob) == ""


def _set(i, value):
    def edit(f):
        f[i] = value
    return edit


def test_operand_past_the_arena_is_refused(hip, c1):
    idx, _ = find(c1.blob, "train", 1)
    arena = c1.header["arena_size"]
    bad = patched(hip, c1.blob, "train", idx, _set(3, arena - 64))  # A ends past the arena
    assert "instruction operand out of bounds" in hip.plan_check(bad)


def test_operand_past_rodata_is_refused(hip, c1):
    idx, w = find(c1.blob, "train", 1)
    assert w[4] & RODATA  # the frozen weight
    bad = patched(hip, c1.blob, "train", idx, _set(4, RODATA | c1.header["rodata_size"]))
    assert "out of bounds" in hip.plan_check(bad)


def test_write_into_rodata_or_the_source_model_is_refused(hip, c1):
    idx, w = find(c1.blob, "train", 1)
    for base in (RODATA, SOURCE):
        bad = patched(hip, c1.blob, "train", idx, _set(5, base | 0))  # C
        assert "out of bounds" in hip.plan_check(bad)


def test_misaligned_and_null_operands_are_refused(hip, c1):
    idx, w = find(c1.blob, "train", 1)
    assert "out of bounds" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(3, w[3] + 2)))
    assert "out of bounds" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(3, NULL)))


def test_overflowing_geometry_is_refused(hip, c1):
    idx, _ = find(c1.blob, "train", 1)
    bad = patched(hip, c1.blob, "train", idx, _set(7, 1 << 40))  # M
    msg = hip.plan_check(bad)
    assert "geometry" in msg or "out of bounds" in msg


def test_aliased_written_operand_is_refused(hip, c1):
    idx, w = find(c1.blob, "train", 1)
    bad = patched(hip, c1.blob, "train", idx, _set(5, w[3]))  # C over A
    assert "alias a written range" in hip.plan_check(bad)


def test_unknown_and_unsupported_opcodes_are_refused(hip, c1):
    idx, _ = find(c1.blob, "train", 1)
    assert "unknown opcode" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(0, 99)))
    # kMseFwd: a real opcode outside this executor
    assert "not supported" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(0, 13)))


def test_flag_bits_each_opcode_does_not_take_are_refused(hip, c1):
    idx, w = find(c1.blob, "train", 1)
    assert "unknown flag bits" in hip.plan_check(
        patched(hip, c1.blob, "train", idx, _set(1, w[1] | (1 << 7))))
    a_idx, a = find(c1.blob, "train", 7)  # ReluFwd takes no flags
    assert "addend" in hip.plan_check(patched(hip, c1.blob, "train", a_idx, _set(1, 1 << 3)))
    assert "relaxed bit" in hip.plan_check(patched(hip, c1.blob, "train", a_idx, _set(1, 1 << 5)))
    nan = struct.unpack("<I", struct.pack("<f", float("nan")))[0]
    assert "alpha" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(2, nan)))


def test_relaxed_instruction_in_the_eval_program_is_refused(hip, c1):
    idx, w = find(c1.blob, "eval", 1)
    bad = patched(hip, c1.blob, "eval", idx, _set(1, w[1] | (1 << 5)))
    assert "relaxed instruction outside the train / step programs" in hip.plan_check(bad)


def test_softmax_labels_must_be_the_staged_slot(hip, c1):
    idx, w = find(c1.blob, "train", 11)
    other = c1.header["input_ref"]
    assert "softmax labels are not the plan's staged label slot" in hip.plan_check(
        patched(hip, c1.blob, "train", idx, _set(4, other)))
    assert "softmax row count disagrees with the plan batch" in hip.plan_check(
        patched(hip, c1.blob, "train", idx, _set(7, w[7] // 2)))


def test_write_into_the_staged_input_slot_is_refused(hip, c1):
    idx, w = find(c1.blob, "train", 7)  # ReluFwd: its output moved onto the input slot
    bad = patched(hip, c1.blob, "train", idx, _set(4, c1.header["input_ref"]))
    assert "writes the staged input slot" in hip.plan_check(bad)


def test_embedding_tokens_must_be_the_staged_input(hip):
    tiny = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=False, **tiny)
    idx, w = find(img.blob, "train", 41)
    assert "embedding tokens are not the plan's staged input slot" in hip.plan_check(
        patched(hip, img.blob, "train", idx, _set(3, img.header["label_ref"])))


def test_emit_entry_outside_the_arena_is_refused(hip, c1):
    h = pw.parse_header(c1.blob)
    assert h["emit_count"] > 0
    out = bytearray(c1.blob)
    off = h["emit_table_offset"]
    smf, size, arena_off = struct.unpack_from("<3Q", out, off)
    struct.pack_into("<3Q", out, off, smf, size, h["arena_size"] - 4)
    assert "emit entry outside the arena" in hip.plan_check(reseal(hip, out))


def test_bad_clip_threshold_is_refused_at_load(hip, c1):
    idx, w = find(c1.blob, "train", 18)
    neg = struct.unpack("<I", struct.pack("<f", -1.0))[0]
    assert "clip threshold" in hip.plan_check(patched(hip, c1.blob, "train", idx, _set(8, neg)))
