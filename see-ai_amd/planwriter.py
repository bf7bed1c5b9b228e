"""Writes .seeu plans (format v26) for the executor's workloads.

The reference compiles plans with its C++ compiler (``seeml-update-compile``:
``MakeMlp`` / ``MakeTokenDecoderStack`` + ``UpdateCompiler``), which is not
runnable in this build.  This module emits the same programs for the graphs
the benchmarks use, instruction for instruction as the reference lowers them
(the config-1 listing: ``seeml-seeu-dump --instrs`` of ``MakeMlp(256, 512,
256)``, rank 8, alpha 16, AdamW), into the reference's container:

* the 320-byte ``PlanHeader`` (``source/plan/schema.h:296-412``), sealed with
  ``PlanSelfHash`` (``source/identity/hash.h:136-158``, computed by the
  library's own implementation);
* 64-byte instruction words (``source/plan/instruction.h:438-449``);
* one arena ``[persistent | I/O | transient]``: LoRA parameters, then the
  AdamW moments, then the staged input, labels and loss slot, then every
  activation and gradient (``arena_binder.h:18-27``);
* rodata holding the frozen base weights, page-aligned in the blob.

The arena offsets are this writer's own (a bump allocator, 64-byte aligned
transients); the reference's memory planner may place transients
differently, which changes no instruction's meaning.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

SEEU_MAGIC = 0x55454553       # schema.h:18
SEEU_VERSION = 26             # schema.h:165
NULL_REF = 0xFFFFFFFFFFFFFFFF
RODATA_BIT = 1 << 63
PLAN_HASH_OFFSET = 216        # offsetof(PlanHeader, plan_hash)

# Opcodes (instruction.h:44-232).
GEMM_NN, GEMM_NT, GEMM_TN, GEMM_ACC_NN = 1, 2, 3, 4
ADD_BIAS, RELU_FWD, RELU_BWD = 6, 7, 8
XENT_FWD, XENT_BWD = 11, 12
ADAMW = 18
FILL = 19
ACCUMULATE = 42
FLAG_ADDEND = 1 << 3          # kFlagGemmAddend

# PlanHeader field order and widths (schema.h:296-384); packed, little-endian.
_HEADER_FIELDS = [
    ("magic", "I"), ("version", "I"), ("arena_size", "Q"), ("persistent_size", "Q"),
    ("input_ref", "Q"), ("input_floats", "Q"), ("label_ref", "Q"), ("label_bytes", "Q"),
    ("label_kind", "I"), ("optimizer_kind", "I"), ("loss_ref", "Q"),
    ("train_instr_offset", "Q"), ("train_instr_count", "Q"),
    ("merge_instr_offset", "Q"), ("merge_instr_count", "Q"),
    ("rodata_offset", "Q"), ("rodata_size", "Q"),
    ("persist_init_offset", "Q"), ("persist_init_size", "Q"),
    ("emit_table_offset", "Q"), ("emit_count", "Q"),
    ("lr", "f"), ("beta1", "f"), ("beta2", "f"), ("eps", "f"), ("weight_decay", "f"),
    ("gemm_tile_k", "I"), ("batch", "Q"), ("default_steps", "Q"),
    ("eval_instr_offset", "Q"), ("eval_instr_count", "Q"),
    ("source_model_hash", "Q"), ("plan_hash", "Q"),
    ("lr_schedule", "I"), ("gemm_tile_n", "I"), ("warmup_steps", "Q"),
    ("min_lr_factor", "f"), ("clip_norm", "f"), ("input_kind", "I"),
    ("grad_accum_steps", "I"), ("seq_len", "Q"),
    ("step_instr_offset", "Q"), ("step_instr_count", "Q"),
    ("tokenizer_hash", "Q"), ("corpus_hash", "Q"), ("split_seed", "Q"),
    ("val_split_hash", "Q"), ("val_frac_bits", "I"), ("data_flags", "I"),
]
HEADER_FORMAT = "<" + "".join(f for _, f in _HEADER_FIELDS)
HEADER_NAMES = [n for n, _ in _HEADER_FIELDS]
assert struct.calcsize(HEADER_FORMAT) == 320


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def ins(opcode: int, ins4=(), outs3=(), flags: int = 0, imm: int = 0) -> bytes:
    """One 64-byte instruction word (instruction.h:438-447)."""
    i4 = list(ins4) + [NULL_REF] * (4 - len(ins4))
    o3 = list(outs3) + [0] * (3 - len(outs3))
    return struct.pack("<HHI4Q3Q", opcode, flags, imm, *[int(x) for x in i4],
                       *[int(x) for x in o3])


def parse_header(blob: bytes) -> dict:
    return dict(zip(HEADER_NAMES, struct.unpack_from(HEADER_FORMAT, blob, 0)))


def pack_header(h: dict) -> bytes:
    return struct.pack(HEADER_FORMAT, *[h[n] for n in HEADER_NAMES])


# --- deterministic inputs ------------------------------------------------------------------------
def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """SplitMix64 outputs start+1 .. start+n from `seed` (uint64)."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


_PAIRS_PER_CHUNK = 1 << 19


_GEN = None


def _gen():
    """The threaded C++ restatement of normal() and quantize_cols()
    (plangen/plangen.cc, built beside the executor), or None."""
    global _GEN
    if _GEN is None:
        import ctypes
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libseeai_plangen.so")
        if not os.path.exists(path):
            _GEN = False
            return None
        lib = ctypes.CDLL(path)
        lib.seeai_plangen_normal.restype = ctypes.c_int
        lib.seeai_plangen_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                                             ctypes.c_void_p]
        lib.seeai_plangen_quantize_cols.restype = ctypes.c_int
        lib.seeai_plangen_quantize_cols.argtypes = [ctypes.c_void_p, ctypes.c_uint64,
                                                    ctypes.c_uint64, ctypes.c_void_p,
                                                    ctypes.c_void_p]
        _GEN = lib
    return _GEN or None


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """N(0, std^2) f32 by Box-Muller in double over SplitMix64 uniforms:
    pair p takes outputs 2p+1 and 2p+2, giving elements 2p and 2p+1
    (normal_numpy states it).  Generated by the threaded C++ restatement
    when it is built, which gives the same bytes."""
    lib = _gen()
    if lib is None:
        return normal_numpy(seed, shape, std)
    out = np.empty(int(np.prod(shape)), np.float32)
    if lib.seeai_plangen_normal(seed & (2**64 - 1), out.size, float(std), out.ctypes.data) != 0:
        raise RuntimeError("plangen normal failed")
    return out.reshape(shape)


def normal_numpy(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """normal() in numpy.  Large arrays are generated in chunks of pairs on a
    thread pool (numpy releases the GIL); every element is the same
    function of its index, so the bytes do not depend on the chunking."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    out = np.empty(2 * m, np.float32)

    def pairs(p0: int, p1: int) -> None:
        u = splitmix64(seed, 2 * (p1 - p0), start=2 * p0)
        u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * (p1 - p0), np.float64)
        z[0::2] = r * np.cos(2.0 * np.pi * u2)
        z[1::2] = r * np.sin(2.0 * np.pi * u2)
        out[2 * p0:2 * p1] = (z * std).astype(np.float32)

    if m <= _PAIRS_PER_CHUNK:
        pairs(0, m)
    else:
        from concurrent.futures import ThreadPoolExecutor
        bounds = [(p, min(p + _PAIRS_PER_CHUNK, m)) for p in range(0, m, _PAIRS_PER_CHUNK)]
        with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
            list(pool.map(lambda b: pairs(*b), bounds))
    return out[:n].reshape(shape)


def uniform_ints(seed: int, n: int, high: int) -> np.ndarray:
    return (splitmix64(seed, n) % np.uint64(high)).astype(np.int32)


def quantize_cols(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-column symmetric int8 of W [K, M] by the reference's rule
    (arena_binder.cc:129-177): column scale max|w| / 127, 1 for an all-zero
    column, at least FLT_MIN; level = clamp(round(w / scale), -127, 127)
    with the quotient in f32 and halves rounded away from zero
    (std::round).  quantize_cols_numpy states it; the C++ restatement runs
    when built."""
    lib = _gen()
    w = np.ascontiguousarray(w, np.float32)
    if lib is None or w.ndim != 2:
        return quantize_cols_numpy(w)
    levels = np.empty(w.shape, np.int8)
    sc = np.empty(w.shape[1], np.float32)
    if lib.seeai_plangen_quantize_cols(w.ctypes.data, w.shape[0], w.shape[1], levels.ctypes.data,
                                       sc.ctypes.data) != 0:
        raise RuntimeError("plangen quantize failed")
    return levels, sc


def quantize_cols_numpy(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantize_cols() in numpy."""
    w = np.ascontiguousarray(w, np.float32)
    mx = np.max(np.abs(w), axis=0)
    sc = np.where(mx == 0, np.float32(1.0),
                  np.maximum(mx / np.float32(127.0), np.finfo(np.float32).tiny)).astype(np.float32)
    levels = np.empty(w.shape, np.int8)
    rows = max(1, (1 << 22) // max(1, w.shape[1]))
    for r0 in range(0, w.shape[0], rows):
        q = (w[r0:r0 + rows] / sc).astype(np.float64)          # the f32 quotient, widened
        q = np.sign(q) * np.floor(np.abs(q) + 0.5)              # halves away from zero
        levels[r0:r0 + rows] = np.clip(q, -127, 127).astype(np.int8)
    return levels, sc


# --- plan assembly -------------------------------------------------------------------------------
@dataclass
class Region:
    """Bump allocation in one address space (arena or rodata)."""
    base_bit: int = 0
    align: int = 64
    size: int = 0
    names: dict = field(default_factory=dict)

    def alloc(self, name: str, nbytes: int, align: int | None = None) -> int:
        a = self.align if align is None else align
        off = (self.size + a - 1) // a * a
        self.size = off + nbytes
        self.names[name] = (off, nbytes)
        return off | self.base_bit

    def ref(self, name: str) -> int:
        return self.names[name][0] | self.base_bit


@dataclass
class PlanImage:
    blob: bytes
    header: dict
    arena: dict          # name -> (offset, bytes)
    rodata: dict         # name -> (offset, bytes)
    train: list
    eval: list
    merge: list
    arrays: dict         # the frozen and initial values, by name


def assemble(header: dict, train: list, eval_: list, merge: list, emit: list,
             persist_init: bytes, rodata: bytes, self_hash, step: list = ()) -> bytes:
    """Lays the sections out after the header and seals the plan.
    `self_hash(blob) -> int` is PlanSelfHash with the hash field zeroed;
    `step` is the step program of a plan that accumulates micro-batches."""
    h = dict(header)
    parts = [(b"".join(train), 64), (b"".join(eval_), 64), (b"".join(merge), 64),
             (b"".join(struct.pack("<3Q", *e) for e in emit), 64), (persist_init, 64),
             (rodata, 4096), (b"".join(step), 64)]
    offs, end = [], 320
    for payload, align in parts:
        end = (end + align - 1) // align * align
        offs.append(end)
        end += len(payload)
    out = bytearray(end)
    view = memoryview(out)
    for (payload, _), off in zip(parts, offs):
        view[off:off + len(payload)] = payload
    del view
    names = ["train_instr", "eval_instr", "merge_instr"]
    for name, off, (payload, _), count in zip(names, offs, parts, (len(train), len(eval_),
                                                                    len(merge))):
        h[name + "_offset"] = off
        h[name + "_count"] = count
    h["emit_table_offset"] = offs[3]
    h["emit_count"] = len(emit)
    h["persist_init_offset"] = offs[4]
    h["persist_init_size"] = len(persist_init)
    h["rodata_offset"] = offs[5]
    h["rodata_size"] = len(rodata)
    h["step_instr_offset"] = offs[6] if step else 0
    h["step_instr_count"] = len(step)
    h["plan_hash"] = 0
    out[0:320] = pack_header(h)
    h["plan_hash"] = self_hash(out)
    out[0:320] = pack_header(h)
    # A plan of a gigabyte and more stays the buffer it was built in (one
    # copy fewer); every reader takes any bytes-like object.
    return out if len(out) >= (1 << 30) else bytes(out)


def mlp_lora(self_hash, batch: int = 32, din: int = 256, hidden: int = 512, dout: int = 256,
             rank: int = 8, alpha: float = 16.0, lr: float = 1e-3, weight_decay: float = 0.01,
             seed: int = 20261201, default_steps: int = 100, grad_accum: int = 1) -> PlanImage:
    """MLP din -> hidden (ReLU) -> dout with AddBias and
    LoRA (rank, alpha) on both MatMuls, softmax-xent over dout classes,
    AdamW.  Base weights and biases N(0, 0.02); LoRA A N(0, 0.02), B = 0.

    The train program is the reference's 25 instructions, eval its first
    10, merge the 4-instruction delta program (fill, GemmAccNN per site).

    grad_accum = G > 1 lowers gradient accumulation as the reference's
    optimizer pass does (compiler/analysis/optimization/optimizer.cc:22-108,
    update_compiler.cc:845-864): the loss seed is 1/G, each adapter's
    gradient folds into a persistent zero-initialised accumulator
    (kAccumulate) at the end of the train (grad) program, and the step
    program runs each AdamW step on the accumulator, then zeroes it."""
    s = alpha / rank
    arrays = {
        "W1": normal(seed + 1, (din, hidden), 0.02), "b1": normal(seed + 2, (hidden,), 0.02),
        "W2": normal(seed + 3, (hidden, dout), 0.02), "b2": normal(seed + 4, (dout,), 0.02),
        "A1": normal(seed + 5, (din, rank), 0.02), "B1": np.zeros((rank, hidden), np.float32),
        "A2": normal(seed + 6, (hidden, rank), 0.02), "B2": np.zeros((rank, dout), np.float32),
    }
    ro = Region(base_bit=RODATA_BIT, align=16)
    for n in ("W1", "b1", "W2", "b2"):
        ro.alloc(n, arrays[n].nbytes)
    ar = Region(align=64)
    params = ["A1", "B1", "A2", "B2"]
    for n in params:                                   # persistent: parameters,
        ar.alloc(n, arrays[n].nbytes, align=4)
    for n in params:                                   # then first moments,
        ar.alloc("m_" + n, arrays[n].nbytes, align=4)
    for n in params:                                   # then second moments
        ar.alloc("v_" + n, arrays[n].nbytes, align=4)
    if grad_accum > 1:                                 # then the accumulators
        for n in params:
            ar.alloc("acc_" + n, arrays[n].nbytes, align=4)
    persistent = ar.size
    ar.alloc("X", batch * din * 4, align=4)            # I/O slots
    ar.alloc("labels", batch * 4, align=4)
    ar.alloc("loss", 4, align=4)
    f = 4
    for name, shape in [("Z1", (batch, hidden)), ("t1", (batch, rank)), ("Z1b", (batch, hidden)),
                        ("Z1c", (batch, hidden)), ("H1", (batch, hidden)),
                        ("Z2", (batch, dout)), ("t2", (batch, rank)), ("Z2b", (batch, dout)),
                        ("logits", (batch, dout)), ("probs", (batch, dout)), ("seed", (1,)),
                        ("dZ", (batch, dout)), ("dt2", (batch, rank)), ("dB2", (rank, dout)),
                        ("dA2", (hidden, rank)), ("dh", (batch, hidden)), ("dh2", (batch, hidden)),
                        ("dH", (batch, hidden)), ("dt1", (batch, rank)), ("dB1", (rank, hidden)),
                        ("dA1", (din, rank)), ("D1", (din, hidden)), ("D2", (hidden, dout))]:
        ar.alloc(name, int(np.prod(shape)) * f)
    R, RO = ar.ref, ro.ref
    sb = f32_bits(s)
    train = [
        ins(GEMM_NN, [R("X"), RO("W1"), R("Z1")], [batch, hidden, din]),
        ins(GEMM_NN, [R("X"), R("A1"), R("t1")], [batch, rank, din]),
        ins(GEMM_NN, [R("t1"), R("B1"), R("Z1b"), R("Z1")], [batch, hidden, rank],
            flags=FLAG_ADDEND, imm=sb),
        ins(ADD_BIAS, [R("Z1b"), RO("b1"), R("Z1c")], [batch, hidden]),
        ins(RELU_FWD, [R("Z1c"), R("H1")], [batch * hidden]),
        ins(GEMM_NN, [R("H1"), RO("W2"), R("Z2")], [batch, dout, hidden]),
        ins(GEMM_NN, [R("H1"), R("A2"), R("t2")], [batch, rank, hidden]),
        ins(GEMM_NN, [R("t2"), R("B2"), R("Z2b"), R("Z2")], [batch, dout, rank],
            flags=FLAG_ADDEND, imm=sb),
        ins(ADD_BIAS, [R("Z2b"), RO("b2"), R("logits")], [batch, dout]),
        ins(XENT_FWD, [R("logits"), R("labels"), R("loss"), R("probs")], [batch, dout]),
        ins(FILL, [R("seed"), f32_bits(1.0 / grad_accum)], [1]),
        ins(XENT_BWD, [R("probs"), R("labels"), R("seed"), R("dZ")], [batch, dout]),
        ins(GEMM_NT, [R("dZ"), R("B2"), R("dt2")], [batch, rank, dout], imm=sb),
        ins(GEMM_TN, [R("t2"), R("dZ"), R("dB2")], [rank, dout, batch], imm=sb),
        ins(GEMM_TN, [R("H1"), R("dt2"), R("dA2")], [hidden, rank, batch]),
        ins(GEMM_NT, [R("dZ"), RO("W2"), R("dh")], [batch, hidden, dout]),
        ins(GEMM_NT, [R("dt2"), R("A2"), R("dh2"), R("dh")], [batch, hidden, rank],
            flags=FLAG_ADDEND),
        ins(RELU_BWD, [R("dh2"), R("Z1c"), R("dH")], [batch * hidden]),
        ins(GEMM_NT, [R("dH"), R("B1"), R("dt1")], [batch, rank, hidden], imm=sb),
        ins(GEMM_TN, [R("t1"), R("dH"), R("dB1")], [rank, hidden, batch], imm=sb),
        ins(GEMM_TN, [R("X"), R("dt1"), R("dA1")], [din, rank, batch]),
    ]
    step = []
    grads = [("A1", "dA1"), ("B1", "dB1"), ("A2", "dA2"), ("B2", "dB2")]
    if grad_accum > 1:
        for p, g in grads:
            train.append(ins(ACCUMULATE, [R("acc_" + p), R(g)], [arrays[p].size]))
        for p, _ in grads:
            step += [ins(ADAMW, [R(p), R("acc_" + p), R("m_" + p), R("v_" + p)],
                         [arrays[p].size, 0]),
                     ins(FILL, [R("acc_" + p), 0], [arrays[p].size])]
    else:
        for p, g in grads:
            train.append(ins(ADAMW, [R(p), R(g), R("m_" + p), R("v_" + p)],
                             [arrays[p].size, 0]))
    eval_ = train[:10]
    merge = [
        ins(FILL, [R("D1"), 0], [din * hidden]),
        ins(GEMM_ACC_NN, [R("A1"), R("B1"), R("D1"), sb], [din, hidden, rank]),
        ins(FILL, [R("D2"), 0], [hidden * dout]),
        ins(GEMM_ACC_NN, [R("A2"), R("B2"), R("D2"), sb], [hidden, dout, rank]),
    ]
    # The emit table names W's byte range in the source model file; this
    # build has no .smf, so the file offsets are the rodata offsets.
    emit = [(ro.names["W1"][0], arrays["W1"].nbytes, ar.names["D1"][0]),
            (ro.names["W2"][0], arrays["W2"].nbytes, ar.names["D2"][0])]
    persist = bytearray(persistent)
    for n in params:
        off, nb = ar.names[n]
        persist[off:off + nb] = arrays[n].tobytes()
    rodata = bytearray(ro.size)
    for n in ("W1", "b1", "W2", "b2"):
        off, nb = ro.names[n]
        rodata[off:off + nb] = arrays[n].tobytes()
    header = {n: 0 for n in HEADER_NAMES}
    header.update(
        magic=SEEU_MAGIC, version=SEEU_VERSION, arena_size=ar.size, persistent_size=persistent,
        input_ref=R("X"), input_floats=batch * din, label_ref=R("labels"), label_bytes=batch * 4,
        label_kind=1, optimizer_kind=1, loss_ref=R("loss"), lr=lr, beta1=0.9, beta2=0.999,
        eps=1e-8, weight_decay=weight_decay, batch=batch, default_steps=default_steps,
        step_instr_offset=0, step_instr_count=0, grad_accum_steps=grad_accum if grad_accum > 1 else 0)
    blob = assemble(header, train, eval_, merge, emit, bytes(persist), bytes(rodata), self_hash,
                    step=step)
    return PlanImage(blob=blob, header=parse_header(blob), arena=dict(ar.names),
                     rodata=dict(ro.names), train=train, eval=eval_, merge=merge, arrays=arrays)


# --- the decoder LoRA training step ----------------------------------------
LAYERNORM_FWD, LAYERNORM_BWD = 26, 27
ADD_EW = 5
GELU_FWD, GELU_BWD = 22, 23
ROPE_FWD, ROPE_BWD, ROPE_TABLE = 33, 34, 45
EMBED_FWD = 41
ATTN_FWD_TILED, ATTN_DQ_TILED, ATTN_DK_TILED, ATTN_DV_TILED = 47, 48, 49, 50
FLAG_RELAXED = 1 << 5        # kFlagRelaxed
MUL_EW = 21
SILU_FWD, SILU_BWD = 24, 25
GEMM_NN_Q8, GEMM_NT_Q8 = 29, 30
RMSNORM_FWD, RMSNORM_BWD = 31, 32
FLAG_Q8_COL_SCALE = 1 << 4   # kFlagQ8ColScale


class Builder:
    """Arena / rodata allocation and the three programs of one plan."""

    def __init__(self):
        self.ro = Region(base_bit=RODATA_BIT, align=16)
        self.ar = Region(align=256)
        self.arrays: dict = {}
        self.params: list = []
        self.train: list = []

    def const(self, name: str, array: np.ndarray) -> int:
        self.arrays[name] = np.ascontiguousarray(array)
        return self.ro.alloc(name, self.arrays[name].nbytes)

    def param(self, name: str, array: np.ndarray) -> int:
        self.arrays[name] = np.ascontiguousarray(array, np.float32)
        self.params.append(name)
        return self.ar.alloc(name, self.arrays[name].nbytes, align=4)

    def const_q8(self, name: str, w: np.ndarray) -> tuple[int, int]:
        """A frozen weight W [K, M] packed as the reference's compiler packs
        an int8 base with per-column scales (arena_binder.cc:129-202,
        283-287): the levels, then one f32 scale per output column right
        after them (4-byte aligned).  Returns the levels' and the scales'
        refs."""
        levels, scales = quantize_cols(w)
        self.arrays[name] = levels
        self.arrays[name + ".s"] = scales
        ref = self.ro.alloc(name, levels.nbytes, align=256)
        sref = self.ro.alloc(name + ".s", scales.nbytes, align=4)
        return ref, sref

    def buf(self, name: str, count: int, itemsize: int = 4) -> int:
        return self.ar.alloc(name, count * itemsize)

    def emit(self, word: bytes):
        self.train.append(word)


def decoder_lora(self_hash, vocab: int = 32000, dim: int = 768, heads: int = 12, ffn: int = 3072,
                 layers: int = 12, seq: int = 1024, batch: int = 8, rank: int = 8,
                 alpha: float = 16.0, relaxed: bool = True, rope_base: float = 10000.0,
                 lr: float = 1e-3, weight_decay: float = 0.01, seed: int = 20261204,
                 default_steps: int = 100) -> PlanImage:
    """a pre-norm decoder of `layers` blocks -- LayerNorm,
    Q / K / V projections with LoRA (rank, alpha) on Q and V, RoPE, causal
    attention (the tiled family), output projection, residual; LayerNorm,
    FFN dim -> ffn (GELU) -> dim, residual -- then a final LayerNorm, the
    vocabulary head and next-token softmax-xent, AdamW on the adapters.
    Frozen weights N(0, 0.02), gains 1, LoRA A N(0, 0.02), B = 0; token ids
    are the input (input_kind 1), next tokens the labels.

    The lowering follows the reference's rules: each adapted MatMul is the
    NN + NN-addend pair forward and the NT / TN / TN / NT-addend family
    backward (lora_grafter.cc:170-207, autodiff.cc:71-93); frozen MatMuls
    contribute only dX (NT); a residual's two gradient paths add (kAddEW);
    the tiled attention backward runs dQ before dK and dV; gradients no
    trainable parameter needs are not formed (the first block's dX chain and
    its dK).  `relaxed` sets kFlagRelaxed on the frozen-weight products and
    on attention (bf16 activations, f32 master weights and adapters).
    """
    assert dim % heads == 0
    T, D, F, H, d = batch * seq, dim, ffn, heads, dim // heads
    s = alpha / rank
    sb = f32_bits(s)
    rf = FLAG_RELAXED if relaxed else 0
    b = Builder()
    R, RO = b.ar.ref, b.ro.ref
    # Frozen weights (rodata) and adapters (persistent).
    b.const("emb", normal(seed, (vocab, D), 0.02))
    ones, zeros = np.ones(D, np.float32), np.zeros(D, np.float32)
    for l in range(layers):
        p = f"l{l}."
        b.const(p + "g1", ones)
        b.const(p + "b1", zeros)
        for w in "qkvo":
            b.const(p + "w" + w, normal(seed + 100 * l + ord(w), (D, D), 0.02))
        b.const(p + "g2", ones)
        b.const(p + "b2", zeros)
        b.const(p + "wu", normal(seed + 100 * l + 1, (D, F), 0.02))
        b.const(p + "wd", normal(seed + 100 * l + 2, (F, D), 0.02))
    b.const("gf", ones)
    b.const("bf", zeros)
    b.const("wh", normal(seed + 7, (D, vocab), 0.02))
    for l in range(layers):
        p = f"l{l}."
        for w in "qv":
            b.param(p + "A" + w, normal(seed + 1000 + 10 * l + ord(w), (D, rank), 0.02))
            b.param(p + "B" + w, np.zeros((rank, D), np.float32))
    for n in list(b.params):
        b.ar.alloc("m_" + n, b.arrays[n].nbytes, align=4)
    for n in list(b.params):
        b.ar.alloc("v_" + n, b.arrays[n].nbytes, align=4)
    persistent = b.ar.size
    b.buf("tokens", T)
    b.buf("labels", T)
    b.buf("loss", 1)
    b.buf("seed", 1)
    b.buf("rope", seq * (d // 2) * 2)
    # Saved activations, per block.
    TD, TF, Tr = T * D, T * F, T * rank
    for l in range(layers):
        p = f"l{l}."
        for n, c in [("x", TD), ("n1", TD), ("mean1", T), ("rstd1", T), ("tq", Tr), ("tv", Tr),
                     ("qr", TD), ("kr", TD), ("v", TD), ("a", TD), ("stats", T * H * 4),
                     ("x1", TD), ("n2", TD), ("mean2", T), ("rstd2", T), ("f", TF)]:
            b.buf(p + n, c)
    for n, c in [("xL", TD), ("nf", TD), ("meanf", T), ("rstdf", T), ("logits", T * vocab),
                 ("probs", T * vocab)]:
        b.buf(n, c)
    # Scratch shared by the blocks (forward products, backward gradients).
    for n, c in [("q0", TD), ("q", TD), ("k", TD), ("v0", TD), ("o", TD), ("h", TF),
                 ("dlogits", T * vocab), ("dnf", TD), ("dx2", TD), ("dh", TF), ("df", TF),
                 ("dn2", TD), ("dx1b", TD), ("dx1", TD), ("da", TD), ("dqr", TD), ("dkr", TD),
                 ("dv", TD), ("dq", TD), ("dk", TD), ("dtq", Tr), ("dtv", Tr),
                 ("dn1a", TD), ("dn1b", TD), ("dxb", TD), ("dx", TD)]:
        b.buf(n, c)
    for l in range(layers):
        p = f"l{l}."
        for w in "qv":
            b.buf(p + "dA" + w, D * rank)
            b.buf(p + "dB" + w, rank * D)

    E = b.emit
    bs, hd = (batch << 32) | seq, (H << 32) | d
    geo = (batch << 48) | (seq << 32) | (H << 16) | d
    base_bits = f32_bits(rope_base)
    # --- forward ---
    E(ins(ROPE_TABLE, [R("rope")], [(seq << 32) | d, base_bits]))
    E(ins(EMBED_FWD, [R("tokens"), RO("emb"), R("l0.x")], [T, (vocab << 32) | D]))

    def adapted(x, w, A, B_, t, out0, out):
        """C = x@W + s*(x@A)@B: NN, NN, NN-addend (the LoRA site, forward)."""
        E(ins(GEMM_NN, [R(x), RO(w), R(out0)], [T, D, D], flags=rf))
        E(ins(GEMM_NN, [R(x), R(A), R(t)], [T, rank, D]))
        E(ins(GEMM_NN, [R(t), R(B_), R(out), R(out0)], [T, D, rank], flags=FLAG_ADDEND, imm=sb))

    for l in range(layers):
        p = f"l{l}."
        nxt = f"l{l + 1}.x" if l + 1 < layers else "xL"
        E(ins(LAYERNORM_FWD, [R(p + "x"), RO(p + "g1"), RO(p + "b1"), R(p + "n1")],
              [(T << 32) | D, R(p + "mean1"), R(p + "rstd1")]))
        adapted(p + "n1", p + "wq", p + "Aq", p + "Bq", p + "tq", "q0", "q")
        E(ins(GEMM_NN, [R(p + "n1"), RO(p + "wk"), R("k")], [T, D, D], flags=rf))
        adapted(p + "n1", p + "wv", p + "Av", p + "Bv", p + "tv", "v0", p + "v")
        E(ins(ROPE_FWD, [R("q"), R(p + "qr"), R("rope")], [bs, hd, base_bits]))
        E(ins(ROPE_FWD, [R("k"), R(p + "kr"), R("rope")], [bs, hd, base_bits]))
        E(ins(ATTN_FWD_TILED, [R(p + "qr"), R(p + "kr"), R(p + "v"), R(p + "a")],
              [R(p + "stats"), bs, hd], flags=rf))
        E(ins(GEMM_NN, [R(p + "a"), RO(p + "wo"), R("o")], [T, D, D], flags=rf))
        E(ins(ADD_EW, [R(p + "x"), R("o"), R(p + "x1")], [TD]))
        E(ins(LAYERNORM_FWD, [R(p + "x1"), RO(p + "g2"), RO(p + "b2"), R(p + "n2")],
              [(T << 32) | D, R(p + "mean2"), R(p + "rstd2")]))
        E(ins(GEMM_NN, [R(p + "n2"), RO(p + "wu"), R(p + "f")], [T, F, D], flags=rf))
        E(ins(GELU_FWD, [R(p + "f"), R("h")], [TF]))
        E(ins(GEMM_NN, [R("h"), RO(p + "wd"), R("o")], [T, D, F], flags=rf))
        E(ins(ADD_EW, [R(p + "x1"), R("o"), R(nxt)], [TD]))
    E(ins(LAYERNORM_FWD, [R("xL"), RO("gf"), RO("bf"), R("nf")],
          [(T << 32) | D, R("meanf"), R("rstdf")]))
    E(ins(GEMM_NN, [R("nf"), RO("wh"), R("logits")], [T, vocab, D], flags=rf))
    E(ins(XENT_FWD, [R("logits"), R("labels"), R("loss"), R("probs")], [T, vocab]))
    n_eval = len(b.train)
    # --- backward ---
    E(ins(FILL, [R("seed"), f32_bits(1.0)], [1]))
    E(ins(XENT_BWD, [R("probs"), R("labels"), R("seed"), R("dlogits")], [T, vocab]))
    E(ins(GEMM_NT, [R("dlogits"), RO("wh"), R("dnf")], [T, D, vocab], flags=rf))
    E(ins(LAYERNORM_BWD, [R("dnf"), R("xL"), RO("gf"), R("dx2")],
          [R("meanf"), R("rstdf"), (T << 32) | D]))
    for l in reversed(range(layers)):
        p = f"l{l}."
        # x2 = x1 + FFN(LN2(x1)): dx1 = dx2 + LN2_bwd(FFN_bwd(dx2))
        E(ins(GEMM_NT, [R("dx2"), RO(p + "wd"), R("dh")], [T, F, D], flags=rf))
        E(ins(GELU_BWD, [R("dh"), R(p + "f"), R("df")], [TF]))
        E(ins(GEMM_NT, [R("df"), RO(p + "wu"), R("dn2")], [T, D, F], flags=rf))
        E(ins(LAYERNORM_BWD, [R("dn2"), R(p + "x1"), RO(p + "g2"), R("dx1b")],
              [R(p + "mean2"), R(p + "rstd2"), (T << 32) | D]))
        E(ins(ADD_EW, [R("dx2"), R("dx1b"), R("dx1")], [TD]))
        # x1 = x + Wo(attn(...)): the attention input gradients
        E(ins(GEMM_NT, [R("dx1"), RO(p + "wo"), R("da")], [T, D, D], flags=rf))
        qkv = [R(p + "qr"), R(p + "kr"), R(p + "v"), R("da")]
        E(ins(ATTN_DQ_TILED, qkv, [R(p + "stats"), R("dqr"), geo], flags=rf))
        if l > 0:
            E(ins(ATTN_DK_TILED, qkv, [R(p + "stats"), R("dkr"), geo], flags=rf))
        E(ins(ATTN_DV_TILED, qkv, [R(p + "stats"), R("dv"), geo], flags=rf))
        E(ins(ROPE_BWD, [R("dqr"), R("dq"), R("rope")], [bs, hd, base_bits]))
        if l > 0:
            E(ins(ROPE_BWD, [R("dkr"), R("dk"), R("rope")], [bs, hd, base_bits]))
        # the LoRA sites (Q, V): dt = s dC B^T, dB = s t^T dC, dA = X^T dt
        for w, dC, t, dt in [("q", "dq", p + "tq", "dtq"), ("v", "dv", p + "tv", "dtv")]:
            E(ins(GEMM_NT, [R(dC), R(p + "B" + w), R(dt)], [T, rank, D], imm=sb))
            E(ins(GEMM_TN, [R(t), R(dC), R(p + "dB" + w)], [rank, D, T], imm=sb))
            E(ins(GEMM_TN, [R(p + "n1"), R(dt), R(p + "dA" + w)], [D, rank, T]))
        if l == 0:
            continue  # nothing trainable below the first block's inputs
        # dn1 = dq Wq^T + dtq Aq^T + dk Wk^T + dv Wv^T + dtv Av^T (NT + addend chain)
        E(ins(GEMM_NT, [R("dq"), RO(p + "wq"), R("dn1a")], [T, D, D], flags=rf))
        E(ins(GEMM_NT, [R("dtq"), R(p + "Aq"), R("dn1b"), R("dn1a")], [T, D, rank],
              flags=FLAG_ADDEND))
        E(ins(GEMM_NT, [R("dk"), RO(p + "wk"), R("dn1a"), R("dn1b")], [T, D, D],
              flags=FLAG_ADDEND | rf))
        E(ins(GEMM_NT, [R("dv"), RO(p + "wv"), R("dn1b"), R("dn1a")], [T, D, D],
              flags=FLAG_ADDEND | rf))
        E(ins(GEMM_NT, [R("dtv"), R(p + "Av"), R("dn1a"), R("dn1b")], [T, D, rank],
              flags=FLAG_ADDEND))
        E(ins(LAYERNORM_BWD, [R("dn1a"), R(p + "x"), RO(p + "g1"), R("dxb")],
              [R(p + "mean1"), R(p + "rstd1"), (T << 32) | D]))
        E(ins(ADD_EW, [R("dx1"), R("dxb"), R("dx2")], [TD]))  # dx2 of the block below
    for n in b.params:
        g = n.replace(".A", ".dA").replace(".B", ".dB")
        E(ins(ADAMW, [R(n), R(g), R("m_" + n), R("v_" + n)], [b.arrays[n].size, 0]))
    train = b.train
    # The eval program scores what ships, in exact arithmetic: the forward
    # without kFlagRelaxed (instruction.h:356-384).
    eval_ = [w[:2] + struct.pack("<H", struct.unpack_from("<H", w, 2)[0] & ~FLAG_RELAXED) + w[4:]
             for w in train[:n_eval]]
    persist = bytearray(persistent)
    for n in b.params:
        off, nb = b.ar.names[n]
        persist[off:off + nb] = b.arrays[n].tobytes()
    rodata = bytearray(b.ro.size)
    for n, (off, nb) in b.ro.names.items():
        rodata[off:off + nb] = b.arrays[n].tobytes()
    header = {n: 0 for n in HEADER_NAMES}
    header.update(
        magic=SEEU_MAGIC, version=SEEU_VERSION, arena_size=b.ar.size, persistent_size=persistent,
        input_ref=R("tokens"), input_floats=T, label_ref=R("labels"), label_bytes=T * 4,
        label_kind=1, optimizer_kind=1, loss_ref=R("loss"), lr=lr, beta1=0.9, beta2=0.999,
        eps=1e-8, weight_decay=weight_decay, batch=T, default_steps=default_steps,
        input_kind=1, seq_len=seq)
    blob = assemble(header, train, eval_, [], [], bytes(persist), rodata, self_hash)
    return PlanImage(blob=blob, header=parse_header(blob), arena=dict(b.ar.names),
                     rodata=dict(b.ro.names), train=train, eval=eval_, merge=[], arrays=b.arrays)


# --- the larger decoder with a frozen int8 base ---------------------------
def decoder_q8_lora(self_hash, vocab: int = 32000, dim: int = 2048, heads: int = 32,
                    ffn: int = 5632, layers: int = 16, seq: int = 2048, batch: int = 4,
                    rank: int = 16, alpha: float = 32.0, relaxed: bool = True,
                    rope_base: float = 10000.0, lr: float = 1e-3, weight_decay: float = 0.01,
                    seed: int = 20261205, default_steps: int = 100) -> PlanImage:
    """a pre-norm decoder of `layers` blocks -- RMSNorm,
    Q / K / V projections, RoPE on Q and K, causal attention (tiled family),
    output projection, residual; RMSNorm, SiLU-gated FFN (gate and up
    dim -> ffn, SiLU(gate) * up, down ffn -> dim), residual -- then RMSNorm,
    the vocabulary head and next-token softmax-xent, AdamW on the adapters.
    The frozen base (Q, K, V, O, gate, up, down) is int8 with per-column
    scales (kGemmNNQ8 / kGemmNTQ8 with kFlagQ8ColScale, packed as the
    reference packs it); embedding, gains and head stay f32.  LoRA (rank,
    alpha) on Q, K, V and O; alpha = 2 rank, so s = 2 is a power of two and
    alpha's placement is exact on every backend.  Weights N(0, 0.02), gains
    1, A N(0, 0.02), B = 0; token ids in, next tokens as labels.

    The lowering follows decoder_lora's (lora_grafter.cc:170-207,
    autodiff.cc:71-93), with the rules the narrow-weight GEMMs add: a q8
    product takes no addend (instruction.h:318-330), so a q8 dX joins its
    LoRA dX through the f32 NT's addend slot, and two q8 dX paths add with
    kAddEW; the gated FFN's backward is two kMulEW (dh * up, dh * SiLU(gate))
    and kSiluBwd.  Every block's dQ, dK, dV feed an adapter, so all three run
    in every block; the first block forms no dX below its norm.  `relaxed`
    sets kFlagRelaxed on the frozen products (q8 and the head) and on
    attention."""
    assert dim % heads == 0
    T, D, F, H, d = batch * seq, dim, ffn, heads, dim // heads
    s = alpha / rank
    sb = f32_bits(s)
    rf = FLAG_RELAXED if relaxed else 0
    qf = FLAG_Q8_COL_SCALE | rf
    b = Builder()
    R, RO = b.ar.ref, b.ro.ref
    b.const("emb", normal(seed, (vocab, D), 0.02))
    ones = np.ones(D, np.float32)
    sites = "qkvo"
    for l in range(layers):
        p = f"l{l}."
        b.const(p + "g1", ones)
        for w in sites:
            b.const_q8(p + "w" + w, normal(seed + 100 * l + ord(w), (D, D), 0.02))
        b.const(p + "g2", ones)
        b.const_q8(p + "wg", normal(seed + 100 * l + 1, (D, F), 0.02))
        b.const_q8(p + "wu", normal(seed + 100 * l + 2, (D, F), 0.02))
        b.const_q8(p + "wd", normal(seed + 100 * l + 3, (F, D), 0.02))
    b.const("gf", ones)
    b.const("wh", normal(seed + 7, (D, vocab), 0.02))
    for l in range(layers):
        p = f"l{l}."
        for w in sites:
            b.param(p + "A" + w, normal(seed + 1000 + 10 * l + ord(w), (D, rank), 0.02))
            b.param(p + "B" + w, np.zeros((rank, D), np.float32))
    for n in list(b.params):
        b.ar.alloc("m_" + n, b.arrays[n].nbytes, align=4)
    for n in list(b.params):
        b.ar.alloc("v_" + n, b.arrays[n].nbytes, align=4)
    persistent = b.ar.size
    b.buf("tokens", T)
    b.buf("labels", T)
    b.buf("loss", 1)
    b.buf("seed", 1)
    b.buf("rope", seq * (d // 2) * 2)
    TD, TF, Tr = T * D, T * F, T * rank
    for l in range(layers):
        p = f"l{l}."
        for n, c in [("x", TD), ("n1", TD), ("rstd1", T), ("tq", Tr), ("tk", Tr), ("tv", Tr),
                     ("to", Tr), ("qr", TD), ("kr", TD), ("v", TD), ("a", TD),
                     ("stats", T * H * 4), ("x1", TD), ("n2", TD), ("rstd2", T), ("gt", TF),
                     ("up", TF), ("sg", TF)]:
            b.buf(p + n, c)
    for n, c in [("xL", TD), ("nf", TD), ("rstdf", T), ("logits", T * vocab),
                 ("probs", T * vocab)]:
        b.buf(n, c)
    for n, c in [("q0", TD), ("q", TD), ("k0", TD), ("k", TD), ("v0", TD), ("o0", TD),
                 ("o", TD), ("h", TF), ("dn", TD),
                 ("dlogits", T * vocab), ("dnf", TD), ("dx2", TD), ("dh", TF), ("dsg", TF),
                 ("dup", TF), ("dgt", TF), ("dn2a", TD), ("dn2b", TD), ("dn2", TD),
                 ("dx1b", TD), ("dx1", TD), ("da0", TD), ("da", TD), ("dqr", TD), ("dkr", TD),
                 ("dv", TD), ("dq", TD), ("dk", TD), ("dtq", Tr), ("dtk", Tr), ("dtv", Tr),
                 ("dto", Tr), ("P1", TD), ("P2", TD), ("P3", TD), ("dxb", TD)]:
        b.buf(n, c)
    for l in range(layers):
        p = f"l{l}."
        for w in sites:
            b.buf(p + "dA" + w, D * rank)
            b.buf(p + "dB" + w, rank * D)

    E = b.emit
    bs, hd = (batch << 32) | seq, (H << 32) | d
    geo = (batch << 48) | (seq << 32) | (H << 16) | d
    nd = (T << 32) | D
    base_bits = f32_bits(rope_base)

    def q8(opcode, x, w, out, m, n, k):
        E(ins(opcode, [R(x), RO(w), R(out), RO(w + ".s")], [m, n, k], flags=qf))

    def adapted(x, w, A, B_, t, out0, out):
        """C = x@W + s*(x@A)@B over the int8 base: NN-q8, NN, NN-addend."""
        q8(GEMM_NN_Q8, x, w, out0, T, D, D)
        E(ins(GEMM_NN, [R(x), R(A), R(t)], [T, rank, D]))
        E(ins(GEMM_NN, [R(t), R(B_), R(out), R(out0)], [T, D, rank], flags=FLAG_ADDEND, imm=sb))

    E(ins(ROPE_TABLE, [R("rope")], [(seq << 32) | d, base_bits]))
    E(ins(EMBED_FWD, [R("tokens"), RO("emb"), R("l0.x")], [T, (vocab << 32) | D]))
    for l in range(layers):
        p = f"l{l}."
        nxt = f"l{l + 1}.x" if l + 1 < layers else "xL"
        E(ins(RMSNORM_FWD, [R(p + "x"), RO(p + "g1"), R(p + "n1"), R(p + "rstd1")], [nd]))
        adapted(p + "n1", p + "wq", p + "Aq", p + "Bq", p + "tq", "q0", "q")
        adapted(p + "n1", p + "wk", p + "Ak", p + "Bk", p + "tk", "k0", "k")
        adapted(p + "n1", p + "wv", p + "Av", p + "Bv", p + "tv", "v0", p + "v")
        E(ins(ROPE_FWD, [R("q"), R(p + "qr"), R("rope")], [bs, hd, base_bits]))
        E(ins(ROPE_FWD, [R("k"), R(p + "kr"), R("rope")], [bs, hd, base_bits]))
        E(ins(ATTN_FWD_TILED, [R(p + "qr"), R(p + "kr"), R(p + "v"), R(p + "a")],
              [R(p + "stats"), bs, hd], flags=rf))
        adapted(p + "a", p + "wo", p + "Ao", p + "Bo", p + "to", "o0", "o")
        E(ins(ADD_EW, [R(p + "x"), R("o"), R(p + "x1")], [TD]))
        E(ins(RMSNORM_FWD, [R(p + "x1"), RO(p + "g2"), R(p + "n2"), R(p + "rstd2")], [nd]))
        q8(GEMM_NN_Q8, p + "n2", p + "wg", p + "gt", T, F, D)
        q8(GEMM_NN_Q8, p + "n2", p + "wu", p + "up", T, F, D)
        E(ins(SILU_FWD, [R(p + "gt"), R(p + "sg")], [TF]))
        E(ins(MUL_EW, [R(p + "sg"), R(p + "up"), R("h")], [TF]))
        q8(GEMM_NN_Q8, "h", p + "wd", "dn", T, D, F)
        E(ins(ADD_EW, [R(p + "x1"), R("dn"), R(nxt)], [TD]))
    E(ins(RMSNORM_FWD, [R("xL"), RO("gf"), R("nf"), R("rstdf")], [nd]))
    E(ins(GEMM_NN, [R("nf"), RO("wh"), R("logits")], [T, vocab, D], flags=rf))
    E(ins(XENT_FWD, [R("logits"), R("labels"), R("loss"), R("probs")], [T, vocab]))
    n_eval = len(b.train)
    # --- backward ---
    E(ins(FILL, [R("seed"), f32_bits(1.0)], [1]))
    E(ins(XENT_BWD, [R("probs"), R("labels"), R("seed"), R("dlogits")], [T, vocab]))
    E(ins(GEMM_NT, [R("dlogits"), RO("wh"), R("dnf")], [T, D, vocab], flags=rf))
    E(ins(RMSNORM_BWD, [R("dnf"), R("xL"), RO("gf"), R("dx2")], [R("rstdf"), nd]))
    for l in reversed(range(layers)):
        p = f"l{l}."
        # x2 = x1 + down(SiLU(gate n2) * up n2), n2 = RMSNorm(x1)
        q8(GEMM_NT_Q8, "dx2", p + "wd", "dh", T, F, D)
        E(ins(MUL_EW, [R("dh"), R(p + "up"), R("dsg")], [TF]))
        E(ins(MUL_EW, [R("dh"), R(p + "sg"), R("dup")], [TF]))
        E(ins(SILU_BWD, [R("dsg"), R(p + "gt"), R("dgt")], [TF]))
        q8(GEMM_NT_Q8, "dgt", p + "wg", "dn2a", T, D, F)
        q8(GEMM_NT_Q8, "dup", p + "wu", "dn2b", T, D, F)
        E(ins(ADD_EW, [R("dn2a"), R("dn2b"), R("dn2")], [TD]))
        E(ins(RMSNORM_BWD, [R("dn2"), R(p + "x1"), RO(p + "g2"), R("dx1b")], [R(p + "rstd2"), nd]))
        E(ins(ADD_EW, [R("dx2"), R("dx1b"), R("dx1")], [TD]))
        # x1 = x + O(attn(...)): the O site, then the attention gradients
        q8(GEMM_NT_Q8, "dx1", p + "wo", "da0", T, D, D)
        E(ins(GEMM_NT, [R("dx1"), R(p + "Bo"), R("dto")], [T, rank, D], imm=sb))
        E(ins(GEMM_TN, [R(p + "to"), R("dx1"), R(p + "dBo")], [rank, D, T], imm=sb))
        E(ins(GEMM_TN, [R(p + "a"), R("dto"), R(p + "dAo")], [D, rank, T]))
        E(ins(GEMM_NT, [R("dto"), R(p + "Ao"), R("da"), R("da0")], [T, D, rank],
              flags=FLAG_ADDEND))
        qkv = [R(p + "qr"), R(p + "kr"), R(p + "v"), R("da")]
        E(ins(ATTN_DQ_TILED, qkv, [R(p + "stats"), R("dqr"), geo], flags=rf))
        E(ins(ATTN_DK_TILED, qkv, [R(p + "stats"), R("dkr"), geo], flags=rf))
        E(ins(ATTN_DV_TILED, qkv, [R(p + "stats"), R("dv"), geo], flags=rf))
        E(ins(ROPE_BWD, [R("dqr"), R("dq"), R("rope")], [bs, hd, base_bits]))
        E(ins(ROPE_BWD, [R("dkr"), R("dk"), R("rope")], [bs, hd, base_bits]))
        for w, dC, dt in [("q", "dq", "dtq"), ("k", "dk", "dtk"), ("v", "dv", "dtv")]:
            E(ins(GEMM_NT, [R(dC), R(p + "B" + w), R(dt)], [T, rank, D], imm=sb))
            E(ins(GEMM_TN, [R(p + "t" + w), R(dC), R(p + "dB" + w)], [rank, D, T], imm=sb))
            E(ins(GEMM_TN, [R(p + "n1"), R(dt), R(p + "dA" + w)], [D, rank, T]))
        if l == 0:
            continue  # nothing trainable below the first block's inputs
        # dn1 = (dq Wq^T + dtq Aq^T) + (dk Wk^T + dtk Ak^T) + (dv Wv^T + dtv Av^T)
        q8(GEMM_NT_Q8, "dq", p + "wq", "P1", T, D, D)
        E(ins(GEMM_NT, [R("dtq"), R(p + "Aq"), R("P2"), R("P1")], [T, D, rank], flags=FLAG_ADDEND))
        q8(GEMM_NT_Q8, "dk", p + "wk", "P1", T, D, D)
        E(ins(GEMM_NT, [R("dtk"), R(p + "Ak"), R("P3"), R("P1")], [T, D, rank], flags=FLAG_ADDEND))
        E(ins(ADD_EW, [R("P2"), R("P3"), R("P1")], [TD]))
        q8(GEMM_NT_Q8, "dv", p + "wv", "P2", T, D, D)
        E(ins(GEMM_NT, [R("dtv"), R(p + "Av"), R("P3"), R("P2")], [T, D, rank], flags=FLAG_ADDEND))
        E(ins(ADD_EW, [R("P1"), R("P3"), R("dn2")], [TD]))
        E(ins(RMSNORM_BWD, [R("dn2"), R(p + "x"), RO(p + "g1"), R("dxb")], [R(p + "rstd1"), nd]))
        E(ins(ADD_EW, [R("dx1"), R("dxb"), R("dx2")], [TD]))  # dx2 of the block below
    for n in b.params:
        g = n.replace(".A", ".dA").replace(".B", ".dB")
        E(ins(ADAMW, [R(n), R(g), R("m_" + n), R("v_" + n)], [b.arrays[n].size, 0]))
    train = b.train
    eval_ = [w[:2] + struct.pack("<H", struct.unpack_from("<H", w, 2)[0] & ~FLAG_RELAXED) + w[4:]
             for w in train[:n_eval]]
    persist = bytearray(persistent)
    for n in b.params:
        off, nb = b.ar.names[n]
        persist[off:off + nb] = b.arrays[n].tobytes()
    rodata = bytearray(b.ro.size)
    view = memoryview(rodata)
    for n, (off, nb) in b.ro.names.items():
        view[off:off + nb] = b.arrays[n].reshape(-1).view(np.uint8)
    del view
    header = {n: 0 for n in HEADER_NAMES}
    header.update(
        magic=SEEU_MAGIC, version=SEEU_VERSION, arena_size=b.ar.size, persistent_size=persistent,
        input_ref=R("tokens"), input_floats=T, label_ref=R("labels"), label_bytes=T * 4,
        label_kind=1, optimizer_kind=1, loss_ref=R("loss"), lr=lr, beta1=0.9, beta2=0.999,
        eps=1e-8, weight_decay=weight_decay, batch=T, default_steps=default_steps,
        input_kind=1, seq_len=seq)
    blob = assemble(header, train, eval_, [], [], bytes(persist), rodata, self_hash)
    return PlanImage(blob=blob, header=parse_header(blob), arena=dict(b.ar.names),
                     rodata=dict(b.ro.names), train=train, eval=eval_, merge=[], arrays=b.arrays)
