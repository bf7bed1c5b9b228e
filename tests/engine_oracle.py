"""The CPU twin of the plan engine, for parity: a .seeu plan interpreted
instruction by instruction through the oracle (orc_execute), with the
engine's step discipline (runtime/dispatcher/update_engine.cc:325-391,
840-870).  Test infrastructure only."""
from __future__ import annotations

import importlib
import math
import struct

import numpy as np

pw = importlib.import_module("see-ai_amd.planwriter")


def effective_lr(h: dict, step: int, horizon: int) -> float:
    """update_engine.cc:370-391 in f32 arithmetic."""
    f = np.float32
    base = f(h["lr"])
    if h["lr_schedule"] != 1:
        return float(base)
    warm = h["warmup_steps"]
    if warm > 0 and step <= warm:
        return float(base * f(step) / f(warm))
    run = horizon or h["default_steps"]
    span = run - warm if run > warm else 0
    floor = base * f(h["min_lr_factor"])
    if span == 0 or step - warm >= span:
        return float(floor)
    t = f(step - warm) / f(span)
    c = f(math.cos(float(f(3.14159265358979323846) * t)))
    return float(floor + (base - floor) * f(0.5) * (f(1.0) + c))


class OracleEngine:
    def __init__(self, orc, blob: bytes):
        self.orc = orc
        self.h = pw.parse_header(blob)
        h = self.h
        size = (h["arena_size"] + 16383) // 16384 * 16384
        self.arena = np.zeros(size, np.uint8)
        pi = np.frombuffer(blob, np.uint8, h["persist_init_size"], h["persist_init_offset"])
        self.arena[:pi.size] = pi
        self.rodata = np.frombuffer(blob, np.uint8, h["rodata_size"], h["rodata_offset"]).copy()
        if self.rodata.size == 0:
            self.rodata = np.zeros(16, np.uint8)

        def section(off, count):
            return [blob[off + 64 * i: off + 64 * (i + 1)] for i in range(count)]
        self.train = section(h["train_instr_offset"], h["train_instr_count"])
        self.eval = section(h["eval_instr_offset"], h["eval_instr_count"])
        self.merge = section(h["merge_instr_offset"], h["merge_instr_count"])
        self.step_program = section(h["step_instr_offset"], h["step_instr_count"])
        self.micro = h["grad_accum_steps"] if h["grad_accum_steps"] > 1 else 1
        self.step = 0
        self.horizon = 0

    def _params(self):
        h = self.h
        return (effective_lr(h, self.step, self.horizon), h["beta1"], h["beta2"], h["eps"],
                h["weight_decay"], self.step)

    def _stage(self, x, labels):
        h = self.h
        off = h["input_ref"]
        xb = np.ascontiguousarray(x, np.float32).view(np.uint8).ravel()
        self.arena[off:off + xb.size] = xb
        if h["label_kind"]:
            lb = np.ascontiguousarray(labels).view(np.uint8).ravel()[:h["label_bytes"]]
            self.arena[h["label_ref"]:h["label_ref"] + lb.size] = lb

    def _run(self, program):
        params = self._params()
        for i, ins in enumerate(program):
            rc = self.orc.execute(ins, self.arena, self.rodata, params)
            assert rc == 0, f"oracle refused instruction {i} (status {rc})"

    def loss(self) -> float:
        o = self.h["loss_ref"]
        return struct.unpack("<f", self.arena[o:o + 4].tobytes())[0]

    def train_step(self, x, labels) -> float:
        """One optimizer step: `x` / `labels` hold the step's micro-batches
        back to back (update_engine.cc:840-870); the mean of their losses."""
        self.step += 1
        if self.micro == 1:
            self._stage(x, labels)
            self._run(self.train)
            return self.loss()
        h = self.h
        xs = np.ascontiguousarray(x, np.float32).reshape(self.micro, -1)
        ls = np.ascontiguousarray(labels).view(np.uint8).reshape(self.micro, -1)
        total = 0.0
        for g in range(self.micro):
            self._stage(xs[g][:h["input_floats"]], ls[g])
            self._run(self.train)
            total += self.loss()
        self._run(self.step_program)
        return float(np.float32(total / self.micro))

    def evaluate(self, x, labels) -> float:
        self._stage(x, labels)
        self._run(self.eval)
        return self.loss()

    def do_merge(self):
        self._run(self.merge)

    def read(self, off: int, nbytes: int) -> bytes:
        return self.arena[off:off + nbytes].tobytes()
