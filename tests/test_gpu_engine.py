"""GPU: the plan engine (include/seeai_engine.h) running the config-1 LoRA
training plan against its CPU twin (the same plan interpreted through the
oracle): losses step by step, the whole persistent segment (LoRA parameters
and AdamW moments) after several steps, the eval program, the merge deltas,
and the cosine-with-warmup schedule."""
from __future__ import annotations

import importlib
import struct

import numpy as np
import pytest

from tests.engine_oracle import OracleEngine

pw = importlib.import_module("see-ai_amd.planwriter")
pytestmark = pytest.mark.gpu
TOL = 1e-5


def maxrel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / den) if den > 0 else float(np.max(np.abs(a - b)))


@pytest.fixture(scope="module")
def c1(hip):
    return pw.mlp_lora(hip.plan_self_hash)


def batch(step):
    return pw.normal(1000 + step, (32, 256)), pw.uniform_ints(2000 + step, 32, 256)


def compare_arena(eng, twin, layout, names):
    for name in names:
        off, nb = layout[name]
        g = np.frombuffer(eng.read(off, nb), np.float32)
        c = np.frombuffer(twin.read(off, nb), np.float32)
        e = maxrel(g, c)
        assert e <= TOL, f"{name}: max-rel {e:.3g}"


PERSISTENT = [p + n for p in ("", "m_", "v_") for n in ("A1", "B1", "A2", "B2")]


def test_c1_training_matches_the_oracle(hip, orc, torch_cuda, c1):
    print("engine: config-1 MLP LoRA plan, 6 steps", flush=True)
    eng = hip.Engine(c1.blob)
    assert eng.header() == c1.blob[:320]
    twin = OracleEngine(orc, c1.blob)
    for s in range(6):
        x, y = batch(s)
        lg, lc = eng.train_step(x, y), twin.train_step(x, y)
        assert abs(lg - lc) <= TOL * abs(lc), f"step {s + 1}: loss {lg} vs {lc}"
    assert eng.step == 6
    compare_arena(eng, twin, c1.arena, PERSISTENT)
    x, y = batch(99)
    assert abs(eng.evaluate(x, y) - twin.evaluate(x, y)) <= TOL * 6
    compare_arena(eng, twin, c1.arena, ["probs", "logits"])
    eng.merge()
    twin.do_merge()
    compare_arena(eng, twin, c1.arena, ["D1", "D2"])
    assert eng.relaxed_executions() == 0
    eng.close()


def test_cosine_schedule_drives_the_optimizer(hip, orc, torch_cuda, c1):
    h = dict(c1.header)
    h.update(lr_schedule=1, warmup_steps=2, default_steps=5, min_lr_factor=0.25, plan_hash=0)
    blob = bytearray(c1.blob)
    blob[:320] = pw.pack_header(h)
    blob[216:224] = struct.pack("<Q", hip.plan_self_hash(bytes(blob)))
    blob = bytes(blob)
    eng = hip.Engine(blob)
    twin = OracleEngine(orc, blob)
    lrs = []
    for s in range(6):
        x, y = batch(s)
        lg, lc = eng.train_step(x, y), twin.train_step(x, y)
        lrs.append(eng.lr())
        assert abs(lg - lc) <= TOL * abs(lc), f"step {s + 1}"
    # warmup 1/2, 2/2 of lr; cosine over steps 3..5; the floor from step 5.
    assert lrs[0] == pytest.approx(5e-4) and lrs[1] == pytest.approx(1e-3)
    assert lrs[2] == pytest.approx(2.5e-4 + 0.75e-3 * 0.5 * (1 + np.cos(np.pi / 3)), rel=1e-6)
    assert lrs[-1] == pytest.approx(2.5e-4)
    compare_arena(eng, twin, c1.arena, PERSISTENT)
    eng.close()


def test_label_outside_the_classes_is_refused(hip, torch_cuda, c1):
    eng = hip.Engine(c1.blob)
    x, y = batch(0)
    y = y.copy()
    y[5] = 256
    with pytest.raises(hip.BackendError) as err:
        eng.train_step(x, y)
    assert err.value.status == hip.INVALID
    assert "label 256 at position 5" in str(err.value)
    eng.close()


def test_corrupt_plan_is_refused_before_the_device(hip, torch_cuda, c1):
    blob = bytearray(c1.blob)
    blob[400] ^= 1
    with pytest.raises(hip.BackendError) as err:
        hip.Engine(bytes(blob))
    assert str(err.value) == "plan hash mismatch — the .seeu blob is corrupt"
