"""GPU: the feeder -- seeai_engine_train_steps over the device feeder
(seeai_feeder_*), the reference's BatchPipeline (runtime/pipeline/
batch_pipeline.h:13-57): the next batch is checked and uploaded on the
feeder's own stream while the current step runs.  The pipeline changes when
batches reach the device, never which batches or in which order, so every
loss and every persistent byte equals serial staging's bit for bit."""
from __future__ import annotations

import ctypes as C
import importlib

import numpy as np
import pytest

pw = importlib.import_module("see-ai_amd.planwriter")
pytestmark = pytest.mark.gpu


def c1_batch(step):
    return pw.normal(3000 + step, (32, 256)), pw.uniform_ints(4000 + step, 32, 256)


TINY = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2, rank=8)


def tokens(step):
    T = TINY["batch"] * TINY["seq"]
    t = pw.uniform_ints(6000 + step, T + 1, TINY["vocab"])
    return t[:T].copy().view(np.float32), t[1:].copy()


def _serial_and_pipelined(hip, blob, batches, persistent):
    a, b = hip.Engine(blob), hip.Engine(blob)
    xs, ys = zip(*batches)
    serial = np.array([a.train_step(x, y) for x, y in zip(xs, ys)], np.float32)
    piped = b.train_steps(np.stack(xs), np.stack(ys))
    assert a.step == b.step == len(batches)
    assert serial.tobytes() == piped.tobytes(), f"losses {serial} vs {piped}"
    assert a.read(0, persistent) == b.read(0, persistent)
    return a, b


def test_c1_pipelined_steps_are_bitwise_the_serial_steps(hip, torch_cuda):
    print("feeder: config-1 plan, 7 steps serial vs pipelined", flush=True)
    img = pw.mlp_lora(hip.plan_self_hash)
    n = img.header["persistent_size"]
    a, b = _serial_and_pipelined(hip, img.blob, [c1_batch(s) for s in range(7)], n)
    # A second run continues the step count and the schedule.
    more = [c1_batch(s) for s in range(7, 10)]
    for x, y in more:
        a.train_step(x, y)
    b.train_steps(np.stack([x for x, _ in more]), np.stack([y for _, y in more]))
    assert a.step == b.step == 10
    assert a.read(0, n) == b.read(0, n)
    a.close()
    b.close()


@pytest.mark.parametrize("relaxed", [False, True])
def test_decoder_pipelined_steps_are_bitwise_the_serial_steps(hip, torch_cuda, relaxed):
    print(f"feeder: tiny decoder plan relaxed={relaxed}, 5 steps", flush=True)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=relaxed, **TINY)
    a, b = _serial_and_pipelined(hip, img.blob, [tokens(s) for s in range(5)],
                                 img.header["persistent_size"])
    a.close()
    b.close()


def test_feeder_stops_at_a_refused_batch(hip, torch_cuda):
    """A batch that breaks the label contract ends the run at that batch,
    with the refusal naming it; the steps before it have run (the engine
    state is three serial steps'), and the engine trains on afterwards."""
    img = pw.mlp_lora(hip.plan_self_hash)
    n = img.header["persistent_size"]
    batches = [c1_batch(s) for s in range(6)]
    bad_y = batches[3][1].copy()
    bad_y[5] = 256  # the plan has 256 classes
    batches[3] = (batches[3][0], bad_y)
    eng, ref = hip.Engine(img.blob), hip.Engine(img.blob)
    with pytest.raises(hip.BackendError, match="batch 3: label 256"):
        eng.train_steps(np.stack([x for x, _ in batches]), np.stack([y for _, y in batches]))
    for x, y in batches[:3]:
        ref.train_step(x, y)
    assert eng.step == 3
    assert eng.read(0, n) == ref.read(0, n)
    x, y = c1_batch(3)
    assert eng.train_step(x, y) == ref.train_step(x, y)
    eng.close()
    ref.close()


def test_accumulating_plan_through_the_feeder(hip, orc, torch_cuda):
    """A plan that accumulates G = 2 micro-batches per optimizer step (the
    reference's grad / step program split, optimizer.cc:22-108): the
    pipelined steps are bitwise the serial ones and within 1e-5 of the
    oracle twin; a refused micro-batch refuses its whole step before the
    step's timestep is spent -- the engine is where the step before left it,
    as TrainStep leaves it (update_engine.cc:840-870) -- and it trains on."""
    from tests.engine_oracle import OracleEngine
    print("feeder: config-1 plan with two micro-batches per step", flush=True)
    img = pw.mlp_lora(hip.plan_self_hash, grad_accum=2)
    n = img.header["persistent_size"]
    batches = [c1_batch(s) for s in range(8)]
    a, b = _serial_and_pipelined_accum(hip, img.blob, batches, n)
    twin = OracleEngine(orc, img.blob)
    for s in range(4):
        xs = np.stack([batches[2 * s][0], batches[2 * s + 1][0]])
        ys = np.stack([batches[2 * s][1], batches[2 * s + 1][1]])
        twin.train_step(xs, ys)
    g = np.frombuffer(a.read(0, n), np.float32).astype(np.float64)
    c = np.frombuffer(twin.read(0, n), np.float32).astype(np.float64)
    for name in ("A1", "B1", "A2", "B2"):
        off, nb = img.arena[name]
        sl = slice(off // 4, (off + nb) // 4)
        e = float(np.max(np.abs(g[sl] - c[sl])) / np.max(np.abs(c[sl])))
        assert e <= 1e-5, f"{name}: {e:.3g}"
    a.close()
    b.close()
    # Micro-batch 1 of step 2 (batch 3) breaks the label contract.
    bad_y = batches[3][1].copy()
    bad_y[5] = 256
    bad = list(batches)
    bad[3] = (batches[3][0], bad_y)
    eng, ref = hip.Engine(img.blob), hip.Engine(img.blob)
    with pytest.raises(hip.BackendError, match="batch 3: label 256"):
        eng.train_steps(np.stack([x for x, _ in bad]), np.stack([y for _, y in bad]))
    ref.train_step(np.stack([batches[0][0], batches[1][0]]),
                   np.stack([batches[0][1], batches[1][1]]))
    assert eng.step == 1 == ref.step
    assert eng.read(0, n) == ref.read(0, n)
    with pytest.raises(hip.BackendError, match="label 256"):
        ref.train_step(np.stack([batches[2][0], batches[3][0]]), np.stack([batches[2][1], bad_y]))
    assert ref.step == 1 and eng.read(0, n) == ref.read(0, n)
    xs = np.stack([batches[2][0], batches[3][0]])
    ys = np.stack([batches[2][1], batches[3][1]])
    assert eng.train_step(xs, ys) == ref.train_step(xs, ys)
    assert eng.read(0, n) == ref.read(0, n)
    eng.close()
    ref.close()


def _serial_and_pipelined_accum(hip, blob, batches, persistent):
    """Serial TrainStep over pairs of micro-batches against TrainSteps over
    the same batches in order: losses and persistent bytes equal."""
    a, b = hip.Engine(blob), hip.Engine(blob)
    xs, ys = zip(*batches)
    serial = np.array([a.train_step(np.stack(xs[i:i + 2]), np.stack(ys[i:i + 2]))
                       for i in range(0, len(batches), 2)], np.float32)
    piped = b.train_steps(np.stack(xs), np.stack(ys))
    assert a.step == b.step == len(batches) // 2
    assert serial.tobytes() == piped.tobytes(), f"losses {serial} vs {piped}"
    assert a.read(0, persistent) == b.read(0, persistent)
    return a, b


def test_device_feeder_holds_two_batches(hip, torch_cuda):
    """The C ABI's two staging slots: a third stage before a hand-over and a
    hand-over with nothing staged are refused; handed-over batches land in
    the arena slots in staging order."""
    import torch
    ctx = hip.Context(0)
    ctx.use_torch_stream()
    lib = hip._lib
    backend_arena = 1 << 16
    ctx.call("seeai_bind", C.c_uint64(backend_arena), None, C.c_uint64(0))
    f = C.c_void_p()
    ctx.call("seeai_feeder_create", C.c_uint64(256), C.c_uint64(64), C.byref(f))
    ins = [np.full(64, 1.0 + i, np.float32) for i in range(3)]
    labs = [np.full(16, 10 + i, np.int32) for i in range(3)]

    def stage(i):
        return lib.seeai_feeder_stage(f, ins[i].ctypes.data, labs[i].ctypes.data)

    assert lib.seeai_feeder_next(f, C.c_uint64(0), C.c_uint64(256)) == hip.INVALID
    assert stage(0) == hip.OK and stage(1) == hip.OK
    assert stage(2) == hip.INVALID
    assert b"two batches" in lib.seeai_feeder_last_error(f)
    arena = lib.seeai_arena(ctx.h)
    for i, (off_in, off_lab) in enumerate([(0, 1024), (4096, 8192)]):
        assert lib.seeai_feeder_next(f, C.c_uint64(off_in), C.c_uint64(off_lab)) == hip.OK
    assert stage(2) == hip.OK
    assert lib.seeai_feeder_next(f, C.c_uint64(12288), C.c_uint64(16384)) == hip.OK
    torch.cuda.synchronize()
    got = bytearray(backend_arena)
    ctx.call("seeai_download", C.c_uint64(0), (C.c_char * backend_arena).from_buffer(got),
             C.c_uint64(backend_arena))
    g = np.frombuffer(bytes(got), np.uint8)
    for i, (off_in, off_lab) in enumerate([(0, 1024), (4096, 8192), (12288, 16384)]):
        assert g[off_in:off_in + 256].tobytes() == ins[i].tobytes()
        assert g[off_lab:off_lab + 64].tobytes() == labs[i].tobytes()
    assert lib.seeai_feeder_next(f, C.c_uint64(backend_arena - 8), C.c_uint64(0)) == hip.INVALID
    lib.seeai_feeder_destroy(f)
    assert arena
    ctx.close()
