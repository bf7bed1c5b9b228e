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
    loss, hits, judged = eng.evaluate_metrics(x, y)
    assert abs(loss - twin.evaluate(x, y)) <= TOL * 6
    compare_arena(eng, twin, c1.arena, ["probs", "logits"])
    # the accuracy tally: the device's argmax over the device's probabilities
    # is the oracle's over the same bytes, and -- where no row's top two
    # classes lie within the 1e-5 parity bar -- the twin's
    off, nb = c1.arena["probs"]
    gp = np.frombuffer(eng.read(off, nb), np.float32).reshape(32, 256)
    cp = np.frombuffer(twin.read(off, nb), np.float32).reshape(32, 256)
    assert (hits, judged) == orc.argmax_tally(gp, y)
    top2 = np.sort(cp, axis=1)[:, -2:]
    if np.all(top2[:, 1] - top2[:, 0] > 1e-5 * top2[:, 1]):
        assert (hits, judged) == orc.argmax_tally(cp, y)
    assert judged == 32
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
    assert eng.step == 0  # the refused step spent no timestep
    eng.close()


def test_corrupt_plan_is_refused_before_the_device(hip, torch_cuda, c1):
    blob = bytearray(c1.blob)
    blob[400] ^= 1
    with pytest.raises(hip.BackendError) as err:
        hip.Engine(bytes(blob))
    assert str(err.value) == "plan hash mismatch — the .seeu blob is corrupt"


# --- the decoder LoRA step (BASELINE configs[3] at a small shape) --------------------------------

TINY = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2, rank=8)


def tokens(step):
    T = TINY["batch"] * TINY["seq"]
    t = pw.uniform_ints(5000 + step, T + 1, TINY["vocab"])
    return t[:T].copy(), t[1:].copy()


def expect_close(what, got, want, rel, abs_floor):
    """Elementwise |got - want| <= abs_floor + rel |want|, NaN failing
    (the reference's ExpectClose, metal_backend_test.cc:85-106)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = ~(err <= abs_floor + rel * np.abs(want))
    assert not bad.any(), (f"{what}[{int(np.argmax(bad))}]: gpu {got[bad][0]} vs cpu {want[bad][0]}"
                           f" ({int(bad.sum())} of {bad.size} outside)")


def persistent_doctrine(img, eng, twin):
    """The reference's persistent-segment doctrine (rel 5e-3 / abs 1e-6 per
    element, metal_backend_test.cc:210-232) after free-running steps,
    applied to an exact family that is not bitwise: AdamW's normalised
    update is ill-conditioned wherever a moment crosses zero, so a few
    elements of a non-bitwise gradient path leave the band.  Asserted: the
    segment's relative L2 error within 5e-3 and at most one element in a
    thousand outside the band (printed); the per-step bars are held by
    tracked_steps below."""
    n = img.header["persistent_size"]
    g = np.frombuffer(eng.read(0, n), np.float32).astype(np.float64)
    c = np.frombuffer(twin.read(0, n), np.float32).astype(np.float64)
    out = ~(np.abs(g - c) <= 1e-6 + 5e-3 * np.abs(c))
    l2 = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    print(f"  persistent: L2 {l2:.2e}, {int(out.sum())} of {out.size} outside rel 5e-3 / abs 1e-6",
          flush=True)
    assert l2 <= 5e-3
    assert int(out.sum()) <= out.size // 1000


def tracked_steps(orc, img, eng, twin, batches, bar):
    """Training steps in lockstep: before each step the twin takes the
    engine's persistent segment, so both start the step from the same
    parameters and moments.  Per step: the loss within `bar`; every
    gradient the AdamW steps read within `bar` per tensor (the north star's
    bar, exact 1e-5 or relaxed 2e-2); and the engine's updated p, m, v
    bitwise the reference AdamW applied to its own gradient and state."""
    h = img.header
    n = h["persistent_size"]
    inv = {off: name for name, (off, nb) in img.arena.items()}
    adam = []
    for w in img.train:
        if struct.unpack_from("<H", w)[0] == 18:
            adam.append(tuple(inv[r] for r in struct.unpack_from("<4Q", w, 8)))
    read = lambda who, name: np.frombuffer(  # noqa: E731
        who.read(*img.arena[name]), np.float32).copy()
    worst = 0.0
    for s, (x, y) in enumerate(batches):
        twin.arena[:n] = np.frombuffer(eng.read(0, n), np.uint8)
        twin.step = eng.step
        before = {p: (read(eng, p), read(eng, m), read(eng, v)) for p, _, m, v in adam}
        lg, lc = eng.train_step(x, y), twin.train_step(x, y)
        assert abs(lg - lc) <= bar * abs(lc), f"step {s + 1}: loss {lg} vs {lc}"
        for p, g, m, v in adam:
            gg = read(eng, g)
            e = maxrel(gg, read(twin, g))
            worst = max(worst, e)
            assert e <= bar, f"step {s + 1} {g}: max-rel {e:.3g}"
            ok, p1, m1, v1 = orc.adamw_step(*before[p][:1], gg, *before[p][1:], h["lr"], h["beta1"],
                                            h["beta2"], h["eps"], h["weight_decay"], eng.step)
            assert ok and p1.tobytes() == read(eng, p).tobytes(), f"step {s + 1} {p}: not AdamW(g)"
            assert m1.tobytes() == read(eng, m).tobytes() and v1.tobytes() == read(eng, v).tobytes()
    print(f"  tracked {len(batches)} steps: gradients worst max-rel {worst:.2e}", flush=True)


def run_decoder(hip, orc, relaxed, steps):
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=relaxed, **TINY)
    eng = hip.Engine(img.blob)
    twin = OracleEngine(orc, img.blob) if orc is not None else None
    curve, want = [], []
    for s in range(steps):
        x, y = tokens(s)
        curve.append(eng.train_step(x.view(np.float32), y))
        if twin:
            want.append(twin.train_step(x.view(np.float32), y))
    return img, eng, twin, np.array(curve), np.array(want)


@pytest.mark.parametrize("relaxed", [False, True])
def test_decoder_training_matches_the_oracle(hip, orc, torch_cuda, relaxed):
    """Eight steps of the decoder plan against its CPU twin.

    Per-instruction the exact family is bit-exact (GEMMs, elementwise) or
    within 1e-5 (attention's f32 dots, the device libm's exp / tanh /
    sin / cos, norm sums); AdamW then divides by sqrt(v) + eps, which turns
    gradient differences far below 1e-5 of the tensor's scale into full-size
    update differences wherever a gradient is near eps.  So the training
    curve is held to the reference's own GPU-vs-CPU doctrine for 8 AdamW
    steps (metal_backend_test.cc:210-232): losses rel 2e-3 / abs 1e-4, the
    persistent segment (adapters and moments) rel 5e-3 / abs 1e-6 -- and
    each step's loss to 1e-5 (exact) or 2e-2 (relaxed, bf16 attention).

    Relaxed, the adapters are not compared elementwise: AdamW's first step
    moves each element by lr * sign(g), and bf16 attention changes the sign
    of gradients that sit at the noise floor, so single elements differ by
    2 lr while the loss curve agrees to 1e-5.  The reference holds its
    relaxed family per instruction (RelaxedGemmsMatchCpuAtTheBf16Tolerance,
    metal_backend_test.cc:745-850), as test_gpu_ops.py does here."""
    print(f"engine: decoder plan {TINY}, relaxed={relaxed}", flush=True)
    img, eng, twin, curve, want = run_decoder(hip, orc, relaxed, 8)
    step_tol = 2e-2 if relaxed else 1e-5
    assert np.all(np.abs(curve - want) <= step_tol * np.abs(want)), (curve, want)
    expect_close("loss curve", curve, want, 2e-3, 1e-4)
    if not relaxed:
        persistent_doctrine(img, eng, twin)
    tracked_steps(orc, img, eng, twin,
                  [(x.view(np.float32), y) for x, y in (tokens(s) for s in range(8, 11))], step_tol)
    assert (eng.relaxed_executions() > 0) == relaxed
    eng.close()


def test_decoder_training_is_bitwise_reproducible(hip, torch_cuda):
    """Run to run on one device the bits repeat: no float atomics, fixed
    reduction orders (metal_backend_test.cc:234-251)."""
    img, a, _, ca, _ = run_decoder(hip, None, True, 5)
    _, b, _, cb, _ = run_decoder(hip, None, True, 5)
    assert ca.tobytes() == cb.tobytes()
    n = img.header["persistent_size"]
    assert a.read(0, n) == b.read(0, n)
    a.close()
    b.close()


def test_decoder_fused_backward_is_bitwise_the_separate_passes(hip, torch_cuda):
    """The engine shows the backend each range (BeginRange), so adjacent
    relaxed dK / dV instructions run as one pass; the losses and every
    persistent byte are those of the plan run with the pairs apart."""
    curves, states, fused = [], [], []
    for allow in (True, False):
        img = pw.decoder_lora(hip.plan_self_hash, relaxed=True, **TINY)
        eng = hip.Engine(img.blob)
        eng.set_attention_bf16(True)  # the dK / dV pair fuses on the bf16 kernels
        eng.set_fusion(allow)
        curve = []
        for s in range(3):
            x, y = tokens(s)
            curve.append(eng.train_step(x.view(np.float32), y))
        curves.append(np.array(curve, np.float32))
        states.append(eng.read(0, img.header["persistent_size"]))
        fused.append(eng.fused_dispatches())
        eng.close()
    assert fused[0] > 0 and fused[1] == 0
    assert curves[0].tobytes() == curves[1].tobytes()
    assert states[0] == states[1]


TINY_Q8 = dict(vocab=96, dim=128, heads=2, ffn=352, layers=2, seq=64, batch=2, rank=16)
# The train program ends in one kAdamWStep per adapter tensor (A and B at four
# sites per block); runs of up to 16 adjacent steps fuse into one launch.
Q8_ADAMW = TINY_Q8["layers"] * 4 * 2
Q8_ADAMW_FUSED = Q8_ADAMW - (Q8_ADAMW + 15) // 16
# Residual adds that run inside their producer, per step: in every block the
# FFN-down product's (x2 = x1 + down), the FFN input gradient's sum (the up
# product's dX plus the gate product's) and the post-attention residual
# gradient behind RMSNorm's backward; below the first block, the block
# input's residual gradient behind the other RMSNorm backward.
Q8_RESIDUAL_ADDS = TINY_Q8["layers"] * 3 + TINY_Q8["layers"] - 1
# ... and the loss: softmax-xent forward, its seed's fill and backward as one.
Q8_XENT = 1


def test_q8_decoder_folded_lora_sites_are_bitwise_the_separate_passes(hip, torch_cuda):
    """On the int8-base decoder the range fusions include the LoRA sites'
    low-rank epilogue (the frozen Q / K / V / O products with the rank-r
    term folded in) and the SwiGLU elementwise chains beside the dK / dV
    pairs: three steps with fusion on and off give the same losses and
    persistent bytes."""
    T = TINY_Q8["batch"] * TINY_Q8["seq"]
    curves, states, fused, dropped = [], [], [], []
    for allow in (True, False):
        img = pw.decoder_q8_lora(hip.plan_self_hash, relaxed=True, **TINY_Q8)
        eng = hip.Engine(img.blob)
        eng.set_attention_bf16(True)  # the dK / dV pair fuses on the bf16 kernels
        eng.set_fusion(allow)
        curve = []
        for s in range(3):
            t = pw.uniform_ints(7100 + s, T + 1, TINY_Q8["vocab"])
            curve.append(eng.train_step(t[:T].copy().view(np.float32), t[1:].copy()))
        curves.append(np.array(curve, np.float32))
        states.append(eng.read(0, img.header["persistent_size"]))
        fused.append(eng.fused_dispatches())
        dropped.append(eng.dropped_stores())
        eng.close()
    # per step and block: 4 LoRA forwards, the dK / dV pair, 2 SwiGLU chains;
    # per step the residual adds and the AdamW runs
    assert fused[0] == 3 * (TINY_Q8["layers"] * 7 + Q8_RESIDUAL_ADDS + Q8_XENT + Q8_ADAMW_FUSED)
    assert fused[1] == 0
    # the base values no later instruction reads (30 here): same bits without them
    assert dropped[0] > 0 and dropped[1] == 0
    assert curves[0].tobytes() == curves[1].tobytes()
    assert states[0] == states[1]


@pytest.mark.parametrize("relaxed", [False, True])
def test_q8_decoder_training_matches_the_oracle(hip, orc, torch_cuda, relaxed):
    """BASELINE configs[4]'s lowering at a small shape -- RMSNorm, the frozen
    int8 base with per-column scales (kGemmNNQ8 / kGemmNTQ8), SiLU-gated
    FFN, LoRA on Q / K / V / O -- six steps against its CPU twin under the
    reference's GPU-vs-CPU doctrine (as the configs[3] test above): losses
    rel 2e-3 / abs 1e-4 and each step's loss to 1e-5 (exact) or 2e-2
    (relaxed); exact, the persistent segment rel 5e-3 / abs 1e-6."""
    print(f"engine: q8 decoder plan {TINY_Q8}, relaxed={relaxed}", flush=True)
    img = pw.decoder_q8_lora(hip.plan_self_hash, relaxed=relaxed, **TINY_Q8)
    eng, twin = hip.Engine(img.blob), OracleEngine(orc, img.blob)
    T = TINY_Q8["batch"] * TINY_Q8["seq"]
    curve, want = [], []
    for s in range(6):
        t = pw.uniform_ints(7000 + s, T + 1, TINY_Q8["vocab"])
        x, y = t[:T].copy(), t[1:].copy()
        curve.append(eng.train_step(x.view(np.float32), y))
        want.append(twin.train_step(x.view(np.float32), y))
    curve, want = np.array(curve), np.array(want)
    step_tol = 2e-2 if relaxed else 1e-5
    assert np.all(np.abs(curve - want) <= step_tol * np.abs(want)), (curve, want)
    expect_close("loss curve", curve, want, 2e-3, 1e-4)
    if not relaxed:
        persistent_doctrine(img, eng, twin)
    assert (eng.relaxed_executions() > 0) == relaxed
    # per step and block: the four LoRA forwards (the dX sites' NT products
    # are below the direct-to-LDS kernel's K), the two SwiGLU chains and the
    # dK / dV pair; the elementwise chains and the attention pair fuse in the
    # exact family too (relaxed attention runs the exact family's f32
    # products here).
    per_block = 7 if relaxed else 3
    assert eng.fused_dispatches() == 6 * (TINY_Q8["layers"] * per_block + Q8_RESIDUAL_ADDS +
                                          Q8_XENT + Q8_ADAMW_FUSED)
    batches = []
    for s in range(6, 9):
        t = pw.uniform_ints(7000 + s, T + 1, TINY_Q8["vocab"])
        batches.append((t[:T].copy().view(np.float32), t[1:].copy()))
    tracked_steps(orc, img, eng, twin, batches, step_tol)
    eng.close()


def test_token_outside_the_vocabulary_is_refused(hip, torch_cuda):
    img = pw.decoder_lora(hip.plan_self_hash, **TINY)
    eng = hip.Engine(img.blob)
    x, y = tokens(0)
    x[7] = TINY["vocab"]
    with pytest.raises(hip.BackendError) as err:
        eng.train_step(x.view(np.float32), y)
    assert "token 96 at position 7" in str(err.value)
    eng.close()


# --- per-tensor parity after one step (every activation and gradient) ----------------------------

def _plant_b(img, eng, twin, seed):
    """Nonzero B adapters (B = 0 at init would leave every dA at zero), the
    same bytes in the engine and its twin (either may be None)."""
    r = np.random.default_rng(seed)
    for name in img.arrays:
        if ".B" in name:
            off, nb = img.arena[name]
            val = (r.standard_normal(img.arrays[name].shape) * 0.05).astype(np.float32)
            if eng is not None:
                eng.write(off, val.tobytes())
            if twin is not None:
                twin.arena[off:off + nb] = val.view(np.uint8).ravel()


def _step_tensor_errors(img, eng, twin):
    """max-rel per arena tensor after one train step, skipping the persistent
    segment (AdamW has moved it: the gradients it read are compared in their
    own slots, which AdamW only reads)."""
    persistent = img.header["persistent_size"]
    errs = {}
    for name, (off, nb) in img.arena.items():
        if off < persistent or nb == 0:
            continue
        g = np.frombuffer(eng.read(off, nb), np.uint8)
        c = np.frombuffer(twin.read(off, nb), np.uint8)
        if name in ("tokens", "labels"):
            assert g.tobytes() == c.tobytes(), name
            continue
        errs[name] = maxrel(g.view(np.float32), c.view(np.float32))
    return errs


# The modes a decoder step is compared in.  "exact": the exact family, fusion
# off.  "relaxed": the relaxed family with fusion off, so every instruction
# stores its output, attention on f32 products.  "bench": what bench.py
# times -- the relaxed family, attention on bf16 copies (the forward's copies
# kept for the backward, RoPE writing them), every range fusion on -- with
# SEEAI_KEEP_DEAD_STORES=1, so each tensor the fused passes compute is still
# stored and compared (storing it or not never changes a value).
STEP_MODES = ["exact", "relaxed", "bench"]
ATTN_OPS = {47, 48, 49, 50, 57}


def _mode_engine(hip, blob, mode):
    import os
    keep = os.environ.get("SEEAI_KEEP_DEAD_STORES")
    if mode == "bench":
        os.environ["SEEAI_KEEP_DEAD_STORES"] = "1"  # read when the context is made
    try:
        eng = hip.Engine(blob)
    finally:
        if keep is None:
            os.environ.pop("SEEAI_KEEP_DEAD_STORES", None)
        else:
            os.environ["SEEAI_KEEP_DEAD_STORES"] = keep
    eng.set_fusion(mode == "bench")
    eng.set_attention_bf16(mode == "bench")
    return eng


_TWINS: dict = {}


def _oracle_step(orc, key, img, plant_seed, tokens, threads=1):
    """One oracle train step of `img` with B planted from `plant_seed`,
    cached per key: the oracle runs the exact family whatever the plan's
    relaxed flags, so the exact and relaxed plans (same layout) share it."""
    if key in _TWINS:
        twin, loss, arena_map = _TWINS[key]
        assert arena_map == img.arena
        return twin, loss
    _TWINS.clear()  # one big twin at a time
    twin = OracleEngine(orc, img.blob)
    _plant_b(img, None, twin, plant_seed)
    x, y = tokens
    orc.set_threads(threads)
    try:
        loss = twin.train_step(x.view(np.float32), y)
    finally:
        orc.set_threads(1)
    _TWINS[key] = (twin, loss, dict(img.arena))
    return twin, loss


def _compare_step(hip, orc, img, mode, key, plant_seed, tokens, threads=1):
    eng = _mode_engine(hip, img.blob, mode)
    _plant_b(img, eng, None, plant_seed)
    x, y = tokens
    relaxed0 = eng.relaxed_executions()
    lg = eng.train_step(x.view(np.float32), y)
    twin, lc = _oracle_step(orc, key, img, plant_seed, tokens, threads)
    errs = _step_tensor_errors(img, eng, twin)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    print(f"{key} {mode}: loss {lg} vs {lc}; fused {eng.fused_dispatches()}; worst " +
          ", ".join(f"{n} {e:.2e}" for n, e in worst), flush=True)
    bar = TOL if mode == "exact" else 2e-2
    assert abs(lg - lc) <= bar * abs(lc)
    bad = {n: e for n, e in errs.items() if not e <= bar}
    assert not bad, bad
    # Relaxed attention counts as a relaxed execution only on the bf16
    # kernels (bench mode); the f32-product family is exact arithmetic.
    n_relaxed = sum(1 for w in img.train
                    if struct.unpack_from("<H", w, 2)[0] & (1 << 5)
                    and (mode == "bench" or struct.unpack_from("<H", w)[0] not in ATTN_OPS))
    assert eng.relaxed_executions() - relaxed0 == (0 if mode == "exact" else n_relaxed)
    if mode == "bench":
        assert eng.fused_dispatches() > 0
    eng.close()


@pytest.mark.parametrize("which", ["c4", "c5"])
@pytest.mark.parametrize("mode", STEP_MODES)
def test_decoder_step_tensors_match_the_oracle(hip, orc, torch_cuda, which, mode):
    """One step of the small decoder plans with B planted nonzero: every
    activation, gradient and scratch tensor of the arena against the
    oracle's, per tensor -- exact family 1e-5, relaxed family 2e-2 -- the
    north star's bars, before AdamW's sign amplification can act; in the
    exact mode, in the relaxed mode with every instruction apart, and in the
    configuration the bench times; each relaxed instruction counted once."""
    make, cfg = (pw.decoder_lora, TINY) if which == "c4" else (pw.decoder_q8_lora, TINY_Q8)
    img = make(hip.plan_self_hash, relaxed=mode != "exact", **cfg)
    T = cfg["batch"] * cfg["seq"]
    t = pw.uniform_ints(7300, T + 1, cfg["vocab"])
    _compare_step(hip, orc, img, mode, f"tiny-{which}", 77, (t[:T].copy(), t[1:].copy()))


def _adamw_pairs(img):
    """(parameter, gradient) arena names of the train program's AdamW steps."""
    inv = {off: n for n, (off, nb) in img.arena.items()}
    out = []
    for w in img.train:
        if struct.unpack_from("<H", w)[0] == 18:
            p, g = struct.unpack_from("<2Q", w, 8)
            out.append((inv[p], inv[g]))
    return out


def _f64(reader, img, name):
    off, nb = img.arena[name]
    return np.frombuffer(reader.read(off, nb), np.float32).astype(np.float64)


@pytest.mark.parametrize("which", ["c4", "c5"])
@pytest.mark.parametrize("mode", ["exact", "bench"])
def test_adapters_after_steps_match_the_oracle(hip, orc, torch_cuda, which, mode):
    """The updated adapters over four AdamW steps (B planted) against the
    exact twin, and where their error comes from.

    At every step the engine's update is bitwise the reference AdamW
    (optimizer.cc:104-132, the oracle's restatement) applied to the engine's
    own gradient and state: the optimizer adds no error of its own.  At the
    first step those gradients are within the family's bar of the twin's
    (exact 1e-5, relaxed 2e-2).  What the update then does to them is
    AdamW's: its step is lr m / (sqrt(v) + eps), about lr g / (|g| + eps) at
    step one, so a gradient element near eps moves its parameter by a
    sizeable fraction of lr for a tiny change of g, and one whose sign
    changes (relaxed: an element at the bf16 noise floor) by 2 lr.  So the
    per-tensor max-rel of the parameters after a step is not the gradients'
    bar: it is printed, held under a regression ceiling (exact 1e-4, relaxed
    5e-2), the relative L2 error under the bar; relaxed, every gradient sign
    change sits below 2e-2 max|g| of its tensor and every parameter element
    outside the bar after four steps had one."""
    make, cfg = (pw.decoder_lora, TINY) if which == "c4" else (pw.decoder_q8_lora, TINY_Q8)
    img = make(hip.plan_self_hash, relaxed=mode != "exact", **cfg)
    eng, twin = _mode_engine(hip, img.blob, mode), OracleEngine(orc, img.blob)
    _plant_b(img, eng, twin, 78)
    T = cfg["batch"] * cfg["seq"]
    h = img.header
    moments = {}
    for w in img.train:
        if struct.unpack_from("<H", w)[0] == 18:
            refs = struct.unpack_from("<4Q", w, 8)
            inv = {off: n for n, (off, nb) in img.arena.items()}
            moments[inv[refs[0]]] = (inv[refs[1]], inv[refs[2]], inv[refs[3]])
    flipped = {p: np.zeros(img.arena[p][1] // 4, bool) for p in moments}
    bar = TOL if mode == "exact" else 2e-2
    f32 = lambda reader, name: _f64(reader, img, name).astype(np.float32)  # noqa: E731
    first = {}
    for s in range(4):
        before = {p: (f32(eng, p), f32(eng, m), f32(eng, v)) for p, (_, m, v) in moments.items()}
        t = pw.uniform_ints(7400 + s, T + 1, cfg["vocab"])
        eng.train_step(t[:T].copy().view(np.float32), t[1:].copy())
        twin.train_step(t[:T].copy().view(np.float32), t[1:].copy())
        for p, (g, m, v) in moments.items():
            ok, p1, m1, v1 = orc.adamw_step(before[p][0], f32(eng, g), before[p][1], before[p][2],
                                            h["lr"], h["beta1"], h["beta2"], h["eps"],
                                            h["weight_decay"], s + 1)
            assert ok
            assert p1.tobytes() == f32(eng, p).tobytes(), f"step {s + 1} {p}: not AdamW(g)"
            assert m1.tobytes() == f32(eng, m).tobytes() and v1.tobytes() == f32(eng, v).tobytes()
            gg, gc = _f64(eng, img, g), _f64(twin, img, g)
            if s == 0:
                first[p] = (maxrel(gg, gc), maxrel(_f64(eng, img, p), _f64(twin, img, p)))
            flip = np.sign(gg) != np.sign(gc)
            if mode != "exact":
                assert np.all(np.abs(gc[flip]) <= bar * np.max(np.abs(gc))), \
                    f"step {s + 1} {g}: a sign change above the noise floor"
            flipped[p] |= flip
    l2, mx, outside = {}, {}, 0
    for p in moments:
        g, c = _f64(eng, img, p), _f64(twin, img, p)
        l2[p] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
        mx[p] = maxrel(g, c)
        out = np.abs(g - c) > bar * np.max(np.abs(c))
        outside += int(out.sum())
        if mode != "exact":
            assert np.all(flipped[p][out]), f"{p}: an element outside the bar with no sign change"
    print(f"{which} {mode}: step 1 gradients max-rel {max(e for e, _ in first.values()):.2e}, "
          f"adapters {max(e for _, e in first.values()):.2e}; after 4 steps adapters L2 "
          f"{max(l2.values()):.2e}, max-rel {max(mx.values()):.2e}, {outside} elements outside "
          f"{bar:g}, {sum(int(f.sum()) for f in flipped.values())} gradient sign changes",
          flush=True)
    assert max(e for e, _ in first.values()) <= bar
    assert max(l2.values()) <= bar
    assert max(mx.values()) <= (1e-4 if mode == "exact" else 5e-2)
    eng.close()


C4_WIDE = dict(vocab=32000, dim=768, heads=12, ffn=3072, layers=1, seq=1024, batch=1, rank=8)


@pytest.mark.parametrize("mode", STEP_MODES)
def test_c4_width_slice_step_tensors_match_the_oracle(hip, orc, torch_cuda, mode):
    """BASELINE configs[3] at its real widths -- d 768, 12 heads, FFN 3072,
    vocab 32000, S 1024 -- one block, one sequence: every arena tensor after
    one step, per tensor, at the bars above, in the three modes (the oracle
    threaded; its bits do not depend on the thread count)."""
    import os
    print(f"engine: C4-width slice {C4_WIDE}, {mode}", flush=True)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=mode != "exact", **C4_WIDE)
    t = pw.uniform_ints(7500, 1025, 32000)
    _compare_step(hip, orc, img, mode, "c4-width", 79, (t[:1024].copy(), t[1:].copy()),
                  threads=min(16, os.cpu_count() or 1))


C5_WIDE = dict(vocab=32000, dim=2048, heads=32, ffn=5632, layers=1, seq=2048, batch=1, rank=16)


@pytest.mark.parametrize("mode", STEP_MODES)
def test_c5_width_slice_step_tensors_match_the_oracle(hip, orc, torch_cuda, mode):
    """BASELINE configs[4] at its real widths -- d 2048, 32 heads, SiLU-gated
    FFN 5632, RMSNorm, the frozen int8 base with per-column scales, LoRA r16
    on Q / K / V / O, vocab 32000, S 2048 -- one block, one sequence (the
    reference's q8 system test, update_system_test.cc:827, at model widths):
    every arena tensor after one step, per tensor, at the bars above, in the
    three modes, against the threaded oracle."""
    import os
    print(f"engine: C5-width slice {C5_WIDE}, {mode}", flush=True)
    img = pw.decoder_q8_lora(hip.plan_self_hash, relaxed=mode != "exact", **C5_WIDE)
    t = pw.uniform_ints(7600, 2049, 32000)
    _compare_step(hip, orc, img, mode, "c5-width", 80, (t[:2048].copy(), t[1:].copy()),
                  threads=min(16, os.cpu_count() or 1))


# Producers that feed a relaxed direct-to-LDS product in one training step of
# the two-block tiny decoders.  c4: LayerNorm forward ahead of Q and of the
# FFN up product (2 + 2), GELU forward (2), the softmax-xent backward (1),
# the final LayerNorm backward (1), GELU backward (2), the residual-gradient
# adds ahead of Wo^T (2) and of the block below's Wd^T (1), and the upper
# block's RoPE backwards of q and k for the input-gradient products past the
# adapter GEMMs (2; the lower block has no input-gradient products).  c5 the
# same with RMSNorm and the SwiGLU passes in place of GELU, the SwiGLU
# backward writing the copies of both its products (2 more).  The final norm
# does not fuse: the head's N = 96 is below the direct-to-LDS kernel's 128.
SINKS_PER_STEP = {"c4": 15, "c5": 17}
# With attention on bf16 copies, per block: the attention forward writes the
# O product's activation, the RoPE forwards of q and k write the attention's
# own copies of them, the V site's low-rank pass writes v's, and the O
# product (c4) or the O site's input-gradient pass (c5) writes the attention
# backward's dO.  Per step, the upper block's dK / dV pass writes dV's for its
# input-gradient product.
ATTN_SINKS_PER_STEP = {"c4": 5 * 2 + 1, "c5": 5 * 2 + 1}


@pytest.mark.parametrize("attn16", [False, True])
@pytest.mark.parametrize("plan", ["c4", "c5"])
def test_conversions_fused_into_producers_are_bitwise_the_passes(hip, torch_cuda, plan, attn16):
    """A producer followed by a relaxed frozen-weight product on the
    direct-to-LDS path writes the product's bf16 activation as it stores
    (GELU forward / backward, the SwiGLU passes, the softmax-xent backward,
    LayerNorm / RMSNorm forward and backward, the residual-gradient adds)
    and drops its f32 store where nothing else reads it; the product skips
    its conversion pass.  The residual adds run inside their producers
    (a product's epilogue, a normalisation's backward) in the same run.  With the NT products on the direct-to-LDS kernel
    at these small K (relaxed_nt_dma_min_k 64), three steps with fusion on
    and off give the same losses and persistent bytes; with attention on
    bf16 copies the attention forward is one of the producers, and the RoPE
    forwards write the attention's q and k copies."""
    print(f"engine: fused conversions, tiny {plan}, attention bf16 {attn16}", flush=True)
    curves, states, sinks = [], [], []
    for allow in (True, False):
        if plan == "c4":
            img = pw.decoder_lora(hip.plan_self_hash, relaxed=True, **TINY)
            T = TINY["batch"] * TINY["seq"]
            vocab = TINY["vocab"]
        else:
            img = pw.decoder_q8_lora(hip.plan_self_hash, relaxed=True, **TINY_Q8)
            T = TINY_Q8["batch"] * TINY_Q8["seq"]
            vocab = TINY_Q8["vocab"]
        eng = hip.Engine(img.blob)
        eng.configure({"relaxed_nt_dma_min_k": 64})
        eng.set_attention_bf16(attn16)
        eng.set_fusion(allow)
        curve = []
        for s in range(3):
            t = pw.uniform_ints(7300 + s, T + 1, vocab)
            curve.append(eng.train_step(t[:T].copy().view(np.float32), t[1:].copy()))
            if s == 0:
                first = eng.fused_conversions()
        curves.append(np.array(curve, np.float32))
        states.append(eng.read(0, img.header["persistent_size"]))
        sinks.append(eng.fused_conversions() - first)
        eng.close()
    # The first step grows the conversion workspace as it goes (a producer
    # ahead of the first product that needs the room does not fuse); steps
    # two and three fuse every one.
    print(f"  {sinks[0]} conversions fused over steps 2-3", flush=True)
    assert sinks[0] == 2 * (SINKS_PER_STEP[plan] + (ATTN_SINKS_PER_STEP[plan] if attn16 else 0))
    assert sinks[1] == 0
    assert curves[0].tobytes() == curves[1].tobytes()
    assert states[0] == states[1]


def test_saved_attention_copies_under_a_cap_keep_the_bits(hip, torch_cuda):
    """The forward's bf16 copies of q, k and v kept for the backward are a
    cost, never a value: with the cap at zero (SEEAI_ATTN_SAVED_MB=0, no
    triple saved, every backward converting again) three steps of the tiny
    decoders on bf16 copies give the losses and persistent bytes of the
    default, which saves one triple per layer."""
    import os
    for make, cfg in ((pw.decoder_lora, TINY), (pw.decoder_q8_lora, TINY_Q8)):
        T = cfg["batch"] * cfg["seq"]
        curves, states = [], []
        for cap in (None, "0"):
            img = make(hip.plan_self_hash, relaxed=True, **cfg)
            if cap is not None:
                os.environ["SEEAI_ATTN_SAVED_MB"] = cap
            try:
                eng = hip.Engine(img.blob)
            finally:
                os.environ.pop("SEEAI_ATTN_SAVED_MB", None)
            eng.set_attention_bf16(True)
            curve = []
            for s in range(3):
                t = pw.uniform_ints(7700 + s, T + 1, cfg["vocab"])
                curve.append(eng.train_step(t[:T].copy().view(np.float32), t[1:].copy()))
            curves.append(np.array(curve, np.float32))
            states.append(eng.read(0, img.header["persistent_size"]))
            eng.close()
        assert curves[0].tobytes() == curves[1].tobytes()
        assert states[0] == states[1]
