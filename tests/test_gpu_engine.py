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
        persistent = img.header["persistent_size"]
        g = np.frombuffer(eng.read(0, persistent), np.float32)
        c = np.frombuffer(twin.read(0, persistent), np.float32)
        expect_close("persistent", g, c, 5e-3, 1e-6)
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
        persistent = img.header["persistent_size"]
        g = np.frombuffer(eng.read(0, persistent), np.float32)
        c = np.frombuffer(twin.read(0, persistent), np.float32)
        expect_close("persistent", g, c, 5e-3, 1e-6)
    assert (eng.relaxed_executions() > 0) == relaxed
    # per step and block: the four LoRA forwards (the dX sites' NT products
    # are below the direct-to-LDS kernel's K) and the two SwiGLU chains; the
    # elementwise chains fuse in the exact family too.  Relaxed attention
    # runs f32 products here, so its dK / dV pair stays two dispatches.
    per_block = 6 if relaxed else 2
    assert eng.fused_dispatches() == 6 * (TINY_Q8["layers"] * per_block + Q8_RESIDUAL_ADDS +
                                          Q8_XENT + Q8_ADAMW_FUSED)
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
    same bytes in the engine and its twin."""
    r = np.random.default_rng(seed)
    for name in img.arrays:
        if ".B" in name:
            off, nb = img.arena[name]
            val = (r.standard_normal(img.arrays[name].shape) * 0.05).astype(np.float32)
            eng.write(off, val.tobytes())
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


@pytest.mark.parametrize("which", ["c4", "c5"])
@pytest.mark.parametrize("relaxed", [False, True])
def test_decoder_step_tensors_match_the_oracle(hip, orc, torch_cuda, which, relaxed):
    """One step of the small decoder plans with B planted nonzero, fusion
    off so every instruction stores its output: every activation, gradient
    and scratch tensor of the arena against the oracle's, per tensor --
    exact family 1e-5, relaxed family (bf16 frozen-weight products) 2e-2 --
    the north star's bars, before AdamW's sign amplification can act."""
    make, cfg = (pw.decoder_lora, TINY) if which == "c4" else (pw.decoder_q8_lora, TINY_Q8)
    img = make(hip.plan_self_hash, relaxed=relaxed, **cfg)
    eng, twin = hip.Engine(img.blob), OracleEngine(orc, img.blob)
    eng.set_fusion(False)
    _plant_b(img, eng, twin, 77)
    T = cfg["batch"] * cfg["seq"]
    t = pw.uniform_ints(7300, T + 1, cfg["vocab"])
    x, y = t[:T].copy(), t[1:].copy()
    lg, lc = eng.train_step(x.view(np.float32), y), twin.train_step(x.view(np.float32), y)
    errs = _step_tensor_errors(img, eng, twin)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    print(f"{which} relaxed={relaxed}: loss {lg} vs {lc}; worst " +
          ", ".join(f"{n} {e:.2e}" for n, e in worst))
    bar = 2e-2 if relaxed else TOL
    assert abs(lg - lc) <= bar * abs(lc)
    bad = {n: e for n, e in errs.items() if not e <= bar}
    assert not bad, bad
    eng.close()


@pytest.mark.parametrize("which", ["c4", "c5"])
def test_relaxed_adapters_after_steps_match_the_oracle(hip, orc, torch_cuda, which):
    """The relaxed plans' adapters after four AdamW steps, B planted, against
    the exact twin: per tensor, the relative L2 error ||gpu - cpu|| / ||cpu||
    within the bf16 bar 2e-2.

    Per element the bar cannot hold, whatever the kernels: AdamW's update is
    lr * m / (sqrt(v) + eps), about lr * sign(g) in the first steps, so a
    gradient element at the bf16 noise floor that changes sign moves its
    parameter by 2 lr per step.  Four steps at lr 1e-3 against adapters of
    magnitude ~0.1 give a per-tensor max-rel near 3e-2 from single elements
    (measured on MI355X: 3.2e-2 and 3.4e-2), printed here beside the L2
    measure that is asserted."""
    make, cfg = (pw.decoder_lora, TINY) if which == "c4" else (pw.decoder_q8_lora, TINY_Q8)
    img = make(hip.plan_self_hash, relaxed=True, **cfg)
    eng, twin = hip.Engine(img.blob), OracleEngine(orc, img.blob)
    _plant_b(img, eng, twin, 78)
    T = cfg["batch"] * cfg["seq"]
    for s in range(4):
        t = pw.uniform_ints(7400 + s, T + 1, cfg["vocab"])
        eng.train_step(t[:T].copy().view(np.float32), t[1:].copy())
        twin.train_step(t[:T].copy().view(np.float32), t[1:].copy())
    l2, mx = {}, {}
    for name in img.arrays:
        if ".A" in name or ".B" in name:
            off, nb = img.arena[name]
            g = np.frombuffer(eng.read(off, nb), np.float32).astype(np.float64)
            c = np.frombuffer(twin.read(off, nb), np.float32).astype(np.float64)
            l2[name] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
            mx[name] = maxrel(g, c)
    print(f"{which} adapters after 4 steps: L2 max {max(l2.values()):.2e}, "
          f"per-element max-rel max {max(mx.values()):.2e}")
    bad = {n: e for n, e in l2.items() if not e <= 2e-2}
    assert not bad, bad
    eng.close()


C4_WIDE = dict(vocab=32000, dim=768, heads=12, ffn=3072, layers=1, seq=1024, batch=1, rank=8)


@pytest.mark.parametrize("relaxed", [False, True])
def test_c4_width_slice_step_tensors_match_the_oracle(hip, orc, torch_cuda, relaxed):
    """BASELINE configs[3] at its real widths -- d 768, 12 heads, FFN 3072,
    vocab 32000, S 1024 -- one block, one sequence: every arena tensor after
    one step, per tensor, at the bars above (the oracle threaded; its bits
    do not depend on the thread count)."""
    import os
    print(f"engine: C4-width slice {C4_WIDE}, relaxed={relaxed}", flush=True)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=relaxed, **C4_WIDE)
    eng, twin = hip.Engine(img.blob), OracleEngine(orc, img.blob)
    eng.set_fusion(False)
    _plant_b(img, eng, twin, 79)
    t = pw.uniform_ints(7500, 1025, 32000)
    x, y = t[:1024].copy(), t[1:].copy()
    lg = eng.train_step(x.view(np.float32), y)
    orc.set_threads(min(16, os.cpu_count() or 1))
    try:
        lc = twin.train_step(x.view(np.float32), y)
    finally:
        orc.set_threads(1)
    errs = _step_tensor_errors(img, eng, twin)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    print(f"C4 width relaxed={relaxed}: loss {lg} vs {lc}; worst " +
          ", ".join(f"{n} {e:.2e}" for n, e in worst))
    bar = 2e-2 if relaxed else TOL
    assert abs(lg - lc) <= bar * abs(lc)
    bad = {n: e for n, e in errs.items() if not e <= bar}
    assert not bad, bad
    eng.close()


# Producers that feed a relaxed direct-to-LDS product in one training step of
# the two-block tiny decoders.  c4: LayerNorm forward ahead of Q and of the
# FFN up product (2 + 2), GELU forward (2), the softmax-xent backward (1),
# the final LayerNorm backward (1), GELU backward (2), the residual-gradient
# adds ahead of Wo^T (2) and of the block below's Wd^T (1).  c5 the same with
# RMSNorm and the SwiGLU passes in place of GELU.  The final norm does not
# fuse: the head's N = 96 is below the direct-to-LDS kernel's 128.
SINKS_PER_STEP = {"c4": 13, "c5": 13}
# With attention on bf16 copies, per block: the attention forward writes the
# O product's activation, and the RoPE forwards of q and k write the
# attention's own copies of them.
ATTN_SINKS_PER_STEP = 3 * 2


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
    assert sinks[0] == 2 * (SINKS_PER_STEP[plan] + (ATTN_SINKS_PER_STEP if attn16 else 0))
    assert sinks[1] == 0
    assert curves[0].tobytes() == curves[1].tobytes()
    assert states[0] == states[1]
