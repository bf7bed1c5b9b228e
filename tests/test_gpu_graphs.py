"""GPU: ranges replayed from captured HIP graphs (seeai_run_range with
seeai_set_graph_replay on).

The engine's ExecuteRange runs a range instruction by instruction the first
time, captures it as a graph the second time and launches the graph from
then on, the step's optimizer values copied to the device ahead of each
launch.  Replay changes how the launches reach the GPU, never which kernels
run with which operands: every loss and every persistent byte equals the
instruction-by-instruction engine's bit for bit, step after step, with the
batches uploaded (and the loss read back) between the replays."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

pw = importlib.import_module("see-ai_amd.planwriter")
pytestmark = pytest.mark.gpu

TINY = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2, rank=8)


def c1_batch(step):
    return pw.normal(7000 + step, (32, 256)), pw.uniform_ints(8000 + step, 32, 256)


def tokens(step):
    T = TINY["batch"] * TINY["seq"]
    t = pw.uniform_ints(9000 + step, T + 1, TINY["vocab"])
    return t[:T].copy().view(np.float32), t[1:].copy()


def _twins(hip, blob):
    graphed, eager = hip.Engine(blob), hip.Engine(blob)
    graphed.set_graph_replay(True)
    eager.set_graph_replay(False)
    return graphed, eager


def _lockstep(graphed, eager, batches, persistent):
    for i, (x, y) in enumerate(batches):
        lg, le = graphed.train_step(x, y), eager.train_step(x, y)
        assert np.float32(lg).tobytes() == np.float32(le).tobytes(), f"step {i}: {lg} vs {le}"
    assert graphed.read(0, persistent) == eager.read(0, persistent)


def test_c1_replayed_steps_are_bitwise_the_eager_steps(hip, torch_cuda):
    print("graphs: config-1 plan, 8 steps graphed vs eager", flush=True)
    img = pw.mlp_lora(hip.plan_self_hash)
    n = img.header["persistent_size"]
    graphed, eager = _twins(hip, img.blob)
    _lockstep(graphed, eager, [c1_batch(s) for s in range(8)], n)
    # The train range ran eagerly once, was captured the second time and
    # replayed from then on; the eager twin never launched a graph.
    assert graphed.graph_launches >= 6
    assert eager.graph_launches == 0
    # Evaluation is a range of its own; training continues on its graph.
    x, y = c1_batch(100)
    assert graphed.evaluate(x, y) == eager.evaluate(x, y)
    _lockstep(graphed, eager, [c1_batch(s) for s in range(8, 11)], n)
    graphed.close()
    eager.close()


def test_c1_feeder_steps_replay_bitwise(hip, torch_cuda):
    print("graphs: config-1 plan through the feeder", flush=True)
    img = pw.mlp_lora(hip.plan_self_hash)
    n = img.header["persistent_size"]
    graphed, eager = _twins(hip, img.blob)
    batches = [c1_batch(s) for s in range(6)]
    xs, ys = np.stack([b[0] for b in batches]), np.stack([b[1] for b in batches])
    lg, le = graphed.train_steps(xs, ys), eager.train_steps(xs, ys)
    assert lg.tobytes() == le.tobytes()
    assert graphed.read(0, n) == eager.read(0, n)
    assert graphed.graph_launches >= 4
    graphed.close()
    eager.close()


@pytest.mark.parametrize("relaxed", [False, True])
def test_decoder_replayed_steps_are_bitwise_the_eager_steps(hip, torch_cuda, relaxed):
    print(f"graphs: tiny decoder relaxed={relaxed}, 5 steps", flush=True)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=relaxed, **TINY)
    graphed, eager = _twins(hip, img.blob)
    _lockstep(graphed, eager, [tokens(s) for s in range(5)], img.header["persistent_size"])
    assert graphed.graph_launches >= 3
    graphed.close()
    eager.close()


def test_a_policy_change_recaptures(hip, torch_cuda):
    """A configure between steps drops the captured graph (it names the old
    geometry's workspaces); the next runs capture again and still match."""
    print("graphs: tiny relaxed decoder, policy change mid-run", flush=True)
    img = pw.decoder_lora(hip.plan_self_hash, relaxed=True, **TINY)
    n = img.header["persistent_size"]
    graphed, eager = _twins(hip, img.blob)
    _lockstep(graphed, eager, [tokens(s) for s in range(3)], n)
    before = graphed.graph_launches
    policy = {"relaxed_min_tiles_256": 1 << 30}
    graphed.configure(policy)
    eager.configure(policy)
    _lockstep(graphed, eager, [tokens(s) for s in range(3, 7)], n)
    assert graphed.graph_launches >= before + 2
    graphed.close()
    eager.close()
