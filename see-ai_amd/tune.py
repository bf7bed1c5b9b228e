"""The offline tuner for the gfx950 member of the kernel-policy table.

    python -m see-ai_amd.tune tune --out table.json [--fields a,b] [--rounds 3]
        [--repeats 3] [--min-gain 0.03] [--quick]
    python -m see-ai_amd.tune show table.json [--key KEY]

It follows the reference's tuner protocol (tool/autotune.py:1-58,
177-212), with kernel launches in place of seeml-bench runs:
- an arm is one value of one policy field; every arm of a field computes
  identical bits, so the table only picks among equivalent schedules;
- the sweep always includes the built-in default, the arm to beat;
- arms are visited round-robin for --rounds rounds, so clock and thermal
  drift land on every arm alike; each (arm, fixture) measurement is the
  median of --repeats timings (HIP events around back-to-back launches on
  the stream the library runs on), and an arm's figure per fixture is the
  median over rounds -- medians of medians;
- an arm's score is the geometric mean over its field's fixtures of its
  rate relative to the default arm's, so no fixture outvotes another by
  being larger;
- the best arm is written only when it beats the default by --min-gain
  (3 %); otherwise the default is recorded, with every number beside it.
The fixtures are the BASELINE shapes each field decides: the W8A8 and
quantizer shapes of the standalone GEMM, the relaxed frozen-weight
products of the decoder steps, and a skinny long-K exact product.

Exit codes: 0 tuned (or the default recorded), 1 a measurement or the table
failed, 2 usage.
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys

policy = importlib.import_module("see-ai_amd.policy")

# field -> arms (the default is always added)
ARMS = {
    "w8a8_large_kernel": [1, 2, 3],
    "w8a8_large_min": [1024, 2048, 4096],
    "quantize_waves_per_cu": [4, 8, 16, 32],
    "relaxed_min_tiles_256": [1, 128, 256, 1 << 30],
    "relaxed_min_fill_256": [0, 50, 80, 95],
    "relaxed_nt_dma_min_k": [256, 512, 768, 1024, 4096],
    "convert_wgs_per_cu": [2, 4, 8, 16, 32],
    "exact_longk_first": [1, 2],
    "relaxed_tile_192": [1, 2, 3],
}


class TuneError(Exception):
    """A failure that ends the run with exit 1 and the message."""


def _median_table(rounds):
    """One arm's rounds [{fixture: rate}, ...] -> {fixture: median rate}; every
    round must measure the same fixtures."""
    names = sorted(rounds[0])
    for r in rounds:
        if sorted(r) != names:
            raise TuneError("the rounds of one arm measured different fixtures")
    return {name: statistics.median([r[name] for r in rounds]) for name in names}


def score_arms(per_arm_runs, default_arm):
    """Score each arm against the default arm.

    per_arm_runs maps an arm to its rounds, each a {fixture: rate} dict.
    Every arm's figure per fixture is its median over rounds; its speedup per
    fixture is that median over the default arm's; its score is the mean of
    the log speedups, exponentiated (the geometric mean), so a large fixture
    counts no more than a small one.  Returns {arm: {"rate", "speedup",
    "score"}}."""
    table = {arm: _median_table(rounds) for arm, rounds in per_arm_runs.items()}
    reference = table[default_arm]
    if any(v <= 0 for v in reference.values()):
        raise TuneError("the default arm measured a non-positive rate")
    scored = {}
    for arm, rates in table.items():
        speedup = {name: rates[name] / reference[name] for name in reference}
        logs = [math.log(x) for x in speedup.values()]
        score = math.exp(math.fsum(logs) / len(logs)) if logs else 0.0
        scored[arm] = {"rate": rates, "speedup": speedup, "score": score}
    return scored


def choose(scored, default_arm, min_gain):
    """(arm to record, why).  The default stays unless another arm's score
    beats it by at least min_gain; a tie goes to the default."""
    base = scored[default_arm]["score"]
    challengers = [a for a in scored if a != default_arm and scored[a]["score"] > base]
    if not challengers:
        return default_arm, "default-is-best"
    top = sorted(challengers, key=lambda a: scored[a]["score"], reverse=True)[0]
    gain = scored[top]["score"] / base - 1.0
    if gain >= min_gain:
        return top, f"tuned: {top} gains {gain:.1%} over the default"
    return default_arm, (f"default-within-margin: best arm {top} gains {gain:.1%}, "
                         f"below --min-gain {min_gain:.1%}")


# --- fixtures ----------------------------------------------------------------

class Bench:
    """Device buffers and timed launches for one field's fixtures."""

    def __init__(self, quick: bool):
        import torch
        self.torch = torch
        self.hip = importlib.import_module("see-ai_amd.hip")
        torch.cuda.set_device(0)
        self.ctx = self.hip.Context(0)
        self.ctx.use_torch_stream()
        self.quick = quick
        self.iters = 5 if quick else 20
        self._relaxed_backends = []

    def time_ms(self, fn, iters=None):
        torch = self.torch
        iters = iters or self.iters
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    # Each fixture: (name, setup() -> (run(), work units per run)); a rate is
    # units per millisecond.
    def fixtures(self, field):
        torch, ctx = self.torch, self.ctx
        g = torch.Generator(device="cuda").manual_seed(20261202)
        if field == "w8a8_large_kernel":
            shapes = [(4096, 4096, 4096), (2048, 2048, 4096), (8192, 4096, 2048)]
            yield from self.fixtures_w8a8(shapes[:1] if self.quick else shapes)
        elif field == "w8a8_large_min":
            yield from self.fixtures_w8a8([(1024, 1024, 4096), (2048, 2048, 4096),
                                           (2048, 4096, 4096)])
        elif field == "quantize_waves_per_cu":
            shapes = [(8192, 768), (4096, 1024), (1024, 16384)]
            if self.quick:
                shapes = shapes[:1]
            for rows, cols in shapes:
                def setup(rows=rows, cols=cols):
                    X = torch.randn((rows, cols), device="cuda", generator=g)
                    Q = torch.empty((rows, cols), dtype=torch.int8, device="cuda")
                    s = torch.empty(rows, device="cuda")
                    keep = (X, Q, s)
                    return (lambda: ctx.call("seeai_w8a8_quantize_rows", X.data_ptr(), Q.data_ptr(),
                                             s.data_ptr(), rows, cols), 5.0 * rows * cols, keep)
                yield f"quantize {rows}x{cols}", setup
        elif field in ("relaxed_min_tiles_256", "relaxed_min_fill_256", "relaxed_tile_192"):
            # The decoder steps' relaxed frozen-weight products (q8, column
            # scales, weights in rodata) -- NN forward and NT dX shapes, the
            # vocabulary head among them.
            shapes = [(0, 8192, 768, 768), (0, 8192, 3072, 768), (1, 8192, 768, 3072),
                      (0, 8192, 32000, 768), (1, 8192, 768, 32000),
                      (0, 8192, 2048, 2048), (0, 8192, 5632, 2048), (1, 8192, 2048, 5632)]
            if self.quick:
                shapes = shapes[:2]
            for nt, M, N, K in shapes:
                def setup(nt=nt, M=M, N=N, K=K):
                    return self._relaxed_q8(nt, M, N, K)
                yield f"relaxed q8 {'NT' if nt else 'NN'} {M}x{N}x{K}", setup
        elif field == "relaxed_nt_dma_min_k":
            # C4's dX products over f32 weights (K = 768 and 3072) and C5's
            # q8 ones (K = 2048, 5632): NT, K either side of the threshold.
            shapes = [("f32", 8192, 768, 768), ("f32", 8192, 3072, 768), ("f32", 8192, 768, 3072),
                      ("q8", 8192, 2048, 2048), ("q8", 8192, 5632, 2048)]
            if self.quick:
                shapes = shapes[:2]
            for kind, M, N, K in shapes:
                def setup(kind=kind, M=M, N=N, K=K):
                    return self._relaxed_nt(kind, M, N, K)
                yield f"relaxed {kind} NT {M}x{N}x{K}", setup
        elif field == "convert_wgs_per_cu":
            # Relaxed products whose A conversion dominates (N = 128): the
            # decoder's activation widths, NN and NT (k-scaled).
            for kind, nt, M, K in [("q8", 0, 8192, 2048), ("q8", 0, 8192, 5632), ("q8", 1, 8192, 2048),
                                   ("f32", 0, 8192, 768)]:
                def setup(kind=kind, nt=nt, M=M, K=K):
                    if nt:
                        return self._relaxed_nt(kind, M, 128, K)
                    if kind == "q8":
                        return self._relaxed_q8(0, M, 128, K)
                    return self._relaxed_f32_nn(M, 128, K)
                yield f"convert {kind} {'NT' if nt else 'NN'} {M}x{K}", setup
        elif field == "exact_longk_first":
            for M, N, K in [(64, 64, 8192), (16, 128, 16384)]:
                def setup(M=M, N=N, K=K):
                    A = torch.randn((M, K), device="cuda", generator=g)
                    B = torch.randn((K, N), device="cuda", generator=g)
                    C = torch.empty((M, N), device="cuda")
                    keep = (A, B, C)
                    return (lambda: ctx.call("seeai_gemm_f32", 0, A.data_ptr(), B.data_ptr(),
                                             C.data_ptr(), M, N, K, None, 0, None,
                                             self.hip._F(1.0), 0), 2.0 * M * N * K, keep)
                yield f"exact NN {M}x{N}x{K}", setup
        else:
            raise TuneError(f"no fixtures for field {field}")

    def fixtures_w8a8(self, shapes):
        torch, ctx = self.torch, self.ctx
        g = torch.Generator(device="cuda").manual_seed(20261203)
        for M, N, K in shapes:
            def setup(M=M, N=N, K=K):
                QA = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
                QW = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
                sa, sw = torch.rand(M, device="cuda"), torch.rand(N, device="cuda")
                C = torch.empty((M, N), device="cuda")
                keep = (QA, QW, sa, sw, C)
                return (lambda: ctx.call("seeai_w8a8_gemm", QA.data_ptr(), sa.data_ptr(),
                                         QW.data_ptr(), sw.data_ptr(), C.data_ptr(), None,
                                         M, N, K), 2.0 * M * N * K, keep)
            yield f"w8a8 {M}x{N}x{K}", setup

    def _relaxed_q8(self, nt, M, N, K):
        import numpy as np
        hip = self.hip
        be = hip.HipBackend(0)
        be.ctx.use_torch_stream()
        r = np.random.default_rng(M + N + K + nt)
        W = r.integers(-127, 128, (N, K) if nt else (K, N)).astype(np.int8)
        sc = r.uniform(1e-3, 5e-2, K if nt else N).astype(np.float32)
        w_off = 0
        s_off = (W.nbytes + 255) // 256 * 256
        rodata = bytearray(s_off + sc.nbytes)
        rodata[:W.nbytes] = W.tobytes()
        rodata[s_off:] = sc.tobytes()
        a_off = 0
        c_off = (4 * M * K + 16383) // 16384 * 16384
        be.Bind(None, c_off + 4 * M * N, bytes(rodata))
        be.Configure(self.ctx.policy())
        be.Upload(a_off, r.standard_normal((M, K)).astype(np.float32).tobytes())
        rb = 1 << 63
        flags = (1 << 5) | (1 << 4)  # kFlagRelaxed | kFlagQ8ColScale
        word = hip.pack_instruction(30 if nt else 29, flags, 0,
                                    [a_off, rb | w_off, c_off, rb | s_off], [M, N, K])
        self._relaxed_backends.append(be)
        return (lambda: be.Execute(word), 2.0 * M * N * K, be)

    def _relaxed_nt(self, kind, M, N, K):
        """A relaxed NT product on a rodata weight [N, K]: f32 (C4's dX) or
        int8 with k-scales (C5's)."""
        import numpy as np
        hip = self.hip
        be = hip.HipBackend(0)
        be.ctx.use_torch_stream()
        r = np.random.default_rng(M + N + K + len(kind))
        if kind == "q8":
            W = r.integers(-127, 128, (N, K)).astype(np.int8)
        else:
            W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
        sc = r.uniform(1e-3, 5e-2, K).astype(np.float32)
        s_off = (W.nbytes + 255) // 256 * 256
        rodata = bytearray(s_off + sc.nbytes)
        rodata[:W.nbytes] = W.tobytes()
        rodata[s_off:] = sc.tobytes()
        c_off = (4 * M * K + 16383) // 16384 * 16384
        be.Bind(None, c_off + 4 * M * N, bytes(rodata))
        be.Configure(self.ctx.policy())
        be.Upload(0, r.standard_normal((M, K)).astype(np.float32).tobytes())
        rb = 1 << 63
        if kind == "q8":
            word = hip.pack_instruction(30, (1 << 5) | (1 << 4), 0, [0, rb, c_off, rb | s_off],
                                        [M, N, K])
        else:
            word = hip.pack_instruction(2, 1 << 5, 0, [0, rb, c_off], [M, N, K])
        self._relaxed_backends.append(be)
        return (lambda: be.Execute(word), 2.0 * M * N * K, be)

    def _relaxed_f32_nn(self, M, N, K):
        """A relaxed NN product on an f32 rodata weight [K, N] (C4's forward)."""
        import numpy as np
        hip = self.hip
        be = hip.HipBackend(0)
        be.ctx.use_torch_stream()
        r = np.random.default_rng(M + N + K + 7)
        W = (r.standard_normal((K, N)) * 0.02).astype(np.float32)
        c_off = (4 * M * K + 16383) // 16384 * 16384
        be.Bind(None, c_off + 4 * M * N, W.tobytes())
        be.Configure(self.ctx.policy())
        be.Upload(0, r.standard_normal((M, K)).astype(np.float32).tobytes())
        word = hip.pack_instruction(1, 1 << 5, 0, [0, 1 << 63, c_off], [M, N, K])
        self._relaxed_backends.append(be)
        return (lambda: be.Execute(word), 2.0 * M * N * K, be)

    def apply(self, field, arm):
        pol = self.ctx.policy()
        pol[field] = arm
        self.ctx.configure(pol)
        for be in self._relaxed_backends:
            be.Configure(pol)


def tune_field(bench, field, rounds, repeats, min_gain, log):
    default = policy.DEFAULTS[field]
    arms = sorted(set(ARMS[field]) | {default})
    fixtures = []
    for name, setup in bench.fixtures(field):
        run, units, keep = setup()
        fixtures.append((name, run, units, keep))
    runs = {arm: [] for arm in arms}
    for rnd in range(rounds):
        for arm in arms:
            bench.apply(field, arm)
            res = {}
            for name, run, units, _ in fixtures:
                ms = statistics.median(bench.time_ms(run) for _ in range(repeats))
                res[name] = units / ms
            runs[arm].append(res)
            log(f"{field} round {rnd + 1}/{rounds} arm {arm}: " +
                ", ".join(f"{k} {v / 1e9:.1f}" for k, v in res.items()) + " (G units/s)")
    scored = score_arms(runs, default)
    chosen, decision = choose(scored, default, min_gain)
    bench.apply(field, chosen)  # later fields are measured on top of this one's decision
    return chosen, {"arms": {str(a): {"score": round(s["score"], 4),
                                      "rate_per_ms": {k: round(v, 1) for k, v in s["rate"].items()}}
                             for a, s in scored.items()},
                    "default": default, "chosen": chosen, "decision": decision}


def cmd_tune(args):
    fields = args.fields.split(",") if args.fields else list(ARMS)
    for f in fields:
        if f not in ARMS:
            print(f"unknown field {f}; known: {', '.join(ARMS)}", file=sys.stderr)
            return 2
    bench = Bench(args.quick)
    key = bench.hip.device_key(0)
    log = (lambda m: print(m, flush=True))
    log(f"device key: {key}")
    entry, tuned = {}, {"protocol": {"rounds": args.rounds, "repeats": args.repeats,
                                     "min_gain": args.min_gain, "iters": bench.iters}}
    for f in fields:
        chosen, record = tune_field(bench, f, args.rounds, args.repeats, args.min_gain, log)
        entry[f] = chosen
        tuned[f] = record
        log(f"{f}: {record['decision']}")
    text = None
    if args.out and os.path.exists(args.out):
        with open(args.out) as fh:
            text = fh.read()
    out = policy.merge_into_table(text, key, entry, tuned)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(out)
    print(json.dumps({"key": key, "gfx950": policy.check_entry(entry, "tuned entry"),
                      "decisions": {f: tuned[f]["decision"] for f in fields}}), flush=True)
    return 0


def cmd_show(args):
    try:
        table = policy.load_table(args.table)
    except policy.PolicyError as e:
        print(e, file=sys.stderr)
        return 1
    for key, entry in table.items():
        if args.key and key != args.key:
            continue
        print(key)
        for k, v in entry.items():
            print(f"  {k} = {v}")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m see-ai_amd.tune")
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("tune")
    t.add_argument("--out", default=None)
    t.add_argument("--fields", default=None)
    t.add_argument("--rounds", type=int, default=3)
    t.add_argument("--repeats", type=int, default=3)
    t.add_argument("--min-gain", type=float, default=0.03)
    t.add_argument("--quick", action="store_true")
    s = sub.add_parser("show")
    s.add_argument("table")
    s.add_argument("--key", default=None)
    args = ap.parse_args(argv)
    try:
        return cmd_tune(args) if args.cmd == "tune" else cmd_show(args)
    except (TuneError, policy.PolicyError) as e:
        print(e, file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
