"""Golden vectors for the oracle, written by the reference kernel library.

``python tests/golden/make_golden.py`` (on a host with /root/reference)
builds oracle/_ref/libseeref.so -- the reference's own kernel sources under
/root/reference/runtime/executor plus our C shim -- runs each kernel below
on small seeded inputs and stores inputs and outputs as .npz fixtures here.
The fixtures are data; the reference code never leaves the build host.

``replay(orc, npz)`` re-runs the same cases through the oracle so the CPU
tests can check it bit-for-bit on any machine.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _cases(k, rng):
    """(family, name, callable(kernels) -> dict of outputs, inputs dict)."""
    out = []

    def add(fam, name, inputs, fn):
        out.append((fam, name, inputs, fn))

    for (M, N, K) in [(3, 5, 7), (67, 129, 66), (5, 300, 17), (32, 64, 40)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        Bt = rng.standard_normal((N, K)).astype(np.float32)
        At = rng.standard_normal((K, M)).astype(np.float32)
        D = rng.standard_normal((M, N)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        Bq = rng.integers(-127, 128, (K, N)).astype(np.int8)
        cs = rng.uniform(0.01, 0.1, N).astype(np.float32)
        ks = rng.uniform(0.01, 0.1, K).astype(np.float32)
        Bqt = rng.integers(-127, 128, (N, K)).astype(np.int8)
        Bh = (B.view(np.uint32) >> 16).astype(np.uint16)
        tag = f"{M}x{N}x{K}"
        inp = dict(A=A, B=B, Bt=Bt, At=At, D=D, bias=bias, Bq=Bq, cs=cs, ks=ks, Bqt=Bqt, Bh=Bh)
        add("gemm", tag, inp, lambda kk, i=inp: {
            "nn_gelu_bias": kk.gemm_nn(i["A"], i["B"], i["bias"], 2, None, 1.0),
            "nn_addend_alpha": kk.gemm_nn(i["A"], i["B"], None, 0, i["D"], 2.0),
            "nt_addend_alpha": kk.gemm_nt(i["A"], i["Bt"], i["D"], 0.5),
            "tn_alpha": kk.gemm_tn(i["At"], i["B"], None, 1.7),
            "acc_nn": kk.gemm_acc_nn(i["A"], i["B"], i["D"], 2.0),
            "nn_q8_cs_silu": kk.gemm_nn_q8(i["A"], i["Bq"], 1.0, 3, i["cs"]),
            "nn_q8_relu": kk.gemm_nn_q8(i["A"], i["Bq"], 0.02, 1),
            "nt_q8_ks": kk.gemm_nt_q8(i["A"], i["Bqt"], 1.0, i["ks"]),
            "nt_q8": kk.gemm_nt_q8(i["A"], i["Bqt"], 0.03),
            "nn_bf16": kk.gemm_nn_bf16(i["A"], i["Bh"], i["bias"], 0),
        })
    for (B_, S, H, d) in [(1, 9, 2, 4), (2, 33, 2, 16), (1, 40, 1, 64)]:
        n = B_ * S * H * d
        q, kq, v, do = (rng.standard_normal(n).astype(np.float32) for _ in range(4))
        toks = rng.integers(0, 4, B_ * S).astype(np.int32)
        inp = dict(q=q, k=kq, v=v, do=do, toks=toks,
                   geo=np.array([B_, S, H, d], np.int64))

        def attn(kk, i=inp):
            B_, S, H, d = (int(x) for x in i["geo"])
            starts = kk.segment_starts(i["toks"], B_, S, 3)
            o, st = kk.attn_fwd_tiled(i["q"], i["k"], i["v"], B_, S, H, d, starts)
            dq, st2 = kk.attn_dq_tiled(i["q"], i["k"], i["v"], i["do"], st, B_, S, H, d)
            dk = kk.attn_dk_tiled(i["q"], i["k"], i["v"], i["do"], st2, B_, S, H, d)
            dv = kk.attn_dv_tiled(i["q"], i["k"], i["do"], st2, B_, S, H, d)
            oc, P = kk.attn_fwd(i["q"], i["k"], i["v"], B_, S, H, d)
            return {"starts": starts, "o": o, "stats": st2, "dq": dq, "dk": dk, "dv": dv,
                    "o_cached": oc, "P": P}
        add("attention", f"{B_}x{S}x{H}x{d}", inp, attn)
    for (N, C) in [(2, 4), (32, 256), (40, 500)]:
        lg = (rng.standard_normal((N, C)) * 3).astype(np.float32)
        lb = rng.integers(0, C, N).astype(np.int32)
        lbm = lb.copy()
        lbm[::3] = -1
        inp = dict(logits=lg, labels=lb, labels_masked=lbm)

        def xent(kk, i=inp):
            l1, p1 = kk.xent_fwd(i["logits"], i["labels"])
            l2, p2 = kk.xent_fwd(i["logits"], i["labels_masked"], True)
            return {"loss": np.float32(l1), "probs": p1, "dl": kk.xent_bwd(p1, i["labels"], 1.0),
                    "loss_masked": np.float32(l2),
                    "dl_masked": kk.xent_bwd(p2, i["labels_masked"], 2.0, True)}
        add("xent", f"{N}x{C}", inp, xent)
    for n in [5, 4000]:
        p, g, m, v = (rng.standard_normal(n).astype(np.float32) for _ in range(4))
        inp = dict(p=p, g=g, m=m, v=np.abs(v))

        def opt(kk, i=inp):
            _, p1, m1, v1 = kk.adamw_step(i["p"], i["g"], i["m"], i["v"], 1e-3, 0.9, 0.999, 1e-8,
                                          0.01, 2, 0.0)
            _, p2, m2, v2 = kk.adamw_step(i["p"], i["g"], i["m"], i["v"], 1e-3, 0.9, 0.999, 1e-8,
                                          0.01, 7, 1.0)
            return {"p": p1, "m": m1, "v": v1, "p_clip": p2, "m_clip": m2, "v_clip": v2,
                    "clipped": kk.clip_norm(i["g"], 1.0)[1],
                    "sqnorm": np.float32(kk.sqnorm_accum(i["g"], 0.25))}
        add("optimizer", f"n{n}", inp, opt)
    x = (rng.standard_normal(2000) * 4).astype(np.float32)
    y = rng.standard_normal(2000).astype(np.float32)
    X = rng.standard_normal((37, 300)).astype(np.float32)
    g = rng.standard_normal(300).astype(np.float32)
    bb = rng.standard_normal(300).astype(np.float32)
    dy = rng.standard_normal((37, 300)).astype(np.float32)
    xr = rng.standard_normal(2 * 9 * 3 * 8).astype(np.float32)
    toks = rng.integers(0, 50, 77).astype(np.int32)
    table = rng.standard_normal((50, 33)).astype(np.float32)
    inp = dict(x=x, y=y, X=X, g=g, b=bb, dy=dy, xr=xr, toks=toks, table=table)

    def ew(kk, i=inp):
        ln = kk.layernorm_fwd(i["X"], i["g"], i["b"])
        rm = kk.rmsnorm_fwd(i["X"], i["g"])
        return {"gelu": kk.gelu_fwd(i["x"]), "gelu_b": kk.gelu_bwd(i["y"], i["x"]),
                "silu": kk.silu_fwd(i["x"]), "silu_b": kk.silu_bwd(i["y"], i["x"]),
                "relu_b": kk.relu_bwd(i["y"], i["x"]), "bias": kk.add_bias(i["X"], i["g"]),
                "rr": kk.reduce_rows(i["X"]), "ln_y": ln[0], "ln_mean": ln[1], "ln_rstd": ln[2],
                "ln_dx": kk.layernorm_bwd(i["dy"], i["X"], i["g"], ln[1], ln[2]),
                "rms_y": rm[0], "rms_rstd": rm[1],
                "rms_dx": kk.rmsnorm_bwd(i["dy"], i["X"], i["g"], rm[1]),
                "rope_f": kk.rope(i["xr"], 2, 9, 3, 8, 10000.0),
                "rope_b": kk.rope(i["xr"], 2, 9, 3, 8, 10000.0, None, True),
                "rope_table": kk.rope_table(9, 8, 10000.0),
                "embed": kk.embed_fwd(i["toks"], i["table"]),
                "fused": kk.fused_map(i["x"], i["y"], None, (0x06 << 16) | (0x13 << 8) | 0x11,
                                      0.25, 3.0)}
    add("elementwise", "mixed", inp, ew)
    return out


def generate() -> list[str]:
    sys.path.insert(0, ROOT)
    from oracle.oracle import reference
    k = reference()
    if k is None:
        raise SystemExit("the reference kernel library cannot be built here")
    rng = np.random.default_rng(20261201)
    written = []
    by_family: dict[str, dict] = {}
    for fam, name, inputs, fn in _cases(k, rng):
        outs = fn(k)
        d = by_family.setdefault(fam, {})
        for key, val in inputs.items():
            d[f"{name}/in/{key}"] = val
        for key, val in outs.items():
            d[f"{name}/out/{key}"] = np.asarray(val)
    for fam, d in by_family.items():
        path = os.path.join(HERE, f"{fam}.npz")
        np.savez_compressed(path, **d)
        written.append(path)
    return written


def replay(orc, z):
    """Yield (name, oracle output, reference output) for every case in z."""
    rng = np.random.default_rng(0)  # inputs come from the file, not from here
    cases = {(fam, name): fn for fam, name, _, fn in _cases(orc, rng)}
    names = sorted({key.split("/")[0] for key in z.files})
    fam = None
    for (f, n) in cases:
        if n in names:
            fam = f
            break
    for name in names:
        inputs = {key.split("/")[2]: z[key] for key in z.files
                  if key.startswith(name + "/in/")}
        fn = cases[(fam, name)]
        got = fn(orc, inputs) if fn.__code__.co_argcount > 1 else fn(orc)
        for key in z.files:
            if key.startswith(name + "/out/"):
                oname = key.split("/")[2]
                yield f"{name}/{oname}", got[oname], z[key]


if __name__ == "__main__":
    for p in generate():
        print(p, os.path.getsize(p))
