"""ctypes front end of the CPU checkers.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, and only as the checker:
the product path (see-ai_amd/) never imports it.

Two libraries share one signature table:
  * ``liboracle.so``        -- the C restatement (oracle.c), functions ``orc_*``;
  * ``_ref/libseeref.so``   -- the reference kernel library compiled from
    /root/reference with our shim (ref_shim.cc), functions ``ref_*``; built
    only where the reference exists (never on the GPU box).

``Kernels(lib, prefix)`` exposes each kernel as a numpy-friendly method that
allocates its outputs, so a test reads ``orc.gemm_nn(A, B)`` and compares the
result with ``ref.gemm_nn(A, B)`` or with the HIP library's.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libseeref.so")
REFERENCE_ROOT = "/root/reference"

_P = C.c_void_p
_Z = C.c_size_t
_F = C.c_float
_I = C.c_int
_U64 = C.c_uint64
_I32 = C.c_int32

# name -> (restype, argtypes); identical for orc_* and ref_*.
SIGS = {
    "gemm_nn": (None, [_P, _P, _P, _Z, _Z, _Z, _P, _I, _P, _F]),
    "gemm_nt": (None, [_P, _P, _P, _Z, _Z, _Z, _P, _F]),
    "gemm_tn": (None, [_P, _P, _P, _Z, _Z, _Z, _P, _F]),
    "gemm_acc_nn": (None, [_P, _P, _P, _Z, _Z, _Z, _F]),
    "gemm_nn_q8": (None, [_P, _P, _P, _Z, _Z, _Z, _F, _I, _P]),
    "gemm_nt_q8": (None, [_P, _P, _P, _Z, _Z, _Z, _F, _P]),
    "gemm_nn_bf16": (None, [_P, _P, _P, _Z, _Z, _Z, _P, _I]),
    "gemm_nt_bf16": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "add_ew": (None, [_P, _P, _P, _Z]),
    "mul_ew": (None, [_P, _P, _P, _Z]),
    "add_bias": (None, [_P, _P, _P, _Z, _Z]),
    "relu_fwd": (None, [_P, _P, _Z]),
    "relu_bwd": (None, [_P, _P, _P, _Z]),
    "gelu_fwd": (None, [_P, _P, _Z]),
    "gelu_bwd": (None, [_P, _P, _P, _Z]),
    "silu_fwd": (None, [_P, _P, _Z]),
    "silu_bwd": (None, [_P, _P, _P, _Z]),
    "scale": (None, [_P, _P, _F, _Z]),
    "reduce_rows": (None, [_P, _P, _Z, _Z]),
    "accumulate": (None, [_P, _P, _Z]),
    "embed_fwd": (None, [_P, _P, _P, _Z, _Z]),
    "fused_map": (None, [_P, _P, _P, _P, _Z, _U64, _F, _F]),
    "layernorm_fwd": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z, _F]),
    "layernorm_bwd": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z]),
    "rmsnorm_fwd": (None, [_P, _P, _P, _P, _Z, _Z, _F]),
    "rmsnorm_bwd": (None, [_P, _P, _P, _P, _P, _Z, _Z]),
    "rope": (None, [_P, _P, _Z, _Z, _Z, _Z, _F, _P, _I]),
    "rope_table": (None, [_P, _Z, _Z, _F]),
    "segment_starts": (None, [_P, _P, _Z, _Z, _I32]),
    "attn_fwd": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _P]),
    "attn_dp": (None, [_P, _P, _P, _Z, _Z, _Z, _Z]),
    "attn_dv": (None, [_P, _P, _P, _Z, _Z, _Z, _Z]),
    "softmax_rows_bwd": (None, [_P, _P, _P, _Z, _Z]),
    "attn_dq": (None, [_P, _P, _P, _Z, _Z, _Z, _Z]),
    "attn_dk": (None, [_P, _P, _P, _Z, _Z, _Z, _Z]),
    "attn_fwd_tiled": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _P]),
    "attn_dq_tiled": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z, _Z]),
    "attn_dk_tiled": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z, _Z]),
    "attn_dv_tiled": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z]),
    "xent_fwd": (None, [_P, _P, _P, _P, _Z, _Z]),
    "xent_bwd": (None, [_P, _P, _P, _P, _Z, _Z]),
    "xent_masked_fwd": (None, [_P, _P, _P, _P, _Z, _Z]),
    "xent_masked_bwd": (None, [_P, _P, _P, _P, _Z, _Z]),
    "clip_norm": (_I, [_P, _Z, _F]),
    "sqnorm_accum": (None, [_P, _Z, _P]),
    "clip_global": (_I, [_P, _Z, _P, _F]),
    "sgd_step": (_I, [_P, _P, _Z, _F, _F, _F]),
    "adamw_step": (_I, [_P, _P, _P, _P, _Z, _F, _F, _F, _F, _F, _U64, _F]),
    "plan_self_hash": (_U64, [_P, _Z, _Z]),
}
# Oracle-only entry points (no reference counterpart or engine-side code).
ORACLE_ONLY = {
    "quantize_rows": (None, [_P, _P, _P, _Z, _Z]),
    "quantize_cols": (None, [_P, _P, _P, _Z, _Z]),
    "gemm_w8a8": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z]),
    "argmax_rows": (None, [_P, _Z, _Z, _P]),
    "argmax_tally": (None, [_P, _P, _Z, _Z, _P, _P]),
    "adamw_bias_corrections": (None, [_F, _F, _U64, _P, _P]),
    "execute": (_I, [_P, _P, _P, _P]),
    "execute_src": (_I, [_P, _P, _P, _P, _P]),
    "set_threads": (None, [_I]),
    "threads": (_I, []),
    "pool_stop": (None, []),
    "chunk_grain": (_Z, [_Z, _Z]),
    "chunk_count": (_Z, [_Z, _Z]),
}


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref where /root/reference exists)."""
    targets = ["oracle"]
    if ref and os.path.isdir(REFERENCE_ROOT):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def _ptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(C.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OrcStepParams(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("eps", C.c_float), ("weight_decay", C.c_float),
                ("pad", C.c_uint32), ("step", C.c_uint64)]


class Kernels:
    """numpy front end over one of the two libraries."""

    def __init__(self, path: str, prefix: str):
        self.lib = C.CDLL(path)
        self.prefix = prefix
        table = dict(SIGS)
        if prefix == "orc_":
            table.update(ORACLE_ONLY)
        for name, (res, args) in table.items():
            fn = getattr(self.lib, prefix + name)
            fn.restype = res
            fn.argtypes = args
        if prefix == "ref_":
            self.lib.ref_set_threads.argtypes = [_Z]
            self.lib.ref_set_threads.restype = None

    def _fn(self, name):
        return getattr(self.lib, self.prefix + name)

    # --- GEMM family ---------------------------------------------------------
    def gemm_nn(self, A, B, bias=None, act=0, addend=None, alpha=1.0):
        A, B = f32(A), f32(B)
        M, K = A.shape
        N = B.shape[1]
        Cm = np.empty((M, N), np.float32)
        bias = None if bias is None else f32(bias)
        addend = None if addend is None else f32(addend)
        self._fn("gemm_nn")(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, _ptr(bias), act,
                            _ptr(addend), alpha)
        return Cm

    def gemm_nt(self, A, B, addend=None, alpha=1.0):
        A, B = f32(A), f32(B)
        M, K = A.shape
        N = B.shape[0]
        Cm = np.empty((M, N), np.float32)
        addend = None if addend is None else f32(addend)
        self._fn("gemm_nt")(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, _ptr(addend), alpha)
        return Cm

    def gemm_tn(self, A, B, addend=None, alpha=1.0):
        A, B = f32(A), f32(B)
        K, M = A.shape
        N = B.shape[1]
        Cm = np.empty((M, N), np.float32)
        addend = None if addend is None else f32(addend)
        self._fn("gemm_tn")(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, _ptr(addend), alpha)
        return Cm

    def gemm_acc_nn(self, A, B, Cin, alpha):
        A, B = f32(A), f32(B)
        Cm = f32(Cin).copy()
        M, K = A.shape
        N = B.shape[1]
        self._fn("gemm_acc_nn")(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, alpha)
        return Cm

    def gemm_nn_q8(self, A, Bq, scale=1.0, act=0, col_scale=None):
        A = f32(A)
        Bq = np.ascontiguousarray(Bq, np.int8)
        M, K = A.shape
        N = Bq.shape[1]
        Cm = np.empty((M, N), np.float32)
        cs = None if col_scale is None else f32(col_scale)
        self._fn("gemm_nn_q8")(_ptr(A), _ptr(Bq), _ptr(Cm), M, N, K, scale, act, _ptr(cs))
        return Cm

    def gemm_nt_q8(self, A, Bq, scale=1.0, k_scale=None):
        A = f32(A)
        Bq = np.ascontiguousarray(Bq, np.int8)
        M, K = A.shape
        N = Bq.shape[0]
        Cm = np.empty((M, N), np.float32)
        ks = None if k_scale is None else f32(k_scale)
        self._fn("gemm_nt_q8")(_ptr(A), _ptr(Bq), _ptr(Cm), M, N, K, scale, _ptr(ks))
        return Cm

    def gemm_nn_bf16(self, A, Bh, bias=None, act=0):
        A = f32(A)
        Bh = np.ascontiguousarray(Bh, np.uint16)
        M, K = A.shape
        N = Bh.shape[1]
        Cm = np.empty((M, N), np.float32)
        bias = None if bias is None else f32(bias)
        self._fn("gemm_nn_bf16")(_ptr(A), _ptr(Bh), _ptr(Cm), M, N, K, _ptr(bias), act)
        return Cm

    def gemm_nt_bf16(self, A, Bh):
        A = f32(A)
        Bh = np.ascontiguousarray(Bh, np.uint16)
        M, K = A.shape
        N = Bh.shape[0]
        Cm = np.empty((M, N), np.float32)
        self._fn("gemm_nt_bf16")(_ptr(A), _ptr(Bh), _ptr(Cm), M, N, K)
        return Cm

    # --- W8A8 (oracle only) ----------------------------------------------------
    def quantize_rows(self, X):
        X = f32(X)
        r, c = X.shape
        Q = np.empty((r, c), np.int8)
        s = np.empty(r, np.float32)
        self._fn("quantize_rows")(_ptr(X), _ptr(Q), _ptr(s), r, c)
        return Q, s

    def quantize_cols(self, W):
        W = f32(W)
        K, N = W.shape
        Q = np.empty((K, N), np.int8)
        s = np.empty(N, np.float32)
        self._fn("quantize_cols")(_ptr(W), _ptr(Q), _ptr(s), K, N)
        return Q, s

    def gemm_w8a8(self, QA, sa, QW, sw):
        QA = np.ascontiguousarray(QA, np.int8)
        QW = np.ascontiguousarray(QW, np.int8)
        sa, sw = f32(sa), f32(sw)
        M, K = QA.shape
        N = QW.shape[1]
        acc = np.empty((M, N), np.int32)
        Cm = np.empty((M, N), np.float32)
        self._fn("gemm_w8a8")(_ptr(QA), _ptr(sa), _ptr(QW), _ptr(sw), _ptr(acc),
                              _ptr(Cm), M, N, K)
        return acc, Cm

    # --- elementwise ------------------------------------------------------------
    def _unary(self, name, x):
        x = f32(x)
        out = np.empty_like(x)
        self._fn(name)(_ptr(x), _ptr(out), x.size)
        return out

    def _binary(self, name, x, y):
        x, y = f32(x), f32(y)
        out = np.empty_like(x)
        self._fn(name)(_ptr(x), _ptr(y), _ptr(out), x.size)
        return out

    def add_ew(self, x, y): return self._binary("add_ew", x, y)
    def mul_ew(self, x, y): return self._binary("mul_ew", x, y)
    def relu_fwd(self, x): return self._unary("relu_fwd", x)
    def gelu_fwd(self, x): return self._unary("gelu_fwd", x)
    def silu_fwd(self, x): return self._unary("silu_fwd", x)
    def relu_bwd(self, dy, x): return self._binary("relu_bwd", dy, x)
    def gelu_bwd(self, dy, x): return self._binary("gelu_bwd", dy, x)
    def silu_bwd(self, dy, x): return self._binary("silu_bwd", dy, x)

    def scale(self, x, alpha):
        x = f32(x)
        out = np.empty_like(x)
        self._fn("scale")(_ptr(x), _ptr(out), alpha, x.size)
        return out

    def add_bias(self, x, b):
        x, b = f32(x), f32(b)
        out = np.empty_like(x)
        self._fn("add_bias")(_ptr(x), _ptr(b), _ptr(out), x.shape[0], x.shape[1])
        return out

    def reduce_rows(self, dy):
        dy = f32(dy)
        db = np.empty(dy.shape[1], np.float32)
        self._fn("reduce_rows")(_ptr(dy), _ptr(db), dy.shape[0], dy.shape[1])
        return db

    def accumulate(self, dst, src):
        dst = f32(dst).copy()
        src = f32(src)
        self._fn("accumulate")(_ptr(dst), _ptr(src), dst.size)
        return dst

    def embed_fwd(self, tokens, table):
        tokens = np.ascontiguousarray(tokens, np.int32)
        table = f32(table)
        out = np.empty((tokens.size, table.shape[1]), np.float32)
        self._fn("embed_fwd")(_ptr(tokens), _ptr(table), _ptr(out), tokens.size,
                              table.shape[1])
        return out

    def fused_map(self, x, o1, o2, stages, imm0=0.0, imm1=0.0):
        x = f32(x)
        o1 = None if o1 is None else f32(o1)
        o2 = None if o2 is None else f32(o2)
        out = np.empty_like(x)
        self._fn("fused_map")(_ptr(x), _ptr(o1), _ptr(o2), _ptr(out), x.size, stages,
                              imm0, imm1)
        return out

    def layernorm_fwd(self, x, g, b, eps=1e-5):
        x, g, b = f32(x), f32(g), f32(b)
        r, c = x.shape
        y = np.empty_like(x)
        mean = np.empty(r, np.float32)
        rstd = np.empty(r, np.float32)
        self._fn("layernorm_fwd")(_ptr(x), _ptr(g), _ptr(b), _ptr(y), _ptr(mean),
                                  _ptr(rstd), r, c, eps)
        return y, mean, rstd

    def layernorm_bwd(self, dy, x, g, mean, rstd):
        dy, x, g, mean, rstd = map(f32, (dy, x, g, mean, rstd))
        dx = np.empty_like(x)
        self._fn("layernorm_bwd")(_ptr(dy), _ptr(x), _ptr(g), _ptr(mean), _ptr(rstd),
                                  _ptr(dx), x.shape[0], x.shape[1])
        return dx

    def rmsnorm_fwd(self, x, g, eps=1e-5):
        x, g = f32(x), f32(g)
        r, c = x.shape
        y = np.empty_like(x)
        rstd = np.empty(r, np.float32)
        self._fn("rmsnorm_fwd")(_ptr(x), _ptr(g), _ptr(y), _ptr(rstd), r, c, eps)
        return y, rstd

    def rmsnorm_bwd(self, dy, x, g, rstd):
        dy, x, g, rstd = map(f32, (dy, x, g, rstd))
        dx = np.empty_like(x)
        self._fn("rmsnorm_bwd")(_ptr(dy), _ptr(x), _ptr(g), _ptr(rstd), _ptr(dx),
                                x.shape[0], x.shape[1])
        return dx

    def rope(self, x, B, S, H, d, base, table=None, backward=False):
        x = f32(x)
        y = np.empty_like(x)
        table = None if table is None else f32(table)
        self._fn("rope")(_ptr(x), _ptr(y), B, S, H, d, base, _ptr(table), int(backward))
        return y

    def rope_table(self, S, d, base):
        t = np.empty((S, d // 2, 2), np.float32)
        self._fn("rope_table")(_ptr(t), S, d, base)
        return t

    # --- attention ----------------------------------------------------------------
    def segment_starts(self, tokens, B, S, eos):
        tokens = np.ascontiguousarray(tokens, np.int32)
        starts = np.empty(B * S, np.int32)
        self._fn("segment_starts")(_ptr(tokens), _ptr(starts), B, S, eos)
        return starts

    def attn_fwd(self, q, k, v, B, S, H, d, starts=None):
        q, k, v = f32(q), f32(k), f32(v)
        o = np.empty_like(q)
        p = np.empty((B * H * S, S), np.float32)
        st = None if starts is None else np.ascontiguousarray(starts, np.int32)
        self._fn("attn_fwd")(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(p), B, S, H, d,
                             _ptr(st))
        return o, p

    def attn_fwd_tiled(self, q, k, v, B, S, H, d, starts=None):
        q, k, v = f32(q), f32(k), f32(v)
        o = np.empty_like(q)
        stats = np.empty((B * H * S, 4), np.float32)
        st = None if starts is None else np.ascontiguousarray(starts, np.int32)
        self._fn("attn_fwd_tiled")(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(stats), B,
                                   S, H, d, _ptr(st))
        return o, stats

    def attn_dq_tiled(self, q, k, v, dout, stats, B, S, H, d):
        q, k, v, dout = map(f32, (q, k, v, dout))
        stats = f32(stats).copy()
        dq = np.empty_like(q)
        self._fn("attn_dq_tiled")(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(stats),
                                  _ptr(dq), B, S, H, d)
        return dq, stats

    def attn_dk_tiled(self, q, k, v, dout, stats, B, S, H, d):
        q, k, v, dout, stats = map(f32, (q, k, v, dout, stats))
        dk = np.empty_like(k)
        self._fn("attn_dk_tiled")(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(stats),
                                  _ptr(dk), B, S, H, d)
        return dk

    def attn_dv_tiled(self, q, k, dout, stats, B, S, H, d):
        q, k, dout, stats = map(f32, (q, k, dout, stats))
        dv = np.empty_like(q)
        self._fn("attn_dv_tiled")(_ptr(q), _ptr(k), _ptr(dout), _ptr(stats), _ptr(dv), B,
                                  S, H, d)
        return dv

    def attn_dp(self, dout, v, B, S, H, d):
        dout, v = f32(dout), f32(v)
        dp = np.empty((B * H * S, S), np.float32)
        self._fn("attn_dp")(_ptr(dout), _ptr(v), _ptr(dp), B, S, H, d)
        return dp

    def attn_dv(self, p, dout, B, S, H, d):
        p, dout = f32(p), f32(dout)
        dv = np.empty_like(dout)
        self._fn("attn_dv")(_ptr(p), _ptr(dout), _ptr(dv), B, S, H, d)
        return dv

    def softmax_rows_bwd(self, p, dp):
        p, dp = f32(p), f32(dp)
        ds = np.empty_like(p)
        self._fn("softmax_rows_bwd")(_ptr(p), _ptr(dp), _ptr(ds), p.shape[0], p.shape[1])
        return ds

    def attn_dq(self, ds, k, B, S, H, d):
        ds, k = f32(ds), f32(k)
        dq = np.empty_like(k)
        self._fn("attn_dq")(_ptr(ds), _ptr(k), _ptr(dq), B, S, H, d)
        return dq

    def attn_dk(self, ds, q, B, S, H, d):
        ds, q = f32(ds), f32(q)
        dk = np.empty_like(q)
        self._fn("attn_dk")(_ptr(ds), _ptr(q), _ptr(dk), B, S, H, d)
        return dk

    # --- losses ---------------------------------------------------------------------
    def xent_fwd(self, logits, labels, masked=False):
        logits = f32(logits)
        labels = np.ascontiguousarray(labels, np.int32)
        N, Cn = logits.shape
        probs = np.empty_like(logits)
        loss = np.zeros(1, np.float32)
        self._fn("xent_masked_fwd" if masked else "xent_fwd")(
            _ptr(logits), _ptr(labels), _ptr(loss), _ptr(probs), N, Cn)
        return loss[0], probs

    def xent_bwd(self, probs, labels, seed=1.0, masked=False):
        probs = f32(probs)
        labels = np.ascontiguousarray(labels, np.int32)
        s = np.array([seed], np.float32)
        dl = np.empty_like(probs)
        self._fn("xent_masked_bwd" if masked else "xent_bwd")(
            _ptr(probs), _ptr(labels), _ptr(s), _ptr(dl), probs.shape[0], probs.shape[1])
        return dl

    # --- optimizer ------------------------------------------------------------------
    def adamw_step(self, p, g, m, v, lr, b1, b2, eps, wd, step, clip=0.0):
        p, m, v = f32(p).copy(), f32(m).copy(), f32(v).copy()
        g = f32(g)
        ok = self._fn("adamw_step")(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.size, lr, b1, b2,
                                    eps, wd, step, clip)
        return bool(ok), p, m, v

    def sgd_step(self, p, g, lr, wd, clip=0.0):
        p = f32(p).copy()
        g = f32(g)
        ok = self._fn("sgd_step")(_ptr(p), _ptr(g), p.size, lr, wd, clip)
        return bool(ok), p

    def clip_norm(self, g, mx):
        g = f32(g).copy()
        ok = self._fn("clip_norm")(_ptr(g), g.size, mx)
        return bool(ok), g

    def sqnorm_accum(self, g, acc0=0.0):
        g = f32(g)
        acc = np.array([acc0], np.float32)
        self._fn("sqnorm_accum")(_ptr(g), g.size, _ptr(acc))
        return acc[0]

    def clip_global(self, g, acc, mx):
        g = f32(g).copy()
        a = np.array([acc], np.float32)
        ok = self._fn("clip_global")(_ptr(g), g.size, _ptr(a), mx)
        return bool(ok), g

    # --- oracle-only ----------------------------------------------------------------
    def argmax_rows(self, probs):
        probs = f32(probs)
        out = np.empty(probs.shape[0], np.int32)
        self._fn("argmax_rows")(_ptr(probs), probs.shape[0], probs.shape[1], _ptr(out))
        return out

    def set_threads(self, n: int):
        """Threads for the chunked loops; the bits do not depend on it."""
        self._fn("set_threads")(int(n))

    def threads(self) -> int:
        return int(self._fn("threads")())

    def pool_stop(self):
        """Ends the worker threads; a later threaded call starts new ones."""
        self._fn("pool_stop")()

    def argmax_tally(self, probs, labels):
        """(hits, judged rows) over rows whose label is not -1
        (update_engine.cc:537-565)."""
        probs = f32(probs)
        labels = np.ascontiguousarray(labels, np.int32)
        hits = np.zeros(1, np.uint64)
        judged = np.zeros(1, np.uint64)
        self._fn("argmax_tally")(_ptr(probs), _ptr(labels), probs.shape[0], probs.shape[1],
                                 _ptr(hits), _ptr(judged))
        return int(hits[0]), int(judged[0])

    def adamw_bias_corrections(self, b1, b2, step):
        a = np.zeros(1, np.float32)
        b = np.zeros(1, np.float32)
        self._fn("adamw_bias_corrections")(b1, b2, step, _ptr(a), _ptr(b))
        return float(a[0]), float(b[0])

    def plan_self_hash(self, blob, hash_offset: int = 216) -> int:
        buf = np.frombuffer(bytes(blob), np.uint8)
        return int(self._fn("plan_self_hash")(_ptr(buf), buf.size, hash_offset))

    def execute(self, ins_bytes: bytes, arena: np.ndarray, rodata: np.ndarray, params,
                source: np.ndarray | None = None):
        """One instruction (cpu_backend.cc:260-646); `source` is the source
        model file's image that bit-62 refs read (none bound: status 3)."""
        buf = C.create_string_buffer(bytes(ins_bytes), 64)
        sp = OrcStepParams(*params[:5], 0, params[5])
        if source is None:
            return self._fn("execute")(buf, _ptr(arena), _ptr(rodata), C.byref(sp))
        return self._fn("execute_src")(buf, _ptr(arena), _ptr(rodata), _ptr(source), C.byref(sp))


_cache: dict = {}


def oracle() -> Kernels:
    """The C restatement (always available once built)."""
    if "orc" not in _cache:
        if not os.path.exists(ORACLE_SO):
            build(ref=False)
        _cache["orc"] = Kernels(ORACLE_SO, "orc_")
    return _cache["orc"]


def reference():
    """The compiled reference kernel library, or None where it cannot exist."""
    if "ref" not in _cache:
        lib = None
        if not os.path.exists(REF_SO) and os.path.isdir(REFERENCE_ROOT):
            try:
                build(ref=True)
            except Exception:  # noqa: BLE001 -- absence is reported as None
                pass
        if os.path.exists(REF_SO):
            lib = Kernels(REF_SO, "ref_")
        _cache["ref"] = lib
    return _cache["ref"]
