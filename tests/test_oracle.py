"""CPU: pin the oracle (oracle/oracle.c) before trusting it.

1. Bit-for-bit against the reference kernel library compiled from
   /root/reference (oracle/_ref) on the reference's ragged shapes -- runs
   where the reference exists (this build host), skipped elsewhere.
2. Bit-for-bit against the golden vectors that library wrote
   (tests/golden/*.npz, made by tests/golden/make_golden.py) -- runs
   everywhere.
3. The reference's own known-answer tests, restated: hand GEMM
   (kernels_test.cc:31-41), uniform logits give log C (:299-308), the xent
   backward is scaled probs minus one-hot (:379-396), AdamW's first step in
   closed form (:541-555) and against a double reference (:557-579),
   single-token attention is V (:1481-1491), RoPE golden angles
   (:1493-1525), and the attention backward against finite differences
   (:1006-1053) -- each chosen so a dropped term, a sign or an index slip
   fails it.
4. The W8A8 pair against definitions: the int32 GEMM against an int64 brute
   force, the quantizer on hand-built rows (ties, clamps, zero rows,
   subnormal maxima).
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

from tests.conftest import ROOT, bits_equal

GOLDEN = os.path.join(ROOT, "tests", "golden")
GEMM_SHAPES = [(1, 1, 1), (3, 5, 7), (4, 4, 4), (5, 9, 3), (67, 129, 66), (130, 257, 63),
               (131, 517, 203), (8, 1100, 300), (2, 700, 900), (257, 33, 64), (66, 131, 65)]


# --- 1. against the compiled reference --------------------------------------------------

@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_family_matches_reference_bits(orc, ref, M, N, K):
    r = np.random.default_rng(M * 131 + N * 7 + K)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    Bt = r.standard_normal((N, K)).astype(np.float32)
    At = r.standard_normal((K, M)).astype(np.float32)
    D = r.standard_normal((M, N)).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    for act in range(4):
        assert bits_equal(orc.gemm_nn(A, B, bias, act, None, 0.7), ref.gemm_nn(A, B, bias, act, None, 0.7))
    assert bits_equal(orc.gemm_nn(A, B, None, 0, D, 2.0), ref.gemm_nn(A, B, None, 0, D, 2.0))
    assert bits_equal(orc.gemm_nt(A, Bt, D, 0.3), ref.gemm_nt(A, Bt, D, 0.3))
    assert bits_equal(orc.gemm_tn(At, B, D, 1.7), ref.gemm_tn(At, B, D, 1.7))
    assert bits_equal(orc.gemm_acc_nn(A, B, D, 2.0), ref.gemm_acc_nn(A, B, D, 2.0))
    Bq = r.integers(-127, 128, (K, N)).astype(np.int8)
    Bqt = r.integers(-127, 128, (N, K)).astype(np.int8)
    cs = r.uniform(0.01, 0.1, N).astype(np.float32)
    ks = r.uniform(0.01, 0.1, K).astype(np.float32)
    assert bits_equal(orc.gemm_nn_q8(A, Bq, 0.02, 1), ref.gemm_nn_q8(A, Bq, 0.02, 1))
    assert bits_equal(orc.gemm_nn_q8(A, Bq, 1.0, 2, cs), ref.gemm_nn_q8(A, Bq, 1.0, 2, cs))
    assert bits_equal(orc.gemm_nt_q8(A, Bqt, 0.02), ref.gemm_nt_q8(A, Bqt, 0.02))
    assert bits_equal(orc.gemm_nt_q8(A, Bqt, 1.0, ks), ref.gemm_nt_q8(A, Bqt, 1.0, ks))
    Bh = (B.view(np.uint32) >> 16).astype(np.uint16)
    Bht = (Bt.view(np.uint32) >> 16).astype(np.uint16)
    assert bits_equal(orc.gemm_nn_bf16(A, Bh, bias, 3), ref.gemm_nn_bf16(A, Bh, bias, 3))
    assert bits_equal(orc.gemm_nt_bf16(A, Bht), ref.gemm_nt_bf16(A, Bht))


@pytest.mark.parametrize("B,S,H,d", [(1, 1, 1, 2), (2, 7, 3, 4), (2, 33, 2, 16), (1, 70, 2, 64)])
def test_attention_matches_reference_bits(orc, ref, B, S, H, d):
    r = np.random.default_rng(S * d)
    n = B * S * H * d
    q, k, v, do = (r.standard_normal(n).astype(np.float32) for _ in range(4))
    toks = r.integers(0, 5, B * S).astype(np.int32)
    starts = orc.segment_starts(toks, B, S, 3)
    assert bits_equal(starts, ref.segment_starts(toks, B, S, 3))
    for st_in in (None, starts):
        o1, s1 = orc.attn_fwd_tiled(q, k, v, B, S, H, d, st_in)
        o2, s2 = ref.attn_fwd_tiled(q, k, v, B, S, H, d, st_in)
        assert bits_equal(o1, o2) and bits_equal(s1, s2)
        dq1, t1 = orc.attn_dq_tiled(q, k, v, do, s1, B, S, H, d)
        dq2, t2 = ref.attn_dq_tiled(q, k, v, do, s2, B, S, H, d)
        assert bits_equal(dq1, dq2) and bits_equal(t1, t2)
        assert bits_equal(orc.attn_dk_tiled(q, k, v, do, t1, B, S, H, d),
                          ref.attn_dk_tiled(q, k, v, do, t2, B, S, H, d))
        assert bits_equal(orc.attn_dv_tiled(q, k, do, t1, B, S, H, d),
                          ref.attn_dv_tiled(q, k, do, t2, B, S, H, d))
        o3, P = orc.attn_fwd(q, k, v, B, S, H, d, st_in)
        o4, P2 = ref.attn_fwd(q, k, v, B, S, H, d, st_in)
        assert bits_equal(o3, o4) and bits_equal(P, P2)
        # The tiled family computes the cached family's bits
        # (kernels_test.cc:1526-1567).
        assert bits_equal(o1, o3)
    dp = orc.attn_dp(do, v, B, S, H, d)
    assert bits_equal(dp, ref.attn_dp(do, v, B, S, H, d))
    ds = orc.softmax_rows_bwd(P, dp)
    assert bits_equal(ds, ref.softmax_rows_bwd(P, dp))
    assert bits_equal(orc.attn_dq(ds, k, B, S, H, d), ref.attn_dq(ds, k, B, S, H, d))
    assert bits_equal(orc.attn_dk(ds, q, B, S, H, d), ref.attn_dk(ds, q, B, S, H, d))
    assert bits_equal(orc.attn_dv(P, do, B, S, H, d), ref.attn_dv(P, do, B, S, H, d))


@pytest.mark.parametrize("N,C", [(1, 1), (2, 4), (32, 256), (300, 1000), (4100, 3)])
def test_losses_match_reference_bits(orc, ref, N, C):
    r = np.random.default_rng(N + C)
    lg = (r.standard_normal((N, C)) * 3).astype(np.float32)
    lb = r.integers(0, C, N).astype(np.int32)
    l1, p1 = orc.xent_fwd(lg, lb)
    l2, p2 = ref.xent_fwd(lg, lb)
    assert bits_equal(np.float32(l1), np.float32(l2)) and bits_equal(p1, p2)
    assert bits_equal(orc.xent_bwd(p1, lb, 1.0), ref.xent_bwd(p1, lb, 1.0))
    lbm = lb.copy()
    lbm[::3] = -1
    l1, p1 = orc.xent_fwd(lg, lbm, True)
    l2, p2 = ref.xent_fwd(lg, lbm, True)
    assert bits_equal(np.float32(l1), np.float32(l2)) and bits_equal(p1, p2)
    assert bits_equal(orc.xent_bwd(p1, lbm, 2.0, True), ref.xent_bwd(p1, lbm, 2.0, True))


@pytest.mark.parametrize("n", [1, 100, 40000, 2000000])
def test_optimizer_matches_reference_bits(orc, ref, n):
    r = np.random.default_rng(n)
    p, g, m, v = (r.standard_normal(n).astype(np.float32) for _ in range(4))
    v = np.abs(v)
    for clip in (0.0, 1.0, 1e6):
        a = orc.adamw_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 3, clip)
        b = ref.adamw_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 3, clip)
        assert a[0] == b[0] and all(bits_equal(x, y) for x, y in zip(a[1:], b[1:]))
    assert bits_equal(orc.clip_norm(g, 1.0)[1], ref.clip_norm(g, 1.0)[1])
    assert bits_equal(np.float32(orc.sqnorm_accum(g, 0.5)), np.float32(ref.sqnorm_accum(g, 0.5)))
    assert bits_equal(orc.clip_global(g, 123.0, 1.0)[1], ref.clip_global(g, 123.0, 1.0)[1])
    assert bits_equal(orc.sgd_step(p, g, 0.1, 0.01, 1.0)[1], ref.sgd_step(p, g, 0.1, 0.01, 1.0)[1])


def test_elementwise_family_matches_reference_bits(orc, ref):
    r = np.random.default_rng(11)
    x = (r.standard_normal(50000) * 4).astype(np.float32)
    y = r.standard_normal(50000).astype(np.float32)
    for nm in ["relu_fwd", "gelu_fwd", "silu_fwd"]:
        assert bits_equal(getattr(orc, nm)(x), getattr(ref, nm)(x)), nm
    for nm in ["relu_bwd", "gelu_bwd", "silu_bwd", "add_ew", "mul_ew"]:
        assert bits_equal(getattr(orc, nm)(y, x), getattr(ref, nm)(y, x)), nm
    X = r.standard_normal((37, 300)).astype(np.float32)
    g = r.standard_normal(300).astype(np.float32)
    b = r.standard_normal(300).astype(np.float32)
    assert bits_equal(orc.add_bias(X, g), ref.add_bias(X, g))
    assert bits_equal(orc.reduce_rows(X), ref.reduce_rows(X))
    for a_, b_ in zip(orc.layernorm_fwd(X, g, b), ref.layernorm_fwd(X, g, b)):
        assert bits_equal(a_, b_)
    _, mu, rs = orc.layernorm_fwd(X, g, b)
    dy = r.standard_normal((37, 300)).astype(np.float32)
    assert bits_equal(orc.layernorm_bwd(dy, X, g, mu, rs), ref.layernorm_bwd(dy, X, g, mu, rs))
    for a_, b_ in zip(orc.rmsnorm_fwd(X, g, 1e-6), ref.rmsnorm_fwd(X, g, 1e-6)):
        assert bits_equal(a_, b_)
    _, rs = orc.rmsnorm_fwd(X, g)
    assert bits_equal(orc.rmsnorm_bwd(dy, X, g, rs), ref.rmsnorm_bwd(dy, X, g, rs))
    xr = r.standard_normal(2 * 9 * 3 * 8).astype(np.float32)
    tab = orc.rope_table(9, 8, 10000.0)
    assert bits_equal(tab, ref.rope_table(9, 8, 10000.0))
    for bw in (0, 1):
        assert bits_equal(orc.rope(xr, 2, 9, 3, 8, 10000.0, None, bw),
                          ref.rope(xr, 2, 9, 3, 8, 10000.0, None, bw))
        # The table path is the recompute path, bit for bit (kernels_test.cc:1621).
        assert bits_equal(orc.rope(xr, 2, 9, 3, 8, 10000.0, tab, bw),
                          orc.rope(xr, 2, 9, 3, 8, 10000.0, None, bw))
    toks = r.integers(0, 50, 77).astype(np.int32)
    table = r.standard_normal((50, 33)).astype(np.float32)
    assert bits_equal(orc.embed_fwd(toks, table), ref.embed_fwd(toks, table))
    for stages in [0x04, 0x11, (0x05 << 8) | 0x11, (0x06 << 16) | (0x13 << 8) | 0x92,
                   (0x04 << 24) | (0x22 << 16) | (0x03 << 8) | 0x05]:
        assert bits_equal(orc.fused_map(x, y, x * 0.5, stages, 0.25, 3.0),
                          ref.fused_map(x, y, x * 0.5, stages, 0.25, 3.0))
    assert bits_equal(orc.accumulate(x, y), ref.accumulate(x, y))
    assert bits_equal(orc.scale(x, 0.3), ref.scale(x, 0.3))


# --- 2. against the committed golden vectors ------------------------------------------------

def golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def test_golden_fixtures_exist():
    assert len(golden_files()) >= 5


@pytest.mark.parametrize("path", golden_files(), ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_golden_vectors(orc, path):
    from tests.golden.make_golden import replay
    z = np.load(path, allow_pickle=False)
    for name, got, want in replay(orc, z):
        assert bits_equal(np.asarray(got), np.asarray(want)), f"{os.path.basename(path)}:{name}"


# --- 3. known-answer tests of the reference, restated ---------------------------------------

def test_gemm_hand_product(orc):
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert np.array_equal(orc.gemm_nn(a, b), [[58, 64], [139, 154]])
    assert np.array_equal(orc.gemm_nt(a, np.ascontiguousarray(b.T)), [[58, 64], [139, 154]])
    assert np.array_equal(orc.gemm_tn(np.ascontiguousarray(a.T), b), [[58, 64], [139, 154]])


def test_gemm_quad_order_is_observable(orc):
    # Catastrophic cancellation makes the NN core's association visible:
    # (1e8*1 + -1e8*1) + 1*1 + ... the k-quad groups four products before
    # touching c; a plain left-to-right chain would lose the small terms.
    A = np.array([[1e8, -1e8, 1.0, 1.0, 1.0]], np.float32)
    B = np.ones((5, 1), np.float32)
    assert orc.gemm_nn(A, B)[0, 0] == np.float32(3.0)
    # NT: lanes k mod 8; the 1e8 / -1e8 pair sits in lanes 0 and 1.
    At = np.array([[1e8, -1e8, 1.0, 1.0]], np.float32)
    assert orc.gemm_nt(At, np.ones((1, 4), np.float32))[0, 0] == np.float32(2.0)


def test_xent_uniform_logits_give_log_c(orc):
    loss, probs = orc.xent_fwd(np.zeros((2, 4), np.float32), np.array([0, 3], np.int32))
    assert abs(loss - np.log(4.0)) < 1e-6
    assert np.allclose(probs, 0.25, atol=1e-6)


def test_xent_backward_is_scaled_probs_minus_onehot(orc):
    probs = np.array([[0.2, 0.3, 0.5], [0.1, 0.8, 0.1]], np.float32)
    dl = orc.xent_bwd(probs, np.array([2, 1], np.int32), 2.0)
    assert abs(dl[0, 0] - 0.2) < 1e-6 and abs(dl[0, 2] - (0.5 - 1.0)) < 1e-6
    assert abs(dl[1, 1] - (0.8 - 1.0)) < 1e-6
    assert np.all(np.abs(dl.sum(1)) < 1e-6)


def test_adamw_first_step_closed_form(orc):
    lr, b1, b2, eps, wd, g0, p0 = 0.01, 0.9, 0.999, 1e-8, 0.1, 0.4, 2.0
    ok, p, m, v = orc.adamw_step([p0], [g0], [0.0], [0.0], lr, b1, b2, eps, wd, 1)
    assert ok
    f = np.float32
    assert abs(m[0] - (f(1) - f(b1)) * f(g0)) < 1e-7
    assert abs(v[0] - (f(1) - f(b2)) * f(g0) * f(g0)) < 1e-9
    assert abs(p[0] - (p0 - lr * (g0 / (np.sqrt(g0 * g0) + eps) + wd * p0))) < 1e-6


def test_adamw_tracks_double_reference(orc):
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.99, 1e-8, 0.01
    p, m, v = np.array([1.5], np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32)
    rp, rm, rv = 1.5, 0.0, 0.0
    for step, gf in [(1, 0.3), (2, -0.2)]:
        ok, p, m, v = orc.adamw_step(p, [gf], m, v, lr, b1, b2, eps, wd, step)
        g = float(np.float32(gf))
        rm = b1 * rm + (1 - b1) * g
        rv = b2 * rv + (1 - b2) * g * g
        mh, vh = rm / (1 - b1 ** step), rv / (1 - b2 ** step)
        rp -= lr * (mh / (np.sqrt(vh) + eps) + wd * rp)
    assert abs(p[0] - rp) < 1e-5


def test_non_finite_gradient_norm_is_refused_untouched(orc):
    g = np.ones(10, np.float32)
    g[3] = np.inf
    ok, p, m, v = orc.adamw_step(np.ones(10), g, np.zeros(10), np.zeros(10), 1e-3, 0.9, 0.999,
                                 1e-8, 0.0, 1, 1.0)
    assert not ok and np.all(p == 1) and not m.any() and not v.any()
    ok, gg = orc.clip_norm(g, 1.0)
    assert not ok and bits_equal(gg, g)
    assert not orc.clip_norm(np.ones(3, np.float32), 0.0)[0]


def test_single_token_attention_is_v(orc):
    r = np.random.default_rng(130)
    B, S, H, d = 2, 1, 2, 3
    q, k, v = (r.standard_normal(B * S * H * d).astype(np.float32) for _ in range(3))
    o, P = orc.attn_fwd(q, k, v, B, S, H, d)
    assert np.all(P == 1.0) and bits_equal(o, v)
    o2, st = orc.attn_fwd_tiled(q, k, v, B, S, H, d)
    assert bits_equal(o2, v) and np.all(st[:, 1] == 1.0)


def test_attention_is_causal_and_matches_naive_softmax(orc):
    r = np.random.default_rng(3)
    B, S, H, d = 1, 6, 2, 4
    q, k, v = (r.standard_normal((B * S, H * d)).astype(np.float32) for _ in range(3))
    o, P = orc.attn_fwd(q, k, v, B, S, H, d)
    P = P.reshape(B, H, S, S)
    assert np.all(np.triu(P[0, 0], 1) == 0)
    for h in range(H):
        qh = q[:, h * d:(h + 1) * d].astype(np.float64)
        kh = k[:, h * d:(h + 1) * d].astype(np.float64)
        vh = v[:, h * d:(h + 1) * d].astype(np.float64)
        s = qh @ kh.T / np.sqrt(d)
        s[np.triu_indices(S, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.allclose(P[0, h], p, atol=1e-6)
        assert np.allclose(o[:, h * d:(h + 1) * d], p @ vh, atol=1e-5)


def test_attention_backward_matches_finite_differences(orc):
    r = np.random.default_rng(21)
    B, S, H, d = 1, 5, 1, 4
    q, k, v = (r.standard_normal((B * S, H * d)).astype(np.float64) for _ in range(3))
    do = r.standard_normal((B * S, H * d))

    def loss(qq, kk, vv):
        o, _ = orc.attn_fwd_tiled(qq, kk, vv, B, S, H, d)
        return float((o.astype(np.float64) * do).sum())

    o, st = orc.attn_fwd_tiled(q, k, v, B, S, H, d)
    dq, st = orc.attn_dq_tiled(q, k, v, do, st, B, S, H, d)
    dk = orc.attn_dk_tiled(q, k, v, do, st, B, S, H, d)
    dv = orc.attn_dv_tiled(q, k, do, st, B, S, H, d)
    eps = 1e-2
    for grad, which in [(dq, 0), (dk, 1), (dv, 2)]:
        for idx in [(0, 0), (2, 1), (4, 3)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            dn = loss(*args)
            fd = (up - dn) / (2 * eps)
            assert abs(fd - grad[idx]) < 2e-2 * max(1.0, abs(fd)), (which, idx, fd, grad[idx])


def test_rope_golden_angles(orc):
    r = np.random.default_rng(72)
    x = r.standard_normal(8).astype(np.float32)
    y = orc.rope(x, 1, 2, 1, 4, 10000.0)
    x1 = x[4:].astype(np.float64)
    for pair, t in [(0, 1.0), (1, 0.01)]:
        a, b = x1[2 * pair], x1[2 * pair + 1]
        assert abs(y[4 + 2 * pair] - (a * np.cos(t) - b * np.sin(t))) < 1e-5
        assert abs(y[4 + 2 * pair + 1] - (a * np.sin(t) + b * np.cos(t))) < 1e-5
    # Backward is the exact adjoint: <R x, y> == <x, R^T y>.
    z = r.standard_normal(8).astype(np.float32)
    lhs = float(np.dot(orc.rope(x, 1, 2, 1, 4, 1e4).astype(np.float64), z))
    rhs = float(np.dot(x.astype(np.float64), orc.rope(z, 1, 2, 1, 4, 1e4, None, True)))
    assert abs(lhs - rhs) < 1e-5


# --- 4. W8A8: definitions -------------------------------------------------------------------

def test_w8a8_gemm_is_the_integer_product(orc):
    r = np.random.default_rng(8)
    for M, N, K in [(1, 1, 1), (5, 9, 7), (33, 65, 300), (64, 64, 4096)]:
        QA = r.integers(-127, 128, (M, K)).astype(np.int8)
        QW = r.integers(-127, 128, (K, N)).astype(np.int8)
        sa = r.uniform(1e-3, 1, M).astype(np.float32)
        sw = r.uniform(1e-3, 1, N).astype(np.float32)
        acc, C = orc.gemm_w8a8(QA, sa, QW, sw)
        want = QA.astype(np.int64) @ QW.astype(np.int64)
        assert np.array_equal(acc.astype(np.int64), want)
        deq = (acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sw[None, :]
        assert bits_equal(C, deq.astype(np.float32))
    # The extreme accumulator: 127^2 * K fits int32 at K = 4096.
    QA = np.full((1, 4096), -127, np.int8)
    acc, _ = orc.gemm_w8a8(QA, np.ones(1, np.float32), np.full((4096, 1), -127, np.int8),
                           np.ones(1, np.float32))
    assert acc[0, 0] == 127 * 127 * 4096


def test_w8a8_quantizer_rule(orc):
    X = np.array([[0.0, 0.0, 0.0, 0.0],
                  [127.0, 63.5, -63.5, -127.0],      # ties round away from zero
                  [1.0, -0.5, 0.25, 2.0],
                  [1e-40, -1e-40, 0.0, 0.0]], np.float32)  # subnormal max -> FLT_MIN scale
    Q, s = orc.quantize_rows(X)
    assert s[0] == 1.0 and not Q[0].any()
    assert s[1] == np.float32(1.0) and list(Q[1]) == [127, 64, -64, -127]
    assert s[2] == np.float32(2.0) / np.float32(127.0)
    assert list(Q[2]) == [64, -32, 16, 127]
    assert s[3] == np.finfo(np.float32).tiny and list(Q[3]) == [0, 0, 0, 0]
    r = np.random.default_rng(1)
    W = r.standard_normal((300, 40)).astype(np.float32)
    Qc, sc = orc.quantize_cols(W)
    Qr, sr = orc.quantize_rows(np.ascontiguousarray(W.T))
    assert bits_equal(Qc.T, Qr) and bits_equal(sc, sr)
    assert np.abs(Qc).max() == 127
