"""The gfx950 tile policy on the device (seeai_configure): every arm of every
field gives the same bits, so a kernel-policy table changes time, never
results (the reference's rule for its CPU tiles, tool/autotune.py:24-28);
out-of-range fields are refused with the policy in force unchanged."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

from tests.arena import Arena
from tests.conftest import bits_equal

pytestmark = pytest.mark.gpu

policy = importlib.import_module("see-ai_amd.policy")


def rng(seed):
    return np.random.default_rng(seed)


@pytest.fixture()
def ctx(hip, torch_cuda):
    c = hip.Context(0)
    c.use_torch_stream()
    yield c
    c.close()


def test_configure_defaults_refusals_and_device_key(hip, ctx):
    assert ctx.policy() == policy.DEFAULTS
    ctx.configure({"w8a8_large_kernel": 2, "quantize_waves_per_cu": 8})
    assert ctx.policy() == dict(policy.DEFAULTS, w8a8_large_kernel=2, quantize_waves_per_cu=8)
    for bad in ({"w8a8_large_kernel": 4}, {"exact_longk_first": 3},
                {"quantize_waves_per_cu": 33}):
        with pytest.raises(hip.BackendError, match="tile policy"):
            ctx.configure(bad)
        assert ctx.policy()["w8a8_large_kernel"] == 2  # unchanged
    ctx.configure(None)
    assert ctx.policy() == policy.DEFAULTS
    key = hip.device_key(0)
    arch, name, *rest = key.split(";")
    assert arch.startswith("gfx") and name
    assert [f.split("=")[0] for f in rest] == ["cus", "lds", "l2", "wave"]
    assert hip.device_key(0) == key


@pytest.mark.parametrize("M,N,K", [(2048, 2304, 512), (2100, 2200, 320)])
def test_w8a8_kernel_arms_are_bitwise_equal(hip, ctx, torch_cuda, M, N, K):
    torch = torch_cuda
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    QA = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
    QW = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    sa = torch.rand(M, device="cuda", generator=g)
    sw = torch.rand(N, device="cuda", generator=g)
    outs = []
    arms = [{"w8a8_large_kernel": k, "w8a8_large_min": 2048} for k in (1, 2, 3)] + [None]
    for arm in arms:
        ctx.configure(arm)
        C = torch.full((M, N), float("nan"), device="cuda")
        acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
        ctx.call("seeai_w8a8_gemm", QA.data_ptr(), sa.data_ptr(), QW.data_ptr(), sw.data_ptr(),
                 C.data_ptr(), acc.data_ptr(), M, N, K)
        torch.cuda.synchronize()
        outs.append((C.cpu().numpy(), acc.cpu().numpy()))
    ref = (QA.cpu().numpy().astype(np.int64)[:64] @ QW.cpu().numpy().astype(np.int64).T)
    assert np.array_equal(outs[0][1][:64], ref)
    for arm, (c, a) in zip(arms[1:], outs[1:]):
        assert bits_equal(a, outs[0][1]), arm
        assert bits_equal(c, outs[0][0]), arm


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (4096, 1024), (37, 2052)])
def test_quantizer_wave_counts_are_bitwise_equal(hip, ctx, torch_cuda, rows, cols):
    torch = torch_cuda
    g = torch.Generator(device="cuda").manual_seed(rows * cols)
    X = torch.randn((rows, cols), device="cuda", generator=g) * 3.0
    outs = []
    for w in (1, 4, 32):
        ctx.configure({"quantize_waves_per_cu": w})
        Q = torch.zeros((rows, cols), dtype=torch.int8, device="cuda")
        s = torch.zeros(rows, device="cuda")
        ctx.call("seeai_w8a8_quantize_rows", X.data_ptr(), Q.data_ptr(), s.data_ptr(), rows, cols)
        torch.cuda.synchronize()
        outs.append((Q.cpu().numpy(), s.cpu().numpy()))
    for q, s in outs[1:]:
        assert bits_equal(q, outs[0][0]) and bits_equal(s, outs[0][1])


@pytest.mark.parametrize("nt", [0, 1])
def test_relaxed_tile_arms_are_bitwise_equal(hip, torch_cuda, nt):
    """The relaxed frozen-weight product on 256 x 256, 128 x 192 and 128 x 128
    tiles (K >= 1024: NT takes the direct-to-LDS kernel from there)."""
    M, N, K = 640, 768, 1024
    r = rng(11 + nt)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = r.integers(-127, 128, (N, K) if nt else (K, N)).astype(np.int8)
    sc = r.uniform(1e-3, 5e-2, K if nt else N).astype(np.float32)
    ar = Arena()
    a = ar.add("A", A)
    w, s = ar.add("W", W, rodata=True), ar.add("sc", sc, rodata=True)
    o = ar.empty("C", (M, N))
    from tests.plan_ops import ins
    word = ins(30 if nt else 29, [a, w, o, s], [M, N, K], flags=(1 << 5) | (1 << 4))
    arena, ro = ar.images()
    outs = []
    for arm in ({"relaxed_min_tiles_256": 1}, {"relaxed_min_tiles_256": 1 << 30}, None,
                {"relaxed_min_tiles_256": 1, "relaxed_min_fill_256": 100},
                {"relaxed_min_tiles_256": 1 << 30, "relaxed_tile_192": 2},
                {"relaxed_min_tiles_256": 1 << 30, "relaxed_tile_192": 3},
                {"convert_wgs_per_cu": 1}, {"convert_wgs_per_cu": 64}):
        be = hip.HipBackend(0)
        be.Bind(arena.tobytes(), arena.nbytes, ro.tobytes())
        be.Configure(arm)
        be.Execute(word)
        be.Flush()
        assert be.relaxed_executions() == 1
        outs.append(ar.get(np.frombuffer(be.Download(0, arena.nbytes), np.uint8), "C"))
        be.ctx.close()
    assert np.isfinite(outs[0]).all()
    for c in outs[1:]:
        assert bits_equal(c, outs[0])


def test_exact_longk_arms_are_bitwise_equal(hip, orc, ctx, torch_cuda):
    torch = torch_cuda
    M, N, K = 64, 64, 8192
    r = rng(5)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    outs = []
    for arm in (1, 2):
        ctx.configure({"exact_longk_first": arm})
        C = torch.full((M, N), float("nan"), device="cuda")
        ctx.call("seeai_gemm_f32", 0, dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, None, 0,
                 None, 1.0, 0)
        torch.cuda.synchronize()
        outs.append(C.cpu().numpy())
    assert bits_equal(outs[1], outs[0])
    assert bits_equal(outs[0], orc.gemm_nn(A, B))  # both are the reference's quad order


@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_relaxed_nt_kernel_arms_are_bitwise_equal(hip, torch_cuda, kind):
    """Relaxed NT products below and above relaxed_nt_dma_min_k: the
    register-staged and the direct-to-LDS bf16 kernels give the same bits
    (operands rounded once to bf16, MFMA k-slices in order, the same
    epilogue)."""
    M, N, K = 384, 768, 768
    r = rng(21 + len(kind))
    A = r.standard_normal((M, K)).astype(np.float32)
    if kind == "q8":
        W = r.integers(-127, 128, (N, K)).astype(np.int8)
    else:
        W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    ks = r.uniform(1e-3, 5e-2, K).astype(np.float32)
    ar = Arena()
    a = ar.add("A", A)
    w, s = ar.add("W", W, rodata=True), ar.add("ks", ks, rodata=True)
    o = ar.empty("C", (M, N))
    from tests.plan_ops import ins
    from tests.arena import f32_bits
    if kind == "q8":
        word = ins(30, [a, w, o, s], [M, N, K], flags=(1 << 5) | (1 << 4))
    else:
        word = ins(2, [a, w, o], [M, N, K], flags=1 << 5, imm=f32_bits(0.37))
    arena, ro = ar.images()
    outs = []
    for arm in ({"relaxed_nt_dma_min_k": 512}, {"relaxed_nt_dma_min_k": 1024}):
        be = hip.HipBackend(0)
        be.Bind(arena.tobytes(), arena.nbytes, ro.tobytes())
        be.Configure(arm)
        be.Execute(word)
        be.Flush()
        outs.append(ar.get(np.frombuffer(be.Download(0, arena.nbytes), np.uint8), "C"))
        be.ctx.close()
    assert np.isfinite(outs[0]).all()
    assert bits_equal(outs[1], outs[0])
