"""CPU: the .seeu plan container -- the self-hash against the reference's
own PlanSelfHash, the plan writer's config-1 program against the reference
compiler's listing, the loader's header contract with the reference's
refusal strings, and one interpreted step of the plan through the oracle."""
from __future__ import annotations

import importlib
import math
import struct

import numpy as np
import pytest

from tests.engine_oracle import OracleEngine, effective_lr

pw = importlib.import_module("see-ai_amd.planwriter")


@pytest.fixture(scope="module")
def c1(hip):
    return pw.mlp_lora(hip.plan_self_hash)


# --- PlanSelfHash (source/identity/hash.h:136-158) ------------------------------------------------

SIZES = [0, 1, 7, 8, 9, 216, 223, 224, 225, (1 << 20) - 1, 1 << 20, (1 << 20) + 1,
         3 * (1 << 20) + 5]


@pytest.mark.parametrize("n", SIZES)
def test_self_hash_matches_the_reference(hip, orc, ref, n):
    blob = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    want = ref.plan_self_hash(blob)
    assert orc.plan_self_hash(blob) == want
    assert hip.plan_self_hash(blob) == want


def test_self_hash_beyond_256_chunks(hip, orc):
    # Past 256 MiB the chunk grows so that there are at most 256 chunks
    # (parallel_for.h:55-59); the hash field sits in the first chunk.
    n = 256 * (1 << 20) + 4097
    blob = np.random.default_rng(1).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert hip.plan_self_hash(blob) == orc.plan_self_hash(blob)


def test_self_hash_reads_the_hash_field_as_zero(hip, orc):
    blob = bytearray(np.random.default_rng(5).integers(0, 256, 4096, dtype=np.uint8).tobytes())
    h0 = hip.plan_self_hash(bytes(blob))
    blob[216:224] = b"\xff" * 8
    assert hip.plan_self_hash(bytes(blob)) == h0
    blob[224] ^= 1
    assert hip.plan_self_hash(bytes(blob)) != h0


def test_fnv_known_answers(orc):
    # FNV-1a 64 of "" and "a" (the published test vectors) are the first
    # lane's building block: a one-byte blob's chain 0 is FNV-1a("a") with
    # chain 0's seed, so check the seed algebra on the empty blob instead:
    # with no bytes every chain keeps its seed.
    basis, prime = 0xcbf29ce484222325, 0x100000001b3

    def fnv_word(h, w):
        for b in range(8):
            h ^= (w >> (8 * b)) & 0xff
            h = (h * prime) & (2 ** 64 - 1)
        return h
    assert fnv_word(basis, 0) != basis
    lanes = [basis ^ ((0x9E3779B97F4A7C15 * (l + 1)) & (2 ** 64 - 1)) for l in range(8)]
    h = basis
    for v in lanes:
        h = fnv_word(h, v)
    striped_empty = fnv_word(h, 0)
    assert orc.plan_self_hash(b"", 0) == fnv_word(fnv_word(basis, striped_empty), 0)
    # FNV-1a("a") = 0xaf63dc4c8601ec8c (published), the loop the lanes run.
    x = (basis ^ 0x61) * prime & (2 ** 64 - 1)
    assert x == 0xaf63dc4c8601ec8c


# --- the config-1 plan (SURVEY Appendix B layout) --------------------------------------------------

def test_c1_plan_matches_the_reference_listing(c1):
    h = c1.header
    assert h["magic"] == 0x55454553 and h["version"] == 26
    assert (h["train_instr_count"], h["eval_instr_count"], h["merge_instr_count"]) == (25, 10, 4)
    assert h["persistent_size"] == 147456
    assert h["rodata_size"] == 1051648
    assert h["input_ref"] == 0x24000 and h["input_floats"] == 8192
    assert h["label_ref"] == 0x2C000 and h["label_bytes"] == 128 and h["label_kind"] == 1
    assert h["loss_ref"] == 0x2C080
    assert h["rodata_offset"] % 4096 == 0
    ops = [struct.unpack_from("<H", w)[0] for w in c1.train]
    assert ops == [1, 1, 1, 6, 7, 1, 1, 1, 6, 11, 19, 12, 2, 3, 3, 2, 2, 8, 2, 3, 3, 18, 18, 18, 18]
    dims = [struct.unpack_from("<3Q", w, 40) for w in c1.train[:21]]
    assert dims[0] == (32, 512, 256) and dims[2] == (32, 512, 8) and dims[13] == (8, 256, 32)
    assert dims[14] == (512, 8, 32) and dims[16] == (32, 512, 8) and dims[20] == (256, 8, 32)
    counts = [struct.unpack_from("<Q", w, 40)[0] for w in c1.train[21:]]
    assert counts == [2048, 4096, 4096, 2048]
    alpha = [struct.unpack_from("<I", w, 4)[0] for w in c1.train]
    two = pw.f32_bits(2.0)
    assert [i for i, a in enumerate(alpha) if a == two] == [2, 7, 12, 13, 18, 19]
    assert c1.eval == c1.train[:10]
    mops = [struct.unpack_from("<H", w)[0] for w in c1.merge]
    assert mops == [19, 4, 19, 4]


def test_c1_plan_is_accepted(hip, c1):
    assert hip.plan_check(c1.blob) == ""


# --- the loader's header contract (plan_loader.cc:19-49, plan_contract.h:35-180) -------------------

def reseal(hip, blob: bytearray) -> bytes:
    blob[216:224] = b"\0" * 8
    blob[216:224] = struct.pack("<Q", hip.plan_self_hash(bytes(blob)))
    return bytes(blob)


def patched(hip, c1, **fields) -> bytes:
    h = dict(c1.header)
    h.update(fields)
    blob = bytearray(c1.blob)
    blob[:320] = pw.pack_header(h)
    return reseal(hip, blob)


def test_refusals(hip, c1):
    assert hip.plan_check(c1.blob[:100]) == "plan smaller than its header"
    assert hip.plan_check(patched(hip, c1, magic=0x12345678)) == "bad plan magic"
    assert hip.plan_check(patched(hip, c1, version=3)) == \
        "unsupported plan version 3 (this runtime reads v4..v26)"
    assert hip.plan_check(patched(hip, c1, version=27)).startswith("unsupported plan version 27")
    corrupt = bytearray(c1.blob)
    corrupt[-1] ^= 0x40
    assert hip.plan_check(bytes(corrupt)) == "plan hash mismatch — the .seeu blob is corrupt"
    assert hip.plan_check(patched(hip, c1, train_instr_count=10 ** 6)) == \
        "plan section out of bounds"
    assert hip.plan_check(patched(hip, c1, train_instr_count=2 ** 60)) == \
        "plan section size overflows"
    assert hip.plan_check(patched(hip, c1, rodata_offset=c1.header["rodata_offset"] + 4)) == \
        "rodata section is not 16-byte aligned"
    assert hip.plan_check(patched(hip, c1, batch=0)) == "plan batch size is zero"
    assert hip.plan_check(patched(hip, c1, lr=float("nan"))) == \
        "plan header lr is not a finite value in its range"
    assert hip.plan_check(patched(hip, c1, beta2=1.0)) == \
        "plan header beta2 is not a finite value in its range"
    assert hip.plan_check(patched(hip, c1, persistent_size=10 ** 9)) == \
        "persistent segment exceeds arena"
    assert hip.plan_check(patched(hip, c1, input_ref=c1.header["arena_size"])) == \
        "plan input slot out of bounds"
    assert hip.plan_check(patched(hip, c1, loss_ref=(1 << 63) | 64)) == \
        "plan loss slot out of bounds"
    assert hip.plan_check(patched(hip, c1, grad_accum_steps=2)) == \
        "plan step program presence disagrees with grad_accum_steps"
    assert hip.plan_check(patched(hip, c1, gemm_tile_k=6)) == \
        "plan gemm_tile_k 6 is not a multiple of the kernel's 4-wide unroll"


# --- one interpreted step through the oracle --------------------------------------------------------

def test_c1_first_step_loss_is_log_classes(orc, c1):
    # B = 0 makes every LoRA branch zero and the base weights are small, so
    # the first loss sits near log(256) (the reference's uniform-logit KAT).
    eng = OracleEngine(orc, c1.blob)
    x = pw.normal(7, (32, 256))
    y = pw.uniform_ints(8, 32, 256)
    loss = eng.train_step(x, y)
    assert abs(loss - math.log(256)) < 0.05
    # AdamW step 1 moves a B element by lr * |g| / (|g| + eps): by lr where
    # the gradient is well above eps, never by more.
    off, nb = c1.arena["B1"]
    B1 = np.abs(np.frombuffer(eng.read(off, nb), np.float32))
    assert np.median(B1) == pytest.approx(1e-3, rel=1e-3)
    assert B1.max() <= 1e-3 * (1 + 1e-5)


def test_effective_lr_schedule():
    h = {"lr": 1e-3, "lr_schedule": 1, "warmup_steps": 10, "default_steps": 110,
         "min_lr_factor": 0.1}
    assert effective_lr(h, 5, 0) == pytest.approx(5e-4)
    assert effective_lr(h, 10, 0) == pytest.approx(1e-3)
    assert effective_lr(h, 60, 0) == pytest.approx(1e-4 + 0.9e-3 * 0.5, rel=1e-6)
    assert effective_lr(h, 110, 0) == pytest.approx(1e-4)
    assert effective_lr({**h, "lr_schedule": 0}, 60, 0) == pytest.approx(1e-3)


# --- the decoder plan (BASELINE configs[3] at a small shape) -----------------------------------------

TINY = dict(vocab=96, dim=128, heads=2, ffn=256, layers=2, seq=64, batch=2, rank=8)


@pytest.fixture(scope="module")
def dec(hip):
    return pw.decoder_lora(hip.plan_self_hash, **TINY)


def test_decoder_plan_structure(hip, dec):
    assert hip.plan_check(dec.blob) == ""
    h = dec.header
    assert h["input_kind"] == 1 and h["seq_len"] == 64 and h["batch"] == 128
    ops = [struct.unpack_from("<HH", w) for w in dec.train]
    opc = [o for o, _ in ops]
    # per block: 1 LoRA site pair each on Q and V = 3 GEMMs forward each,
    # and the tiled attention forward; the backward's dK only above block 0
    assert opc.count(47) == 2 and opc.count(48) == 2 and opc.count(49) == 1 and opc.count(50) == 2
    assert opc.count(18) == 2 * 2 * 2  # AdamW on Aq, Bq, Av, Bv of each block
    assert opc.count(41) == 1 and opc.count(45) == 1
    # relaxed: the frozen-weight products and attention; never the adapters
    for w, (op, flags) in zip(dec.train, ops):
        ins4 = struct.unpack_from("<4Q", w, 8)
        if op in (47, 48, 49, 50):
            assert flags & (1 << 5)
        if op in (1, 2, 3) and not any(r >> 63 for r in ins4[:2]):
            assert not flags & (1 << 5), "an adapter product carries the relaxed flag"
    # eval = the forward, in exact arithmetic (instruction.h:356-384)
    assert len(dec.eval) == 2 + 2 * 18 + 3
    for e, t in zip(dec.eval, dec.train):
        assert e[:2] == t[:2] and e[4:] == t[4:]
        assert not struct.unpack_from("<H", e, 2)[0] & (1 << 5)
    assert struct.unpack_from("<H", dec.eval[-1])[0] == 11


def test_decoder_first_step_through_the_oracle(orc, dec):
    eng = OracleEngine(orc, dec.blob)
    T = TINY["batch"] * TINY["seq"]
    toks = pw.uniform_ints(11, T, TINY["vocab"])
    labels = np.roll(toks, -1)
    loss = eng.train_step(toks.view(np.float32), labels)
    assert abs(loss - math.log(TINY["vocab"])) < 0.05


# --- the int8-base decoder plan (BASELINE configs[4] at a small shape) ------------------------------

TINY_Q8 = dict(vocab=96, dim=128, heads=2, ffn=352, layers=2, seq=64, batch=2, rank=16)


@pytest.fixture(scope="module")
def dq8(hip):
    return pw.decoder_q8_lora(hip.plan_self_hash, **TINY_Q8)


def test_quantize_cols_follows_the_reference_packing_rule():
    """arena_binder.cc:129-177: scale = max|w| / 127 per column (1 for a zero
    column, FLT_MIN for a subnormal quotient); level = clamp(round(w / s),
    -127, 127) with halves away from zero."""
    tiny = np.float32(np.finfo(np.float32).tiny)
    u = 2.0 ** -7  # column 0's scale exactly: max |w| = 127 u
    w = np.array([[127 * u, 0.0, 3e-38],
                  [0.5 * u, 0.0, -1.2e-38],
                  [-1.5 * u, 0.0, 0.0],
                  [2.5 * u, 0.0, 0.0]], np.float32)
    levels, sc = pw.quantize_cols(w)
    assert sc[0] == np.float32(u) and sc[1] == 1.0 and sc[2] == tiny
    assert list(levels[:, 0]) == [127, 1, -2, 3]   # halves away from zero, not to even
    assert list(levels[:, 1]) == [0, 0, 0, 0]      # an all-zero column
    assert list(levels[:, 2]) == [3, -1, 0, 0]     # subnormal max / 127: the FLT_MIN scale
    # brute force on random columns against a plain-Python restatement
    r = np.random.default_rng(3).standard_normal((37, 11)).astype(np.float32) * 0.02
    lv, s2 = pw.quantize_cols(r)
    for j in range(r.shape[1]):
        m = max(abs(float(x)) for x in r[:, j])
        assert s2[j] == np.float32(np.float32(m) / np.float32(127.0))
        for i in range(r.shape[0]):
            x = float(np.float32(r[i, j] / s2[j]))
            want = math.floor(abs(x) + 0.5) * (1 if x >= 0 else -1)
            assert lv[i, j] == max(-127, min(127, want))


def test_q8_decoder_plan_structure(hip, dq8):
    assert hip.plan_check(dq8.blob) == ""
    ops = [struct.unpack_from("<HH", w) for w in dq8.train]
    opc = [o for o, _ in ops]
    L = TINY_Q8["layers"]
    # Q, K, V, O adapted in every block; gate, up, down on the int8 base
    assert opc.count(29) == L * 7                       # NN q8: q, k, v, o, gate, up, down
    assert opc.count(30) == L * 4 + (L - 1) * 3         # NT q8: down, gate, up, o; q, k, v above 0
    assert opc.count(47) == L and opc.count(48) == L and opc.count(49) == L and opc.count(50) == L
    assert opc.count(31) == 2 * L + 1 and opc.count(32) == 1 + L + (L - 1)  # no norm dX below block 0
    assert opc.count(24) == L and opc.count(25) == L and opc.count(21) == 3 * L
    assert opc.count(18) == L * 4 * 2                   # AdamW on A and B of four sites
    n_params = sum(dq8.arrays[n].size for n in dq8.arrays if ".A" in n or ".B" in n)
    assert n_params == L * 4 * 2 * TINY_Q8["dim"] * TINY_Q8["rank"]
    for w, (op, flags) in zip(dq8.train, ops):
        ins4 = struct.unpack_from("<4Q", w, 8)
        if op in (29, 30):
            assert flags & (1 << 4) and flags & (1 << 5)
            lv, sc = ins4[1], ins4[3]
            assert lv >> 63 and sc >> 63
            # the scales sit right after the levels (arena_binder.cc:283-287)
            name = next(n for n, (off, _) in dq8.rodata.items() if off == (lv & ~(1 << 63)))
            off, nb = dq8.rodata[name]
            assert (sc & ~(1 << 63)) == (off + nb + 3) // 4 * 4
        if op in (1, 2, 3) and not any(r >> 63 for r in ins4[:2]):
            assert not flags & (1 << 5), "an adapter product carries the relaxed flag"
    # adjacent dQ, dK, dV per block: the backward pair fuses
    idx = [i for i, o in enumerate(opc) if o == 48]
    assert all(opc[i + 1] == 49 and opc[i + 2] == 50 for i in idx)
    for e, t in zip(dq8.eval, dq8.train):
        assert e[:2] == t[:2] and e[4:] == t[4:]
        assert not struct.unpack_from("<H", e, 2)[0] & (1 << 5)
    assert struct.unpack_from("<H", dq8.eval[-1])[0] == 11
    # the packed levels are the quantizer applied to the generated weights
    lv, sc = pw.quantize_cols(pw.normal(20261205 + ord("q"), (TINY_Q8["dim"], TINY_Q8["dim"]), 0.02))
    assert np.array_equal(dq8.arrays["l0.wq"], lv) and np.array_equal(dq8.arrays["l0.wq.s"], sc)


def test_q8_decoder_first_step_through_the_oracle(orc, dq8):
    eng = OracleEngine(orc, dq8.blob)
    T = TINY_Q8["batch"] * TINY_Q8["seq"]
    toks = pw.uniform_ints(12, T, TINY_Q8["vocab"])
    labels = np.roll(toks, -1)
    loss = eng.train_step(toks.view(np.float32), labels)
    assert abs(loss - math.log(TINY_Q8["vocab"])) < 0.1
    loss2 = eng.train_step(toks.view(np.float32), labels)
    assert loss2 < loss  # the adapters learned from the first step


def test_plan_generator_matches_its_numpy_definition():
    """The threaded C++ generator (plangen.cc) gives the numpy definitions'
    bytes: normals (SplitMix64 -> Box-Muller in double) and int8 packing."""
    assert pw._gen() is not None, "libseeai_plangen.so is not built"
    for seed, shape, std in [(5, (513, 771), 0.02), (2 ** 63 + 11, (300001,), 2.0), (7, (3, 5), 0.5)]:
        a, b = pw.normal(seed, shape, std), pw.normal_numpy(seed, shape, std)
        assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    w = pw.normal(9, (700, 333), 0.02)
    w[:, 5] = 0.0
    w[:, 7] *= 1e-38
    l1, s1 = pw.quantize_cols(w)
    l2, s2 = pw.quantize_cols_numpy(w)
    assert np.array_equal(l1, l2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


# --- the oracle's threads (the reference's "same bits, any thread count") -------------------------

@pytest.mark.parametrize("which", ["c1", "dec", "dq8"])
def test_oracle_threads_do_not_change_bits(hip, orc, which):
    """Two training steps of each plan through the oracle at 1 and at 5
    threads: the whole arena is the same bytes (chunks are the reference's
    ParallelFor chunks; partials combine in chunk order)."""
    if which == "c1":
        img = pw.mlp_lora(hip.plan_self_hash)
        batches = [(pw.normal(300 + s, (32, 256)), pw.uniform_ints(400 + s, 32, 256)) for s in range(2)]
    else:
        make = pw.decoder_lora if which == "dec" else pw.decoder_q8_lora
        cfg = TINY if which == "dec" else TINY_Q8
        img = make(hip.plan_self_hash, relaxed=False, **cfg)
        T = cfg["batch"] * cfg["seq"]
        batches = []
        for s in range(2):
            t = pw.uniform_ints(500 + s, T + 1, cfg["vocab"])
            batches.append((t[:T].copy().view(np.float32), t[1:].copy()))
    arenas = []
    try:
        for threads in (1, 5):
            orc.set_threads(threads)
            eng = OracleEngine(orc, img.blob)
            for x, y in batches:
                eng.train_step(x, y)
            arenas.append(eng.arena.tobytes())
    finally:
        orc.set_threads(1)
    assert arenas[0] == arenas[1]
