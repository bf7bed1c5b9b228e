"""The gfx950 kernel-policy table (see-ai_amd/policy.py) and the tuner's
decision rule (see-ai_amd/tune.py), on the CPU.

The reader's contract is the reference's ParseKernelPolicyTable /
ResolveKernelPolicy (compiler/backend/architecture/kernel_policy_table.cc:
280-404): schema 1, hosts keyed by the device key, unknown members skipped,
a missing entry a note and the defaults; the tuner's is autotune.py:177-212
(medians of medians, geometric-mean score against the default arm, a 3 %
margin before a non-default arm is written)."""
from __future__ import annotations

import importlib
import json

import pytest

policy = importlib.import_module("see-ai_amd.policy")

KEY = "gfx950;AMD Instinct MI355X;cus=256;lds=163840;l2=4194304;wave=64"


def table(**hosts):
    return json.dumps({"schema": 1, "hosts": hosts})


def test_reader_takes_the_gfx950_member_and_skips_the_rest():
    t = policy.parse_table(table(**{
        KEY: {"cpu": {"gemm_tile_k": 64, "gemm_tile_n": 256}, "tuned": {"x": 1},
              "gfx950": {"w8a8_large_kernel": 2, "quantize_waves_per_cu": 8}},
        "arm64;Apple M2;cores=8": {"cpu": {"gemm_tile_k": 128, "gemm_tile_n": 512}},
    }))
    assert list(t) == [KEY]  # a host without the member is skipped, as the CPU reader skips
    want = dict(policy.DEFAULTS, w8a8_large_kernel=2, quantize_waves_per_cu=8)
    assert t[KEY] == want


@pytest.mark.parametrize("text,words", [
    ("not json", "not valid JSON"),
    ("[1, 2]", "must be a JSON object"),
    (json.dumps({"schema": 2, "hosts": {}}), "\"schema\" must be 1"),
    (json.dumps({"schema": True, "hosts": {}}), "\"schema\" must be 1"),
    (json.dumps({"schema": 1}), "\"hosts\" must be an object"),
    (json.dumps({"schema": 1, "hosts": {"k": 3}}), "host \"k\" must be an object"),
    (table(k={"gfx950": 5}), "must be an object"),
    (table(k={"gfx950": {"w8a8_large_kernel": 4}}), "w8a8_large_kernel = 4"),
    (table(k={"gfx950": {"w8a8_large_kernel": 0}}), "w8a8_large_kernel = 0"),
    (table(k={"gfx950": {"quantize_waves_per_cu": 33}}), "quantize_waves_per_cu = 33"),
    (table(k={"gfx950": {"exact_longk_first": 3}}), "exact_longk_first = 3"),
    (table(k={"gfx950": {"relaxed_min_tiles_256": 1.5}}), "whole number"),
    (table(k={"gfx950": {"relaxed_min_tiles_256": True}}), "whole number"),
    (table(k={"gfx950": {"w8a8_tile": 1}}), "unknown field \"w8a8_tile\""),
])
def test_reader_refuses_what_no_kernel_implements(text, words):
    with pytest.raises(policy.PolicyError, match=None) as e:
        policy.parse_table(text)
    assert words in str(e.value)


def test_resolve_order_and_the_missing_entry_note(tmp_path):
    path = tmp_path / "t.json"
    path.write_text(table(**{KEY: {"gfx950": {"relaxed_min_tiles_256": 96}}}))
    pol, src, note = policy.resolve(KEY, str(path))
    assert src == "table" and pol["relaxed_min_tiles_256"] == 96 and note == ""
    pol, src, note = policy.resolve("gfx950;other", str(path))
    assert src == "default" and pol == policy.DEFAULTS
    assert "has no \"gfx950\" entry for device \"gfx950;other\"" in note
    pol, src, _ = policy.resolve(KEY, str(path), explicit={"exact_longk_first": 2})
    assert src == "flag" and pol["exact_longk_first"] == 2
    assert policy.resolve(KEY) == (policy.DEFAULTS, "default", "")
    with pytest.raises(policy.PolicyError, match="cannot read kernel-policy table"):
        policy.resolve(KEY, str(tmp_path / "missing.json"))
    bad = tmp_path / "bad.json"
    bad.write_text("{}")
    with pytest.raises(policy.PolicyError, match=r"\['.*bad.json'\]"):
        policy.load_table(str(bad))


def test_merge_keeps_every_other_host_and_member():
    base = table(**{KEY: {"cpu": {"gemm_tile_k": 64, "gemm_tile_n": 256}},
                    "other": {"gfx950": {"w8a8_large_kernel": 3}}})
    out = policy.merge_into_table(base, KEY, {"w8a8_large_kernel": 2}, {"note": "measured"})
    doc = json.loads(out)
    assert doc["hosts"][KEY]["cpu"] == {"gemm_tile_k": 64, "gemm_tile_n": 256}
    assert doc["hosts"][KEY]["tuned_gfx950"] == {"note": "measured"}
    assert doc["hosts"]["other"]["gfx950"]["w8a8_large_kernel"] == 3
    assert policy.parse_table(out)[KEY]["w8a8_large_kernel"] == 2
    with pytest.raises(policy.PolicyError):
        policy.merge_into_table(base, KEY, {"w8a8_large_kernel": 9}, {})


def test_tuner_decision_rule():
    tune = importlib.import_module("see-ai_amd.tune")
    # medians over rounds, then the geometric mean of per-fixture ratios
    runs = {1: [{"a": 100.0, "b": 10.0}, {"a": 90.0, "b": 11.0}, {"a": 110.0, "b": 9.0}],
            2: [{"a": 200.0, "b": 5.0}, {"a": 210.0, "b": 5.5}, {"a": 190.0, "b": 4.5}],
            3: [{"a": 103.0, "b": 10.2}] * 3}
    s = tune.score_arms(runs, 1)
    assert s[1]["score"] == pytest.approx(1.0)
    assert s[2]["speedup"] == {"a": pytest.approx(2.0), "b": pytest.approx(0.5)}
    assert s[2]["score"] == pytest.approx(1.0)  # 2x on one fixture does not outvote 0.5x
    assert s[3]["score"] == pytest.approx((1.03 * 1.02) ** 0.5)
    arm, why = tune.choose(s, 1, 0.03)
    assert arm == 1 and why.startswith("default-within-margin")  # 2.5 % < 3 %
    arm, why = tune.choose(s, 1, 0.02)
    assert arm == 3 and why.startswith("tuned: 3 gains")
    arm, why = tune.choose({1: {"score": 1.0}, 2: {"score": 0.9}}, 1, 0.03)
    assert (arm, why) == (1, "default-is-best")
    # a tie with the default keeps the default
    arm, _ = tune.choose({1: {"score": 1.0}, 2: {"score": 1.0}}, 1, 0.0)
    assert arm == 1
    assert set(tune.ARMS) == set(policy.FIELDS)
    for field, arms in tune.ARMS.items():
        for a in arms:
            policy.check_entry({field: a}, "arm")
