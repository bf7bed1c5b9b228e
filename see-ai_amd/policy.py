"""The gfx950 member of the kernel-policy table.

The reference keeps one measured, host-keyed JSON table (schema 1) that its
compiler reads (compiler/backend/architecture/kernel_policy_table.cc:294-404)
and its offline tuner writes (tool/autotune.py:45-58):

    {"schema": 1,
     "hosts": {"<host key>": {"cpu": {"gemm_tile_k": K, "gemm_tile_n": N},
                              "tuned": {...}}}}

The reader skips members it does not know (kernel_policy_table.cc:319-321),
so the GPU's geometry travels in the same file, beside "cpu", under the
device's key (``hip.device_key()``, the counterpart of HostKey,
host_arch.h:41-50):

    "hosts": {"gfx950;AMD Instinct MI355X;cus=256;...":
                 {"gfx950": {"w8a8_large_kernel": 1, ...},
                  "tuned_gfx950": {...every measurement...}}}

Every field picks among kernels that give identical bits (as the CPU tiles
do, autotune.py:24-28), so a table changes time, never results.  This
module is pure Python: parsing, validation and resolution, with the
reference's error behaviour (``PolicyError`` messages, a missing entry is a
note and the defaults, not an error).
"""
from __future__ import annotations

import json

SCHEMA = 1
MEMBER = "gfx950"

# field -> (default, ("choice", values) or ("range", lo, hi), meaning)
FIELDS = {
    "w8a8_large_kernel": (1, ("choice", 1, 2, 3),
                          "W8A8 from M, N >= w8a8_large_min: 1 direct-to-LDS 256x256, "
                          "2 register-staged 256x256, 3 register-staged 128x128"),
    "w8a8_large_min": (4096, ("range", 1, 1 << 30), "M and N from which w8a8_large_kernel applies"),
    "quantize_waves_per_cu": (32, ("range", 1, 32),
                              "waves per CU walking the activation quantizer's rows of at most "
                              "1024 or more than 8192 floats (rows in between: four waves each)"),
    "relaxed_min_tiles_256": (256, ("range", 1, 1 << 30),
                              "relaxed bf16 GEMM: 256x256 tiles once the grid has this many"),
    "relaxed_min_fill_256": (0, ("range", 0, 100),
                             "relaxed bf16 GEMM: 256x256 tiles only when their last round over "
                             "the CUs is at least this percent full"),
    "relaxed_nt_dma_min_k": (768, ("range", 64, 1 << 30),
                             "relaxed NT on rodata weights: the direct-to-LDS kernel from this K"),
    "convert_wgs_per_cu": (8, ("range", 1, 64),
                           "workgroups per CU of the relaxed GEMMs' activation conversion"),
    "exact_longk_first": (1, ("choice", 1, 2),
                          "exact skinny long-K GEMM: 1 two-pass workspace form first, "
                          "2 chain kernel first"),
    "relaxed_tile_192": (2, ("choice", 1, 2, 3),
                         "relaxed bf16 GEMM below 256x256: 1 128x192 tiles where they take fewer "
                         "CU rounds per unit of work, 2 never, 3 always (N >= 192)"),
}
DEFAULTS = {k: v[0] for k, v in FIELDS.items()}


class PolicyError(ValueError):
    """A table or entry the backend refuses (the reference's PolicyError)."""


def check_entry(entry: dict, what: str) -> dict:
    """CheckEntry (kernel_policy_table.cc:280-289) for the gfx950 fields:
    whole numbers in range; unknown fields are refused (a misspelt field
    would silently leave a default in force)."""
    if not isinstance(entry, dict):
        raise PolicyError(f"{what}: \"{MEMBER}\" must be an object")
    out = dict(DEFAULTS)
    for key, value in entry.items():
        if key not in FIELDS:
            raise PolicyError(f"{what}: unknown field \"{key}\"")
        if isinstance(value, bool) or not isinstance(value, int):
            raise PolicyError(f"{what}: {key} must be a whole number, got {value!r}")
        spec = FIELDS[key][1]
        ok = spec[1] <= value <= spec[2] if spec[0] == "range" else value in spec[1:]
        if not ok:
            raise PolicyError(f"{what}: {key} = {value} is outside what the kernels implement "
                              f"({FIELDS[key][2]})")
        out[key] = value
    return out


def parse_table(text: str) -> dict:
    """ParseKernelPolicyTable (kernel_policy_table.cc:299-334) for the gfx950
    member: {device key: policy dict}.  Hosts without the member are skipped,
    as the reference skips hosts without "cpu"."""
    try:
        doc = json.loads(text)
    except json.JSONDecodeError as e:
        raise PolicyError(f"table is not valid JSON ({e})") from None
    if not isinstance(doc, dict):
        raise PolicyError("table must be a JSON object")
    if doc.get("schema") != SCHEMA or isinstance(doc.get("schema"), bool):
        raise PolicyError("table \"schema\" must be 1")
    hosts = doc.get("hosts")
    if not isinstance(hosts, dict):
        raise PolicyError("table \"hosts\" must be an object keyed by host")
    table = {}
    for key, host in hosts.items():
        if not isinstance(host, dict):
            raise PolicyError(f"host \"{key}\" must be an object")
        if MEMBER not in host:
            continue
        table[key] = check_entry(host[MEMBER], f"host \"{key}\"")
    return table


def load_table(path: str) -> dict:
    """LoadKernelPolicyTable (kernel_policy_table.cc:336-347)."""
    try:
        with open(path, "rb") as f:
            text = f.read().decode("utf-8")
    except OSError:
        raise PolicyError(f"cannot read kernel-policy table '{path}'") from None
    try:
        return parse_table(text)
    except PolicyError as e:
        raise PolicyError(f"{e} ['{path}']") from None


def resolve(key: str, table_path: str | None = None, explicit: dict | None = None):
    """ResolveKernelPolicy (kernel_policy_table.cc:372-402): an explicit
    policy wins, then the table's entry for `key`; otherwise the defaults
    with a note.  Returns (policy, source, note)."""
    if explicit is not None:
        return check_entry(explicit, "explicit policy"), "flag", ""
    if table_path:
        table = load_table(table_path)
        if key in table:
            return table[key], "table", ""
        note = (f"kernel-policy table '{table_path}' has no \"{MEMBER}\" entry for device "
                f"\"{key}\"; the built-in kernel geometry applies (run "
                f"python -m see-ai_amd.tune on this device to add one)")
        return dict(DEFAULTS), "default", note
    return dict(DEFAULTS), "default", ""


def merge_into_table(text: str | None, key: str, entry: dict, tuned: dict) -> str:
    """The tuner's write (autotune.py's table step): this device's gfx950
    member and its measurements, every other host and member untouched."""
    doc = {"schema": SCHEMA, "hosts": {}}
    if text:
        doc = json.loads(text)
        parse_table(text)  # refuse to extend a table the reader would refuse
    host = doc["hosts"].setdefault(key, {})
    host[MEMBER] = check_entry(entry, "tuned entry")
    host["tuned_" + MEMBER] = tuned
    return json.dumps(doc, indent=2, sort_keys=True) + "\n"
