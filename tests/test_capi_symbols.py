"""CPU: the C-ABI library loads and exports every symbol include/*.h declares
(no compute call -- there is no GPU here)."""
from __future__ import annotations

import ctypes
import glob
import os
import re

from tests.conftest import ROOT


def declared_symbols():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(seeai_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(os.path.join(ROOT, "see-ai_amd", "libseeai_hip.so"))
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_table_matches_the_header(hip):
    assert set(hip.EXPORTS) == declared_symbols()


def test_instruction_word_is_64_bytes(hip):
    w = hip.pack_instruction(1, 0, 0, [0, 1, 2], [3, 4, 5])
    assert len(w) == 64
