"""Instruction-word construction for tests (source/plan/instruction.h:438-447)."""
from __future__ import annotations

import struct

NULL = 0xFFFFFFFFFFFFFFFF


def ins(opcode: int, ins4=(), outs3=(), flags: int = 0, imm: int = 0) -> bytes:
    i4 = list(ins4) + [NULL] * (4 - len(ins4))
    o3 = list(outs3) + [0] * (3 - len(outs3))
    return struct.pack("<HHI4Q3Q", opcode, flags, imm, *[int(x) for x in i4],
                       *[int(x) for x in o3])
