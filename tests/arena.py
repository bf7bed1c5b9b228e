"""A host-side arena builder for instruction-level parity tests.

Places named tensors at 256-byte-aligned offsets of one arena image (and,
for frozen weights, of a rodata image), and hands out the 64-bit tensor
references the plan ABI uses (source/plan/instruction.h:25-42: bit 63 marks
a rodata reference).  The same bytes are then executed by the oracle's
instruction interpreter and by the HIP executor, and compared extent by
extent.
"""
from __future__ import annotations

import numpy as np

RODATA_BIT = 1 << 63
NULL = 0xFFFFFFFFFFFFFFFF


def f32_bits(x: float) -> int:
    return int(np.array([x], np.float32).view(np.uint32)[0])


class Arena:
    def __init__(self):
        self.arena_parts: list[tuple[int, np.ndarray]] = []
        self.ro_parts: list[tuple[int, np.ndarray]] = []
        self.arena_size = 0
        self.ro_size = 0
        self.meta: dict[str, tuple[bool, int, np.dtype, tuple]] = {}

    @staticmethod
    def _align(n: int) -> int:
        return (n + 255) // 256 * 256

    def add(self, name: str, arr, rodata: bool = False) -> int:
        arr = np.ascontiguousarray(arr)
        if rodata:
            off = self.ro_size
            self.ro_parts.append((off, arr))
            self.ro_size = self._align(off + arr.nbytes)
            ref = off | RODATA_BIT
        else:
            off = self.arena_size
            self.arena_parts.append((off, arr))
            self.arena_size = self._align(off + arr.nbytes)
            ref = off
        self.meta[name] = (rodata, off, arr.dtype, arr.shape)
        return ref

    def empty(self, name: str, shape, dtype=np.float32, fill=np.nan) -> int:
        a = np.full(shape, fill, dtype) if np.dtype(dtype).kind == "f" else np.zeros(shape, dtype)
        return self.add(name, a)

    def images(self) -> tuple[np.ndarray, np.ndarray]:
        arena = np.zeros(max(self.arena_size, 256), np.uint8)
        for off, a in self.arena_parts:
            arena[off:off + a.nbytes] = a.view(np.uint8).reshape(-1)
        ro = np.zeros(max(self.ro_size, 256), np.uint8)
        for off, a in self.ro_parts:
            ro[off:off + a.nbytes] = a.view(np.uint8).reshape(-1)
        return arena, ro

    def get(self, image: np.ndarray, name: str) -> np.ndarray:
        rodata, off, dtype, shape = self.meta[name]
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return np.frombuffer(image[off:off + n].tobytes(), dtype).reshape(shape)
