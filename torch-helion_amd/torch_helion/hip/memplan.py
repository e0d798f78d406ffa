"""Liveness-based reuse of device memory for a Program's intermediates.

The reference interpreter keeps every tensor of the program alive
(codegen/interpret.py:54-65, the kernel order of optimizer/partition.py:286-300).
On the device a deep program would then hold every layer's activations at
once (the 24-layer Mamba-2 backbone: ~12 GB at B=8, L=2048). Kernels run in
program order on one stream, so a buffer whose tensor is read for the last
time by kernel i can hold a tensor produced by kernel i+1 or later.

``lifetimes`` gives each tensor the kernel that produces it and the last
kernel that reads it; ``BufferPool`` is a linear-scan allocator over those
intervals: before kernel i is bound, every block whose tensor's last reader is
before i returns to the free list, and a request takes the smallest free block
that holds it (else a new block).
"""

from __future__ import annotations

from typing import Callable

ALIGN = 256


def lifetimes(program) -> tuple[dict[str, int], dict[str, int]]:
    """(producer kernel index, last reading kernel index) per tensor. Program
    outputs live to the end; a produced tensor nobody reads dies at its producer."""
    born: dict[str, int] = {}
    last: dict[str, int] = {}
    n = len(program.kernels)
    for i, k in enumerate(program.kernels):
        for a in k.args:
            last[a.tensor] = max(last.get(a.tensor, -1), i)
        for o in k.outputs:
            born.setdefault(o.tensor, i)
            last[o.tensor] = max(last.get(o.tensor, -1), i)
    for o in program.outputs:
        last[o] = n
    return born, last


class BufferPool:
    """Linear-scan allocator of device blocks over [born, last] kernel intervals.

    ``factory(nbytes)`` makes a new block (a 1-D uint8 tensor); blocks are never
    freed to the device, only recycled, so bound kernels keep valid pointers."""

    def __init__(self, factory: Callable[[int], object]) -> None:
        self._factory = factory
        self._free: list[tuple[int, object]] = []
        self._live: list[tuple[int, int, object]] = []  # (last kernel, bytes, block)
        self.block_bytes = 0                              # device memory held by the pool
        self.requested_bytes = 0                          # what allocation without reuse would hold

    def release_before(self, i: int) -> None:
        """Return the blocks of tensors whose last reader runs before kernel ``i``."""
        keep = []
        for last, size, blk in self._live:
            if last < i:
                self._free.append((size, blk))
            else:
                keep.append((last, size, blk))
        self._live = keep

    def alloc(self, nbytes: int, last: int):
        """A block of at least ``nbytes`` that stays unused by others through kernel ``last``."""
        size = max(ALIGN, (nbytes + ALIGN - 1) // ALIGN * ALIGN)
        self.requested_bytes += size
        best = None
        for j, (fsize, _) in enumerate(self._free):
            if fsize >= size and (best is None or fsize < self._free[best][0]):
                best = j
        if best is not None:
            fsize, blk = self._free.pop(best)
        else:
            fsize, blk = size, self._factory(size)
            self.block_bytes += size
        self._live.append((last, fsize, blk))
        return blk
