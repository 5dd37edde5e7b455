"""Growable host byte arena backing the uniform-block `MTCMatrix` layout.

Same contract as mtc/core/arena.py:9-75 (MemoryArena): a uint8 buffer with a
bump pointer, 2x growth on overflow, and alignment on request. It only holds
the reference's uniform-block payload layout on the host; the device-side
weight stream lives in a separate GPU buffer owned by the packed matrix.
"""

import numpy as np


class MemoryArena:
    def __init__(self, capacity_bytes: int = 64 * 1024 * 1024):
        self._capacity = int(capacity_bytes)
        self._buffer = np.zeros(self._capacity, dtype=np.uint8)
        self._offset = 0

    @property
    def capacity(self) -> int:
        return self._capacity

    @property
    def bytes_allocated(self) -> int:
        return self._offset

    @property
    def utilization_pct(self) -> float:
        return 100.0 * self._offset / self._capacity if self._capacity else 0.0

    @property
    def raw_buffer(self) -> np.ndarray:
        return self._buffer

    def allocate(self, size_bytes: int, alignment: int = 1) -> int:
        start = self._offset
        if alignment > 1 and start % alignment:
            start += alignment - start % alignment
        end = start + int(size_bytes)
        if end > self._capacity:
            grown = max(2 * self._capacity, end + (1 << 20))
            buf = np.zeros(grown, dtype=np.uint8)
            buf[: self._offset] = self._buffer[: self._offset]
            self._buffer, self._capacity = buf, grown
        self._offset = end
        return start

    def write_bytes(self, data, alignment: int = 1) -> int:
        flat = np.ascontiguousarray(data, dtype=np.uint8).ravel()
        off = self.allocate(flat.nbytes, alignment)
        self._buffer[off: off + flat.nbytes] = flat
        return off

    def view(self, offset: int, length: int) -> np.ndarray:
        return self._buffer[offset: offset + length]

    def reset(self):
        self._offset = 0
