"""Append-only segment files of raw PaxBlock64 records (src/segment.rs)."""
from __future__ import annotations

import os

import numpy as np

from .block import BLOCK_BYTES, as_blocks


class SegmentError(RuntimeError):
    pass


class SegmentWriter:
    """segment.rs:21-79"""

    def __init__(self, path, append: bool = False):
        self.path = str(path)
        os.makedirs(os.path.dirname(self.path) or ".", exist_ok=True)
        if append and os.path.exists(self.path):
            size = os.path.getsize(self.path)
            if size % BLOCK_BYTES:
                raise SegmentError(f"corrupt segment size {size} (not multiple of 4096)")
            self.blocks = size // BLOCK_BYTES
            self._f = open(self.path, "ab")
        else:
            self.blocks = 0
            self._f = open(self.path, "wb")

    @classmethod
    def create(cls, path):
        return cls(path, append=False)

    @classmethod
    def open_append(cls, path):
        return cls(path, append=True)

    def append_block(self, block) -> int:
        b = as_blocks(block)
        idx = self.blocks
        self._f.write(b.tobytes())
        self._f.flush()
        self.blocks += b.shape[0]
        return idx

    def block_count(self) -> int:
        return self.blocks

    def close(self):
        self._f.close()


def read_segment(path) -> np.ndarray:
    """Host copy of a segment (SegmentReader with an owned buffer)."""
    if not os.path.exists(path):
        return np.zeros((0, BLOCK_BYTES), dtype=np.uint8)
    data = np.fromfile(path, dtype=np.uint8)
    if data.size % BLOCK_BYTES:
        raise SegmentError(f"corrupt segment size {data.size} (not multiple of 4096)")
    return data.reshape(-1, BLOCK_BYTES)
