"""PaxBlock64 layout constants and ids (src/block.rs)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

VECTORS_PER_BLOCK = 64
BLOCK_BYTES = 4096
MRL_PREFIX_DIMS = 64
RABITQ_DIMS = 128
MID_PREFIX_DIMS = 64
TAIL_START = MRL_PREFIX_DIMS + RABITQ_DIMS
TAIL_FOLD_DIMS = 64
TAIL_FOLD_BLOCKS = 9
EMBED_DIMS_768 = 768

# byte offsets inside one block (block.rs:34-44,133-142)
OFF_MIN_TIMESTAMP = 0
OFF_MAX_TIMESTAMP = 4
OFF_SOURCE_MASK = 8
OFF_COARSE_CLUSTER_ID = 12
OFF_BLOCK_FLAGS = 14
OFF_TOMBSTONE_MASK = 16
OFF_CRC32C = 24
OFF_META = 64
OFF_STRATUM0_SIGN = 512
OFF_STRATUM1_RABITQ = 1024
OFF_STRATUM2_MSB1 = 2048
OFF_STRATUM3_MSB2 = 2560
OFF_STRATUM4_MID = 3072
OFF_STRATUM5_LSB = 3584


class source:
    """block.rs:24-29"""
    SLACK = 1 << 0
    EMAIL = 1 << 1
    CODE = 1 << 2
    DOC = 1 << 3


@dataclass(frozen=True)
class VectorId:
    """block.rs:200-223"""
    block: int
    slot: int

    def as_u64(self) -> int:
        return (self.block << 16) | self.slot

    @classmethod
    def from_u64(cls, v: int) -> "VectorId":
        return cls(int(v) >> 16, int(v) & 0xFFFF)


def as_blocks(data) -> np.ndarray:
    """View bytes / a uint8 array as an (n, 4096) uint8 block array."""
    a = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) else np.asarray(data)
    if a.dtype != np.uint8:
        raise TypeError("blocks must be uint8")
    if a.size % BLOCK_BYTES:
        raise ValueError(f"corrupt segment size {a.size} (not multiple of 4096)")
    return np.ascontiguousarray(a.reshape(-1, BLOCK_BYTES))


def tombstone_mask(blocks: np.ndarray) -> np.ndarray:
    return blocks[:, OFF_TOMBSTONE_MASK:OFF_TOMBSTONE_MASK + 8].copy().view("<u8").reshape(-1)


def active_count(block: np.ndarray) -> int:
    """PaxBlock64::active_count (block.rs:178-180)."""
    t = int(block[OFF_TOMBSTONE_MASK:OFF_TOMBSTONE_MASK + 8].view("<u8")[0])
    return bin(~t & 0xFFFFFFFFFFFFFFFF).count("1")
