"""Ingestion ring buffer (src/ring.rs) with its exact search on the GPU.

The ring holds the vectors not yet flushed into a PaxBlock64 (fewer than 64
after every push, ring.rs:76-84).  ``search_exact`` scores them against a query
on the device (mrl_ring_search), and ``merge_into`` pushes each query's ring
hits into the device-resident scan shortlists the way
IndexEngine::query_filtered does (src/engine.rs:584-594).

``push`` / ``flush_partial`` are a thin host-side holder of the pending rows
(ring.rs:76-93), kept only so that the pending rows exist for
``search_exact`` and the merge; their block encoding is the host encoder's
and is not part of the scan path.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from . import _lib
from .block import VECTORS_PER_BLOCK, source
from .eden import EdenFit
from .quantize import encode_block
from .scan import Device, DeviceResults, default_device


@dataclass
class PendingVector:
    """ring.rs:13-25 (the fp16 / int8 mirrors live in a RerankStore instead)."""
    passage_id: int
    embedding: np.ndarray
    timestamp: int
    source: int
    text: str = ""


class RingBuffer:
    """ring.rs:47-120"""

    def __init__(self, capacity: int, device: Optional[Device] = None):
        self._capacity = max(capacity, VECTORS_PER_BLOCK)
        self.pending: List[PendingVector] = []
        self.device = device

    def __len__(self):
        return len(self.pending)

    def is_empty(self) -> bool:
        return not self.pending

    def capacity(self) -> int:
        return self._capacity

    def push(self, item: PendingVector, eden: Optional[EdenFit] = None) -> Optional[np.ndarray]:
        """ring.rs:76-84: returns the flushed block once 64 vectors are pending."""
        self.pending.append(item)
        if len(self.pending) >= VECTORS_PER_BLOCK:
            return self._flush_block(eden)
        return None

    def flush_partial(self, eden: Optional[EdenFit] = None) -> Optional[np.ndarray]:
        """ring.rs:87-93"""
        return self._flush_block(eden) if self.pending else None

    def _flush_block(self, eden: Optional[EdenFit]) -> np.ndarray:
        """ring.rs:95-106 (encode_pending_embeddings_eden, encoder.rs:252-268)."""
        take = min(len(self.pending), VECTORS_PER_BLOCK)
        batch, self.pending = self.pending[:take], self.pending[take:]
        vecs = np.stack([np.asarray(p.embedding, dtype=np.float32) for p in batch])
        ts = np.array([p.timestamp for p in batch], dtype=np.uint32)
        src = np.array([source.DOC if p.source == 0 else p.source for p in batch], dtype=np.uint32)
        return encode_block(vecs, ts, src, vecs.shape[1], eden)

    def pending_matrix(self) -> np.ndarray:
        if not self.pending:
            return np.zeros((0, 0), dtype=np.float32)
        return np.ascontiguousarray(np.stack([np.asarray(p.embedding, dtype=np.float32) for p in self.pending]))

    def search_exact(self, query, top_k: int):
        """ring.rs:109-119: [(local index, score, PendingVector)], score descending."""
        if not self.pending:
            return []
        rows = self.pending_matrix()
        q = np.ascontiguousarray(np.asarray(query, dtype=np.float32)[None, :])
        if q.shape[1] != rows.shape[1]:
            raise ValueError("query dims differ from the pending rows'")
        keep = min(top_k, rows.shape[0])
        loc = np.zeros((1, max(keep, 1)), dtype=np.uint64)
        sc = np.zeros((1, max(keep, 1)), dtype=np.float32)
        cnt = np.zeros(1, dtype=np.uint32)
        dev = self.device or default_device()
        _lib.check(_lib.lib.mrl_ring_search(dev.handle, _lib.fptr(rows), rows.shape[0], rows.shape[1], _lib.fptr(q),
                                            1, top_k, _lib.u64ptr(loc), _lib.fptr(sc), _lib.u32ptr(cnt)))
        return [(int(loc[0, i]), float(sc[0, i]), self.pending[int(loc[0, i])]) for i in range(int(cnt[0]))]

    def merge_into(self, results: DeviceResults) -> None:
        """engine.rs:584-594 for every query of the results' last scan, on the device."""
        if not self.pending:
            return
        rows = self.pending_matrix()
        _lib.check(_lib.lib.mrl_results_merge_ring(results.device.handle, results._h, _lib.fptr(rows),
                                                   rows.shape[0], rows.shape[1]))
