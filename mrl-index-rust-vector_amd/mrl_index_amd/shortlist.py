"""Shortlist (src/scan.rs:310-399): the fixed-capacity top-K tracker a caller
owns and QueryPipeline.scan_segments_into pushes into."""
from __future__ import annotations

import math
from typing import List

import numpy as np

from .scan import ScoredHit


class Shortlist:
    def __init__(self, capacity: int, floor_tau: float = -math.inf):
        """Shortlist::new / with_floor (scan.rs:320-338): capacity 0 acts as 1."""
        self.capacity = max(int(capacity), 1)
        self.heap: List[ScoredHit] = []
        self.min_idx = 0
        self.min_score = math.inf
        self.floor_tau = float(np.float32(floor_tau))

    @classmethod
    def with_floor(cls, capacity: int, floor_tau: float) -> "Shortlist":
        return cls(capacity, floor_tau)

    def threshold(self) -> float:
        """scan.rs:340-347"""
        if len(self.heap) < self.capacity:
            return self.floor_tau
        return max(self.min_score, self.floor_tau)

    def push(self, hit: ScoredHit) -> None:
        """scan.rs:349-366: below the floor is dropped; while filling, the
        first strict minimum is tracked; once full, a hit replaces the
        minimum only if strictly greater."""
        s = float(hit.score)
        if s < self.floor_tau:
            return
        if len(self.heap) < self.capacity:
            if s < self.min_score:
                self.min_score = s
                self.min_idx = len(self.heap)
            self.heap.append(hit)
            return
        if s > self.min_score:
            self.heap[self.min_idx] = hit
            self._recompute_min()

    def _recompute_min(self) -> None:
        """scan.rs:368-380"""
        self.min_idx, self.min_score = 0, math.inf
        for i, h in enumerate(self.heap):
            if float(h.score) < self.min_score:
                self.min_score = float(h.score)
                self.min_idx = i

    def merge(self, other: "Shortlist") -> None:
        """scan.rs:382-386"""
        for h in other.heap:
            self.push(h)

    def into_sorted(self) -> List[ScoredHit]:
        """scan.rs:388-393: a stable sort, descending.  The reference's
        partial_cmp().unwrap() panics when a NaN score is compared, i.e. with
        a NaN among two or more hits; that raises ValueError here."""
        if len(self.heap) > 1 and any(math.isnan(float(h.score)) for h in self.heap):
            raise ValueError("NaN score in Shortlist::into_sorted")
        return sorted(self.heap, key=lambda h: -float(h.score))

    def __len__(self) -> int:
        return len(self.heap)
