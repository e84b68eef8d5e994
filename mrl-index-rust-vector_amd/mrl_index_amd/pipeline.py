"""QueryPipeline (src/pipeline.rs): plan selection + scan, the seam every
caller of the reference goes through."""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from .block import VECTORS_PER_BLOCK, VectorId
from .config import EngineConfig, MidCodec, PrefixCodec
from .eden import EdenFit
from .lowprec import RerankStore, rerank_rows
from .scan import DeviceIndex, QueryPlan, ScanStats, ScoredHit, scan_blocks_stats


@dataclass
class ScanPhase:
    """pipeline.rs:25-32"""
    plan: QueryPlan
    hits: list
    scan_ms: float
    blocks_scanned: int


class QueryPipeline:
    def __init__(self, cfg: EngineConfig, eden: Optional[EdenFit] = None, eden_mid: Optional[EdenFit] = None):
        self.cfg = cfg
        self.eden = eden
        self.eden_mid = eden_mid

    @classmethod
    def with_eden(cls, cfg, fit):
        return cls(cfg, fit, None)

    @classmethod
    def with_eden_dual(cls, cfg, prefix, mid):
        return cls(cfg, prefix, mid)

    def build_plan(self, query) -> QueryPlan:
        """pipeline.rs:63-74 (match order kept)."""
        c = self.cfg
        if c.prefix_codec == PrefixCodec.EDEN_PROD and c.mid_codec == MidCodec.EDEN_B1 and self.eden is not None \
                and self.eden_mid is not None:
            return QueryPlan.from_query_eden_dual(query, c.embed_dims, self.eden, self.eden_mid)
        if c.prefix_codec == PrefixCodec.EDEN_PROD and self.eden is not None:
            return QueryPlan.from_query_eden(query, c.embed_dims, self.eden)
        return QueryPlan.from_query(query, c.embed_dims)

    def scan_slab(self, query, blocks, time_lo=None, time_hi=None, stats: Optional[ScanStats] = None) -> ScanPhase:
        """pipeline.rs:77-98: plan time is outside scan_ms."""
        plan = self.build_plan(query)
        t = time.perf_counter()
        hits = scan_blocks_stats(blocks, plan, self.cfg, time_lo, time_hi, stats)
        ms = (time.perf_counter() - t) * 1000.0
        n = blocks.block_count() if isinstance(blocks, DeviceIndex) else len(np.asarray(blocks).reshape(-1, 4096))
        return ScanPhase(plan, hits, ms, n)

    def scan_segments(self, query, index: DeviceIndex, time_lo=None, time_hi=None):
        """pipeline.rs:136-154 for a segment opened with DeviceIndex.open_segment."""
        plan = self.build_plan(query)
        t = time.perf_counter()
        hits = scan_blocks_stats(index, plan, self.cfg, time_lo, time_hi, None)
        return plan, hits, (time.perf_counter() - t) * 1000.0, index.block_count()

    @staticmethod
    def rerank_exact_rows(query, candidate_ids, corpus_row):
        """pipeline.rs:157-169 on the GPU: (row, dot(query, row)) for every
        candidate, stably sorted by score, descending.  ``corpus_row`` is a
        RerankStore (rows resident in HBM), or a callable row -> vector as in
        the reference, whose rows are gathered into a transient fp32 store."""
        ids = [int(i) for i in candidate_ids]
        if isinstance(corpus_row, RerankStore):
            return rerank_rows(query, ids, corpus_row)
        if not ids:
            return []
        uniq = sorted(set(ids))
        pos = {r: k for k, r in enumerate(uniq)}
        store = RerankStore.create(np.stack([np.asarray(corpus_row(r), dtype=np.float32) for r in uniq]))
        try:
            ranked = rerank_rows(query, [pos[i] for i in ids], store)
        finally:
            store.close()
        return [(uniq[r], s) for r, s in ranked]


def scored_hits_to_row_ids(hits: List[ScoredHit]) -> List[int]:
    """pipeline.rs:175-180"""
    return [h.id.block * VECTORS_PER_BLOCK + h.id.slot for h in hits if h.id.block != 0xFFFFFFFF]


def row_id_to_vector_id(row: int) -> VectorId:
    """pipeline.rs:183-188"""
    return VectorId(row // VECTORS_PER_BLOCK, row % VECTORS_PER_BLOCK)
