"""QueryPipeline (src/pipeline.rs): plan selection + scan, the seam every
caller of the reference goes through."""
from __future__ import annotations

import json
import os
import time
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from .block import BLOCK_BYTES, VECTORS_PER_BLOCK, VectorId
from .config import EngineConfig, MidCodec, PrefixCodec
from .eden import EdenFit
from .lowprec import RerankStore, rerank_rows
from .scan import DeviceIndex, QueryPlan, ScanStats, ScoredHit, default_device, scan_blocks_stats
from .shortlist import Shortlist

EDEN_PREFIX_FILE = "eden_prefix.json"  # engine.rs:22
MANIFEST_FILE = "manifest.json"
SEGMENT_PATH = os.path.join("segments", "000001.pax")  # engine.rs:143


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

    def scan_segments_into(self, plan: QueryPlan, reader: DeviceIndex, shortlist: Shortlist, time_lo=None,
                           time_hi=None) -> int:
        """pipeline.rs:104-133: scans the segment (resident in HBM) and pushes
        every hit, best first, into the caller's shortlist; the caller merges
        ring hits afterwards and calls into_sorted.  Returns the block count."""
        for hit in scan_blocks_stats(reader, plan, self.cfg, time_lo, time_hi, None):
            shortlist.push(hit)
        return reader.block_count()

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


@dataclass
class IndexManifest:
    """engine.rs:38-44 (manifest.json)."""
    version: str
    config: EngineConfig
    next_passage_id: int
    blocks_written: int

    @classmethod
    def load(cls, path) -> "IndexManifest":
        with open(path) as f:
            d = json.loads(f.read(), parse_float=str)
        try:
            ver, cfg = d["version"], d["config"]
            npid, bw = d["next_passage_id"], d["blocks_written"]
        except (KeyError, TypeError) as e:
            raise ValueError(f"manifest: missing {e}") from None
        if not isinstance(ver, str):
            raise ValueError("manifest: `version` expects a string")
        for name, v, hi in (("next_passage_id", npid, 2 ** 64 - 1), ("blocks_written", bw, 2 ** 32 - 1)):
            if isinstance(v, bool) or not isinstance(v, int) or not 0 <= v <= hi:
                raise ValueError(f"manifest: `{name}` expects an unsigned integer")
        return cls(ver, EngineConfig.from_serde(cfg), npid, bw)

    def save(self, path) -> None:
        """engine.rs:213-225 (pretty JSON)."""
        d = {"version": self.version, "config": self.config.to_serde(), "next_passage_id": int(self.next_passage_id),
             "blocks_written": int(self.blocks_written)}
        with open(path, "w") as f:
            f.write(json.dumps(d, indent=2))


def live_slots(segment_path) -> int:
    """Slots not tombstoned in a segment file (the id_map rebuild of
    engine.rs:149-161 counts them): tombstone bits are the u64 at byte 16 of
    each block header (block.rs:34-44)."""
    if not os.path.exists(segment_path):
        return 0
    size = os.path.getsize(segment_path)
    if size == 0 or size % BLOCK_BYTES:
        return 0
    mm = np.memmap(segment_path, dtype=np.uint8, mode="r")
    tomb = np.ascontiguousarray(mm.reshape(-1, BLOCK_BYTES)[:, 16:24]).view("<u8").ravel()
    del mm
    return int(VECTORS_PER_BLOCK * tomb.size - int(np.unpackbits(tomb.view(np.uint8)).sum()))


PASSAGE_INDEX_FILE = "passages.idx"
PASSAGE_INDEX_ENTRY_BYTES = 24  # PassageIndexEntry (passage.rs:44)


def passage_count(directory) -> Optional[int]:
    """PassageStore::len() of an index directory (passage.rs:152-202): the
    number of 24-byte entries in passages.idx; None when the file is absent."""
    path = os.path.join(str(directory), PASSAGE_INDEX_FILE)
    if not os.path.exists(path):
        return None
    size = os.path.getsize(path)
    if size % PASSAGE_INDEX_ENTRY_BYTES:
        raise ValueError(f"{path}: corrupt passage index (size {size} is not a multiple of 24)")
    return size // PASSAGE_INDEX_ENTRY_BYTES


def open_index(directory, device=None, verify_crc: bool = False) -> Tuple[QueryPipeline, DeviceIndex, IndexManifest]:
    """The scan path of IndexEngine::open (engine.rs:132-192) on an index
    directory: manifest.json's config (validated), segments/000001.pax
    streamed into HBM, and the prefix fit -- eden_prefix.json if present,
    else EdenFit::default_prefix(eden_seed) -- when the codec is EdenProd.
    The reopen check compares the segment's live slots with
    PassageStore::len(): the entries of passages.idx (24 bytes each, a size
    that is not a multiple of 24 is PassageError::CorruptIndex;
    passage.rs:152-202).  A directory without passages.idx (the passage
    store is not on the scan path) is checked against the manifest's
    next_passage_id, the passage count it was written with.  Errors raise
    ValueError (config, JSON, passage index, reopen check) or MrlError
    (segment)."""
    directory = str(directory)
    man = IndexManifest.load(os.path.join(directory, MANIFEST_FILE))
    man.config.validate()
    seg = os.path.join(directory, SEGMENT_PATH)
    live = live_slots(seg)
    n_passages = passage_count(directory)
    if n_passages is None:
        n_passages = man.next_passage_id
    if live > n_passages:
        raise ValueError(f"segment/passage mismatch: {live} live slots vs {n_passages} passages")
    index = DeviceIndex.open_segment(seg, device or default_device(), verify_crc)
    fit = None
    if man.config.prefix_codec == PrefixCodec.EDEN_PROD:
        path = os.path.join(directory, EDEN_PREFIX_FILE)
        fit = EdenFit.load_json(path) if os.path.exists(path) else EdenFit.default_prefix(man.config.eden_seed)
    return QueryPipeline(man.config, fit, None), index, man


def scored_hits_to_row_ids(hits: List[ScoredHit]) -> List[int]:
    """pipeline.rs:175-180"""
    return [h.id.block * VECTORS_PER_BLOCK + h.id.slot for h in hits if h.id.block != 0xFFFFFFFF]


def row_id_to_vector_id(row: int) -> VectorId:
    """pipeline.rs:183-188"""
    return VectorId(row // VECTORS_PER_BLOCK, row % VECTORS_PER_BLOCK)
