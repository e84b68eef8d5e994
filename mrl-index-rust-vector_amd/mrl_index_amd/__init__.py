"""MI355X (gfx950) backend for the PaxBlock64 progressive bitplane scan of
tcondello/mrl-index-rust-vector.  The compute lives in libmrl_scan.so (HIP
kernels behind a C ABI); this package mirrors the reference's Rust scan API
on top of it."""
from ._lib import LIB_PATH, MrlError
from .block import (BLOCK_BYTES, MRL_PREFIX_DIMS, RABITQ_DIMS, TAIL_FOLD_DIMS, TAIL_START, VECTORS_PER_BLOCK,
                    VectorId, source)
from .config import EngineConfig, MidCodec, PrefixCodec, ScanConfig, StrataDepth
from .eden import EdenFit
from .lowprec import RerankPrecision, RerankStore, rerank_batch, rerank_rows
from .ring import PendingVector, RingBuffer
from .pipeline import (IndexManifest, QueryPipeline, ScanPhase, live_slots, open_index, passage_count, row_id_to_vector_id,
                       scored_hits_to_row_ids)
from .quantize import encode_block, encode_corpus, encode_corpus_clustered, encode_corpus_device
from .scan import (Device, DeviceBuffer, DeviceIndex, DeviceResults, QueryPlan, ScanResult, ScanStats, ScoredHit, StageTrace, default_device,
                   index_block_bounds, scan_batch, scan_blocks, scan_blocks_stats, scan_fixed_tau,
                   scan_mma_bounds)
from .segment import SegmentWriter, read_segment
from .shortlist import Shortlist

__all__ = [
    "LIB_PATH", "MrlError", "BLOCK_BYTES", "MRL_PREFIX_DIMS", "RABITQ_DIMS", "TAIL_FOLD_DIMS", "TAIL_START",
    "VECTORS_PER_BLOCK", "VectorId", "source", "EngineConfig", "MidCodec", "PrefixCodec", "ScanConfig",
    "StrataDepth", "EdenFit", "QueryPipeline", "ScanPhase", "row_id_to_vector_id", "scored_hits_to_row_ids",
    "encode_block", "encode_corpus", "encode_corpus_clustered", "encode_corpus_device", "Device", "DeviceBuffer", "DeviceIndex", "QueryPlan", "ScanResult", "ScanStats", "ScoredHit",
    "StageTrace", "default_device", "scan_batch", "scan_blocks", "scan_blocks_stats", "scan_fixed_tau", "scan_mma_bounds",
    "index_block_bounds",
    "SegmentWriter", "read_segment", "DeviceResults", "RerankPrecision", "RerankStore", "rerank_batch",
    "rerank_rows", "PendingVector", "RingBuffer", "IndexManifest", "open_index", "passage_count", "live_slots", "Shortlist",
]
