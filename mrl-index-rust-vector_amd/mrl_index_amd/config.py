"""Scan configuration types, mirroring src/config.rs of the reference."""
from __future__ import annotations

from dataclasses import dataclass, field, replace
from enum import IntEnum

from . import _lib


class PrefixCodec(IntEnum):
    """src/config.rs:10-16"""
    MIN_MAX4 = 0
    EDEN_PROD = 1


class MidCodec(IntEnum):
    """src/config.rs:21-28"""
    RABITQ = 0
    EDEN_B1 = 1


class StrataDepth(IntEnum):
    """src/config.rs:36-67"""
    L0_ONLY = 0
    L1_RABITQ = 1
    FULL64B = 2

    def includes_prefix_4bit(self) -> bool:
        return self is not StrataDepth.L0_ONLY

    def includes_rabitq(self) -> bool:
        return self in (StrataDepth.L1_RABITQ, StrataDepth.FULL64B)

    def includes_tail_fold(self) -> bool:
        return self is StrataDepth.FULL64B


# rotate.rs:120
DEFAULT_STRATUM4_WEIGHT = 0.20


@dataclass
class ScanConfig:
    """src/config.rs:81-114.  ``exhaustive`` is build-specific: score every
    active vector through every gated stage instead of bound pruning (the
    top-K result is the same; only the work differs)."""
    shortlist_cand: int = 64
    cs_tolerance: float = 1.0
    stratum4_weight: float = DEFAULT_STRATUM4_WEIGHT
    strata_depth: StrataDepth = StrataDepth.FULL64B
    temporal_filter_enable: bool = True
    numa_sharding: bool = True
    exhaustive: bool = False

    @classmethod
    def from_engine(cls, cfg: "EngineConfig") -> "ScanConfig":
        return cls(cfg.shortlist_cand, cfg.cs_tolerance, cfg.stratum4_weight, cfg.strata_depth,
                   cfg.temporal_filter_enable, cfg.numa_sharding, cfg.exhaustive)

    def validate(self) -> None:
        """ScanConfig::validate (config.rs:102-113).  Like the reference, the
        scan itself does not call this."""
        if not 16 <= self.shortlist_cand <= 4096:
            raise ValueError("shortlist_cand must be in [16, 4096]")
        if not 0.80 <= self.cs_tolerance <= 1.20:
            raise ValueError("cs_tolerance must be in [0.80, 1.20]")
        if not 0.05 <= self.stratum4_weight <= 1.50:
            raise ValueError("stratum4_weight must be in [0.05, 1.50]")

    def to_c(self) -> _lib.ScanConfigC:
        return _lib.ScanConfigC(int(self.shortlist_cand), float(self.cs_tolerance), float(self.stratum4_weight),
                                int(self.strata_depth), int(bool(self.temporal_filter_enable)),
                                int(bool(self.numa_sharding)), int(bool(self.exhaustive)), 0)


@dataclass
class EngineConfig:
    """src/config.rs:124-201 (defaults as EngineConfig::default)."""
    strata_depth: StrataDepth = StrataDepth.FULL64B
    slab_residency: str = "mmap_willneed"
    numa_sharding: bool = True
    shortlist_cand: int = 64
    cs_tolerance: float = 1.0
    stratum4_weight: float = DEFAULT_STRATUM4_WEIGHT
    rabitq_confidence: float = 2.576
    jit_batch_size: int = 64
    io_read_workers: int = 4
    max_latency_budget_ms: int = 100
    ring_buffer_size: int = 1024
    tombstone_compact_ratio: float = 0.25
    temporal_filter_enable: bool = True
    embed_dims: int = 384
    mrl_prefix: int = 64
    final_top_k: int = 10
    use_gemma2: bool = False
    prefix_codec: PrefixCodec = PrefixCodec.EDEN_PROD
    eden_seed: int = 1
    mid_codec: MidCodec = MidCodec.RABITQ
    exhaustive: bool = False

    def scan_config(self) -> ScanConfig:
        return ScanConfig.from_engine(self)

    def validate(self) -> None:
        """EngineConfig::validate (config.rs:204-217)."""
        self.scan_config().validate()
        if self.embed_dims < 192:
            raise ValueError(f"embed_dims ({self.embed_dims}) must be >= tail_start (192)")
        if self.use_gemma2 and self.embed_dims != 768:
            raise ValueError("use_gemma2 (--gemma2) requires embed_dims == 768")
        if self.mrl_prefix != 64:
            raise ValueError("mrl_prefix must be 64 for PaxBlock64 layout")
        if self.ring_buffer_size < 64:
            raise ValueError("ring_buffer_size must be >= 64")

    def active_strata(self):
        """config.rs:231-240"""
        return {StrataDepth.L0_ONLY: (0,), StrataDepth.L1_RABITQ: (0, 1, 2, 3, 5),
                StrataDepth.FULL64B: (0, 1, 2, 3, 4, 5)}[StrataDepth(self.strata_depth)]

    def copy(self, **kw) -> "EngineConfig":
        return replace(self, **kw)
