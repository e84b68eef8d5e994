"""Scan configuration types, mirroring src/config.rs of the reference."""
from __future__ import annotations

from dataclasses import dataclass, field, replace
from enum import IntEnum

from . import _lib
from .jsonf32 import f32_from_text, f32_text


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

    def to_serde(self) -> dict:
        """The serde form of EngineConfig (config.rs:124-167): the Rust field
        order, enums in snake_case (``exhaustive`` is this build's own and is
        not written)."""
        d = {}
        for name, kind in _SERDE_FIELDS:
            v = getattr(self, name)
            if kind == "enum":
                v = _SERDE_ENUMS[name][type(_SERDE_DEFAULTS_ENUM[name])(v)]
            elif kind == "f32":
                v = float(f32_text(v))  # the shortest text of the f32 (json.dumps writes it back)
            elif kind == "bool":
                v = bool(v)
            elif kind == "residency":
                if v not in _RESIDENCY:
                    raise ValueError(f"slab_residency {v!r}")
            else:
                v = int(v)
            d[name] = v
        return d

    @classmethod
    def from_serde(cls, d: dict) -> "EngineConfig":
        """Deserialize the serde form: every field is required except those
        with #[serde(default)] (use_gemma2 false, prefix_codec min_max4 -- the
        enum's own default, not EngineConfig::default's --, eden_seed 1,
        mid_codec rabitq); unknown fields are ignored; f32 fields are rounded
        once from their decimal text.  Type errors raise ValueError."""
        if not isinstance(d, dict):
            raise ValueError("config: expected an object")
        kw = {}
        for name, kind in _SERDE_FIELDS:
            if name not in d:
                if name in _SERDE_OPTIONAL:
                    kw[name] = _SERDE_OPTIONAL[name]
                    continue
                raise ValueError(f"config: missing field `{name}`")
            v = d[name]
            if kind == "enum":
                inv = {t: e for e, t in _SERDE_ENUMS[name].items()}
                if v not in inv:
                    raise ValueError(f"config: unknown variant {v!r} for `{name}`")
                v = inv[v]
            elif kind == "residency":
                if v not in _RESIDENCY:
                    raise ValueError(f"config: unknown variant {v!r} for `slab_residency`")
            elif kind == "bool":
                if not isinstance(v, bool):
                    raise ValueError(f"config: `{name}` expects a bool")
            elif kind == "f32":
                if isinstance(v, bool) or not isinstance(v, (int, float, str)):
                    raise ValueError(f"config: `{name}` expects a number")
                v = float(f32_text(f32_from_text(str(v))))
            else:
                if isinstance(v, bool) or not isinstance(v, int) or v < 0:
                    raise ValueError(f"config: `{name}` expects an unsigned integer")
            kw[name] = v
        return cls(**kw)


# serde field order and kinds of EngineConfig (config.rs:124-167)
_SERDE_FIELDS = (
    ("strata_depth", "enum"), ("slab_residency", "residency"), ("numa_sharding", "bool"),
    ("shortlist_cand", "usize"), ("cs_tolerance", "f32"), ("stratum4_weight", "f32"),
    ("rabitq_confidence", "f32"), ("jit_batch_size", "usize"), ("io_read_workers", "usize"),
    ("max_latency_budget_ms", "usize"), ("ring_buffer_size", "usize"), ("tombstone_compact_ratio", "f32"),
    ("temporal_filter_enable", "bool"), ("embed_dims", "usize"), ("mrl_prefix", "usize"),
    ("final_top_k", "usize"), ("use_gemma2", "bool"), ("prefix_codec", "enum"), ("eden_seed", "usize"),
    ("mid_codec", "enum"),
)
# #[serde(rename_all = "snake_case")] variant names (config.rs:8-77)
_SERDE_ENUMS = {
    "strata_depth": {StrataDepth.L0_ONLY: "l0_only", StrataDepth.L1_RABITQ: "l1_rabitq",
                     StrataDepth.FULL64B: "full64b"},
    "prefix_codec": {PrefixCodec.MIN_MAX4: "min_max4", PrefixCodec.EDEN_PROD: "eden_prod"},
    "mid_codec": {MidCodec.RABITQ: "rabitq", MidCodec.EDEN_B1: "eden_b1"},
}
_SERDE_DEFAULTS_ENUM = {"strata_depth": StrataDepth.FULL64B, "prefix_codec": PrefixCodec.MIN_MAX4,
                        "mid_codec": MidCodec.RABITQ}
_RESIDENCY = ("ram_locked", "mmap_willneed", "direct_nvme")
# fields with #[serde(default)] (config.rs:155-166)
_SERDE_OPTIONAL = {"use_gemma2": False, "prefix_codec": PrefixCodec.MIN_MAX4, "eden_seed": 1,
                   "mid_codec": MidCodec.RABITQ}
