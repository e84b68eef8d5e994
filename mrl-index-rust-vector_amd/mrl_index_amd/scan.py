"""The scan API of src/scan.rs, served by the MI355X library.

Names and argument meaning follow the reference: ``QueryPlan.from_query*``
(scan.rs:74-266), ``scan_blocks`` / ``scan_blocks_stats`` (scan.rs:802-886),
``ScoredHit``, ``ScanStats``.  Differences:

* a plan may hold a batch of queries (one row per query), built by one HIP
  kernel launch; ``scan_blocks`` then returns one hit list per query;
* blocks are handed over as a ``DeviceIndex`` (uploaded to HBM once) or as a
  uint8 array that is uploaded for the call;
* errors raise ``MrlError`` where the reference panics.
"""
from __future__ import annotations

import ctypes as C
import threading
from dataclasses import dataclass
from typing import List, Optional, Sequence, Union

import numpy as np

from . import _lib
from .block import BLOCK_BYTES, VectorId, as_blocks
from .config import EngineConfig, MidCodec, PrefixCodec, ScanConfig
from .eden import EdenFit


class Device:
    """One HIP device with its stream (mrl_ctx)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _lib.check(_lib.lib.mrl_ctx_create(device, C.byref(h)))
        self._h = h
        self.device = device

    @property
    def handle(self):
        return self._h

    def synchronize(self) -> None:
        _lib.check(_lib.lib.mrl_ctx_synchronize(self._h))

    S4_BOUND_AUTO, S4_BOUND_ALWAYS, S4_BOUND_NEVER = 0, 1, 2

    def set_s4_bound(self, policy: int) -> None:
        """Cost policy of the MFMA final pass (mrl_ctx_set_s4_bound): AUTO,
        ALWAYS or NEVER replace its four S4 K-steps by a bound of the S4
        score; the results are the same under each."""
        _lib.check(_lib.lib.mrl_ctx_set_s4_bound(self._h, int(policy)))

    def close(self) -> None:
        if self._h:
            _lib.lib.mrl_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default = None
_default_lock = threading.Lock()


class DeviceBuffer:
    """Device memory on `device` (mrl_device_alloc); `ptr` is its device address."""

    def __init__(self, nbytes: int, device: Optional[Device] = None):
        self._dev = device or default_device()
        p = C.c_void_p()
        _lib.check(_lib.lib.mrl_device_alloc(self._dev.handle, nbytes, C.byref(p)))
        self.ptr = p.value or 0
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, a: np.ndarray, device: Optional[Device] = None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        _lib.check(_lib.lib.mrl_copy_to_device(b._dev.handle, C.c_void_p(b.ptr), _lib.vptr(a), a.nbytes))
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        _lib.check(_lib.lib.mrl_copy_to_host(self._dev.handle, _lib.vptr(out), C.c_void_p(self.ptr), out.nbytes))
        return out

    def close(self):
        if self.ptr:
            _lib.lib.mrl_device_free(self._dev.handle, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def default_device() -> Device:
    global _default
    with _default_lock:
        if _default is None:
            _default = Device(0)
        return _default


class DeviceIndex:
    """A slab of PaxBlock64 blocks resident in HBM (mrl_index)."""

    def __init__(self, handle, device: Device):
        self._h = handle
        self.device = device

    @classmethod
    def upload(cls, blocks, device: Optional[Device] = None, verify_crc: bool = False) -> "DeviceIndex":
        device = device or default_device()
        b = as_blocks(blocks)
        h = C.c_void_p()
        _lib.check(_lib.lib.mrl_index_upload(device.handle, _lib.vptr(b), b.shape[0], int(verify_crc),
                                             C.byref(h)))
        return cls(h, device)

    @classmethod
    def from_device(cls, d_blocks: int, n_blocks: int, device: Optional[Device] = None) -> "DeviceIndex":
        """Index over records already in device memory (address d_blocks), e.g. from the GPU encoder."""
        device = device or default_device()
        h = C.c_void_p()
        _lib.check(_lib.lib.mrl_index_from_device(device.handle, C.c_void_p(d_blocks), n_blocks, C.byref(h)))
        return cls(h, device)

    @classmethod
    def open_segment(cls, path: str, device: Optional[Device] = None, verify_crc: bool = False) -> "DeviceIndex":
        """SegmentReader::open (segment.rs:89-162) straight into HBM."""
        device = device or default_device()
        h = C.c_void_p()
        _lib.check(_lib.lib.mrl_index_open_segment(device.handle, str(path).encode(), int(verify_crc), C.byref(h)))
        return cls(h, device)

    @property
    def handle(self):
        return self._h

    def block_count(self) -> int:
        n = C.c_uint64()
        _lib.check(_lib.lib.mrl_index_block_count(self._h, C.byref(n)))
        return n.value

    def __len__(self):
        return self.block_count()

    def download(self) -> np.ndarray:
        out = np.zeros((self.block_count(), BLOCK_BYTES), dtype=np.uint8)
        _lib.check(_lib.lib.mrl_index_download(self.device.handle, self._h, _lib.vptr(out)))
        return out

    def close(self):
        if self._h:
            _lib.lib.mrl_index_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _fit_ref(fit: Optional[EdenFit]):
    return C.byref(fit.to_c()) if fit is not None else None


class QueryPlan:
    """Precomputed query side (scan.rs:20-71), built on the GPU for a batch."""

    def __init__(self, handle, device: Device, n_queries: int, dims: int, prefix_codec, mid_codec, fits):
        self._h = handle
        self.device = device
        self.n_queries = n_queries
        self.dims = dims
        self.prefix_codec = PrefixCodec(prefix_codec)
        self.mid_codec = MidCodec(mid_codec)
        self._fits = fits  # keep the means alive for rebuilds

    @classmethod
    def from_query_codec(cls, query, dims: int, prefix_codec, mid_codec, eden: Optional[EdenFit] = None,
                         eden_mid: Optional[EdenFit] = None, device: Optional[Device] = None) -> "QueryPlan":
        device = device or default_device()
        q = np.ascontiguousarray(query, dtype=np.float32)
        if q.ndim == 1:
            q = q[None, :]
        if q.shape[1] != dims:
            raise _lib.MrlError(_lib.MRL_ERR_INVALID_ARG, "query.len() != dims")  # scan.rs:113
        h = C.c_void_p()
        ef = eden.to_c() if eden is not None else None
        mf = eden_mid.to_c() if eden_mid is not None else None
        _lib.check(_lib.lib.mrl_plans_build(device.handle, _lib.fptr(q), q.shape[0], dims, int(prefix_codec),
                                            int(mid_codec), C.byref(ef) if ef else None,
                                            C.byref(mf) if mf else None, C.byref(h)))
        return cls(h, device, q.shape[0], dims, prefix_codec, mid_codec, (eden, eden_mid))

    @classmethod
    def from_query(cls, query, dims: int, device: Optional[Device] = None) -> "QueryPlan":
        return cls.from_query_codec(query, dims, PrefixCodec.MIN_MAX4, MidCodec.RABITQ, device=device)

    @classmethod
    def from_query_eden(cls, query, dims: int, fit: EdenFit, device: Optional[Device] = None) -> "QueryPlan":
        return cls.from_query_codec(query, dims, PrefixCodec.EDEN_PROD, MidCodec.RABITQ, fit, None, device)

    @classmethod
    def from_query_eden_dual(cls, query, dims: int, prefix: EdenFit, mid: EdenFit,
                             device: Optional[Device] = None) -> "QueryPlan":
        return cls.from_query_codec(query, dims, PrefixCodec.EDEN_PROD, MidCodec.EDEN_B1, prefix, mid, device)

    @property
    def handle(self):
        return self._h

    def export(self, first: int = 0, count: Optional[int] = None) -> List[_lib.QueryPlanC]:
        count = self.n_queries - first if count is None else count
        arr = (_lib.QueryPlanC * max(count, 1))()
        _lib.check(_lib.lib.mrl_plans_export(self.device.handle, self._h, first, count, arr))
        return [arr[i] for i in range(count)]

    def close(self):
        if self._h:
            _lib.lib.mrl_plans_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class ScoredHit:
    """scan.rs:304-308"""
    id: VectorId
    score: float


@dataclass
class ScanStats:
    """scan.rs:270-302 (summed over the queries of one call)."""
    blocks: int = 0
    active_vecs: int = 0
    after_prefix: int = 0
    after_s1: int = 0
    after_s4_budget: int = 0
    pushed: int = 0
    # no reference counterpart: queries the final selection flagged for a
    # re-run at the safe floor / a dense re-run (mrl_scan_stats)
    reruns_safe: int = 0
    reruns_dense: int = 0

    @classmethod
    def from_c(cls, st: "_lib.ScanStatsC") -> "ScanStats":
        return cls(*[getattr(st, f) for f, _ in _lib.ScanStatsC._fields_])

    def merge(self, other: "ScanStats") -> None:
        for f, _ in _lib.ScanStatsC._fields_:
            setattr(self, f, getattr(self, f) + getattr(other, f))

    def summary(self) -> str:
        a = max(self.active_vecs, 1)
        return (f"scan-stats: blocks={self.blocks} active={self.active_vecs}  "
                f"keep_prefix={100.0 * self.after_prefix / a:.2f}%  keep_s1={100.0 * self.after_s1 / a:.2f}%  "
                f"keep_s4bud={100.0 * self.after_s4_budget / a:.2f}%  pushed={100.0 * self.pushed / a:.2f}%")


def _scan_cfg(cfg) -> ScanConfig:
    return cfg.scan_config() if isinstance(cfg, EngineConfig) else cfg


def _time(time_lo, time_hi) -> _lib.TimeRangeC:
    return _lib.TimeRangeC(int(time_lo is not None), int(time_lo or 0), int(time_hi is not None), int(time_hi or 0))


def _as_index(blocks, device: Device):
    if isinstance(blocks, DeviceIndex):
        return blocks, False
    return DeviceIndex.upload(blocks, device), True


@dataclass
class ScanResult:
    """Raw arrays of one batched scan: ids (n_q, K) as VectorId::as_u64,
    scores (n_q, K) and counts (n_q,)."""
    ids: np.ndarray
    scores: np.ndarray
    counts: np.ndarray
    stats: ScanStats

    def hits(self, q: int = 0) -> List[ScoredHit]:
        n = int(self.counts[q])
        return [ScoredHit(VectorId.from_u64(int(i)), float(s)) for i, s in zip(self.ids[q, :n], self.scores[q, :n])]


def scan_batch(blocks: Union["DeviceIndex", np.ndarray], plan: QueryPlan, cfg, time_lo: Optional[int] = None,
               time_hi: Optional[int] = None) -> ScanResult:
    """All plans of ``plan`` against the slab; one call, one device pass per
    pass level."""
    sc = _scan_cfg(cfg)
    idx, owned = _as_index(blocks, plan.device)
    try:
        k = max(int(sc.shortlist_cand), 1)
        nq = plan.n_queries
        ids = np.zeros((nq, k), dtype=np.uint64)
        scores = np.zeros((nq, k), dtype=np.float32)
        counts = np.zeros(nq, dtype=np.uint32)
        st = _lib.ScanStatsC()
        c = sc.to_c()
        t = _time(time_lo, time_hi)
        _lib.check(_lib.lib.mrl_scan(plan.device.handle, idx.handle, plan.handle, C.byref(c), C.byref(t),
                                     _lib.u64ptr(ids), _lib.fptr(scores), _lib.u32ptr(counts), C.byref(st)))
        return ScanResult(ids, scores, counts, ScanStats.from_c(st))
    finally:
        if owned:
            idx.close()


def scan_blocks_stats(blocks, plan: QueryPlan, cfg, time_lo=None, time_hi=None,
                      stats: Optional[ScanStats] = None):
    """scan_blocks_stats (scan.rs:813-886).  Single-query plans return a list
    of ScoredHit; batched plans return one list per query."""
    r = scan_batch(blocks, plan, cfg, time_lo, time_hi)
    if stats is not None:
        stats.merge(r.stats)
    if plan.n_queries == 1:
        return r.hits(0)
    return [r.hits(q) for q in range(plan.n_queries)]


def scan_blocks(blocks, plan: QueryPlan, cfg, time_lo=None, time_hi=None):
    """scan_blocks (scan.rs:802-810)."""
    return scan_blocks_stats(blocks, plan, cfg, time_lo, time_hi, None)


class DeviceResults:
    """Device-resident shortlists of an asynchronous scan (mrl_results): scan
    now, then fetch the hits and / or rerank them on the GPU without the
    shortlist leaving HBM."""

    def __init__(self, n_queries: int, k: int, device: Optional[Device] = None):
        self.device = device or default_device()
        h = C.c_void_p()
        _lib.check(_lib.lib.mrl_results_create(self.device.handle, n_queries, k, C.byref(h)))
        self._h = h
        self.n_queries = n_queries
        self.k = k
        self._plan = None
        self._index = None

    def scan(self, index: "DeviceIndex", plan: QueryPlan, cfg, time_lo=None, time_hi=None) -> None:
        """Enqueue the scan of every plan row (mrl_scan_async); returns at once."""
        c = _scan_cfg(cfg).to_c()
        t = _time(time_lo, time_hi)
        _lib.check(_lib.lib.mrl_scan_async(self.device.handle, index.handle, plan.handle, C.byref(c), C.byref(t),
                                           self._h))
        self._plan, self._index = plan, index  # the results refer to both until fetched
        self._nq = plan.n_queries

    def fetch(self) -> ScanResult:
        nq, k = self._nq, self.k
        ids = np.zeros((nq, k), dtype=np.uint64)
        scores = np.zeros((nq, k), dtype=np.float32)
        counts = np.zeros(nq, dtype=np.uint32)
        st = _lib.ScanStatsC()
        _lib.check(_lib.lib.mrl_results_fetch(self.device.handle, self._h, _lib.u64ptr(ids), _lib.fptr(scores),
                                              _lib.u32ptr(counts), C.byref(st)))
        return ScanResult(ids, scores, counts, ScanStats.from_c(st))

    def floors(self) -> np.ndarray:
        """Per query of the last fetched scan, the floor its list was selected
        at (mrl_results_floors; -inf where none was used)."""
        out = np.zeros(max(self._nq, 1), dtype=np.float32)
        _lib.check(_lib.lib.mrl_results_floors(self.device.handle, self._h, _lib.fptr(out)))
        return out[:self._nq]

    def rerank(self, store) -> "tuple[np.ndarray, np.ndarray, np.ndarray]":
        """scored_hits_to_row_ids + rerank_exact_rows (pipeline.rs:157-180) of
        every query's shortlist against ``store`` (a RerankStore): returns
        (rows (n_q, K), scores (n_q, K), counts (n_q,))."""
        nq, k = self._nq, self.k
        rows = np.zeros((nq, k), dtype=np.uint64)
        scores = np.zeros((nq, k), dtype=np.float32)
        counts = np.zeros(nq, dtype=np.uint32)
        _lib.check(_lib.lib.mrl_results_rerank(self.device.handle, self._h, store.handle, _lib.u64ptr(rows),
                                               _lib.fptr(scores), _lib.u32ptr(counts)))
        return rows, scores, counts

    def close(self):
        if self._h:
            _lib.lib.mrl_results_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class StageTrace:
    """Per (query, block) output of the fixed-threshold diagnostic scan:
    masks[..., 5] = active, after prefix, after S1+CS, after S4 budget, pushed."""
    masks: np.ndarray
    prefix_ip: np.ndarray
    scores: np.ndarray


def scan_fixed_tau(blocks, plan: QueryPlan, cfg, tau, time_lo=None, time_hi=None) -> StageTrace:
    """The stage functions at a fixed threshold per query (mrl_scan_fixed_tau)."""
    sc = _scan_cfg(cfg)
    idx, owned = _as_index(blocks, plan.device)
    try:
        nq, nb = plan.n_queries, idx.block_count()
        tau = np.ascontiguousarray(np.broadcast_to(np.asarray(tau, dtype=np.float32), (nq,)))
        masks = np.zeros((nq, nb, 5), dtype=np.uint64)
        pre = np.zeros((nq, nb, 64), dtype=np.float32)
        scr = np.zeros((nq, nb, 64), dtype=np.float32)
        c = sc.to_c()
        t = _time(time_lo, time_hi)
        _lib.check(_lib.lib.mrl_scan_fixed_tau(plan.device.handle, idx.handle, plan.handle, C.byref(c), C.byref(t),
                                               _lib.fptr(tau), _lib.u64ptr(masks), _lib.fptr(pre), _lib.fptr(scr)))
        return StageTrace(masks, pre, scr)
    finally:
        if owned:
            idx.close()


def index_block_bounds(index: "DeviceIndex", plan: QueryPlan, cfg) -> np.ndarray:
    """Upper bounds of every (query, block) pair's full scores on a
    cluster-grouped index (mrl_index_block_bounds): float32 [query, block],
    NaN for blocks without a bound."""
    sc = _scan_cfg(cfg)
    nq, nb = plan.n_queries, index.block_count()
    out = np.zeros((nq, nb), dtype=np.float32)
    c = sc.to_c()
    _lib.check(_lib.lib.mrl_index_block_bounds(plan.device.handle, index.handle, plan.handle, C.byref(c),
                                               _lib.fptr(out)))
    return out


def scan_mma_bounds(blocks, plan: QueryPlan, cfg, time_lo=None, time_hi=None):
    """Upper and lower bounds of every (query, slot) pair's full score from
    the batched path's f16 MFMA tiles (mrl_scan_mma_bounds): two float32
    arrays [query, block * 64 + slot], NaN where a slot is inactive."""
    sc = _scan_cfg(cfg)
    idx, owned = _as_index(blocks, plan.device)
    try:
        nq, n = plan.n_queries, idx.block_count() * 64
        up = np.zeros((nq, n), dtype=np.float32)
        lo = np.zeros((nq, n), dtype=np.float32)
        c = sc.to_c()
        t = _time(time_lo, time_hi)
        _lib.check(_lib.lib.mrl_scan_mma_bounds(plan.device.handle, idx.handle, plan.handle, C.byref(c), C.byref(t),
                                                _lib.fptr(up), _lib.fptr(lo)))
        return up, lo
    finally:
        if owned:
            idx.close()
