"""Post-scan rerank at fp32 / fp16 / int8 (src/lowprec.rs, src/pipeline.rs:157-169),
served by the MI355X library.

``RerankStore`` holds the corpus rows in HBM at one ``RerankPrecision``.  The
reference converts a row with ``Fp16Vec768::from_f32`` / ``Int8Vec768::from_f32``
inside every ``rerank_dot`` call (lowprec.rs:103-121); the conversion depends
only on the row, so the store does it once, on the GPU, with the same
arithmetic, and every rerank reads the converted rows.
"""
from __future__ import annotations

import ctypes as C
from enum import IntEnum
from typing import Optional, Sequence, Tuple

import numpy as np

from . import _lib
from .scan import Device, DeviceBuffer, default_device

EMBED_DIMS_768 = 768
BYTES_FP32_768 = EMBED_DIMS_768 * 4
BYTES_FP16_768 = EMBED_DIMS_768 * 2
BYTES_INT8_768 = EMBED_DIMS_768 + 2


class RerankPrecision(IntEnum):
    """lowprec.rs:18-41"""
    FP32 = 0
    FP16 = 1
    INT8 = 2

    def as_str(self) -> str:
        return ("fp32", "fp16", "int8")[int(self)]

    def bytes_per_vec(self) -> int:
        return (BYTES_FP32_768, BYTES_FP16_768, BYTES_INT8_768)[int(self)]


class RerankStore:
    """Corpus rows resident in HBM at one rerank precision (mrl_rerank_store)."""

    def __init__(self, handle, device: Device, n_rows: int, dims: int, precision: RerankPrecision):
        self._h = handle
        self.device = device
        self.n_rows = n_rows
        self.dims = dims
        self.precision = RerankPrecision(precision)

    @classmethod
    def create(cls, rows, precision=RerankPrecision.FP32, device: Optional[Device] = None,
               n_rows: Optional[int] = None, dims: Optional[int] = None) -> "RerankStore":
        """rows: an (n, dims) float32 array, or a DeviceBuffer holding n_rows x
        dims float32 (then n_rows and dims are required)."""
        dev = device or default_device()
        h = C.c_void_p()
        if isinstance(rows, DeviceBuffer):
            if n_rows is None or dims is None:
                raise ValueError("n_rows and dims are required for a DeviceBuffer")
            if n_rows * dims * 4 > rows.nbytes:
                raise ValueError("buffer smaller than n_rows x dims float32")
            _lib.check(_lib.lib.mrl_rerank_store_create(dev.handle, C.c_void_p(rows.ptr), 1, n_rows, dims,
                                                        int(precision), C.byref(h)))
        else:
            a = np.ascontiguousarray(rows, dtype=np.float32)
            if a.ndim != 2:
                raise ValueError("rows must be (n, dims)")
            n_rows, dims = a.shape
            _lib.check(_lib.lib.mrl_rerank_store_create(dev.handle, _lib.vptr(a), 0, n_rows, dims,
                                                        int(precision), C.byref(h)))
        return cls(h, dev, int(n_rows), int(dims), precision)

    @property
    def handle(self):
        return self._h

    def download(self):
        """The stored rows in the reference's form: FP32 (n, dims) float32;
        FP16 (n, 768) float16 (Fp16Vec768.data); INT8 ((n, 768) int8 codes,
        (n,) float16 scales) (Int8Vec768)."""
        n = self.n_rows
        if self.precision == RerankPrecision.FP32:
            out = np.empty((n, self.dims), dtype=np.float32)
            _lib.check(_lib.lib.mrl_rerank_store_download(self.device.handle, self._h, _lib.vptr(out), None))
            return out
        if self.precision == RerankPrecision.FP16:
            out = np.empty((n, 768), dtype=np.uint16)
            _lib.check(_lib.lib.mrl_rerank_store_download(self.device.handle, self._h, _lib.vptr(out), None))
            return out.view(np.float16)
        codes = np.empty((n, 768), dtype=np.int8)
        scales = np.empty(n, dtype=np.uint16)
        _lib.check(_lib.lib.mrl_rerank_store_download(self.device.handle, self._h, _lib.vptr(codes),
                                                      scales.ctypes.data_as(C.POINTER(C.c_uint16))))
        return codes, scales.view(np.float16)

    def close(self):
        if self._h:
            _lib.lib.mrl_rerank_store_destroy(self._h)
            self._h = None

    def __len__(self):
        return self.n_rows

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rerank_batch(store: RerankStore, queries, cand_rows, counts=None) -> Tuple[np.ndarray, np.ndarray]:
    """rerank_exact_rows (pipeline.rs:157-169) at the store's precision for a
    batch: queries (n_q, dims); cand_rows (n_q, stride) row ids, the first
    counts[q] of row q used (all when counts is None).  Returns (rows, scores),
    each (n_q, stride); row q's first counts[q] entries are its candidates
    sorted by score, descending, ties in input order."""
    q = np.ascontiguousarray(np.atleast_2d(np.asarray(queries, dtype=np.float32)))
    c = np.ascontiguousarray(np.atleast_2d(np.asarray(cand_rows, dtype=np.uint64)))
    n_q, stride = c.shape
    if q.shape != (n_q, store.dims):
        raise ValueError("queries must be (n_q, dims) with one row per candidate list")
    cnt = np.full(n_q, stride, dtype=np.uint32) if counts is None else np.ascontiguousarray(counts, dtype=np.uint32)
    rows = np.zeros((n_q, stride), dtype=np.uint64)
    scores = np.zeros((n_q, stride), dtype=np.float32)
    _lib.check(_lib.lib.mrl_rerank_rows(store.device.handle, store.handle, _lib.fptr(q), n_q, store.dims,
                                        _lib.u64ptr(c), _lib.u32ptr(cnt), stride, _lib.u64ptr(rows),
                                        _lib.fptr(scores)))
    return rows, scores


def rerank_rows(query, candidate_ids: Sequence[int], store: RerankStore):
    """One query: list of (row, score), score descending (pipeline.rs:157-169)."""
    ids = np.asarray(list(candidate_ids), dtype=np.uint64)
    if ids.size == 0:
        return []
    rows, scores = rerank_batch(store, np.asarray(query, dtype=np.float32)[None, :], ids[None, :])
    return [(int(r), float(s)) for r, s in zip(rows[0], scores[0])]
