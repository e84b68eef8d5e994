"""Synthetic workloads of the benchmark configurations.

Generator: x_d = (1+d)^-1/2 z_d (+ mean offset), L2-normalised; clustered
corpora add isotropic noise of norm sigma around seeded centroids; queries
are noisy copies of seeded documents (noise norm sigma, i.e. per-dim
sigma/sqrt(dims)) or fresh draws.  Seeds: documents 42, queries 43,
centroids 44, assignment 45; EDEN Hadamard seed 1 with the prefix mean
fitted on the first 65,536 documents.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import _lib
from .block import BLOCK_BYTES, source
from .config import MidCodec, PrefixCodec, StrataDepth
from .eden import EdenFit

SEED_DOCS, SEED_QUERIES, SEED_CENTROIDS, SEED_ASSIGN = 42, 43, 44, 45
EDEN_FIT_ROWS = 65536


@dataclass
class Workload:
    name: str
    n_docs: int
    dims: int
    n_queries: int
    k: int
    prefix_codec: PrefixCodec = PrefixCodec.EDEN_PROD
    mean_offset: float = 0.0
    n_centroids: int = 0
    centroid_noise: float = 0.0
    query_noise: float = 0.1
    fresh_queries: bool = False
    exhaustive: bool = False
    strata: StrataDepth = StrataDepth.FULL64B

    def spec(self) -> _lib.SynthSpecC:
        return _lib.SynthSpecC(self.n_docs, self.dims, self.mean_offset, SEED_DOCS, self.n_centroids,
                               SEED_CENTROIDS, SEED_ASSIGN, self.centroid_noise)

    def scaled(self, n_docs: int, n_queries: Optional[int] = None) -> "Workload":
        from dataclasses import replace
        return replace(self, n_docs=n_docs, n_queries=n_queries or self.n_queries,
                       name=f"{self.name}@{n_docs}")


# BASELINE.json configs[0..4]
CONFIGS = {
    1: Workload("cpu-bench-131072x384-eden", 131072, 384, 1, 256, fresh_queries=True),
    2: Workload("1m-768-b1", 1_000_000, 768, 1, 256, mean_offset=0.05),
    3: Workload("1m-768-b256", 1_000_000, 768, 256, 256, mean_offset=0.05),
    4: Workload("8.8m-768-clustered-b64", 8_800_000, 768, 64, 256, mean_offset=0.05, n_centroids=1000,
                centroid_noise=0.3),
    5: Workload("1m-768-minmax4-exhaustive-b1024", 1_000_000, 768, 1024, 1024, PrefixCodec.MIN_MAX4,
                mean_offset=0.05, exhaustive=True),
}


def eden_fit(w: Workload) -> Optional[EdenFit]:
    if w.prefix_codec != PrefixCodec.EDEN_PROD:
        return None
    mean = np.zeros(64, dtype=np.float32)
    spec = w.spec()
    rows = min(EDEN_FIT_ROWS, w.n_docs)
    _lib.check(_lib.lib.mrl_synth_eden_fit(C.byref(spec), rows, _lib.fptr(mean)))
    return EdenFit(64, 4, 1, mean, rows)


def docs(w: Workload, first: int = 0, n: Optional[int] = None, n_threads: int = 0) -> np.ndarray:
    n = w.n_docs - first if n is None else n
    out = np.zeros((n, w.dims), dtype=np.float32)
    spec = w.spec()
    _lib.check(_lib.lib.mrl_synth_docs(C.byref(spec), first, n, n_threads, _lib.fptr(out)))
    return out


def queries(w: Workload, n_queries: Optional[int] = None, seed: int = SEED_QUERIES):
    n = w.n_queries if n_queries is None else n_queries
    out = np.zeros((n, w.dims), dtype=np.float32)
    src = np.zeros(n, dtype=np.uint64)
    spec = w.spec()
    _lib.check(_lib.lib.mrl_synth_queries(C.byref(spec), seed, w.query_noise, int(w.fresh_queries), n,
                                          _lib.fptr(out), _lib.u64ptr(src)))
    return out, src


def encode_clustered(w: Workload, fit: Optional[EdenFit], n_threads: int = 0):
    """The same documents in the cluster-grouped layout
    (mrl_synth_encode_clustered): (blocks, rows) with rows[p] the document at
    position p (its id in `encode`'s layout)."""
    out = np.zeros(((w.n_docs + 63) // 64, BLOCK_BYTES), dtype=np.uint8)
    rows = np.zeros(w.n_docs, dtype=np.uint64)
    spec = w.spec()
    f = fit.to_c() if fit is not None else None
    _lib.check(_lib.lib.mrl_synth_encode_clustered(C.byref(spec), C.byref(f) if f else None, None, source.DOC,
                                                   n_threads, _lib.vptr(out), _lib.u64ptr(rows)))
    return out, rows


def encode(w: Workload, fit: Optional[EdenFit], n_threads: int = 0) -> np.ndarray:
    out = np.zeros(((w.n_docs + 63) // 64, BLOCK_BYTES), dtype=np.uint8)
    spec = w.spec()
    f = fit.to_c() if fit is not None else None
    _lib.check(_lib.lib.mrl_synth_encode(C.byref(spec), C.byref(f) if f else None, None, source.DOC, n_threads,
                                         _lib.vptr(out)))
    return out
