"""Host encoder (src/quantize.rs, src/encoder.rs) through the C ABI."""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import _lib
from .block import BLOCK_BYTES, source
from .eden import EdenFit


def _fitp(fit: Optional[EdenFit]):
    import ctypes as C
    return C.byref(fit.to_c()) if fit is not None else None


def encode_block(vectors, timestamps, sources, dims: int, eden: Optional[EdenFit] = None,
                 eden_mid: Optional[EdenFit] = None) -> np.ndarray:
    """encode_block_with_fits (quantize.rs:36-96): up to 64 rows -> one 4096-byte block."""
    v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1, dims)
    ts = np.ascontiguousarray(timestamps, dtype=np.uint32)
    src = np.ascontiguousarray(sources, dtype=np.uint32)
    out = np.zeros(BLOCK_BYTES, dtype=np.uint8)
    ef = eden.to_c() if eden is not None else None
    mf = eden_mid.to_c() if eden_mid is not None else None
    import ctypes as C
    _lib.check(_lib.lib.mrl_encode_block(_lib.fptr(v), v.shape[0], dims, _lib.u32ptr(ts), _lib.u32ptr(src),
                                         C.byref(ef) if ef else None, C.byref(mf) if mf else None, _lib.vptr(out)))
    return out


def encode_corpus(matrix, default_source: int = source.DOC, eden: Optional[EdenFit] = None,
                  eden_mid: Optional[EdenFit] = None, n_threads: int = 0) -> np.ndarray:
    """encode_f32_corpus_par (encoder.rs:195-219): timestamps = row index."""
    m = np.ascontiguousarray(matrix, dtype=np.float32)
    n, dims = m.shape
    out = np.zeros(((n + 63) // 64, BLOCK_BYTES), dtype=np.uint8)
    ef = eden.to_c() if eden is not None else None
    mf = eden_mid.to_c() if eden_mid is not None else None
    import ctypes as C
    _lib.check(_lib.lib.mrl_encode_corpus(_lib.fptr(m), n, dims, default_source, C.byref(ef) if ef else None,
                                          C.byref(mf) if mf else None, n_threads, _lib.vptr(out)))
    return out


def encode_corpus_clustered(matrix, cluster, default_source: int = source.DOC, eden: Optional[EdenFit] = None,
                            eden_mid: Optional[EdenFit] = None, n_threads: int = 0) -> np.ndarray:
    """encode_corpus with the cluster-grouped layout convention
    (mrl_encode_corpus_clustered): cluster[i] is row i's coarse cluster, rows
    grouped by cluster; single-cluster blocks record it in their header."""
    m = np.ascontiguousarray(matrix, dtype=np.float32)
    cl = np.ascontiguousarray(cluster, dtype=np.uint32)
    n, dims = m.shape
    if cl.shape != (n,):
        raise ValueError("one cluster per row")
    out = np.zeros(((n + 63) // 64, BLOCK_BYTES), dtype=np.uint8)
    ef = eden.to_c() if eden is not None else None
    mf = eden_mid.to_c() if eden_mid is not None else None
    import ctypes as C
    _lib.check(_lib.lib.mrl_encode_corpus_clustered(_lib.fptr(m), n, dims, _lib.u32ptr(cl), default_source,
                                                    C.byref(ef) if ef else None, C.byref(mf) if mf else None,
                                                    n_threads, _lib.vptr(out)))
    return out


def encode_corpus_device(d_matrix: int, n: int, dims: int, d_out: int, device, default_source: int = source.DOC,
                         eden: Optional[EdenFit] = None, eden_mid: Optional[EdenFit] = None,
                         d_cluster: int = 0) -> None:
    """encode_f32_corpus_par on the GPU: `d_matrix` is the device address of n x dims
    float32 rows, `d_out` of ceil(n/64) * 4096 bytes; byte-identical to encode_corpus."""
    import ctypes as C
    ef = eden.to_c() if eden is not None else None
    mf = eden_mid.to_c() if eden_mid is not None else None
    if d_cluster:
        _lib.check(_lib.lib.mrl_encode_corpus_device_clustered(
            device.handle, C.c_void_p(d_matrix), n, dims, C.c_void_p(d_cluster), default_source,
            C.byref(ef) if ef else None, C.byref(mf) if mf else None, C.c_void_p(d_out)))
        return
    _lib.check(_lib.lib.mrl_encode_corpus_device(device.handle, C.c_void_p(d_matrix), n, dims, default_source,
                                                 C.byref(ef) if ef else None, C.byref(mf) if mf else None,
                                                 C.c_void_p(d_out)))
