"""ctypes wrapper of the CPU oracle (oracle/_build/libmrl_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  Build with
``make -C oracle``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmrl_oracle.so")

PREFIX_MINMAX4, PREFIX_EDEN_PROD = 0, 1
MID_RABITQ, MID_EDEN_B1 = 0, 1
L0_ONLY, L1_RABITQ, FULL64B = 0, 1, 2
ERR_NAN = 3


def build(quiet: bool = True) -> str:
    subprocess.run(["make", "-C", HERE], check=True, stdout=subprocess.DEVNULL if quiet else None)
    return LIB_PATH


class EdenFitC(C.Structure):
    _fields_ = [("dim", C.c_uint32), ("bits", C.c_uint32), ("seed", C.c_uint64),
                ("mean", C.POINTER(C.c_float)), ("n_observed", C.c_uint64)]


class ScanConfigC(C.Structure):
    _fields_ = [("shortlist_cand", C.c_uint32), ("cs_tolerance", C.c_float), ("stratum4_weight", C.c_float),
                ("strata_depth", C.c_int32), ("temporal_filter_enable", C.c_int32), ("numa_sharding", C.c_int32),
                ("n_threads", C.c_int32), ("reserved", C.c_int32)]


class ScanStatsC(C.Structure):
    _fields_ = [("blocks", C.c_uint64), ("active_vecs", C.c_uint64), ("after_prefix", C.c_uint64),
                ("after_s1", C.c_uint64), ("after_s4_budget", C.c_uint64), ("pushed", C.c_uint64)]


PLAN_FIELDS = [
    ("dims", C.c_uint32), ("prefix_codec", C.c_int32), ("mid_codec", C.c_int32), ("has_tail_fold", C.c_uint32),
    ("prefix", C.c_float * 64), ("bit_weights", (C.c_float * 4) * 64), ("rabitq_q", C.c_float * 128),
    ("rabitq_scale", C.c_float), ("rabitq_weights2", C.c_float * 128), ("rabitq_base", C.c_float),
    ("rabitq_lut", (C.c_float * 16) * 32), ("tail_fold_q", C.c_float * 64),
    ("tail_fold_weights2", C.c_float * 64), ("tail_fold_base", C.c_float), ("q_tail_norm", C.c_float),
    ("q_mid_norm", C.c_float), ("q_after_prefix", C.c_float), ("q_after_s1", C.c_float),
    ("s4_abs_budget", C.c_float), ("prefix_l1", C.c_float), ("prefix_sum", C.c_float),
    ("eden_q_rot", C.c_float * 64), ("eden_mean_ip", C.c_float), ("eden_inv_sqrt_d", C.c_float),
    ("eden_codebook", C.c_float * 16), ("eden_mid_q_rot", C.c_float * 128), ("eden_mid_mean_ip", C.c_float),
    ("eden_mid_inv_sqrt_d", C.c_float), ("eden_mid_codebook", C.c_float * 2), ("prefix_weight", C.c_float * 64),
    ("eden_mid_base", C.c_float), ("eden_mid_deltas", C.c_float * 128), ("pad", C.c_float * 27),
]


class PlanC(C.Structure):
    _fields_ = PLAN_FIELDS


_F = C.POINTER(C.c_float)
_U8 = C.POINTER(C.c_uint8)
_U16 = C.POINTER(C.c_uint16)
_U32 = C.POINTER(C.c_uint32)
_U64 = C.POINTER(C.c_uint64)
_FIT = C.POINTER(EdenFitC)

_SIGS = {
    "ora_plan_size": (C.c_size_t, []),
    "ora_f16_to_f32": (C.c_float, [C.c_uint16]),
    "ora_f32_to_f16": (C.c_uint16, [C.c_float]),
    "ora_f16_to_f32_array": (None, [_U16, _F, C.c_size_t]),
    "ora_f32_to_f16_array": (None, [_F, _U16, C.c_size_t]),
    "ora_meta_decode": (None, [_U8, C.c_int, _F]),
    "ora_pack_rho_flags": (C.c_uint8, [C.c_float, C.c_float]),
    "ora_crc32": (C.c_uint32, [_U8, C.c_size_t]),
    "ora_verify_crc": (C.c_int, [_U8]),
    "ora_fwht_inplace": (None, [_F, C.c_int]),
    "ora_rotate_mid_band": (None, [_F, _F]),
    "ora_rabitq_bit_scale": (C.c_float, []),
    "ora_tail_rademacher": (C.c_float, [C.c_uint64, C.c_uint64]),
    "ora_fold_tail": (None, [_F, C.c_int, _F]),
    "ora_rotate_tail_fold": (None, [_F, C.c_int, _F]),
    "ora_tail_fold_bit_scale": (C.c_float, []),
    "ora_lloyd_max_normal": (C.c_int, [C.c_int, C.POINTER(_F)]),
    "ora_nearest_centroid": (C.c_int, [_F, C.c_int, C.c_float]),
    "ora_rademacher_diag": (C.c_float, [C.c_uint64, C.c_uint64]),
    "ora_structured_hadamard_inplace": (None, [_F, C.c_int, C.c_uint64]),
    "ora_eden_fit_band": (C.c_int, [_F, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, _F]),
    "ora_eden_observe": (None, [_F, C.c_uint32, _U64, _F]),
    "ora_eden_encode_slice": (C.c_int, [_FIT, _F, _U8, _F, _F]),
    "ora_eden_rotate_query": (None, [_FIT, _F, _F]),
    "ora_eden_score_ip": (C.c_float, [_FIT, _F, _F, _U8, C.c_float]),
    "ora_encode_block": (C.c_int, [_F, C.c_int, C.c_int, _U32, _U32, _FIT, _FIT, _U8]),
    "ora_extract_bits4": (None, [_U8, C.c_int, _U8]),
    "ora_plan_build": (C.c_int, [_F, C.c_int, C.c_int, C.c_int, _FIT, _FIT, C.POINTER(PlanC)]),
    "ora_block_stages": (C.c_int, [_U8, C.POINTER(PlanC), C.POINTER(ScanConfigC), C.c_float, C.c_int, C.c_uint32,
                                   C.c_int, C.c_uint32, _U64, _F, _F]),
    "ora_scan_blocks": (C.c_int64, [_U8, C.c_uint64, C.POINTER(PlanC), C.POINTER(ScanConfigC), C.c_int,
                                    C.c_uint32, C.c_int, C.c_uint32, _U64, _F, C.POINTER(ScanStatsC)]),
    "ora_exhaustive_scores": (None, [_U8, C.c_uint64, C.POINTER(PlanC), C.POINTER(ScanConfigC), C.c_int,
                                     C.c_uint32, C.c_int, C.c_uint32, _F, _U8]),
    "ora_dot": (C.c_float, [_F, _F, C.c_uint32]),
    "ora_dot_fp16_768": (C.c_float, [_F, _F]),
    "ora_int8_quantize_768": (None, [_F, C.POINTER(C.c_int8), C.POINTER(C.c_uint16)]),
    "ora_dot_int8_768": (C.c_float, [_F, C.POINTER(C.c_int8), C.c_uint16]),
    "ora_rerank_dot": (C.c_float, [C.c_int, _F, _F, C.c_uint32]),
    "ora_rerank": (C.c_int, [C.c_int, _F, _F, C.c_uint32, _U64, C.c_uint32, _U64, _F]),
    "ora_ring_search_exact": (C.c_int, [_F, C.c_uint32, C.c_uint32, _F, C.c_uint32, _U64, _F]),
    "ora_shortlist_push_sorted": (C.c_int, [C.c_uint32, _U64, _F, C.c_uint32, _U64, _F, C.c_uint32, _U64, _F]),
}

RERANK_FP32, RERANK_FP16, RERANK_INT8 = 0, 1, 2


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def fp(a):
    return a.ctypes.data_as(_F)


def u8p(a):
    return a.ctypes.data_as(_U8)


def u32p(a):
    return a.ctypes.data_as(_U32)


def u64p(a):
    return a.ctypes.data_as(_U64)


class Fit:
    """Holds an EdenFit mean alive next to its C view."""

    def __init__(self, mean, bits, seed, n_observed=0):
        self.mean = np.ascontiguousarray(mean, dtype=np.float32)
        self.c = EdenFitC(self.mean.shape[0], bits, seed, fp(self.mean), n_observed)

    def ref(self):
        return C.byref(self.c)


def _fitref(f):
    return f.ref() if f is not None else None


def plan_build(query, dims, prefix_codec=PREFIX_MINMAX4, mid_codec=MID_RABITQ, eden=None, eden_mid=None):
    q = np.ascontiguousarray(query, dtype=np.float32)
    p = PlanC()
    rc = lib.ora_plan_build(fp(q), dims, prefix_codec, mid_codec, _fitref(eden), _fitref(eden_mid), C.byref(p))
    if rc != 0:
        raise ValueError(f"ora_plan_build rc={rc}")
    return p


def scan_config(k=64, alpha=1.0, w_s4=0.2, depth=FULL64B, temporal=True, sharding=False, threads=1):
    return ScanConfigC(k, alpha, w_s4, depth, int(temporal), int(sharding), threads, 0)


def encode_block(vecs, dims, timestamps=None, sources=None, eden=None, eden_mid=None):
    v = np.ascontiguousarray(vecs, dtype=np.float32).reshape(-1, dims)
    n = v.shape[0]
    ts = np.ascontiguousarray(np.arange(n) if timestamps is None else timestamps, dtype=np.uint32)
    src = np.ascontiguousarray(np.ones(n) if sources is None else sources, dtype=np.uint32)
    out = np.zeros(4096, dtype=np.uint8)
    rc = lib.ora_encode_block(fp(v), n, dims, u32p(ts), u32p(src), _fitref(eden), _fitref(eden_mid), u8p(out))
    if rc != 0:
        raise ValueError(f"ora_encode_block rc={rc}")
    return out


def block_stages(block, plan, cfg, tau, lo=None, hi=None):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    masks = np.zeros(5, dtype=np.uint64)
    pre = np.zeros(64, dtype=np.float32)
    sc = np.zeros(64, dtype=np.float32)
    scored = lib.ora_block_stages(u8p(b), C.byref(plan), C.byref(cfg), tau, int(lo is not None), int(lo or 0),
                                  int(hi is not None), int(hi or 0), u64p(masks), fp(pre), fp(sc))
    return scored, masks, pre, sc


def scan_blocks(blocks, plan, cfg, lo=None, hi=None, stats=False):
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 4096)
    k = max(cfg.shortlist_cand, 1)
    ids = np.zeros(k, dtype=np.uint64)
    scores = np.zeros(k, dtype=np.float32)
    st = ScanStatsC()
    n = lib.ora_scan_blocks(u8p(b), b.shape[0], C.byref(plan), C.byref(cfg), int(lo is not None), int(lo or 0),
                            int(hi is not None), int(hi or 0), u64p(ids), fp(scores),
                            C.byref(st) if stats else None)
    if n < 0:
        raise FloatingPointError("NaN score reached Shortlist::into_sorted")
    out = (ids[:n].copy(), scores[:n].copy())
    if stats:
        return out + ({f: getattr(st, f) for f, _ in ScanStatsC._fields_},)
    return out


def exhaustive_scores(blocks, plan, cfg, lo=None, hi=None):
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 4096)
    sc = np.zeros(b.shape[0] * 64, dtype=np.float32)
    valid = np.zeros(b.shape[0] * 64, dtype=np.uint8)
    lib.ora_exhaustive_scores(u8p(b), b.shape[0], C.byref(plan), C.byref(cfg), int(lo is not None), int(lo or 0),
                              int(hi is not None), int(hi or 0), fp(sc), u8p(valid))
    return sc, valid.astype(bool)


def exhaustive_topk(blocks, plan, cfg, k, lo=None, hi=None):
    """Top-K of the exhaustive scores, ordered by (score desc, id asc)."""
    sc, valid = exhaustive_scores(blocks, plan, cfg, lo, hi)
    rows = np.nonzero(valid)[0]
    s = sc[rows]
    order = np.lexsort((rows, -s.astype(np.float64)))[:k]
    rows = rows[order]
    ids = ((rows // 64).astype(np.uint64) << np.uint64(16)) | (rows % 64).astype(np.uint64)
    return ids, s[order]


def plan_to_dict(p):
    return {name: np.ctypeslib.as_array(getattr(p, name)).copy() if hasattr(getattr(p, name), "_length_")
            else getattr(p, name) for name, _ in PLAN_FIELDS}


# ---- post-scan rerank (src/pipeline.rs:157-169, src/lowprec.rs, src/embed.rs:115-206) ----
def dot(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib.ora_dot(fp(a), fp(b), a.size)


def dot_fp16_768(q, v):
    q = np.ascontiguousarray(q, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    return lib.ora_dot_fp16_768(fp(q), fp(v))


def int8_quantize_768(v):
    """Int8Vec768::from_f32 -> (codes int8[768], scale f16 bits)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    codes = np.zeros(768, dtype=np.int8)
    sc = C.c_uint16(0)
    lib.ora_int8_quantize_768(fp(v), codes.ctypes.data_as(C.POINTER(C.c_int8)), C.byref(sc))
    return codes, sc.value


def dot_int8_768(q, codes, scale_bits):
    q = np.ascontiguousarray(q, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    return lib.ora_dot_int8_768(fp(q), codes.ctypes.data_as(C.POINTER(C.c_int8)), scale_bits)


def rerank_dot(precision, q, row):
    q = np.ascontiguousarray(q, dtype=np.float32)
    row = np.ascontiguousarray(row, dtype=np.float32)
    return lib.ora_rerank_dot(precision, fp(q), fp(row), q.size)


def rerank(precision, q, rows, cand):
    """rerank_exact_rows at a precision: (rows, scores) sorted; None where the
    reference would panic on a NaN score."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    cand = np.ascontiguousarray(cand, dtype=np.uint64)
    n = cand.size
    out_r = np.zeros(max(n, 1), dtype=np.uint64)
    out_s = np.zeros(max(n, 1), dtype=np.float32)
    rc = lib.ora_rerank(precision, fp(q), fp(rows), rows.shape[1], u64p(cand), n, u64p(out_r), fp(out_s))
    if rc != 0:
        return None
    return out_r[:n], out_s[:n]


def ring_search_exact(pending, q, top_k):
    """(local indices, scores) of RingBuffer::search_exact; None on NaN."""
    p = np.ascontiguousarray(pending, dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n = p.shape[0]
    out_l = np.zeros(max(n, 1), dtype=np.uint64)
    out_s = np.zeros(max(n, 1), dtype=np.float32)
    rc = lib.ora_ring_search_exact(fp(p), n, p.shape[1] if p.ndim == 2 else q.size, fp(q), top_k, u64p(out_l),
                                   fp(out_s))
    if rc < 0:
        return None
    return out_l[:rc], out_s[:rc]


def shortlist_push_sorted(capacity, ids, scores, push_ids, push_scores):
    """Shortlist holding (ids, scores) in that internal order, push the others
    in order, into_sorted.  None on NaN."""
    ids = np.ascontiguousarray(ids, dtype=np.uint64)
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    pi = np.ascontiguousarray(push_ids, dtype=np.uint64)
    ps = np.ascontiguousarray(push_scores, dtype=np.float32)
    cap = max(capacity, 1)
    out_i = np.zeros(cap, dtype=np.uint64)
    out_s = np.zeros(cap, dtype=np.float32)
    rc = lib.ora_shortlist_push_sorted(capacity, u64p(ids), fp(scores), ids.size, u64p(pi), fp(ps), pi.size,
                                       u64p(out_i), fp(out_s))
    if rc < 0:
        return None
    return out_i[:rc], out_s[:rc]
