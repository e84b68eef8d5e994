"""ctypes binding of libmrl_scan.so (the C ABI declared in include/mrl_scan.h
and include/mrl_synth.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
mrl-index-rust-vector_amd/csrc``).  There is no fallback: if the library is
missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "_build", "libmrl_scan.so")


class MrlError(RuntimeError):
    """A non-zero mrl_status returned through the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"mrl status {code}: {message}")
        self.code = code
        self.message = message


MRL_OK = 0
MRL_ERR_INVALID_ARG = 1
MRL_ERR_HIP = 2
MRL_ERR_NAN = 3
MRL_ERR_OUT_OF_MEMORY = 4
MRL_ERR_NO_DEVICE = 5
MRL_ERR_CORRUPT = 6
MRL_ERR_IO = 7


class EdenFitC(C.Structure):
    _fields_ = [
        ("dim", C.c_uint32),
        ("bits", C.c_uint32),
        ("seed", C.c_uint64),
        ("mean", C.POINTER(C.c_float)),
        ("n_observed", C.c_uint64),
    ]


class ScanConfigC(C.Structure):
    _fields_ = [
        ("shortlist_cand", C.c_uint32),
        ("cs_tolerance", C.c_float),
        ("stratum4_weight", C.c_float),
        ("strata_depth", C.c_int32),
        ("temporal_filter_enable", C.c_int32),
        ("numa_sharding", C.c_int32),
        ("exhaustive", C.c_int32),
        ("reserved", C.c_int32),
    ]


class TimeRangeC(C.Structure):
    _fields_ = [
        ("has_lo", C.c_int32),
        ("lo", C.c_uint32),
        ("has_hi", C.c_int32),
        ("hi", C.c_uint32),
    ]


class ScanStatsC(C.Structure):
    _fields_ = [
        ("blocks", C.c_uint64),
        ("active_vecs", C.c_uint64),
        ("after_prefix", C.c_uint64),
        ("after_s1", C.c_uint64),
        ("after_s4_budget", C.c_uint64),
        ("pushed", C.c_uint64),
        ("reruns_safe", C.c_uint64),
        ("reruns_dense", C.c_uint64),
    ]


# Field list of QueryPlan (src/scan.rs:20-71) + the stage-derived values.
PLAN_FIELDS = [
    ("dims", C.c_uint32),
    ("prefix_codec", C.c_int32),
    ("mid_codec", C.c_int32),
    ("has_tail_fold", C.c_uint32),
    ("prefix", C.c_float * 64),
    ("bit_weights", (C.c_float * 4) * 64),
    ("rabitq_q", C.c_float * 128),
    ("rabitq_scale", C.c_float),
    ("rabitq_weights2", C.c_float * 128),
    ("rabitq_base", C.c_float),
    ("rabitq_lut", (C.c_float * 16) * 32),
    ("tail_fold_q", C.c_float * 64),
    ("tail_fold_weights2", C.c_float * 64),
    ("tail_fold_base", C.c_float),
    ("q_tail_norm", C.c_float),
    ("q_mid_norm", C.c_float),
    ("q_after_prefix", C.c_float),
    ("q_after_s1", C.c_float),
    ("s4_abs_budget", C.c_float),
    ("prefix_l1", C.c_float),
    ("prefix_sum", C.c_float),
    ("eden_q_rot", C.c_float * 64),
    ("eden_mean_ip", C.c_float),
    ("eden_inv_sqrt_d", C.c_float),
    ("eden_codebook", C.c_float * 16),
    ("eden_mid_q_rot", C.c_float * 128),
    ("eden_mid_mean_ip", C.c_float),
    ("eden_mid_inv_sqrt_d", C.c_float),
    ("eden_mid_codebook", C.c_float * 2),
    ("prefix_weight", C.c_float * 64),
    ("eden_mid_base", C.c_float),
    ("eden_mid_deltas", C.c_float * 128),
    ("pad", C.c_float * 27),
]


class QueryPlanC(C.Structure):
    _fields_ = PLAN_FIELDS


class KernelTimeC(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("pass_", C.c_int32),
        ("n_blocks", C.c_uint32),
        ("n_queries", C.c_uint32),
        ("ms", C.c_float),
        ("flags", C.c_uint32),  # MRL_KT_S4_BOUNDED = 1
    ]


(KERNEL_PLAN, KERNEL_SCAN, KERNEL_SELECT, KERNEL_THRESH, KERNEL_RERANK, KERNEL_RERANK_SORT, KERNEL_FINISH,
 KERNEL_MMA_PREP, KERNEL_EXACT, KERNEL_BOUNDS, KERNEL_PLAN_SCAN, KERNEL_PLAN_PREP) = 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11


class SynthSpecC(C.Structure):
    _fields_ = [
        ("n_docs", C.c_uint64),
        ("dims", C.c_uint32),
        ("mean_offset", C.c_float),
        ("seed", C.c_uint64),
        ("n_centroids", C.c_uint32),
        ("seed_centroids", C.c_uint64),
        ("seed_assign", C.c_uint64),
        ("noise_sigma", C.c_float),
    ]


_P = C.c_void_p
_PP = C.POINTER(C.c_void_p)
_F = C.POINTER(C.c_float)
_U32 = C.POINTER(C.c_uint32)
_U64 = C.POINTER(C.c_uint64)

# name -> (restype, argtypes); every symbol declared in include/*.h
SIGNATURES = {
    "mrl_abi_version": (C.c_int, []),
    "mrl_last_error": (C.c_char_p, []),
    "mrl_query_plan_size": (C.c_size_t, []),
    "mrl_ctx_create": (C.c_int, [C.c_int, _PP]),
    "mrl_ctx_destroy": (None, [_P]),
    "mrl_ctx_synchronize": (C.c_int, [_P]),
    "mrl_index_upload": (C.c_int, [_P, _P, C.c_uint64, C.c_int, _PP]),
    "mrl_index_open_segment": (C.c_int, [_P, C.c_char_p, C.c_int, _PP]),
    "mrl_index_block_count": (C.c_int, [_P, _U64]),
    "mrl_index_download": (C.c_int, [_P, _P, _P]),
    "mrl_index_destroy": (None, [_P]),
    "mrl_plans_build": (C.c_int, [_P, _F, C.c_uint32, C.c_uint32, C.c_int, C.c_int,
                                   C.POINTER(EdenFitC), C.POINTER(EdenFitC), _PP]),
    "mrl_plans_build_device": (C.c_int, [_P, _P, C.c_uint32, C.c_uint32, C.c_int, C.c_int,
                                          C.POINTER(EdenFitC), C.POINTER(EdenFitC), _PP]),
    "mrl_plans_rebuild": (C.c_int, [_P, _P]),
    "mrl_plans_count": (C.c_int, [_P, _U32]),
    "mrl_plans_export": (C.c_int, [_P, _P, C.c_uint32, C.c_uint32, C.POINTER(QueryPlanC)]),
    "mrl_plans_destroy": (None, [_P]),
    "mrl_scan": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), C.POINTER(TimeRangeC), _U64, _F, _U32,
                           C.POINTER(ScanStatsC)]),
    "mrl_results_create": (C.c_int, [_P, C.c_uint32, C.c_uint32, _PP]),
    "mrl_results_destroy": (None, [_P]),
    "mrl_scan_async": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), C.POINTER(TimeRangeC), _P]),
    "mrl_results_fetch": (C.c_int, [_P, _P, _U64, _F, _U32, C.POINTER(ScanStatsC)]),
    "mrl_results_floors": (C.c_int, [_P, _P, _F]),
    "mrl_scan_noalloc": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), C.POINTER(TimeRangeC), _P, _P, _P, _P]),
    "mrl_scan_fixed_tau": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), C.POINTER(TimeRangeC), _F, _U64,
                                     _F, _F]),
    "mrl_scan_mma_bounds": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), C.POINTER(TimeRangeC), _F, _F]),
    "mrl_index_block_bounds": (C.c_int, [_P, _P, _P, C.POINTER(ScanConfigC), _F]),
    "mrl_ctx_set_profiling": (C.c_int, [_P, C.c_int]),
    "mrl_ctx_profile_collect": (C.c_int, [_P, C.POINTER(KernelTimeC), C.c_uint32, _U32]),
    "mrl_ctx_evict_caches": (C.c_int, [_P, C.c_uint64]),
    "mrl_ctx_set_s4_bound": (C.c_int, [_P, C.c_int]),
    "mrl_encode_block": (C.c_int, [_F, C.c_uint32, C.c_uint32, _U32, _U32, C.POINTER(EdenFitC),
                                   C.POINTER(EdenFitC), _P]),
    "mrl_encode_corpus": (C.c_int, [_F, C.c_uint64, C.c_uint32, C.c_uint32, C.POINTER(EdenFitC),
                                    C.POINTER(EdenFitC), C.c_int, _P]),
    "mrl_eden_fit_band": (C.c_int, [_F, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, _F]),
    "mrl_encode_corpus_device": (C.c_int, [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, C.POINTER(EdenFitC),
                                           C.POINTER(EdenFitC), _P]),
    "mrl_encode_corpus_clustered": (C.c_int, [_F, C.c_uint64, C.c_uint32, _U32, C.c_uint32, C.POINTER(EdenFitC),
                                              C.POINTER(EdenFitC), C.c_int, _P]),
    "mrl_encode_corpus_device_clustered": (C.c_int, [_P, _P, C.c_uint64, C.c_uint32, _P, C.c_uint32,
                                                     C.POINTER(EdenFitC), C.POINTER(EdenFitC), _P]),
    "mrl_index_from_device": (C.c_int, [_P, _P, C.c_uint64, _PP]),
    "mrl_device_alloc": (C.c_int, [_P, C.c_size_t, _PP]),
    "mrl_device_free": (None, [_P, _P]),
    "mrl_device_mem_info": (C.c_int, [_P, _U64, _U64]),
    "mrl_copy_to_device": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "mrl_copy_to_host": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "mrl_rerank_store_create": (C.c_int, [_P, _P, C.c_int, C.c_uint64, C.c_uint32, C.c_int, _PP]),
    "mrl_rerank_store_destroy": (None, [_P]),
    "mrl_rerank_store_download": (C.c_int, [_P, _P, _P, C.POINTER(C.c_uint16)]),
    "mrl_rerank_rows": (C.c_int, [_P, _P, _F, C.c_uint32, C.c_uint32, _U64, _U32, C.c_uint32, _U64, _F]),
    "mrl_results_rerank": (C.c_int, [_P, _P, _P, _U64, _F, _U32]),
    "mrl_ring_search": (C.c_int, [_P, _F, C.c_uint32, C.c_uint32, _F, C.c_uint32, C.c_uint32, _U64, _F, _U32]),
    "mrl_results_merge_ring": (C.c_int, [_P, _P, _F, C.c_uint32, C.c_uint32]),
    "mrl_synth_docs": (C.c_int, [C.POINTER(SynthSpecC), C.c_uint64, C.c_uint64, C.c_int, _F]),
    "mrl_synth_queries": (C.c_int, [C.POINTER(SynthSpecC), C.c_uint64, C.c_float, C.c_int, C.c_uint32, _F,
                                    _U64]),
    "mrl_synth_eden_fit": (C.c_int, [C.POINTER(SynthSpecC), C.c_uint64, _F]),
    "mrl_synth_encode": (C.c_int, [C.POINTER(SynthSpecC), C.POINTER(EdenFitC), C.POINTER(EdenFitC),
                                   C.c_uint32, C.c_int, _P]),
    "mrl_synth_encode_clustered": (C.c_int, [C.POINTER(SynthSpecC), C.POINTER(EdenFitC), C.POINTER(EdenFitC),
                                             C.c_uint32, C.c_int, _P, _U64]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() or "
            "make -C mrl-index-rust-vector_amd/csrc")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int) -> None:
    if rc != MRL_OK:
        msg = lib.mrl_last_error()
        raise MrlError(rc, msg.decode() if msg else "")


def fptr(a):
    """float* view of a contiguous float32 numpy array."""
    return a.ctypes.data_as(_F)


def u32ptr(a):
    return a.ctypes.data_as(_U32)


def u64ptr(a):
    return a.ctypes.data_as(_U64)


def vptr(a):
    return C.c_void_p(a.ctypes.data)
