"""C-ABI library on the CPU: it loads, exports every symbol the headers
declare, agrees on struct layouts, and its host-only entry points work
without a GPU (no device compute is called here)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import _lib, synth
import ora

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in ("mrl_scan.h", "mrl_synth.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(mrl_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_lib.LIB_PATH)
    declared = header_functions()
    assert len(declared) >= 30
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} not exported"
    assert declared == set(_lib.SIGNATURES), "ctypes binding and headers disagree"


def test_abi_version_and_plan_layout():
    assert _lib.lib.mrl_abi_version() == 2
    assert C.sizeof(_lib.ScanStatsC) == 64
    assert _lib.lib.mrl_query_plan_size() == C.sizeof(_lib.QueryPlanC) == 6656
    assert ora.lib.ora_plan_size() == 6656
    # identical field layout with the oracle's plan (field by field)
    for (n1, t1), (n2, t2) in zip(_lib.PLAN_FIELDS, ora.PLAN_FIELDS):
        assert n1 == n2 and getattr(_lib.QueryPlanC, n1).offset == getattr(ora.PlanC, n2).offset


def test_no_device_is_an_error_not_a_crash():
    from conftest import gpu_available
    if gpu_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = _lib.lib.mrl_ctx_create(0, C.byref(h))
    assert rc == _lib.MRL_ERR_NO_DEVICE
    assert b"device" in _lib.lib.mrl_last_error()


def test_null_arguments_are_rejected():
    assert _lib.lib.mrl_ctx_create(0, None) == _lib.MRL_ERR_INVALID_ARG
    assert _lib.lib.mrl_index_block_count(None, None) == _lib.MRL_ERR_INVALID_ARG
    assert _lib.lib.mrl_plans_count(None, None) == _lib.MRL_ERR_INVALID_ARG


def test_encode_block_argument_checks():
    v = np.zeros((65, 384), dtype=np.float32)
    with pytest.raises(m.MrlError):
        m.encode_block(v, np.zeros(65), np.zeros(65), 384)       # more than 64 rows
    with pytest.raises(m.MrlError):
        m.encode_block(np.zeros((2, 100)), [0, 1], [0, 1], 100)  # dims < 192


def test_eden_fit_and_json_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    rows = rng.standard_normal((300, 384)).astype(np.float32)
    f = m.EdenFit.fit_prefix(rows, 4, 1)
    assert np.max(np.abs(f.mean - rows[:, :64].mean(axis=0))) < 1e-5
    f.save_json(tmp_path / "eden_prefix.json")
    g = m.EdenFit.load_json(tmp_path / "eden_prefix.json")
    assert np.array_equal(f.mean, g.mean) and g.n_observed == 300 and g.seed == 1


def test_engine_config_defaults_and_validation():
    """config.rs:181-217"""
    c = m.EngineConfig()
    assert c.strata_depth == m.StrataDepth.FULL64B and c.shortlist_cand == 64 and c.cs_tolerance == 1.0
    assert c.stratum4_weight == np.float32(0.2) or abs(c.stratum4_weight - 0.2) < 1e-9
    assert c.prefix_codec == m.PrefixCodec.EDEN_PROD and c.eden_seed == 1 and c.mid_codec == m.MidCodec.RABITQ
    c.validate()
    for bad in (dict(shortlist_cand=8), dict(cs_tolerance=1.5), dict(stratum4_weight=2.0), dict(mrl_prefix=32),
                dict(ring_buffer_size=10), dict(use_gemma2=True)):
        with pytest.raises(ValueError):
            c.copy(**bad).validate()
    assert c.active_strata() == (0, 1, 2, 3, 4, 5)


def test_segment_writer_and_corrupt_size(tmp_path):
    rng = np.random.default_rng(1)
    rows = rng.standard_normal((130, 384)).astype(np.float32)
    blocks = m.encode_corpus(rows)
    w = m.SegmentWriter.create(tmp_path / "segments" / "000001.pax")
    for b in blocks:
        w.append_block(b)
    w.close()
    assert np.array_equal(m.read_segment(tmp_path / "segments" / "000001.pax"), blocks)
    w2 = m.SegmentWriter.open_append(tmp_path / "segments" / "000001.pax")
    assert w2.block_count() == 3
    w2.close()
    with open(tmp_path / "bad.pax", "wb") as f:
        f.write(b"x" * 4097)
    from mrl_index_amd.segment import SegmentError
    with pytest.raises(SegmentError):
        m.read_segment(tmp_path / "bad.pax")


def test_synthetic_generator_is_deterministic_and_shaped():
    w = synth.CONFIGS[2].scaled(640, 3)
    a = synth.docs(w, 0, 128)
    b = synth.docs(w, 64, 64)
    assert np.array_equal(a[64:], b)                       # row r depends only on (seed, r)
    assert np.allclose(np.linalg.norm(a, axis=1), 1.0, atol=1e-5)
    q, src = synth.queries(w)
    assert q.shape == (3, 768) and np.all(src < 640)
    cos = np.sum(q * synth.docs(w, 0, 640)[src.astype(int)], axis=1)
    assert np.all(cos > 0.98)                              # noise norm 0.1 around a document
    blocks = synth.encode(w, synth.eden_fit(w))
    assert blocks.shape == (10, 4096)
    fit = synth.eden_fit(w)
    from helpers import oracle_encode_corpus
    of = ora.Fit(fit.mean, 4, 1, fit.n_observed)
    assert np.array_equal(blocks, oracle_encode_corpus(synth.docs(w), 768, of))
    wc = synth.CONFIGS[4].scaled(640, 2)
    d = synth.docs(wc)
    assert np.allclose(np.linalg.norm(d, axis=1), 1.0, atol=1e-5)
