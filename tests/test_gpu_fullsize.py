"""GPU parity at the benchmark configurations' full sizes, plus the segment
loader, the QueryPipeline seam and an exhaustive f16 meta decode check.

Full-size checks: for every query of every configuration the GPU top-K
equals the oracle's scan_blocks top-K (exact ties excepted) with bit-identical
scores; the first queries against the sharded scan (scan.rs:838-886), the
rest against the serial one (scan.rs:822-836), run query-parallel."""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import _lib, synth
import ora
from helpers import assert_topk_equal

pytestmark = pytest.mark.gpu


def _oracle_all(blocks, qs, w, ofit, n_sharded):
    """The oracle's top K of every query: the first n_sharded through the
    sharded scan on all host threads, the others through serial scans, one
    query per host thread."""
    threads = max(1, min(16, os.cpu_count() or 1))
    sharded = ora.scan_config(w.k, depth=int(w.strata), sharding=True, threads=threads)
    serial = ora.scan_config(w.k, depth=int(w.strata), sharding=False)
    b = np.ascontiguousarray(blocks)

    def one(qi):
        op = ora.plan_build(qs[qi], w.dims, int(w.prefix_codec), 0, ofit, None)
        return ora.scan_blocks(b, op, sharded if qi < n_sharded else serial)

    out = [one(qi) for qi in range(min(n_sharded, w.n_queries))]
    with ThreadPoolExecutor(threads) as ex:
        out += list(ex.map(one, range(len(out), w.n_queries)))
    return out


def _check_config(device, cfg_id, n_sharded, n_queries=None, s4_policy=None, s4_bounded=None):
    """s4_policy: the MFMA final pass's policy for this scan (mrl_ctx_set_s4_bound);
    None keeps the library's own choice.  s4_bounded: whether the final pass
    must have bounded the S4 stage (from its profile record's flag)."""
    if s4_policy is not None:
        device.set_s4_bound(s4_policy)
    try:
        return _check_config_now(device, cfg_id, n_sharded, n_queries, s4_bounded)
    finally:
        device.set_s4_bound(device.S4_BOUND_AUTO)


def _final_pass_flags(device):
    """The flags of the last scan's final pass (the scan record with the
    highest pass index) from the context's profile records."""
    kt = (_lib.KernelTimeC * 256)()
    n = C.c_uint32()
    _lib.check(_lib.lib.mrl_ctx_profile_collect(device.handle, kt, 256, C.byref(n)))
    scans = [kt[i] for i in range(min(n.value, 256)) if kt[i].kind == _lib.KERNEL_SCAN]
    return max(scans, key=lambda r: r.pass_).flags


def _check_config_now(device, cfg_id, n_sharded, n_queries, s4_bounded):
    w = synth.CONFIGS[cfg_id]
    if n_queries:
        w = w.scaled(w.n_docs, n_queries)
    print(f"[fullsize] config {cfg_id}: {w.n_docs} x {w.dims}, {w.n_queries} queries, K={w.k}", flush=True)
    fit = synth.eden_fit(w)
    blocks = synth.encode(w, fit, 16)
    qs, _ = synth.queries(w)
    ix = m.DeviceIndex.upload(blocks, device)
    plan = m.QueryPlan.from_query_codec(qs, w.dims, w.prefix_codec, m.MidCodec.RABITQ, fit, None, device)
    cfg = m.ScanConfig(shortlist_cand=w.k, strata_depth=w.strata, exhaustive=w.exhaustive)
    if s4_bounded is not None:
        _lib.check(_lib.lib.mrl_ctx_set_profiling(device.handle, 1))
    try:
        res = m.scan_batch(ix, plan, cfg)
        if s4_bounded is not None:
            assert bool(_final_pass_flags(device) & 1) == s4_bounded, "final pass variant"
    finally:
        if s4_bounded is not None:
            _lib.check(_lib.lib.mrl_ctx_set_profiling(device.handle, 0))
    ofit = ora.Fit(fit.mean, 4, 1, fit.n_observed) if fit is not None else None
    refs = _oracle_all(blocks, qs, w, ofit, n_sharded)
    for qi in range(w.n_queries):
        n = int(res.counts[qi])
        ids, sc = res.ids[qi, :n], res.scores[qi, :n]
        assert n == min(w.k, w.n_docs)
        assert len(set(ids.tolist())) == n and np.all(sc[:-1] >= sc[1:])
        assert_topk_equal(ids, sc, refs[qi][0], refs[qi][1], w.k, f"config {cfg_id} q={qi}")
    return res


def test_config1_cpu_bench_size(device):
    _check_config(device, 1, 1)


def test_config2_1m_batch1_k256(device):
    """The bench line's own workload at full size: 15,625 blocks, one query,
    K = 256, against the oracle's sharded scan_blocks."""
    _check_config(device, 2, 1)


def test_config3_1m_batch256(device):
    """(the library's rule keeps config 3's final pass on the full tiles)"""
    _check_config(device, 3, 8, s4_bounded=False)


def test_config3_s4_bounded_final_pass(device):
    """Config 3 with its final pass forced to bound the S4 stage."""
    _check_config(device, 3, 8, s4_policy=device.S4_BOUND_ALWAYS, s4_bounded=True)


def test_config4_8_8m_clustered_batch64(device):
    """(the library's rule gives config 4 the S4-bounded final pass)"""
    _check_config(device, 4, 4, s4_bounded=True)


def test_config4_full_tiles(device):
    """Config 4 with its final pass on the full tiles."""
    _check_config(device, 4, 4, s4_policy=device.S4_BOUND_NEVER, s4_bounded=False)


def test_config5_minmax4_exhaustive_batch1024_k1024(device):
    _check_config(device, 5, 4)


def test_f16_meta_decode_exhaustive(device):
    """All 65536 f16 patterns as scale, offset and tail norm of active slots,
    scored at tau = -inf: masks, prefix_ip and scores match the oracle."""
    pats = np.arange(65536, dtype=np.uint16).reshape(1024, 64)
    blocks = np.zeros((3 * 1024, 4096), dtype=np.uint8)
    for part in range(3):
        for b in range(1024):
            blk = blocks[part * 1024 + b]
            meta = blk[64:512].reshape(64, 7)
            vals = pats[b].view(np.uint8).reshape(64, 2)
            meta[:, 2 * part:2 * part + 2] = vals
            if part != 0:
                meta[:, 0:2] = np.frombuffer(np.float16(0.5).tobytes(), dtype=np.uint8)
            meta[:, 6] = (np.arange(64) * 4) % 256
            blk[512 + 0] = 0xFF        # S0 bit for dim 0, all slots -> level 8
            blk[1024:1024 + 8 * 5] = 0xAA
            blk[3072:3072 + 8 * 7] = 0x55
    q = np.zeros(768, dtype=np.float32)
    q[0] = 1.0
    q[64:80] = 0.1
    q[300:310] = 0.2
    plan = m.QueryPlan.from_query(q, 768, device)
    tr = m.scan_fixed_tau(blocks, plan, m.ScanConfig(shortlist_cand=16), -np.inf)
    op = ora.plan_build(q, 768)
    cfg = ora.scan_config(16)
    for b in range(blocks.shape[0]):
        _, mk, pre, sc = ora.block_stages(blocks[b], op, cfg, -np.inf)
        assert np.array_equal(tr.masks[0, b], mk), b
        g, o = tr.prefix_ip[0, b], pre
        same = (g.view(np.uint32) == o.view(np.uint32)) | (np.isnan(g) & np.isnan(o))
        assert same.all(), b
        push = [v for v in range(64) if int(mk[4]) >> v & 1]
        g, o = tr.scores[0, b, push], sc[push]
        same = (g.view(np.uint32) == o.view(np.uint32)) | (np.isnan(g) & np.isnan(o))
        assert same.all(), b


def test_segment_file_and_pipeline(device, tmp_path):
    w = synth.CONFIGS[2].scaled(64 * 50, 2)
    fit = synth.eden_fit(w)
    blocks = synth.encode(w, fit)
    seg = m.SegmentWriter.create(tmp_path / "segments" / "000001.pax")
    for b in blocks:
        seg.append_block(b)
    seg.close()
    ix = m.DeviceIndex.open_segment(str(tmp_path / "segments" / "000001.pax"), device, verify_crc=True)
    assert np.array_equal(ix.download(), blocks)
    empty = m.DeviceIndex.open_segment(str(tmp_path / "missing.pax"), device)
    assert empty.block_count() == 0
    with open(tmp_path / "bad.pax", "wb") as f:
        f.write(b"\0" * 5000)
    with pytest.raises(m.MrlError) as e:
        m.DeviceIndex.open_segment(str(tmp_path / "bad.pax"), device)
    assert e.value.code == 6
    corrupt = blocks.copy()
    corrupt[3, 2000] ^= 0xFF
    with pytest.raises(m.MrlError) as e:
        m.DeviceIndex.upload(corrupt, device, verify_crc=True)
    assert e.value.code == 6
    cfg = m.EngineConfig(embed_dims=768, shortlist_cand=32)
    pipe = m.QueryPipeline.with_eden(cfg, fit)
    qs, _ = synth.queries(w)
    phase = pipe.scan_slab(qs[0], ix)
    direct = m.scan_blocks(ix, m.QueryPlan.from_query_eden(qs[0], 768, fit, device), cfg)
    assert [(h.id, h.score) for h in phase.hits] == [(h.id, h.score) for h in direct]
    rows = m.scored_hits_to_row_ids(phase.hits)
    assert all(m.row_id_to_vector_id(r) == h.id for r, h in zip(rows, phase.hits))
    op = ora.plan_build(qs[0], 768, ora.PREFIX_EDEN_PROD, 0, ora.Fit(fit.mean, 4, 1), None)
    rids, rsc = ora.scan_blocks(blocks, op, ora.scan_config(32))
    assert_topk_equal([h.id.as_u64() for h in phase.hits], [h.score for h in phase.hits], rids, rsc, 32)
