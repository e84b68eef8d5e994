"""The allocation-free scan entry point (mrl_scan_noalloc) against the
existing one (mrl_scan_async + mrl_results_fetch), through the C ABI.

Two calls in a row on one context, the second with a smaller input (fewer
queries and a smaller index), for the one-query kernel and for the MFMA
path; queries re-run at the safe floor on the device, alone and in an MFMA
batch; the batch limit.  Results must be identical: ids, scores (bit for
bit) and counts; and the device's free memory (hipMemGetInfo) is the same
before and after the calls."""
import contextlib
import ctypes as C
import gc

import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import _lib
from helpers import normalized, oracle_fit

pytestmark = pytest.mark.gpu

L = _lib.lib


class DevOut:
    """Device-memory outputs for n queries of K entries (allocated by the
    test, the caller of the entry point)."""

    def __init__(self, device, n, k):
        self.device, self.n, self.k = device, n, k
        self.ids = m.DeviceBuffer(max(n * k * 8, 8), device)
        self.scores = m.DeviceBuffer(max(n * k * 4, 4), device)
        self.counts = m.DeviceBuffer(max(n * 4, 4), device)
        self.status = m.DeviceBuffer(max(n * 4, 4), device)

    def fetch(self):
        n, k = self.n, self.k
        return (self.ids.to_array(np.uint64, (n, k)), self.scores.to_array(np.float32, (n, k)),
                self.counts.to_array(np.uint32, (n,)), self.status.to_array(np.uint32, (n,)))


def noalloc(device, ix, plan, cfg, out):
    c = cfg.to_c()
    t = _lib.TimeRangeC(0, 0, 0, 0)
    _lib.check(L.mrl_scan_noalloc(device.handle, ix.handle, plan.handle, C.byref(c), C.byref(t),
                                  C.c_void_p(out.ids.ptr), C.c_void_p(out.scores.ptr), C.c_void_p(out.counts.ptr),
                                  C.c_void_p(out.status.ptr)))
    device.synchronize()
    return out.fetch()


def free_bytes(device):
    f, t = C.c_uint64(), C.c_uint64()
    _lib.check(L.mrl_device_mem_info(device.handle, C.byref(f), C.byref(t)))
    return f.value


@contextlib.contextmanager
def collector_paused():
    """Python's cycle collector paused around a free-memory window: a
    collection inside it could free an earlier test's device buffers and
    change the figure for a reason other than the entry point."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def existing(device, ix, plan, cfg):
    res = m.DeviceResults(plan.n_queries, max(cfg.shortlist_cand, 1), device)
    res.scan(ix, plan, cfg)
    r = res.fetch()
    res.close()
    return r


def assert_same(got, ref, what):
    ids, scores, counts, status = got
    assert np.array_equal(counts, ref.counts), f"{what}: counts"
    assert not (status & 3).any(), f"{what}: status {status}"
    for q in range(len(counts)):
        n = int(counts[q])
        assert np.array_equal(ids[q, :n], ref.ids[q, :n]), f"{what}: ids of query {q}"
        assert np.array_equal(scores[q, :n].view(np.uint32), ref.scores[q, :n].view(np.uint32)), \
            f"{what}: scores of query {q}"


@pytest.fixture(scope="module")
def data(device):
    rng = np.random.default_rng(77)
    rows = normalized(rng, 600 * 64, 768)
    fit = oracle_fit(rows[:4096])
    pf = m.EdenFit(64, 4, 1, fit.mean, 4096)
    blocks = m.encode_corpus(rows, 8, pf)
    return rows, pf, m.DeviceIndex.upload(blocks, device), m.DeviceIndex.upload(blocks[:300], device)


def _plan(rows, pf, n, seed, device):
    rng = np.random.default_rng(seed)
    q = rows[rng.integers(0, rows.shape[0], n)] + np.float32(0.01) * rng.standard_normal((n, 768)).astype(np.float32)
    return m.QueryPlan.from_query_eden(q, 768, pf, device)


@pytest.fixture
def s4_policy(device):
    """Sets the device's S4-bound policy for one test and restores AUTO."""
    def set_policy(p):
        device.set_s4_bound(p)
    yield set_policy
    device.set_s4_bound(device.S4_BOUND_AUTO)


@pytest.mark.parametrize("n_first,n_second,s4", [(5, 2, 0), (40, 9, 0), (64, 1, 0), (40, 9, 1)])
def test_noalloc_matches_existing_entry_point(device, data, s4_policy, n_first, n_second, s4):
    """s4 = 1: the MFMA final pass forced to bound the S4 stage
    (mrl_ctx_set_s4_bound ALWAYS) for both entry points."""
    rows, pf, ix_big, ix_small = data
    s4_policy(s4)
    cfg = m.ScanConfig(shortlist_cand=100)
    out = DevOut(device, n_first, 100)
    p1 = _plan(rows, pf, n_first, n_first, device)
    out2 = DevOut(device, n_second, 100)
    p2 = _plan(rows, pf, n_second, 1000 + n_second, device)
    with collector_paused():
        free0 = free_bytes(device)
        g1 = noalloc(device, ix_big, p1, cfg, out)
        # second call: fewer queries, smaller index, the same array
        g2 = noalloc(device, ix_small, p2, cfg, out2)
        free1 = free_bytes(device)
    assert free1 == free0, "the calls changed the device's free memory"
    assert_same(g1, existing(device, ix_big, p1, cfg), f"first {n_first}")
    assert_same(g2, existing(device, ix_small, p2, cfg), f"second {n_second}")


def test_noalloc_safe_floor_rerun_on_device(device):
    """Near vectors only in sampled blocks: the final floor leaves the query
    short of K; the device re-runs it at the safe floor (the existing entry
    point re-runs it from the host)."""
    rng = np.random.default_rng(15)
    n_blocks, dims, k = 4096, 192, 64
    rows = normalized(rng, n_blocks * 64, dims)
    q = normalized(rng, 1, dims)[0]
    near = (np.arange(40) // 8) * 16 * 64 + (np.arange(40) % 8)
    rows[near] = q[None, :] + np.float32(0.02) * normalized(rng, 40, dims)
    rows[near] /= np.linalg.norm(rows[near], axis=1, keepdims=True).astype(np.float32)
    ix = m.DeviceIndex.upload(m.encode_corpus(rows, 8), device)
    plan = m.QueryPlan.from_query(q, dims, device)
    cfg = m.ScanConfig(shortlist_cand=k)
    ref = existing(device, ix, plan, cfg)
    assert ref.stats.reruns_safe == 1
    out = DevOut(device, 1, k)
    with collector_paused():
        free0 = free_bytes(device)
        got = noalloc(device, ix, plan, cfg, out)
        free1 = free_bytes(device)
    assert free1 == free0
    assert_same(got, ref, "safe-floor re-run")
    assert int(got[2][0]) == k


def test_noalloc_safe_floor_rerun_in_a_batch(device):
    """Nine queries (the MFMA path), each with its near vectors only in
    sampled blocks: every query is flagged and re-run on the device with the
    one-query kernel, gated per query, inside the full candidate room."""
    rng = np.random.default_rng(19)
    n_blocks, dims, k, nq = 4096, 192, 64, 9
    rows = normalized(rng, n_blocks * 64, dims)
    qs = normalized(rng, nq, dims)
    for qi in range(nq):
        blks = 32 * (5 * qi + np.arange(40) // 8)
        near = blks * 64 + np.arange(40) % 8
        rows[near] = qs[qi][None, :] + np.float32(0.02) * normalized(rng, 40, dims)
        rows[near] /= np.linalg.norm(rows[near], axis=1, keepdims=True).astype(np.float32)
    ix = m.DeviceIndex.upload(m.encode_corpus(rows, 8), device)
    plan = m.QueryPlan.from_query(qs, dims, device)
    cfg = m.ScanConfig(shortlist_cand=k)
    ref = existing(device, ix, plan, cfg)
    assert ref.stats.reruns_safe >= 1
    out = DevOut(device, nq, k)
    with collector_paused():
        free0 = free_bytes(device)
        got = noalloc(device, ix, plan, cfg, out)
        free1 = free_bytes(device)
    assert free1 == free0
    assert_same(got, ref, "batched safe-floor re-run")
    assert np.all(got[2] == k)


def test_noalloc_rejects_a_batch_beyond_its_scratch(device, data):
    rows, pf, ix_big, _ = data
    plan = _plan(rows, pf, 65, 3, device)
    out = DevOut(device, 65, 16)
    c = m.ScanConfig(shortlist_cand=16).to_c()
    rc = L.mrl_scan_noalloc(device.handle, ix_big.handle, plan.handle, C.byref(c), None, C.c_void_p(out.ids.ptr),
                            C.c_void_p(out.scores.ptr), C.c_void_p(out.counts.ptr), C.c_void_p(out.status.ptr))
    assert rc == _lib.MRL_ERR_INVALID_ARG
    assert b"at most 64" in L.mrl_last_error()
