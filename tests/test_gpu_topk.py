"""GPU top-K edge cases: exact ties, segment overflow, empty and partial inputs,
K limits, NaN reporting."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized, oracle_encode_corpus, oracle_fit

pytestmark = pytest.mark.gpu


def _identical_blocks(n_blocks, dims=384, seed=3):
    rng = np.random.default_rng(seed)
    v = normalized(rng, 1, dims)
    blk = m.encode_block(np.repeat(v, 64, axis=0), np.arange(64), np.full(64, 8), dims)
    out = np.repeat(blk[None, :], n_blocks, axis=0).copy()
    # distinct timestamps do not matter for the scan; keep the encoder's bytes
    return v[0], out


def _minmax_plan(q, dims, device):
    return m.QueryPlan.from_query(q, dims, device)


@pytest.mark.parametrize("k", [16, 256])
def test_exact_ties_keep_smallest_ids(device, k):
    q, blocks = _identical_blocks(300)
    plan = _minmax_plan(q, 384, device)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=k))
    n = int(res.counts[0])
    assert n == k
    ids = res.ids[0, :n]
    rows = (ids >> np.uint64(16)) * np.uint64(64) + (ids & np.uint64(0xFFFF))
    assert np.array_equal(np.sort(rows), np.arange(k, dtype=np.uint64)), "ties resolve to the smallest ids"
    op = ora.plan_build(q, 384)
    ref_ids, ref_sc = ora.scan_blocks(blocks, op, ora.scan_config(k))
    assert np.all(res.scores[0, :n].view(np.uint32) == ref_sc[0].view(np.uint32))


def test_segment_overflow_dense_rerun(device):
    # 2000 blocks of one vector: every pass appends everything, segments overflow
    q, blocks = _identical_blocks(2000)
    plan = _minmax_plan(q, 384, device)
    k = 4096
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=k))
    n = int(res.counts[0])
    assert n == k
    ids = res.ids[0, :n]
    rows = (ids >> np.uint64(16)) * np.uint64(64) + (ids & np.uint64(0xFFFF))
    assert np.array_equal(np.sort(rows), np.arange(k, dtype=np.uint64))


def test_k_larger_than_corpus_and_partial_block(device):
    rng = np.random.default_rng(8)
    rows = normalized(rng, 100, 768)  # 1 full block + 36 in a tombstoned-tail block
    fit = oracle_fit(rows)
    blocks = oracle_encode_corpus(rows, 768, fit)
    q = rows[7]
    plan = m.QueryPlan.from_query_eden(q, 768, m.EdenFit(64, 4, 1, fit.mean, 100), device)
    res = m.scan_batch(blocks, plan, m.ScanConfig(shortlist_cand=4096))
    op = ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
    ref_ids, ref_sc = ora.scan_blocks(blocks, op, ora.scan_config(4096))
    assert int(res.counts[0]) == len(ref_ids) <= 100
    assert_topk_equal(res.ids[0, :len(ref_ids)], res.scores[0, :len(ref_ids)], ref_ids, ref_sc, 4096)


def test_empty_index_and_all_tombstoned(device):
    rng = np.random.default_rng(9)
    q = normalized(rng, 1, 384)[0]
    plan = _minmax_plan(q, 384, device)
    empty = np.zeros((0, 4096), dtype=np.uint8)
    res = m.scan_batch(empty, plan, m.ScanConfig(shortlist_cand=16))
    assert int(res.counts[0]) == 0
    _, blocks = _identical_blocks(3)
    blocks[:, 16:24] = 0xFF
    res = m.scan_batch(blocks, plan, m.ScanConfig(shortlist_cand=16))
    assert int(res.counts[0]) == 0


def test_k_zero_behaves_as_one_and_k_limit(device):
    rng = np.random.default_rng(10)
    rows = normalized(rng, 640, 384)
    blocks = oracle_encode_corpus(rows, 384)
    plan = _minmax_plan(rows[3], 384, device)
    res = m.scan_batch(blocks, plan, m.ScanConfig(shortlist_cand=0))
    op = ora.plan_build(rows[3], 384)
    ref_ids, ref_sc = ora.scan_blocks(blocks, op, ora.scan_config(0))
    assert int(res.counts[0]) == 1 == len(ref_ids)
    assert res.ids[0, 0] == ref_ids[0] and res.scores[0, 0].view(np.uint32) == ref_sc[0].view(np.uint32)
    with pytest.raises(m.MrlError) as e:
        m.scan_batch(blocks, plan, m.ScanConfig(shortlist_cand=4097))
    assert e.value.code == 1


def test_nan_score_is_an_error(device):
    """A NaN score among survivors is MRL_ERR_NAN (the reference panics in
    Shortlist::into_sorted, scan.rs:390-394)."""
    rng = np.random.default_rng(14)
    rows = normalized(rng, 64, 768)
    blocks = oracle_encode_corpus(rows, 768)
    q = rows[0].copy()
    q[700] = np.inf
    op = ora.plan_build(q, 768)
    sc, valid = ora.exhaustive_scores(blocks, op, ora.scan_config(64))
    assert np.isnan(sc[valid]).any()
    plan = _minmax_plan(q, 768, device)
    with pytest.raises(m.MrlError) as e:
        m.scan_batch(blocks, plan, m.ScanConfig(shortlist_cand=64))
    assert e.value.code == 3


def test_final_floor_shortfall_reruns_at_the_safe_floor(device):
    """The final pass prunes and appends at a floor taken from the sampling
    pass (a higher rank than K).  Here the vectors near the query all sit in
    sampled blocks (every 16th of 4096), so that floor lies above the true
    K-th score and too few candidates remain: the query must be re-run at the
    safe floor and still return the exact top K."""
    rng = np.random.default_rng(15)
    n_blocks, dims, k = 4096, 192, 64
    rows = normalized(rng, n_blocks * 64, dims)
    q = normalized(rng, 1, dims)[0]
    near = (np.arange(40) // 8) * 16 * 64 + (np.arange(40) % 8)  # 8 slots in each of 5 sampled blocks
    rows[near] = q[None, :] + np.float32(0.02) * normalized(rng, 40, dims)
    rows[near] /= np.linalg.norm(rows[near], axis=1, keepdims=True).astype(np.float32)
    blocks = m.encode_corpus(rows, 8)
    plan = _minmax_plan(q, dims, device)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=k))
    op = ora.plan_build(q, dims)
    ref_ids, ref_sc = ora.scan_blocks(blocks, op, ora.scan_config(k))
    n = int(res.counts[0])
    assert n == len(ref_ids) == k
    assert_topk_equal(res.ids[0, :n], res.scores[0, :n], ref_ids, ref_sc, k)
