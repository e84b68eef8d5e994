"""Block skipping on cluster-grouped indexes (the encoder convention of
mrl_encode_corpus_clustered: coarse_cluster_id and MRL_BLOCK_FLAG_ONE_CLUSTER
in the header bytes the reference's scan never reads, src/block.rs:37-43).

- the GPU encoder writes the same bytes as the host encoder;
- every block bound (mrl_index_block_bounds) is at least the oracle's full
  score (src/scan.rs:453-634, every stage run) of each active slot of the
  block, for both prefix codecs and both S1 depths, and mixed blocks carry no
  bound;
- scans of a cluster-grouped index skip blocks (fewer blocks scanned) and
  still return the oracle's top K: the one-query kernel, k_scan_tile and the
  MFMA path.
"""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized, oracle_fit

pytestmark = pytest.mark.gpu


def clustered_rows(seed, n_clusters, per_cluster, dims, noise=0.3):
    """Rows grouped by cluster (centroid + isotropic noise of norm `noise`,
    renormalised) and their cluster ids; cluster sizes vary."""
    rng = np.random.default_rng(seed)
    cents = normalized(rng, n_clusters, dims)
    sizes = rng.integers(per_cluster // 2, per_cluster * 3 // 2, n_clusters)
    cl = np.repeat(np.arange(n_clusters, dtype=np.uint32), sizes)
    rows = cents[cl] + np.float32(noise / np.sqrt(dims)) * rng.standard_normal((cl.size, dims)).astype(np.float32)
    rows /= np.linalg.norm(rows, axis=1, keepdims=True).astype(np.float32)
    return rows.astype(np.float32), cl


@pytest.fixture(scope="module")
def eden_index(device):
    rows, cl = clustered_rows(31, 48, 640, 768)
    fit = oracle_fit(rows[:8192])
    pf = m.EdenFit(64, 4, 1, fit.mean, 8192)
    blocks = m.encode_corpus_clustered(rows, cl, 8, pf)
    return rows, cl, fit, pf, blocks, m.DeviceIndex.upload(blocks, device)


def test_gpu_encoder_writes_the_cluster_convention(device):
    rows, cl = clustered_rows(5, 9, 150, 384)
    cl[200:230] = 70000  # ids beyond 16 bits are never recorded
    host = m.encode_corpus_clustered(rows, cl, 8)
    d_rows = m.DeviceBuffer.from_array(rows, device)
    d_cl = m.DeviceBuffer.from_array(cl, device)
    d_out = m.DeviceBuffer(host.nbytes, device)
    m.encode_corpus_device(d_rows.ptr, rows.shape[0], 384, d_out.ptr, device, 8, None, None, d_cl.ptr)
    assert np.array_equal(d_out.to_array(np.uint8, host.shape), host)
    plain = m.encode_corpus(rows, 8)
    diff = np.nonzero((plain != host).any(0))[0]
    assert set(diff.tolist()) <= {12, 13, 14, 15, 24, 25, 26, 27}
    h = host[:, 12:16].copy().view(np.uint16).reshape(-1, 2)
    for b in range(host.shape[0]):
        c = cl[64 * b:64 * b + 64]
        one = bool((c == c[0]).all() and c[0] < 65536)
        assert h[b, 1] == (1 if one else 0) and h[b, 0] == (c[0] if one else 0), b
        assert ora.lib.ora_verify_crc(ora.u8p(np.ascontiguousarray(host[b]))) == 1


def _check_bounds(device, blocks, ix, qs, plan, op_fn, cfg_p, cfg_o, cl, what):
    bnd = m.index_block_bounds(ix, plan, cfg_p)
    nb = blocks.shape[0]
    pure = np.array([(cl[64 * b:64 * b + 64] == cl[64 * b]).all() for b in range(nb)])
    gap = []
    for qi in range(qs.shape[0]):
        sc, valid = ora.exhaustive_scores(blocks, op_fn(qs[qi]), cfg_o)
        sc = sc.reshape(nb, 64)
        valid = valid.reshape(nb, 64)
        best = np.where(valid, sc, -np.inf).max(1)
        assert np.isnan(bnd[qi, ~pure]).all(), f"{what}: a mixed block has a bound"
        ok = bnd[qi, pure] >= best[pure]
        assert ok.all(), f"{what} q={qi}: bound below a slot's score in blocks {np.nonzero(pure)[0][~ok][:5]}"
        gap.append(bnd[qi, pure] - best[pure])
    return np.concatenate(gap)


@pytest.mark.parametrize("depth", [m.StrataDepth.FULL64B, m.StrataDepth.L1_RABITQ])
def test_block_bounds_cover_every_slot_eden(device, eden_index, depth):
    rows, cl, fit, pf, blocks, ix = eden_index
    rng = np.random.default_rng(int(depth))
    qs = rows[rng.integers(0, rows.shape[0], 6)] + np.float32(0.05) * rng.standard_normal((6, 768)).astype(np.float32)
    qs[5] *= np.float32(7.0)  # far from unit norm
    plan = m.QueryPlan.from_query_eden(qs, 768, pf, device)
    gap = _check_bounds(device, blocks, ix, qs, plan,
                        lambda q: ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit),
                        m.ScanConfig(shortlist_cand=64, strata_depth=depth), ora.scan_config(64, depth=int(depth)),
                        cl, f"eden depth={depth}")
    assert np.median(gap) < 1.0  # the bound follows the clusters (it is not vacuous)


def test_block_bounds_cover_every_slot_minmax(device):
    rows, cl = clustered_rows(41, 20, 400, 384)
    blocks = m.encode_corpus_clustered(rows, cl, 8)
    ix = m.DeviceIndex.upload(blocks, device)
    rng = np.random.default_rng(2)
    qs = normalized(rng, 5, 384)
    plan = m.QueryPlan.from_query(qs, 384, device)
    for w_s4 in (0.2, 1.3):
        _check_bounds(device, blocks, ix, qs, plan, lambda q: ora.plan_build(q, 384),
                      m.ScanConfig(shortlist_cand=32, stratum4_weight=w_s4),
                      ora.scan_config(32, w_s4=w_s4), cl, f"minmax w_s4={w_s4}")


def test_block_bounds_absent_without_the_convention(device):
    rows, _ = clustered_rows(43, 4, 200, 384)
    ix = m.DeviceIndex.upload(m.encode_corpus(rows, 8), device)
    plan = m.QueryPlan.from_query(rows[:2], 384, device)
    assert np.isnan(m.index_block_bounds(ix, plan, m.ScanConfig())).all()


def _scan_vs_oracle(device, blocks, ix, qs, plan, op_fn, cfg_p, cfg_o, k, what):
    res = m.scan_batch(ix, plan, cfg_p)
    for qi in range(qs.shape[0]):
        rid, rsc = ora.scan_blocks(blocks, op_fn(qs[qi]), cfg_o)
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"{what} q={qi}")
    return res


@pytest.mark.parametrize("nq", [1, 3, 24, 64])
def test_cluster_grouped_scan_skips_blocks_and_matches(device, eden_index, nq):
    """Queries near a few clusters: the final pass scans a fraction of the
    blocks (the one-query kernel at 1 and 3 queries, the MFMA path at 24 and
    64) and the top K is the oracle's."""
    rows, cl, fit, pf, blocks, ix = eden_index
    rng = np.random.default_rng(100 + nq)
    k = 64
    near = np.nonzero(cl < 6)[0]  # queries near 6 of the 48 clusters
    qs = rows[rng.choice(near, nq)] + np.float32(0.1 / np.sqrt(768)) * rng.standard_normal(
        (nq, 768)).astype(np.float32)
    plan = m.QueryPlan.from_query_eden(qs, 768, pf, device)
    res = _scan_vs_oracle(device, blocks, ix, qs, plan,
                          lambda q: ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit),
                          m.ScanConfig(shortlist_cand=k), ora.scan_config(k), k, f"nq={nq}")
    # blocks scanned by the final pass, per query (the sampling pass adds at most half the index)
    nb = blocks.shape[0]
    assert res.stats.blocks < 0.5 * nb * nq + 1, (res.stats.blocks, nb * nq)


def test_cluster_grouped_scan_tile_kernel_contract(device, eden_index):
    """alpha = 0.9 at 9 queries: k_scan_tile with block lists, under the
    fixed-floor contract (the reference's stage checks at the reported floor)."""
    from test_gpu_paths import fixed_floor_topk
    rows, cl, fit, pf, blocks, ix = eden_index
    rng = np.random.default_rng(7)
    qs = rows[rng.choice(np.nonzero(cl < 6)[0], 9)]
    plan = m.QueryPlan.from_query_eden(qs, 768, pf, device)
    cfg = m.ScanConfig(shortlist_cand=48, cs_tolerance=0.9)
    res = m.DeviceResults(9, 48, device)
    res.scan(ix, plan, cfg)
    out = res.fetch()
    floors = res.floors()
    res.close()
    assert out.stats.blocks < 0.5 * blocks.shape[0] * 9
    for qi in range(9):
        op = ora.plan_build(qs[qi], 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
        rid, rsc = fixed_floor_topk(blocks, op, ora.scan_config(48, alpha=0.9), floors[qi], 48)
        n = int(out.counts[qi])
        assert_topk_equal(out.ids[qi, :n], out.scores[qi, :n], rid, rsc, 48, f"tile q={qi}")


def test_cluster_grouped_mma_two_stage_lists(device):
    """An index of more than 2048 blocks at 64 queries: the MFMA path's
    second sampling stage runs over block lists and lists its counted lower
    bounds per workgroup (k_mma_floors_seg); queries near 5 of the 40
    clusters (each spans a few of the stage's every-32nd blocks, so its
    floor comes from the query's own cluster), top K equal to the oracle's,
    blocks skipped."""
    rows, cl = clustered_rows(57, 40, 4400, 768)
    fit = oracle_fit(rows[:8192])
    pf = m.EdenFit(64, 4, 1, fit.mean, 8192)
    blocks = m.encode_corpus_clustered(rows, cl, 8, pf)
    nb = blocks.shape[0]
    assert nb > 2048, nb
    ix = m.DeviceIndex.upload(blocks, device)
    rng = np.random.default_rng(58)
    nq, k = 64, 128
    near = np.nonzero(cl < 5)[0]
    qs = rows[rng.choice(near, nq)] + np.float32(0.1 / np.sqrt(768)) * rng.standard_normal(
        (nq, 768)).astype(np.float32)
    plan = m.QueryPlan.from_query_eden(qs, 768, pf, device)
    res = _scan_vs_oracle(device, blocks, ix, qs, plan,
                          lambda q: ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit),
                          m.ScanConfig(shortlist_cand=k), ora.scan_config(k), k, "two-stage lists")
    assert res.stats.blocks < 0.5 * nb * nq, (res.stats.blocks, nb * nq)
    assert res.stats.reruns_dense == 0
    ix.close()
