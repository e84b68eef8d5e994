"""GPU top-K parity of the production paths the other suites leave out, and
the contract for settings under which the reference's stage bounds are not
admissible.

Paths (through mrl_scan / mrl_scan_async, the kernels that production runs):
- the one-query kernel with the EdenB1 mid-band and with L0Only;
- k_scan_tile (8 or more queries off the MFMA path's conditions);
- k_scan<8> for L0Only batches;
- the MFMA path with alpha > 1, with queries far from unit norm, with a
  final floor left short of K (re-run at the safe floor) and with K = 4096
  on a sampled, clustered index.

Contract where the reference's bounds are inadmissible (EdenB1, alpha < 1,
w_s4 > alpha / 2.4; src/config.rs:102-113 accepts these): the reference's
own top K then depends on the order its running threshold rises in.  The GPU
returns the top K of the vectors that the reference's stage functions
(src/scan.rs:453-634) keep at one fixed floor, the one mrl_results_floors
reports, with their scores.  The check runs the oracle's stage functions at
that floor over every block.  Like the reference's shortlist, whose
threshold stays at -inf until it holds K hits, every query returns
min(K, active) hits: a query that the stage functions leave short at the
safe floor is re-run with no floor (-inf).
"""
import json
import os

import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized, oracle_fit, oracle_fit_mid

pytestmark = pytest.mark.gpu

DIMS = 768


def _pfit(f, seed=1):
    return m.EdenFit(64, 4, seed, f.mean, int(f.c.n_observed))


def _mfit(f, seed=7):
    return m.EdenFit(128, 1, seed, f.mean, int(f.c.n_observed))


@pytest.fixture(scope="module")
def corpus(device):
    """320 blocks (> 256: a sampling pass sets the final floor) of 768-d
    rows, encoded twice: EDEN prefix + RaBitQ, and EDEN prefix + EdenB1."""
    rng = np.random.default_rng(2027)
    rows = normalized(rng, 320 * 64 - 9, DIMS)
    pf, mf = oracle_fit(rows[:4096]), oracle_fit_mid(rows[:4096], seed=7)
    blocks = m.encode_corpus(rows, 8, _pfit(pf))
    blocks_b1 = m.encode_corpus(rows, 8, _pfit(pf), _mfit(mf))
    return {"rows": rows, "pf": pf, "mf": mf, "blocks": blocks, "blocks_b1": blocks_b1,
            "ix": m.DeviceIndex.upload(blocks, device), "ix_b1": m.DeviceIndex.upload(blocks_b1, device)}


def _queries(rows, n, seed, noise=0.01):
    rng = np.random.default_rng(seed)
    q = rows[rng.integers(0, rows.shape[0], n)] + np.float32(noise) * rng.standard_normal((n, rows.shape[1]))
    return q.astype(np.float32)


def _scan_async(device, ix, plan, cfg):
    res = m.DeviceResults(plan.n_queries, max(cfg.shortlist_cand, 1), device)
    res.scan(ix, plan, cfg)
    out = res.fetch()
    floors = res.floors()
    res.close()
    return out, floors


def fixed_floor_topk(blocks, op, ocfg, floor, k):
    """Top K (score desc, id asc) of the vectors the oracle's stage functions
    push at the fixed threshold `floor` and whose score reaches it."""
    ids, scs = [], []
    bit = np.uint64(1) << np.arange(64, dtype=np.uint64)
    for b in range(blocks.shape[0]):
        _, mk, _, sc = ora.block_stages(blocks[b], op, ocfg, float(floor))
        pushed = np.nonzero(np.uint64(mk[4]) & bit)[0]
        if pushed.size == 0:
            continue
        s = sc[pushed]
        keep = s >= np.float32(floor)
        ids.append((np.uint64(b) << np.uint64(16)) | pushed[keep].astype(np.uint64))
        scs.append(s[keep])
    if not ids:
        return np.zeros(0, np.uint64), np.zeros(0, np.float32)
    ids, scs = np.concatenate(ids), np.concatenate(scs)
    assert not np.isnan(scs).any()
    order = np.lexsort((ids, -scs.astype(np.float64)))[:k]
    return ids[order], scs[order]


def _n_active(blocks):
    tomb = blocks[:, 16:24].copy().view("<u8")[:, 0]
    return int(sum(64 - bin(int(t)).count("1") for t in tomb))


def _check_contract(res, floors, blocks, plans_o, ocfg, k, what, sampled=True):
    n_active = _n_active(blocks)
    for qi, op in enumerate(plans_o):
        if sampled:  # a finite floor, or -inf after a re-run with no floor
            assert np.isfinite(floors[qi]) or floors[qi] == -np.inf, f"{what} q={qi}: floor {floors[qi]}"
        rid, rsc = fixed_floor_topk(blocks, op, ocfg, floors[qi], k)
        n = int(res.counts[qi])
        assert n == min(k, n_active), f"{what} q={qi}: {n} hits, {min(k, n_active)} expected"
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"{what} q={qi}")


@pytest.mark.parametrize("nq", [1, 8, 13])
def test_edenb1_mid_band_contract(device, corpus, nq):
    """EdenB1 at batch 1 (the one-query kernel's EdenB1 branch) and at 8 / 13
    queries (k_scan_tile, a full and a partial tile)."""
    c = corpus
    k = 64
    qs = _queries(c["rows"], nq, 100 + nq)
    plan = m.QueryPlan.from_query_codec(qs, DIMS, m.PrefixCodec.EDEN_PROD, m.MidCodec.EDEN_B1, _pfit(c["pf"]),
                                        _mfit(c["mf"]), device)
    res, floors = _scan_async(device, c["ix_b1"], plan, m.ScanConfig(shortlist_cand=k))
    plans_o = [ora.plan_build(q, DIMS, ora.PREFIX_EDEN_PROD, ora.MID_EDEN_B1, c["pf"], c["mf"]) for q in qs]
    _check_contract(res, floors, c["blocks_b1"], plans_o, ora.scan_config(k), k, f"EdenB1 nq={nq}")


@pytest.mark.parametrize("alpha,w_s4", [(0.85, 0.2), (1.0, 0.6), (0.8, 3.0)])
@pytest.mark.parametrize("nq", [1, 9])
def test_inadmissible_weights_contract(device, corpus, alpha, w_s4, nq):
    """alpha < 1, or w_s4 > alpha / 2.4, with the RaBitQ mid-band: the
    one-query kernel and k_scan_tile keep the reference's own stage checks.
    At alpha 0.8 / w_s4 3.0 the S1 + CS check rejects nearly every vector
    above the safe floor (0-3 of K = 48 stay, computed with the oracle), so
    those queries are re-run with no floor."""
    c = corpus
    k = 48
    qs = _queries(c["rows"], nq, 200 + nq)
    plan = m.QueryPlan.from_query_eden(qs, DIMS, _pfit(c["pf"]), device)
    cfg = m.ScanConfig(shortlist_cand=k, cs_tolerance=alpha, stratum4_weight=w_s4)
    res, floors = _scan_async(device, c["ix"], plan, cfg)
    plans_o = [ora.plan_build(q, DIMS, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, c["pf"]) for q in qs]
    _check_contract(res, floors, c["blocks"], plans_o, ora.scan_config(k, alpha=alpha, w_s4=w_s4), k,
                    f"alpha={alpha} w_s4={w_s4} nq={nq}")
    if w_s4 >= 3.0:
        assert res.stats.reruns_dense >= 1 and np.any(floors == -np.inf)


@pytest.mark.parametrize("nq", [1, 9])
def test_l0_only_topk(device, corpus, nq):
    """L0Only (scan.rs:753-790): the production kernels k_scan<1, L0> and
    k_scan<8, L0>.  Its bound dominates its score, so the top K is the
    reference's."""
    c = corpus
    k = 40
    qs = _queries(c["rows"], nq, 300 + nq)
    plan = m.QueryPlan.from_query_eden(qs, DIMS, _pfit(c["pf"]), device)
    res = m.scan_batch(c["ix"], plan, m.ScanConfig(shortlist_cand=k, strata_depth=m.StrataDepth.L0_ONLY))
    for qi, q in enumerate(qs):
        op = ora.plan_build(q, DIMS, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, c["pf"])
        rid, rsc = ora.scan_blocks(c["blocks"], op, ora.scan_config(k, depth=ora.L0_ONLY))
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"L0Only nq={nq} q={qi}")


def test_mfma_path_with_alpha_above_one(device, corpus):
    """alpha = 1.2, w_s4 = 0.4 (admissible): the MFMA path's tight checks."""
    c = corpus
    k = 64
    qs = _queries(c["rows"], 10, 401)
    plan = m.QueryPlan.from_query_eden(qs, DIMS, _pfit(c["pf"]), device)
    cfg = m.ScanConfig(shortlist_cand=k, cs_tolerance=1.2, stratum4_weight=0.4)
    res = m.scan_batch(c["ix"], plan, cfg)
    for qi, q in enumerate(qs):
        op = ora.plan_build(q, DIMS, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, c["pf"])
        rid, rsc = ora.scan_blocks(c["blocks"], op, ora.scan_config(k, alpha=1.2, w_s4=0.4))
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"alpha=1.2 q={qi}")


@pytest.mark.parametrize("nq", [1, 16])
def test_queries_far_from_unit_norm(device, corpus, nq):
    """Queries of norm 5 to 10 (the reference does not renormalize them,
    eden.rs:9): exact top K, no dense re-run, and about as many final-pass
    candidates as the same queries at unit norm (the sampling histogram
    follows the query's norm)."""
    c = corpus
    k = 64
    qs = _queries(c["rows"], nq, 500 + nq)
    qs /= np.linalg.norm(qs, axis=1, keepdims=True).astype(np.float32)
    big = (qs * np.linspace(5.0, 10.0, nq, dtype=np.float32)[:, None]).astype(np.float32)
    stats = {}
    for name, q in (("unit", qs), ("big", big)):
        plan = m.QueryPlan.from_query_eden(q, DIMS, _pfit(c["pf"]), device)
        res = m.scan_batch(c["ix"], plan, m.ScanConfig(shortlist_cand=k))
        stats[name] = res.stats
        for qi in range(nq):
            op = ora.plan_build(q[qi], DIMS, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, c["pf"])
            rid, rsc = ora.scan_blocks(c["blocks"], op, ora.scan_config(k))
            n = int(res.counts[qi])
            assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"{name} nq={nq} q={qi}")
    assert stats["big"].reruns_dense == 0
    # final-pass candidates (the one-query kernel's pushed survivors, the
    # MFMA path's appended pairs)
    u = stats["unit"].after_prefix if nq >= 8 else stats["unit"].pushed
    b = stats["big"].after_prefix if nq >= 8 else stats["big"].pushed
    assert b <= 3 * u + 4 * k * nq, (u, b)


def _shortfall_corpus(nq, dims=192, n_blocks=4096, seed=16):
    """Each query's 40 nearest vectors all sit in blocks that the sampling
    stages score (block ids that are multiples of 32), so the floor taken
    from the sample lies above the true K-th score."""
    rng = np.random.default_rng(seed)
    rows = normalized(rng, n_blocks * 64, dims)
    qs = normalized(rng, nq, dims)
    for qi in range(nq):
        # 8 slots in each of 5 sampled blocks
        blks = 32 * (5 * qi + np.arange(40) // 8)
        near = blks * 64 + np.arange(40) % 8
        rows[near] = qs[qi][None, :] + np.float32(0.02) * normalized(rng, 40, dims)
        rows[near] /= np.linalg.norm(rows[near], axis=1, keepdims=True).astype(np.float32)
    return m.encode_corpus(rows, 8), qs


def _check_exact(blocks, qs, res, k):
    for qi in range(qs.shape[0]):
        rid, rsc = ora.scan_blocks(blocks, ora.plan_build(qs[qi], qs.shape[1]), ora.scan_config(k))
        n = int(res.counts[qi])
        assert n == len(rid) == k
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"q={qi}")


def test_mfma_final_floor_shortfall_reruns_at_the_safe_floor(device):
    """The MFMA path's sampling stage scores every 32nd block; every query is
    flagged, re-run at the safe floor, and still returns the exact top K."""
    k = 64
    blocks, qs = _shortfall_corpus(8)
    plan = m.QueryPlan.from_query(qs, qs.shape[1], device)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=k))
    assert res.stats.reruns_safe >= 1
    _check_exact(blocks, qs, res, k)


def _records(dev):
    import ctypes as C
    L = m._lib.lib
    kt = (m._lib.KernelTimeC * 512)()
    n = C.c_uint32()
    m._lib.check(L.mrl_ctx_profile_collect(dev.handle, kt, 512, C.byref(n)))
    return [(kt[i].kind, kt[i].pass_) for i in range(min(n.value, 512))]


@pytest.mark.parametrize("nq", [1, 8])
def test_async_scan_reruns_on_the_device(device, nq):
    """mrl_scan_async itself enqueues the safe-floor re-run (the gated scan
    and selection, recorded as pass -1): once the stream is done the lists
    are final, and mrl_results_fetch launches nothing more.  nq 1: the
    one-query kernel; 8: the MFMA path."""
    L = m._lib.lib
    k = 64
    blocks, qs = _shortfall_corpus(nq, seed=17 + nq)
    dev = m.Device(0)
    ix = m.DeviceIndex.upload(blocks, dev)
    plan = m.QueryPlan.from_query(qs, qs.shape[1], dev)
    res = m.DeviceResults(nq, k, dev)
    m._lib.check(L.mrl_ctx_set_profiling(dev.handle, 1))
    res.scan(ix, plan, m.ScanConfig(shortlist_cand=k))
    dev.synchronize()
    before = _records(dev)
    out = res.fetch()
    after = _records(dev)
    m._lib.check(L.mrl_ctx_set_profiling(dev.handle, 0))
    assert (1, -1) in before and (2, -1) in before, before
    assert after == [], f"fetch launched {after}"
    assert out.stats.reruns_safe >= 1 and out.stats.reruns_dense == 0
    _check_exact(blocks, qs, out, k)
    # the floors reported are the safe floors the lists were selected at
    fl = res.floors()
    assert np.all(np.isfinite(fl))
    for qi in range(nq):
        assert out.scores[qi, k - 1] >= fl[qi]
    res.close()
    plan.close()
    ix.close()
    dev.close()


def test_mfma_k4096_sampled_clustered(device):
    """K = 4096 on a sampled index of near-duplicate clusters through the
    MFMA path: the exact-scoring lists stay within their room (no dense
    re-run) and the top K is the reference's."""
    rng = np.random.default_rng(17)
    n_blocks, dims, k, nq = 2048, 384, 4096, 8
    cents = normalized(rng, 32, dims)
    assign = rng.integers(0, 32, n_blocks * 64)
    rows = cents[assign] + np.float32(0.3 / np.sqrt(dims)) * rng.standard_normal((n_blocks * 64, dims)).astype(
        np.float32)
    rows /= np.linalg.norm(rows, axis=1, keepdims=True).astype(np.float32)
    fit = oracle_fit(rows[:8192])
    blocks = m.encode_corpus(rows, 8, _pfit(fit))
    qs = _queries(rows, nq, 18, noise=0.1 / np.sqrt(dims))
    plan = m.QueryPlan.from_query_eden(qs, dims, _pfit(fit), device)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=k))
    assert res.stats.reruns_dense == 0
    for qi in range(2):
        op = ora.plan_build(qs[qi], dims, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
        rid, rsc = ora.scan_blocks(blocks, op, ora.scan_config(k))
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rid, rsc, k, f"q={qi}")


def test_plan_codebooks_are_the_reference_literals(device):
    """The plan's EDEN codebooks (eden.rs:15-44, B4 and B1) bit-exact to the
    fixture made from the reference's literals."""
    with open(os.path.join(os.path.dirname(__file__), "golden", "eden_codebooks.json")) as f:
        fx = json.load(f)
    rng = np.random.default_rng(3)
    rows = normalized(rng, 256, DIMS)
    pf, mf = oracle_fit(rows), oracle_fit_mid(rows)
    plan = m.QueryPlan.from_query_codec(rows[:1], DIMS, m.PrefixCodec.EDEN_PROD, m.MidCodec.EDEN_B1, _pfit(pf),
                                        _mfit(mf), device)
    p = plan.export()[0]
    b4 = np.array([int(h, 16) for h in fx["B4"]["f32_bits"]], dtype=np.uint32)
    b1 = np.array([int(h, 16) for h in fx["B1"]["f32_bits"]], dtype=np.uint32)
    assert np.array_equal(np.ctypeslib.as_array(p.eden_codebook).astype(np.float32).view(np.uint32), b4)
    assert np.array_equal(np.ctypeslib.as_array(p.eden_mid_codebook).astype(np.float32).view(np.uint32), b1)
