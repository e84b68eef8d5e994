"""MFMA-bounded batched scan (batches of 8 or more queries with the RaBitQ
mid-band): the top K of every query equals the oracle's scan_blocks top K
(exact ties excepted) with bit-identical scores.  Covers both prefix codecs,
the Full64b and L1Rabitq depths, indexes with and without a sampling pass,
one and two 32-query tiles per wave and a partial last query chunk, tombstones
and the temporal filter, vectors whose meta is beyond the f16 operand range,
near-duplicate clusters, K above the index size, and a non-finite query (an
error, as on the exact path).  Every case runs twice: under the library's own
choice of final pass, and with the final pass forced to bound the S4 stage
(mrl_ctx_set_s4_bound ALWAYS: its staged pairs are made exact before they
are written out, a wave past its append allowance returns to the full
tiles, and a pair beyond the staging room keeps the bound)."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "s4-bounded"], autouse=True)
def s4_policy(request, device):
    device.set_s4_bound(device.S4_BOUND_AUTO if request.param == "auto" else device.S4_BOUND_ALWAYS)
    yield request.param
    device.set_s4_bound(device.S4_BOUND_AUTO)


def _rows(n, dims, seed, clusters=0):
    rng = np.random.default_rng(seed)
    rows = normalized(rng, n, dims)
    if clusters:
        cent = normalized(rng, clusters, dims)
        noise = rng.standard_normal((n, dims)).astype(np.float32) * np.float32(0.3 / np.sqrt(dims))
        rows = cent[rng.integers(0, clusters, n)] + noise
        rows /= np.linalg.norm(rows, axis=1, keepdims=True).astype(np.float32)
    return rows.astype(np.float32), rng


def _queries(rows, rng, n_q, noise=0.1):
    src = rng.integers(0, rows.shape[0], n_q)
    q = rows[src] + rng.standard_normal((n_q, rows.shape[1])).astype(np.float32) * np.float32(
        noise / np.sqrt(rows.shape[1]))
    return (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)


def _check(device, blocks, qs, dims, fit, k, depth=m.StrataDepth.FULL64B, lo=None, hi=None, temporal=True,
           exhaustive=False, checked=None, what="", alpha=1.0, w_s4=0.2):
    eden = fit is not None
    codec = m.PrefixCodec.EDEN_PROD if eden else m.PrefixCodec.MIN_MAX4
    plan = m.QueryPlan.from_query_codec(qs, dims, codec, m.MidCodec.RABITQ, fit, None, device)
    cfg = m.ScanConfig(shortlist_cand=k, strata_depth=depth, temporal_filter_enable=temporal, exhaustive=exhaustive,
                       cs_tolerance=alpha, stratum4_weight=w_s4)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, cfg, lo, hi)
    ofit = ora.Fit(fit.mean, 4, 1, fit.n_observed) if eden else None
    ocfg = ora.scan_config(k, alpha=alpha, w_s4=w_s4, depth=int(depth), temporal=temporal, sharding=True, threads=8)
    for qi in (range(len(qs)) if checked is None else checked):
        op = ora.plan_build(qs[qi], dims, int(codec), 0, ofit, None)
        rids, rsc = ora.scan_blocks(blocks, op, ocfg, lo, hi)
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], rids, rsc, k, f"{what} q={qi}")
    return res


@pytest.mark.parametrize("n_q", [8, 40, 70])
def test_eden_sampled_index(device, n_q):
    """300 blocks (a sampling pass, then the final pass at its floor)."""
    print(f"[mma] eden sampled n_q={n_q}", flush=True)
    rows, rng = _rows(300 * 64, 768, 21)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    _check(device, blocks, _queries(rows, rng, n_q), 768, fit, 64, what=f"eden n_q={n_q}")


def test_minmax_single_pass_index(device):
    """120 blocks: no sampling pass, every active pair is a candidate."""
    print("[mma] minmax single pass", flush=True)
    rows, rng = _rows(120 * 64 - 17, 384, 22)
    blocks = m.encode_corpus(rows, 8)
    _check(device, blocks, _queries(rows, rng, 24), 384, None, 128, what="minmax single")


def test_minmax_sampled_l1_depth(device):
    print("[mma] minmax sampled L1Rabitq", flush=True)
    rows, rng = _rows(700 * 64, 256, 23)
    blocks = m.encode_corpus(rows, 8)
    _check(device, blocks, _queries(rows, rng, 33), 256, None, 256, depth=m.StrataDepth.L1_RABITQ,
           what="minmax L1")


def test_clustered_near_duplicates(device):
    print("[mma] clustered", flush=True)
    rows, rng = _rows(600 * 64, 768, 24, clusters=20)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    _check(device, blocks, _queries(rows, rng, 64, noise=0.02), 768, fit, 256, what="clustered")


def test_tombstones_and_temporal_filter(device):
    print("[mma] tombstones + temporal", flush=True)
    rows, rng = _rows(400 * 64, 768, 25)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    tomb = rng.integers(0, 2**63, size=blocks.shape[0], dtype=np.uint64) | np.uint64(1 << 63)
    tomb[::7] = 0
    blocks[:, 16:24] = tomb.view(np.uint8).reshape(-1, 8)
    blocks[5, 16:24] = 0xFF  # a fully tombstoned block
    qs = _queries(rows, rng, 16)
    _check(device, blocks, qs, 768, fit, 64, what="tombstones")
    # timestamps are row indices: keep rows 3000 .. 20000 (blocks 46 .. 312)
    _check(device, blocks, qs, 768, fit, 64, lo=3000, hi=20000, what="temporal")


def test_dense_appends_past_the_staging_room(device):
    """K 1024 over 300 blocks: the sampled floor passes ~9 % of the
    vectors, about 170 pairs per 32-vector tile, more than a wave's staging
    region takes in one tile.  Pairs go straight to their segments (with the
    S4 bound still in them when the pass bounds S4), and every wave of an
    S4-bounded pass returns to the full tiles after its first tiles."""
    print("[mma] dense appends", flush=True)
    rows, rng = _rows(300 * 64, 768, 29)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    _check(device, blocks, _queries(rows, rng, 64), 768, fit, 1024, what="dense appends")


@pytest.mark.parametrize("alpha,w_s4", [(10.0, 4.0), (12.0, 5.0)])
def test_large_stratum_weights(device, alpha, w_s4):
    """Admissible (2.4 w_s4 <= alpha) weights at and past the largest
    stratum weight the S4 bound covers (4): past it the final pass keeps the
    full tiles whatever the policy."""
    print(f"[mma] alpha {alpha} w_s4 {w_s4}", flush=True)
    rows, rng = _rows(400 * 64, 768, 30)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    _check(device, blocks, _queries(rows, rng, 40), 768, fit, 64, alpha=alpha, w_s4=w_s4,
           what=f"alpha {alpha} w_s4 {w_s4}")


def test_exhaustive_flag_and_k_above_index(device):
    print("[mma] exhaustive, K > N", flush=True)
    rows, rng = _rows(50 * 64 - 9, 384, 26)
    blocks = m.encode_corpus(rows, 8)
    qs = _queries(rows, rng, 12)
    _check(device, blocks, qs, 384, None, 4096, exhaustive=True, what="k>n")


def test_vectors_beyond_the_operand_range(device):
    """Slots whose scale / tail norm exceed the f16 operand range (and NaN
    meta, which the reference prunes) are always candidates and scored
    exactly."""
    print("[mma] extreme meta", flush=True)
    rows, rng = _rows(300 * 64, 768, 27)
    blocks = m.encode_corpus(rows, 8)
    meta = blocks[:, 64:512].reshape(-1, 64, 7)
    big = np.frombuffer(np.float16(30000.0).tobytes(), dtype=np.uint8)
    meta[3, 5, 0:2] = big           # scale
    meta[10, 9, 4:6] = big          # tail norm
    meta[20, 1, 0:2] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)
    meta[40, 2, 2:4] = big          # offset (MinMax4)
    _check(device, blocks, _queries(rows, rng, 16), 768, None, 64, what="extreme meta")


def test_nonfinite_query_is_an_error(device):
    rows, rng = _rows(300 * 64, 768, 28)
    blocks = m.encode_corpus(rows, 8)
    qs = _queries(rows, rng, 16)
    qs[3, 700] = np.inf
    plan = m.QueryPlan.from_query(qs, 768, device)
    with pytest.raises(m.MrlError) as e:
        m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, m.ScanConfig(shortlist_cand=64))
    assert e.value.code == 3
