"""GPU post-scan rerank (mrl_rerank_store_* / mrl_rerank_rows / mrl_results_rerank)
against the oracle's restatement of rerank_exact_rows and rerank_dot
(src/pipeline.rs:157-169, src/lowprec.rs:49-121, src/embed.rs:115-206):
stored rows byte-identical, scores bit-identical, order identical (stable)."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized

pytestmark = pytest.mark.gpu

PRECS = [(m.RerankPrecision.FP32, ora.RERANK_FP32), (m.RerankPrecision.FP16, ora.RERANK_FP16),
         (m.RerankPrecision.INT8, ora.RERANK_INT8)]


def _rows(seed, n, dims=768):
    return normalized(np.random.default_rng(seed), n, dims)


def _check_batch(prec_o, queries, rows, cand, counts, got_rows, got_scores, what=""):
    for q in range(cand.shape[0]):
        c = int(counts[q])
        want = ora.rerank(prec_o, queries[q], rows, cand[q, :c])
        assert want is not None
        wr, ws = want
        assert np.array_equal(got_rows[q, :c], wr), f"{what} q={q}: order differs"
        assert np.array_equal(got_scores[q, :c].view(np.uint32), ws.view(np.uint32)), f"{what} q={q}: scores differ"


def test_store_bytes_match_the_reference_conversions(device):
    rows = _rows(1, 300)
    rows[3] = 0.0
    rows[4] *= np.float32(1e-6)                  # f16 subnormals
    rows[5] *= np.float32(2e4)                   # f16 near its maximum
    rows[6, 0] = np.float32(1e6)                 # f16 overflow -> inf
    rows[7, 1] = -0.0
    rows[8, 2] = np.nan                          # int8: max ignores it, code 0
    rows[9, 10:20] = np.float32(1e-13)
    st32 = m.RerankStore.create(rows, m.RerankPrecision.FP32, device)
    assert np.array_equal(st32.download().view(np.uint32), rows.view(np.uint32))
    st16 = m.RerankStore.create(rows, m.RerankPrecision.FP16, device)
    f16 = st16.download()
    want16 = rows.astype(np.float16)
    nan = np.isnan(want16)
    assert np.array_equal(np.isnan(f16), nan)
    assert np.array_equal(f16.view(np.uint16)[~nan], want16.view(np.uint16)[~nan])
    st8 = m.RerankStore.create(rows, m.RerankPrecision.INT8, device)
    codes, scales = st8.download()
    for r in range(rows.shape[0]):
        c, s = ora.int8_quantize_768(rows[r])
        assert np.array_equal(codes[r], c), f"row {r} codes"
        assert int(scales.view(np.uint16)[r]) == s, f"row {r} scale"


def test_store_from_device_rows_equals_host_upload(device):
    rows = _rows(2, 130)
    buf = m.DeviceBuffer.from_array(rows, device)
    for prec, _ in PRECS:
        a = m.RerankStore.create(rows, prec, device)
        b = m.RerankStore.create(buf, prec, device, n_rows=130, dims=768)
        da, db = a.download(), b.download()
        if prec == m.RerankPrecision.INT8:
            assert np.array_equal(da[0], db[0]) and np.array_equal(da[1].view(np.uint16), db[1].view(np.uint16))
        else:
            assert np.array_equal(np.asarray(da).view(np.uint8), np.asarray(db).view(np.uint8))


@pytest.mark.parametrize("prec,prec_o", PRECS)
@pytest.mark.parametrize("stride", [1, 37, 256, 513, 1500])
def test_rerank_rows_matches_oracle(device, prec, prec_o, stride):
    """Ragged counts (0 .. stride) cover the rank sort (<= 512) and the
    bitonic sort, partial workgroups and empty lists."""
    n_rows = 2000
    rows = _rows(3, n_rows)
    rng = np.random.default_rng(stride)
    nq = 5
    queries = normalized(rng, nq, 768)
    cand = rng.integers(0, n_rows, (nq, stride)).astype(np.uint64)
    counts = np.array([stride, 0, max(stride // 2, 1), 1, stride], dtype=np.uint32)[:nq]
    store = m.RerankStore.create(rows, prec, device)
    got_r, got_s = m.rerank_batch(store, queries, cand, counts)
    _check_batch(prec_o, queries, rows, cand, counts, got_r, got_s, f"{prec.as_str()} stride={stride}")


def test_rerank_max_shortlist(device):
    rows = _rows(4, 5000)
    rng = np.random.default_rng(4)
    q = normalized(rng, 2, 768)
    cand = np.stack([rng.permutation(5000)[:4096], rng.integers(0, 5000, 4096)]).astype(np.uint64)
    store = m.RerankStore.create(rows, m.RerankPrecision.FP32, device)
    got_r, got_s = m.rerank_batch(store, q, cand)
    _check_batch(ora.RERANK_FP32, q, rows, cand, np.full(2, 4096), got_r, got_s, "K=4096")
    with pytest.raises(m.MrlError):
        m.rerank_batch(store, q[:1], np.zeros((1, 4097), dtype=np.uint64))


@pytest.mark.parametrize("dims", [192, 384, 1000])
def test_rerank_generic_dims_fp32(device, dims):
    rows = _rows(5, 700, dims)
    rng = np.random.default_rng(dims)
    q = normalized(rng, 3, dims)
    cand = rng.integers(0, 700, (3, 300)).astype(np.uint64)
    counts = np.array([300, 17, 0], dtype=np.uint32)
    store = m.RerankStore.create(rows, m.RerankPrecision.FP32, device)
    got_r, got_s = m.rerank_batch(store, q, cand, counts)
    _check_batch(ora.RERANK_FP32, q, rows, cand, counts, got_r, got_s, f"dims={dims}")
    with pytest.raises(m.MrlError):
        m.RerankStore.create(rows, m.RerankPrecision.FP16, device)  # fp16 / int8 need 768 dims


@pytest.mark.parametrize("prec,prec_o", PRECS)
def test_rerank_ties_keep_input_order(device, prec, prec_o):
    rows = _rows(6, 64)
    rows[10] = rows[20]
    rows[30] = 0.0
    rows[31] = 0.0
    q = normalized(np.random.default_rng(6), 1, 768)
    cand = np.array([[20, 5, 31, 10, 30, 7, 20, 10, 31, 30]], dtype=np.uint64)
    store = m.RerankStore.create(rows, prec, device)
    got_r, got_s = m.rerank_batch(store, q, cand)
    _check_batch(prec_o, q, rows, cand, [cand.shape[1]], got_r, got_s, "ties")
    assert m.QueryPipeline.rerank_exact_rows(q[0], cand[0], store) == list(zip(got_r[0].tolist(),
                                                                               got_s[0].tolist()))


def test_rerank_errors(device):
    rows = _rows(7, 100)
    rows[50, 3] = np.nan
    q = normalized(np.random.default_rng(7), 1, 768)
    for prec in (m.RerankPrecision.FP32, m.RerankPrecision.FP16):
        store = m.RerankStore.create(rows, prec, device)
        with pytest.raises(m.MrlError) as e:
            m.rerank_batch(store, q, np.array([[1, 50]], dtype=np.uint64))
        assert e.value.code == 3  # NaN: partial_cmp().unwrap() panics in the reference
        with pytest.raises(m.MrlError) as e:
            m.rerank_batch(store, q, np.array([[1, 100]], dtype=np.uint64))
        assert e.value.code == 1  # row out of range
    st8 = m.RerankStore.create(rows, m.RerankPrecision.INT8, device)
    got_r, got_s = m.rerank_batch(st8, q, np.array([[1, 50, 2]], dtype=np.uint64))
    _check_batch(ora.RERANK_INT8, q, rows, np.array([[1, 50, 2]], dtype=np.uint64), [3], got_r, got_s, "int8 NaN")
    with pytest.raises(m.MrlError):
        m.rerank_batch(st8, q, np.zeros((1, 4), dtype=np.uint64), counts=np.array([5], dtype=np.uint32))


def test_pipeline_rerank_with_a_row_callable(device):
    rows = _rows(8, 400)
    q = normalized(np.random.default_rng(8), 1, 768)[0]
    ids = [399, 3, 250, 3, 17]
    got = m.QueryPipeline.rerank_exact_rows(q, ids, lambda i: rows[i])
    wr, ws = ora.rerank(ora.RERANK_FP32, q, rows, np.array(ids, dtype=np.uint64))
    assert [r for r, _ in got] == wr.tolist()
    assert np.array_equal(np.array([s for _, s in got], dtype=np.float32).view(np.uint32), ws.view(np.uint32))
    assert m.QueryPipeline.rerank_exact_rows(q, [], lambda i: rows[i]) == []


@pytest.mark.parametrize("prec,prec_o", PRECS)
def test_scan_then_rerank_on_device(device, prec, prec_o):
    """The bench's scan -> scored_hits_to_row_ids -> rerank chain with the
    shortlist kept in HBM (retrieval_bench.rs:736-745)."""
    n = 64 * 150 - 20
    rows = _rows(9, n)
    rng = np.random.default_rng(9)
    queries = rows[rng.integers(0, n, 6)] + np.float32(0.01) * normalized(rng, 6, 768)
    queries = np.ascontiguousarray(queries, dtype=np.float32)
    blocks = m.encode_corpus(rows, 8)
    index = m.DeviceIndex.upload(blocks, device)
    plan = m.QueryPlan.from_query(queries, 768, device)
    k = 200
    cfg = m.ScanConfig(shortlist_cand=k)
    res = m.DeviceResults(6, k, device)
    res.scan(index, plan, cfg)
    hits = res.fetch()
    store = m.RerankStore.create(rows, prec, device)
    got_r, got_s, counts = res.rerank(store)
    assert np.array_equal(counts, hits.counts)
    cand = (hits.ids >> np.uint64(16)) * np.uint64(64) + (hits.ids & np.uint64(0xFFFF))
    _check_batch(prec_o, queries, rows, cand, counts, got_r, got_s, f"scan+{prec.as_str()}")
    # rerank straight after the scan, without a fetch in between
    res.scan(index, plan, cfg)
    got_r2, got_s2, _ = res.rerank(store)
    assert np.array_equal(got_r2, got_r) and np.array_equal(got_s2.view(np.uint32), got_s.view(np.uint32))
    # a store shorter than the index's rows is an error, not a fault
    short = m.RerankStore.create(rows[:100], prec, device)
    with pytest.raises(m.MrlError):
        res.rerank(short)
    res.close()


@pytest.mark.parametrize("dims", [768, 384])
@pytest.mark.parametrize("n_pending,top_k", [(1, 256), (17, 5), (63, 256), (300, 100), (1100, 1024)])
def test_ring_search_matches_oracle(device, dims, n_pending, top_k):
    rng = np.random.default_rng(n_pending + dims)
    pending = normalized(rng, n_pending, dims)
    if n_pending > 2:
        pending[2] = pending[0]          # exact tie: the lower index first
    queries = normalized(rng, 3, dims)
    ring = m.RingBuffer(1024, device)
    keep = min(top_k, n_pending)
    loc = np.zeros((3, keep), dtype=np.uint64)
    sc = np.zeros((3, keep), dtype=np.float32)
    cnt = np.zeros(3, dtype=np.uint32)
    from mrl_index_amd import _lib
    _lib.check(_lib.lib.mrl_ring_search(device.handle, _lib.fptr(pending), n_pending, dims, _lib.fptr(queries), 3,
                                        top_k, _lib.u64ptr(loc), _lib.fptr(sc), _lib.u32ptr(cnt)))
    for q in range(3):
        wl, ws = ora.ring_search_exact(pending, queries[q], top_k)
        assert int(cnt[q]) == keep
        assert np.array_equal(loc[q], wl) and np.array_equal(sc[q].view(np.uint32), ws.view(np.uint32))
    # the RingBuffer mirror (pending < 64 after every push)
    for i in range(min(n_pending, 63)):
        assert ring.push(m.PendingVector(i, pending[i], i, 0)) is None
    hits = ring.search_exact(queries[0], top_k)
    wl, ws = ora.ring_search_exact(pending[:min(n_pending, 63)], queries[0], top_k)
    assert [h[0] for h in hits] == wl.tolist()
    assert np.array_equal(np.array([h[1] for h in hits], dtype=np.float32).view(np.uint32), ws.view(np.uint32))


def test_ring_buffer_flushes_at_64(device):
    rows = normalized(np.random.default_rng(30), 70, 384)
    ring = m.RingBuffer(1024, device)
    blocks = [ring.push(m.PendingVector(i, rows[i], 100 + i, 0)) for i in range(70)]
    flushed = [b for b in blocks if b is not None]
    assert len(flushed) == 1 and len(ring) == 6
    assert np.array_equal(flushed[0], m.encode_block(rows[:64], 100 + np.arange(64), np.full(64, m.source.DOC), 384))
    tail = ring.flush_partial()
    assert np.array_equal(tail, m.encode_block(rows[64:], 164 + np.arange(6), np.full(6, m.source.DOC), 384))
    assert ring.is_empty() and ring.search_exact(rows[0], 10) == []


@pytest.mark.parametrize("n_pending", [5, 63, 600])
def test_ring_merge_into_scan_shortlists(device, n_pending):
    """engine.rs:584-594: ring hits pushed into each query's scan shortlist,
    then the rerank of the merged list skips them (pipeline.rs:175-180)."""
    n = 64 * 120
    rng = np.random.default_rng(31 + n_pending)
    rows = _rows(31, n)
    queries = np.ascontiguousarray(rows[rng.integers(0, n, 4)] + np.float32(0.02) * normalized(rng, 4, 768),
                                   dtype=np.float32)
    # pending rows close to the queries so that ring hits interleave with scan hits
    pending = np.ascontiguousarray(np.repeat(queries, (n_pending + 3) // 4, axis=0)[:n_pending]
                                   + np.float32(0.05) * normalized(rng, n_pending, 768), dtype=np.float32)
    index = m.DeviceIndex.upload(m.encode_corpus(rows, 8), device)
    plan = m.QueryPlan.from_query(queries, 768, device)
    k = 128
    res = m.DeviceResults(4, k, device)
    res.scan(index, plan, m.ScanConfig(shortlist_cand=k))
    before = res.fetch()
    from mrl_index_amd import _lib
    _lib.check(_lib.lib.mrl_results_merge_ring(device.handle, res._h, _lib.fptr(pending), n_pending, 768))
    after = res.fetch()
    n_ring_hits = 0
    for q in range(4):
        c = int(before.counts[q])
        rl, rs = ora.ring_search_exact(pending, queries[q], k)
        ring_ids = (np.uint64(0xFFFFFFFF) << np.uint64(16)) | rl
        wi, ws = ora.shortlist_push_sorted(k, before.ids[q, :c], before.scores[q, :c], ring_ids, rs)
        ca = int(after.counts[q])
        assert ca == wi.size
        union = np.concatenate([before.scores[q, :c], rs])
        if np.unique(union).size == union.size:  # no exact ties: identical lists
            assert np.array_equal(after.ids[q, :ca], wi), f"q={q}: merged ids differ"
            assert np.array_equal(after.scores[q, :ca].view(np.uint32), ws.view(np.uint32))
        else:  # which tied entry is kept follows the reference's heap order
            assert_topk_equal(after.ids[q, :ca], after.scores[q, :ca], wi, ws, k, f"q={q}")
        n_ring_hits += int(np.sum((after.ids[q, :ca] >> np.uint64(16)) == np.uint64(0xFFFFFFFF)))
    assert n_ring_hits > 0
    store = m.RerankStore.create(rows, m.RerankPrecision.FP32, device)
    rr, rsc, rc = res.rerank(store)
    for q in range(4):
        ids = after.ids[q, :int(after.counts[q])]
        keep = ids[(ids >> np.uint64(16)) != np.uint64(0xFFFFFFFF)]
        cand = (keep >> np.uint64(16)) * np.uint64(64) + (keep & np.uint64(0xFFFF))
        assert int(rc[q]) == cand.size
        wr, ws = ora.rerank(ora.RERANK_FP32, queries[q], rows, cand)
        assert np.array_equal(rr[q, :cand.size], wr)
        assert np.array_equal(rsc[q, :cand.size].view(np.uint32), ws.view(np.uint32))
    bad = pending.copy()
    bad[1, 4] = np.nan
    res.scan(index, plan, m.ScanConfig(shortlist_cand=k))
    with pytest.raises(m.MrlError) as e:
        _lib.check(_lib.lib.mrl_results_merge_ring(device.handle, res._h, _lib.fptr(bad), n_pending, 768))
    assert e.value.code == 3
    res.close()
