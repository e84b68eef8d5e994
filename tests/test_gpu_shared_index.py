"""One device index scanned through several contexts at once (one stream
each), the GPU analogue of the reference engine serving `&self` queries from
many threads over one slab (src/engine.rs:572-580): every context's results
equal one context's, bit for bit, with the scans enqueued back to back on
all streams, and from concurrent host threads; on the standard and the
cluster-grouped layout (whose block lists are per-context scratch)."""
import threading

import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import synth

pytestmark = pytest.mark.gpu


def _corpus(layout):
    w = synth.CONFIGS[4].scaled(64 * 1500, 24)
    fit = synth.eden_fit(w)
    if layout == "clustered":
        blocks, _ = synth.encode_clustered(w, fit, 8)
    else:
        blocks = synth.encode(w, fit, 8)
    qs, _ = synth.queries(w)
    return w, fit, blocks, qs


def _lanes(device, ix, w, fit, qs, n):
    """n contexts, each with plans for a different slice of the queries."""
    out = []
    for i in range(n):
        dev = device if i == 0 else m.Device(0)
        sel = np.roll(qs, 5 * i, axis=0)[:(9 if i % 2 else w.n_queries)]
        plan = m.QueryPlan.from_query_codec(sel, w.dims, w.prefix_codec, m.MidCodec.RABITQ, fit, None, dev)
        res = m.DeviceResults(sel.shape[0], w.k, dev)
        out.append((dev, plan, res))
    return out


@pytest.mark.parametrize("layout", ["standard", "clustered"])
def test_contexts_share_one_index(device, layout):
    print(f"[shared index] {layout}", flush=True)
    w, fit, blocks, qs = _corpus(layout)
    ix = m.DeviceIndex.upload(blocks, device)
    cfg = m.ScanConfig(shortlist_cand=w.k)
    lanes = _lanes(device, ix, w, fit, qs, 3)
    # reference: each lane's plans alone, one scan at a time
    ref = []
    for dev, plan, res in lanes:
        res.scan(ix, plan, cfg)
        ref.append(res.fetch())
    # all lanes enqueued back to back, three rounds, fetched at the end
    for _ in range(3):
        for dev, plan, res in lanes:
            res.scan(ix, plan, cfg)
    for (dev, plan, res), r in zip(lanes, ref):
        got = res.fetch()
        assert np.array_equal(got.counts, r.counts)
        assert np.array_equal(got.ids, r.ids)
        assert np.array_equal(got.scores.view(np.uint32), r.scores.view(np.uint32))
    # concurrent host threads, each driving its own context
    errs, outs = [], [None] * len(lanes)

    def run(i):
        try:
            dev, plan, res = lanes[i]
            for _ in range(4):
                res.scan(ix, plan, cfg)
                outs[i] = res.fetch()
        except Exception as e:  # reported below
            errs.append(e)

    th = [threading.Thread(target=run, args=(i,)) for i in range(len(lanes))]
    for t in th:
        t.start()
    for t in th:
        t.join(100)
    assert not errs, errs
    for got, r in zip(outs, ref):
        assert np.array_equal(got.ids, r.ids) and np.array_equal(got.scores.view(np.uint32), r.scores.view(np.uint32))
    for dev, plan, res in lanes:
        res.close()
        plan.close()
    ix.close()  # waits for every stream of the device


def test_plans_and_results_stay_with_their_context(device):
    w, fit, blocks, qs = _corpus("standard")
    ix = m.DeviceIndex.upload(blocks[:300], device)
    other = m.Device(0)
    plan = m.QueryPlan.from_query_codec(qs[:2], w.dims, w.prefix_codec, m.MidCodec.RABITQ, fit, None, device)
    res = m.DeviceResults(2, w.k, other)
    with pytest.raises(m.MrlError) as e:
        res.scan(ix, plan, m.ScanConfig(shortlist_cand=w.k))
    assert e.value.code == 1
