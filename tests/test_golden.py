"""Committed golden vectors (tests/golden/*.npz, written by
tests/golden/make_golden.py with the CPU oracle): the oracle must keep
reproducing them (CPU), and the HIP path must match them (GPU)."""
import os

import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["eden768_32blk", "minmax384_partial"]


def load(name):
    return dict(np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False))


def oracle_fit(f):
    return ora.Fit(f["fit_mean"], 4, 1) if "fit_mean" in f else None


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_golden(name):
    f = load(name)
    dims, codec = int(f["dims"]), int(f["prefix_codec"])
    fit = oracle_fit(f)
    cfg = ora.scan_config(64)
    for qi, q in enumerate(f["queries"]):
        p = ora.plan_build(q, dims, codec, ora.MID_RABITQ, fit, None)
        assert np.array_equal(np.frombuffer(bytes(p), dtype=np.uint8), f["plans"][qi])
        for ti, t in enumerate(f["taus"]):
            for b, blk in enumerate(f["blocks"]):
                _, mk, pre, sc = ora.block_stages(blk, p, cfg, float(t))
                assert np.array_equal(mk, f["masks"][qi, ti, b])
                assert np.array_equal(pre.view(np.uint32), f["prefix_ip"][qi, ti, b].view(np.uint32))
                assert np.array_equal(sc.view(np.uint32), f["stage_scores"][qi, ti, b].view(np.uint32))
        e, v = ora.exhaustive_scores(f["blocks"], p, cfg)
        assert np.array_equal(v, f["exhaustive_valid"][qi])
        assert np.array_equal(e[v].view(np.uint32), f["exhaustive"][qi][v].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_gpu_matches_golden(device, name):
    f = load(name)
    dims, codec = int(f["dims"]), int(f["prefix_codec"])
    fit = m.EdenFit(64, 4, 1, f["fit_mean"]) if "fit_mean" in f else None
    plan = m.QueryPlan.from_query_codec(f["queries"], dims, codec, m.MidCodec.RABITQ, fit, None, device)
    got = plan.export()
    for qi in range(len(f["queries"])):
        assert np.array_equal(np.frombuffer(bytes(got[qi]), dtype=np.uint8), f["plans"][qi]), f"plan {qi}"
    ix = m.DeviceIndex.upload(f["blocks"], device)
    assert np.array_equal(ix.download(), f["blocks"])
    for ti, t in enumerate(f["taus"]):
        tr = m.scan_fixed_tau(ix, plan, m.ScanConfig(shortlist_cand=64), np.full(len(f["queries"]), t, np.float32))
        assert np.array_equal(tr.masks, f["masks"][:, ti])
        for qi in range(len(f["queries"])):
            for b in range(len(f["blocks"])):
                act = [v for v in range(64) if int(f["masks"][qi, ti, b, 0]) >> v & 1]
                push = [v for v in range(64) if int(f["masks"][qi, ti, b, 4]) >> v & 1]
                assert np.array_equal(tr.prefix_ip[qi, b, act].view(np.uint32),
                                      f["prefix_ip"][qi, ti, b, act].view(np.uint32))
                assert np.array_equal(tr.scores[qi, b, push].view(np.uint32),
                                      f["stage_scores"][qi, ti, b, push].view(np.uint32))
    for k in f["ks"]:
        k = int(k)
        res = m.scan_batch(ix, plan, m.ScanConfig(shortlist_cand=k))
        for qi in range(len(f["queries"])):
            ref_ids = f[f"topk_ids_{k}"][qi]
            keep = ref_ids != np.iinfo(np.uint64).max
            n = int(res.counts[qi])
            assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], ref_ids[keep], f[f"topk_scores_{k}"][qi][keep], k,
                              f"{name} k={k} q={qi}")
