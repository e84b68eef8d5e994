"""GPU parity: the HIP path through the C ABI against the CPU oracle."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized, oracle_encode_corpus, oracle_fit, oracle_fit_mid

pytestmark = pytest.mark.gpu

PLAN_FLOAT_FIELDS = [n for n, _ in ora.PLAN_FIELDS if n not in ("dims", "prefix_codec", "mid_codec",
                                                                 "has_tail_fold", "pad")]


def _fit_for_product(f):
    return m.EdenFit(f.mean.shape[0], f.c.bits, f.c.seed, f.mean, f.c.n_observed)


def _plan_equal(gp, op, what):
    for name in ("dims", "prefix_codec", "mid_codec", "has_tail_fold"):
        assert getattr(gp, name) == getattr(op, name), f"{what}: {name}"
    for name in PLAN_FLOAT_FIELDS:
        g = np.ctypeslib.as_array(getattr(gp, name)) if hasattr(getattr(gp, name), "_length_") else \
            np.float32(getattr(gp, name))
        o = np.ctypeslib.as_array(getattr(op, name)) if hasattr(getattr(op, name), "_length_") else \
            np.float32(getattr(op, name))
        g = np.asarray(g, dtype=np.float32)
        o = np.asarray(o, dtype=np.float32)
        assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), f"{what}: field {name} differs"


@pytest.fixture(scope="module")
def corpus768(device):
    rng = np.random.default_rng(1234)
    rows = normalized(rng, 64 * 96 - 17, 768)  # ragged last block
    fit = oracle_fit(rows[:4096])
    blocks = oracle_encode_corpus(rows, 768, fit)
    return rows, fit, blocks


def test_relayout_roundtrip_exact(device, corpus768):
    _, _, blocks = corpus768
    ix = m.DeviceIndex.upload(blocks, device)
    assert ix.block_count() == blocks.shape[0]
    assert np.array_equal(ix.download(), blocks)
    # arbitrary bytes are a bijection too
    rnd = np.random.default_rng(5).integers(0, 256, size=(37, 4096), dtype=np.uint8)
    ix2 = m.DeviceIndex.upload(rnd, device)
    assert np.array_equal(ix2.download(), rnd)


@pytest.mark.parametrize("dims", [192, 200, 256, 384, 768, 1024])
@pytest.mark.parametrize("codec", ["minmax", "eden", "eden_dual"])
def test_plan_bit_exact(device, dims, codec):
    rng = np.random.default_rng(dims * 7 + len(codec))
    qs = normalized(rng, 9, dims, offset=0.01)
    qs[3] = 0.0                      # all-zero query
    qs[4, :64] = 0.0                 # zero prefix
    qs[5] *= np.float32(1e-30)       # denormal-range squares
    rows = normalized(rng, 256, dims)
    pf = oracle_fit(rows)
    mf = oracle_fit_mid(rows, seed=11)
    kw = {"minmax": (ora.PREFIX_MINMAX4, ora.MID_RABITQ, None, None),
          "eden": (ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, pf, None),
          "eden_dual": (ora.PREFIX_EDEN_PROD, ora.MID_EDEN_B1, pf, mf)}[codec]
    plan = m.QueryPlan.from_query_codec(qs, dims, kw[0], kw[1], _fit_for_product(kw[2]) if kw[2] else None,
                                        _fit_for_product(kw[3]) if kw[3] else None, device)
    got = plan.export()
    for i in range(qs.shape[0]):
        op = ora.plan_build(qs[i], dims, kw[0], kw[1], kw[2], kw[3])
        _plan_equal(got[i], op, f"dims={dims} codec={codec} q={i}")


def _trace_vs_oracle(blocks, plan_gpu, plans_ora, cfg_p, cfg_o, taus, lo=None, hi=None, what=""):
    tr = m.scan_fixed_tau(blocks, plan_gpu, cfg_p, taus, lo, hi)
    for qi, op in enumerate(plans_ora):
        for b in range(blocks.shape[0]):
            scored, masks, pre, sc = ora.block_stages(blocks[b], op, cfg_o, float(taus[qi]), lo, hi)
            gm = tr.masks[qi, b]
            assert np.array_equal(gm, masks), f"{what} q={qi} b={b}: masks {gm} vs {masks}"
            act = int(masks[0])
            lanes = [v for v in range(64) if (act >> v) & 1]
            assert np.array_equal(tr.prefix_ip[qi, b, lanes].view(np.uint32), pre[lanes].view(np.uint32)), \
                f"{what} q={qi} b={b}: prefix_ip"
            pushed = [v for v in range(64) if (int(masks[4]) >> v) & 1]
            assert np.array_equal(tr.scores[qi, b, pushed].view(np.uint32), sc[pushed].view(np.uint32)), \
                f"{what} q={qi} b={b}: scores"


@pytest.mark.parametrize("depth", [m.StrataDepth.L0_ONLY, m.StrataDepth.L1_RABITQ, m.StrataDepth.FULL64B])
def test_fixed_tau_stages_bit_exact(device, corpus768, depth):
    rows, fit, blocks = corpus768
    rng = np.random.default_rng(int(depth) + 3)
    qs = rows[rng.integers(0, rows.shape[0], 3)] + np.float32(0.01) * rng.standard_normal((3, 768)).astype(np.float32)
    plan = m.QueryPlan.from_query_eden(qs, 768, _fit_for_product(fit), device)
    plans_o = [ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit) for q in qs]
    sub = blocks[:24]
    for tau in (-np.inf, 0.3, 0.6):
        cfg_p = m.ScanConfig(shortlist_cand=64, strata_depth=depth)
        cfg_o = ora.scan_config(64, depth=int(depth))
        _trace_vs_oracle(sub, plan, plans_o, cfg_p, cfg_o, np.full(3, tau, np.float32), what=f"tau={tau}")


def test_fixed_tau_minmax_and_edenb1(device):
    rng = np.random.default_rng(99)
    rows = normalized(rng, 64 * 6, 384)
    pf, mf = oracle_fit(rows), oracle_fit_mid(rows)
    for enc, pc, mc, efit, mfit in ((None, ora.PREFIX_MINMAX4, ora.MID_RABITQ, None, None),
                                    ("dual", ora.PREFIX_EDEN_PROD, ora.MID_EDEN_B1, pf, mf)):
        blocks = oracle_encode_corpus(rows, 384, efit, mfit)
        qs = normalized(rng, 2, 384)
        plan = m.QueryPlan.from_query_codec(qs, 384, pc, mc, _fit_for_product(efit) if efit else None,
                                            _fit_for_product(mfit) if mfit else None, device)
        plans_o = [ora.plan_build(q, 384, pc, mc, efit, mfit) for q in qs]
        for tau in (-np.inf, 0.2):
            _trace_vs_oracle(blocks, plan, plans_o, m.ScanConfig(shortlist_cand=16), ora.scan_config(16),
                             np.full(2, tau, np.float32), what=f"codec={pc}/{mc} tau={tau}")


def test_fixed_tau_tombstones_and_time_filter(device, corpus768):
    rows, fit, blocks = corpus768
    b = blocks[:8].copy()
    b[2, 16:24] = 0xFF                                     # all tombstoned
    b[3, 16:24] = np.frombuffer(np.uint64(0xF0F0F0F00000FFFF).tobytes(), dtype=np.uint8)
    qs = rows[:2]
    plan = m.QueryPlan.from_query_eden(qs, 768, _fit_for_product(fit), device)
    plans_o = [ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit) for q in qs]
    cfg_p, cfg_o = m.ScanConfig(shortlist_cand=16), ora.scan_config(16)
    _trace_vs_oracle(b, plan, plans_o, cfg_p, cfg_o, np.full(2, 0.1, np.float32), lo=100, hi=300, what="time")


@pytest.mark.parametrize("k", [1, 16, 256])
@pytest.mark.parametrize("sharding", [False, True])
def test_scan_topk_vs_oracle(device, corpus768, k, sharding):
    rows, fit, blocks = corpus768
    rng = np.random.default_rng(k)
    qs = rows[rng.integers(0, rows.shape[0], 4)] + np.float32(0.003) * rng.standard_normal((4, 768)).astype(np.float32)
    ix = m.DeviceIndex.upload(blocks, device)
    plan = m.QueryPlan.from_query_eden(qs, 768, _fit_for_product(fit), device)
    res = m.scan_batch(ix, plan, m.EngineConfig(embed_dims=768, shortlist_cand=k))
    for qi, q in enumerate(qs):
        op = ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
        ids, sc = ora.scan_blocks(blocks, op, ora.scan_config(k, sharding=sharding, threads=4))
        n = int(res.counts[qi])
        assert_topk_equal(res.ids[qi, :n], res.scores[qi, :n], ids, sc, k, f"k={k} q={qi}")
        # the GPU ordering is score desc, id asc
        g = res.scores[qi, :n]
        assert np.all(g[:-1] >= g[1:])
