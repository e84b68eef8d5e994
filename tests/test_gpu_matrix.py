"""Top-K parity over a matrix of shapes chosen at the boundaries of the scan
paths: batches of 1 and 7 (the one-query kernel), 8 (the first MFMA batch),
31 / 33 (one or two 32-query tiles per wave), 63 / 65 (a partial and a second
64-query workgroup row), 255 / 256 / 257 (the largest batch whose plans and
query operands are built in one launch, and the first that takes two), K
from 1 to 4096, indexes with a partial last block, at and just above the
256 blocks below which no sampling pass runs, dims 384 / 512 / 768 / 1024,
both prefix codecs, the L0Only / L1Rabitq / Full64b depths and the
exhaustive flag, and indexes of 1,500 and 2,100 blocks (a final-pass grid
between one and two workgroups per CU, and the full two).  Every query's top K must equal the oracle's sharded
scan_blocks (scan.rs:802-886) with bit-identical scores (exact ties at the
K-th score excepted), under the library's own choice of MFMA final pass and
with the S4-bounded pass forced."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized

pytestmark = pytest.mark.gpu

FULL, L1, L0 = m.StrataDepth.FULL64B, m.StrataDepth.L1_RABITQ, m.StrataDepth.L0_ONLY

# (dims, vectors, queries, K, EDEN-prod prefix, depth, exhaustive, clusters)
CASES = [
    (768, 700 * 64 - 3, 1, 100, True, FULL, False, 0),
    (768, 700 * 64 - 3, 7, 100, True, FULL, False, 0),
    (768, 700 * 64, 8, 256, True, FULL, False, 40),
    (768, 600 * 64 + 17, 31, 1, True, FULL, False, 0),
    (768, 600 * 64, 33, 4096, False, FULL, False, 0),
    (512, 500 * 64, 63, 300, True, L1, False, 30),
    (768, 800 * 64, 65, 257, True, FULL, False, 300),
    (384, 400 * 64 - 1, 129, 50, False, L1, False, 0),
    (768, 300 * 64, 255, 64, True, FULL, False, 0),
    (768, 300 * 64, 256, 64, True, FULL, False, 0),
    (768, 300 * 64, 257, 64, True, FULL, False, 0),
    (1024, 200 * 64, 100, 200, True, FULL, True, 0),
    (768, 256 * 64, 9, 256, True, FULL, False, 0),
    (768, 257 * 64, 9, 256, True, FULL, False, 0),
    (768, 40 * 64 + 5, 16, 1000, True, FULL, False, 0),
    (768, 500 * 64, 12, 128, True, L0, False, 0),
    # grids between one and two workgroups per CU (the final pass's CU pairs split their columns) and
    # at the full two (a partial last block, clustered rows)
    (768, 1500 * 64 - 7, 64, 256, True, FULL, False, 50),
    (512, 2100 * 64, 40, 100, True, FULL, False, 0),
]


def _ids(c):
    dims, n, nq, k, eden, depth, exh, cl = c
    return f"d{dims}-n{n}-q{nq}-k{k}-{'eden' if eden else 'minmax'}-{depth.name.lower()}{'-exh' if exh else ''}" \
           f"{f'-c{cl}' if cl else ''}"


@pytest.fixture(params=["auto", "s4-bounded"])
def s4_policy(request, device):
    device.set_s4_bound(device.S4_BOUND_AUTO if request.param == "auto" else device.S4_BOUND_ALWAYS)
    yield request.param
    device.set_s4_bound(device.S4_BOUND_AUTO)


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_shape_matrix(device, s4_policy, case):
    dims, n, n_q, k, eden, depth, exhaustive, clusters = case
    print(f"[matrix] {_ids(case)} {s4_policy}", flush=True)
    rng = np.random.default_rng(dims * 7919 + n_q * 31 + k)
    rows = normalized(rng, n, dims)
    if clusters:
        cent = normalized(rng, clusters, dims)
        rows = cent[rng.integers(0, clusters, n)] + rng.standard_normal((n, dims)).astype(np.float32) * np.float32(
            0.3 / np.sqrt(dims))
        rows = (rows / np.linalg.norm(rows, axis=1, keepdims=True)).astype(np.float32)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1) if eden else None
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    src = rng.integers(0, n, n_q)
    qs = rows[src] + rng.standard_normal((n_q, dims)).astype(np.float32) * np.float32(0.1 / np.sqrt(dims))
    qs = (qs / np.linalg.norm(qs, axis=1, keepdims=True)).astype(np.float32)

    codec = m.PrefixCodec.EDEN_PROD if eden else m.PrefixCodec.MIN_MAX4
    plan = m.QueryPlan.from_query_codec(qs, dims, codec, m.MidCodec.RABITQ, fit, None, device)
    cfg = m.ScanConfig(shortlist_cand=k, strata_depth=depth, exhaustive=exhaustive)
    res = m.scan_batch(m.DeviceIndex.upload(blocks, device), plan, cfg)

    ofit = ora.Fit(fit.mean, 4, 1, fit.n_observed) if eden else None
    ocfg = ora.scan_config(k, depth=int(depth), sharding=True, threads=8)
    for qi in range(n_q):
        op = ora.plan_build(qs[qi], dims, int(codec), 0, ofit, None)
        rids, rsc = ora.scan_blocks(blocks, op, ocfg)
        c = int(res.counts[qi])
        assert c == min(k, n), f"{_ids(case)} q={qi}: {c} hits"
        assert_topk_equal(res.ids[qi, :c], res.scores[qi, :c], rids, rsc, k, f"{_ids(case)} q={qi}")
        g = res.scores[qi, :c]
        assert np.all(g[:-1] >= g[1:]), f"{_ids(case)} q={qi}: not sorted"
