"""Writes tests/golden/*.npz: fixed inputs and the CPU oracle's outputs for
them.  Inputs are seeded numpy draws encoded by the oracle's encoder; the
outputs are the oracle's plans, per-stage survivor masks at fixed
thresholds, exhaustive scores and serial scan_blocks top-K lists.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import ora  # noqa: E402
from helpers import normalized, oracle_encode_corpus, oracle_fit  # noqa: E402

TAUS = np.array([-np.inf, 0.2, 0.5], dtype=np.float32)
KS = (16, 64)


def fixture(name, dims, n_rows, codec, seed, tombstone_block=None):
    rng = np.random.default_rng(seed)
    rows = normalized(rng, n_rows, dims)
    fit = oracle_fit(rows) if codec == ora.PREFIX_EDEN_PROD else None
    blocks = oracle_encode_corpus(rows, dims, fit)
    if tombstone_block is not None:
        blocks[tombstone_block, 16:24] = np.frombuffer(np.uint64(0xFFFF0000FFFF0000).tobytes(), dtype=np.uint8)
    src = rng.integers(0, n_rows, 4)
    queries = (rows[src] + np.float32(0.02) * rng.standard_normal((4, dims)).astype(np.float32)).astype(np.float32)
    out = {"blocks": blocks, "queries": queries, "dims": np.int32(dims), "prefix_codec": np.int32(codec),
           "taus": TAUS, "ks": np.array(KS, dtype=np.int32)}
    if fit is not None:
        out["fit_mean"] = fit.mean
    plans, masks, pre, sc, exh, exv = [], [], [], [], [], []
    topk_ids = {k: [] for k in KS}
    topk_sc = {k: [] for k in KS}
    for q in queries:
        p = ora.plan_build(q, dims, codec, ora.MID_RABITQ, fit, None)
        plans.append(np.frombuffer(bytes(p), dtype=np.uint8))
        cfg = ora.scan_config(64)
        mq, pq, sq = [], [], []
        for t in TAUS:
            mb, pb, sb = [], [], []
            for b in blocks:
                _, mk, pi, s = ora.block_stages(b, p, cfg, float(t))
                mb.append(mk), pb.append(pi), sb.append(s)
            mq.append(mb), pq.append(pb), sq.append(sb)
        masks.append(mq), pre.append(pq), sc.append(sq)
        e, v = ora.exhaustive_scores(blocks, p, cfg)
        exh.append(e), exv.append(v)
        for k in KS:
            ids, s = ora.scan_blocks(blocks, p, ora.scan_config(k))
            pad = np.full(k, np.iinfo(np.uint64).max, dtype=np.uint64)
            pad[:len(ids)] = ids
            spad = np.full(k, np.nan, dtype=np.float32)
            spad[:len(s)] = s
            topk_ids[k].append(pad), topk_sc[k].append(spad)
    out.update(plans=np.stack(plans), masks=np.array(masks, dtype=np.uint64), prefix_ip=np.array(pre, np.float32),
               stage_scores=np.array(sc, np.float32), exhaustive=np.array(exh, np.float32),
               exhaustive_valid=np.array(exv, bool))
    for k in KS:
        out[f"topk_ids_{k}"] = np.stack(topk_ids[k])
        out[f"topk_scores_{k}"] = np.stack(topk_sc[k])
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
    print(name, {k: v.shape for k, v in out.items() if hasattr(v, "shape")})


if __name__ == "__main__":
    fixture("eden768_32blk", 768, 32 * 64, ora.PREFIX_EDEN_PROD, 2026)
    fixture("minmax384_partial", 384, 12 * 64 - 23, ora.PREFIX_MINMAX4, 2027, tombstone_block=5)
