"""Pins the oracle's scan: the reference's own scan tests (scan.rs:888-1038,
pipeline.rs:203-243), every scored vector against a float64 closed form of
the stage formulas, and the admissibility of pruning (the pruned serial and
sharded scans return the exhaustive top-K)."""
import ctypes as C

import numpy as np
import pytest

import ora
from helpers import assert_topk_equal, normalized, oracle_encode_corpus, oracle_fit, oracle_fit_mid

L = ora.lib


def synth_block(seed, n, dims):
    """scan.rs:901-922: the reference's LCG-like deterministic rows."""
    rows = np.zeros((n, dims), dtype=np.float32)
    M = 1 << 32
    for i in range(n):
        for d in range(dims):
            x = ((seed * 1103515245 + 12345) % M + (i * 9973) % M + (d * 7919) % M) % M
            rows[i, d] = np.float32(np.float32(x % 10007) / np.float32(5003.5)) - np.float32(1.0)
        nrm = max(float(np.sqrt(np.sum(rows[i] * rows[i], dtype=np.float32))), 1e-12)
        rows[i] = rows[i] / np.float32(nrm)
    blk = ora.encode_block(rows, dims, np.arange(n), np.ones(n))
    return blk, rows


def test_default_kernel_stages_narrow_monotonically():
    """scan.rs:924-957"""
    blk, rows = synth_block(42, 64, 768)
    p = ora.plan_build(rows[0], 768)
    cfg = ora.scan_config(64)
    scored, masks, pre, sc = ora.block_stages(blk, p, cfg, -1.0)
    after_prefix, after_s1, after_bud, pushed = (bin(int(x)).count("1") for x in masks[1:])
    assert after_prefix > 0 and after_s1 <= after_prefix and after_bud <= after_s1
    assert int(masks[3]) & ~int(masks[2]) == 0
    assert pushed > 0


def test_scan_blocks_deterministic_and_stats_consistent():
    """scan.rs:959-993"""
    blk, rows = synth_block(7, 32, 768)
    p = ora.plan_build(rows[3], 768)
    cfg = ora.scan_config(16)
    a = ora.scan_blocks(blk, p, cfg)
    b = ora.scan_blocks(blk, p, cfg)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    ids, sc, st = ora.scan_blocks(blk, p, cfg, stats=True)
    assert np.array_equal(ids, a[0]) and np.array_equal(sc.view(np.uint32), a[1].view(np.uint32))
    assert st["blocks"] == 1 and st["active_vecs"] >= 32
    assert st["active_vecs"] >= st["after_prefix"] >= st["after_s1"] >= st["after_s4_budget"] >= st["pushed"]
    assert len(ids) <= 16 and len(ids) <= st["pushed"]


def test_strata_depth_gates_s4_scores():
    """scan.rs:1010-1037"""
    blk, rows = synth_block(99, 64, 768)
    p = ora.plan_build(rows[0], 768)
    full = ora.scan_blocks(blk, p, ora.scan_config(64, depth=ora.FULL64B))
    l1 = ora.scan_blocks(blk, p, ora.scan_config(64, depth=ora.L1_RABITQ))
    assert len(full[0]) > 0 and len(full[0]) == len(l1[0])
    assert not np.array_equal(full[1].view(np.uint32), l1[1].view(np.uint32))


def _closed_form(block, plan, v, depth, w_s4):
    """float64 restatement of one vector's full score (stages of scan.rs:453-634)."""
    d = ora.plan_to_dict(plan)
    mt = np.zeros(6, dtype=np.float32)
    L.ora_meta_decode(ora.u8p(block), v, ora.fp(mt))
    scale, offset, tail, rho = (float(x) for x in mt[:4])
    lv = np.zeros(64, dtype=np.uint8)
    L.ora_extract_bits4(ora.u8p(block), v, ora.u8p(lv))
    t = max(tail, 0.0)
    mid_n = max(np.sqrt(max(1 - rho * rho, 0.0)) * t, 1e-6)
    hn = max(rho * t, 0.0)
    q = d["prefix"].astype(np.float64)
    if depth == ora.L0_ONLY:
        cd = np.sum((lv >> 3 & 1) * q * 8.0)
        return cd * scale + offset * float(d["prefix_sum"])
    if plan.prefix_codec == ora.PREFIX_EDEN_PROD:
        w = d["eden_q_rot"].astype(np.float64) * float(d["eden_inv_sqrt_d"])
        score = float(d["eden_mean_ip"]) + scale * np.sum(d["eden_codebook"].astype(np.float64)[lv] * w)
    else:
        score = np.sum(lv * q) * scale + offset * float(d["prefix_sum"])
    s1w = block[1024:2048].view("<u8")
    bits1 = np.array([(int(s1w[k]) >> v) & 1 for k in range(128)])
    if plan.mid_codec == ora.MID_EDEN_B1:
        cw = float(d["eden_mid_base"]) + np.sum(bits1 * d["eden_mid_deltas"].astype(np.float64))
        score += float(d["eden_mid_mean_ip"]) + offset * cw
    else:
        s1 = float(d["rabitq_base"]) + np.sum(bits1 * d["rabitq_weights2"].astype(np.float64))
        score += s1 * mid_n
    if depth == ora.FULL64B and plan.has_tail_fold:
        s4w = block[3072:3584].view("<u8")
        bits4 = np.array([(int(s4w[k]) >> v) & 1 for k in range(64)])
        s4 = float(d["tail_fold_base"]) + np.sum(bits4 * d["tail_fold_weights2"].astype(np.float64))
        score += s4 * max(hn, 1e-6) * w_s4
    return score


@pytest.mark.parametrize("codec", ["minmax", "eden", "dual"])
@pytest.mark.parametrize("depth", [ora.L0_ONLY, ora.L1_RABITQ, ora.FULL64B])
def test_every_score_matches_the_float64_closed_form(codec, depth):
    rng = np.random.default_rng(int(depth) * 10 + len(codec))
    dims = 768
    rows = normalized(rng, 128, dims)
    pf, mf = oracle_fit(rows), oracle_fit_mid(rows)
    ef, emf, pc, mc = {"minmax": (None, None, ora.PREFIX_MINMAX4, ora.MID_RABITQ),
                       "eden": (pf, None, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ),
                       "dual": (pf, mf, ora.PREFIX_EDEN_PROD, ora.MID_EDEN_B1)}[codec]
    blocks = oracle_encode_corpus(rows, dims, ef, emf)
    q = normalized(rng, 1, dims)[0]
    p = ora.plan_build(q, dims, pc, mc, ef, emf)
    cfg = ora.scan_config(64, depth=depth, w_s4=0.2)
    sc, valid = ora.exhaustive_scores(blocks, p, cfg)
    assert valid.sum() == 128
    for r in range(128):
        ref = _closed_form(blocks[r // 64], p, r % 64, depth, 0.2)
        assert abs(float(sc[r]) - ref) < 2e-5, (r, float(sc[r]), ref)


def test_hand_built_block_single_bits():
    """One active vector whose levels and plane bits are set by hand."""
    blk = np.zeros(4096, dtype=np.uint8)
    blk[16:24] = np.frombuffer(np.uint64(~np.uint64(1)).tobytes(), dtype=np.uint8)  # only slot 0 active
    meta = blk[64:71]
    meta[0:2] = np.frombuffer(np.float16(0.5).tobytes(), dtype=np.uint8)   # scale
    meta[2:4] = np.frombuffer(np.float16(0.25).tobytes(), dtype=np.uint8)  # offset
    meta[4:6] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)   # tail norm
    meta[6] = 51                                                            # rho = 0.2
    # level of dim 3 = 0b1011 (S0, S3, S5 bits), S1 bit at d=5, S4 bit at d=9
    for off in (512, 2560, 3584):
        blk[off + 8 * 3] = 1
    blk[1024 + 8 * 5] = 1
    blk[3072 + 8 * 9] = 1
    q = np.zeros(768, dtype=np.float32)
    q[3] = 0.5
    q[64 + 7] = 0.3
    q[200] = 0.4
    p = ora.plan_build(q, 768)
    cfg = ora.scan_config(16)
    sc, valid = ora.exhaustive_scores(blk[None], p, cfg)
    d = ora.plan_to_dict(p)
    mid_n = np.sqrt(1 - (51 / 255) ** 2)
    hn = 51 / 255
    expect = (11 * 0.5) * 0.5 + 0.25 * 0.5
    expect += (float(d["rabitq_base"]) + float(d["rabitq_weights2"][5])) * mid_n
    expect += (float(d["tail_fold_base"]) + float(d["tail_fold_weights2"][9])) * hn * 0.2
    assert valid[0] and not valid[1:].any()
    assert abs(float(sc[0]) - expect) < 1e-6


@pytest.mark.parametrize("k", [1, 16, 100, 256, 1024])
@pytest.mark.parametrize("depth", [ora.L0_ONLY, ora.L1_RABITQ, ora.FULL64B])
def test_pruned_scans_return_the_exhaustive_topk(k, depth):
    rng = np.random.default_rng(k + 7 * int(depth))
    rows = normalized(rng, 64 * 40, 768)
    fit = oracle_fit(rows)
    blocks = oracle_encode_corpus(rows, 768, fit)
    blocks[3, 16:24] = 0xFF  # a fully tombstoned block
    q = rows[11] + np.float32(0.01) * rng.standard_normal(768).astype(np.float32)
    p = ora.plan_build(q, 768, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
    for sharding in (False, True):
        cfg = ora.scan_config(k, depth=depth, sharding=sharding, threads=3)
        ids, sc = ora.scan_blocks(blocks, p, cfg)
        eids, esc = ora.exhaustive_topk(blocks, p, cfg, k)
        assert_topk_equal(ids, sc, eids, esc, k, f"k={k} depth={depth} sharding={sharding}")


def test_temporal_filter_skips_blocks_by_header_bounds():
    rng = np.random.default_rng(12)
    rows = normalized(rng, 64 * 6, 384)
    blocks = oracle_encode_corpus(rows, 384)  # timestamps = row index
    q = rows[0]
    p = ora.plan_build(q, 384)
    cfg = ora.scan_config(64)
    ids, _ = ora.scan_blocks(blocks, p, cfg, lo=64 * 2, hi=64 * 4 - 1)
    blk = ids >> np.uint64(16)
    assert set(blk.tolist()) <= {2, 3}
    cfg_off = ora.scan_config(64, temporal=False)
    ids2, _ = ora.scan_blocks(blocks, p, cfg_off, lo=64 * 2, hi=64 * 4 - 1)
    assert len(set((ids2 >> np.uint64(16)).tolist()) - {2, 3}) > 0


def test_exact_ties_keep_the_first_pushed_in_serial_order():
    """Shortlist::push replaces only on a strictly greater score (scan.rs:351-368)."""
    rng = np.random.default_rng(13)
    v = normalized(rng, 1, 384)
    blk = ora.encode_block(np.repeat(v, 64, axis=0), 384)
    blocks = np.repeat(blk[None], 5, axis=0)
    p = ora.plan_build(v[0], 384)
    ids, sc = ora.scan_blocks(blocks, p, ora.scan_config(16))
    rows = (ids >> np.uint64(16)) * np.uint64(64) + (ids & np.uint64(0xFFFF))
    assert np.array_equal(np.sort(rows), np.arange(16, dtype=np.uint64))
    assert len(set(sc.view(np.uint32).tolist())) == 1


def test_nan_in_shortlist_is_reported():
    """into_sorted panics on NaN (scan.rs:390-394); the oracle returns an error."""
    rng = np.random.default_rng(14)
    rows = normalized(rng, 64, 768)
    blk = oracle_encode_corpus(rows, 768)[0].copy()
    q = rows[0].copy()
    q[700] = np.inf  # tail fold weights become inf/NaN; q_tail_norm = inf keeps bounds open
    p = ora.plan_build(q, 768)
    sc, valid = ora.exhaustive_scores(blk[None], p, ora.scan_config(64))
    if not np.isnan(sc[valid]).any():
        pytest.skip("no NaN survivor produced")
    with pytest.raises(FloatingPointError):
        ora.scan_blocks(blk[None], p, ora.scan_config(64))
