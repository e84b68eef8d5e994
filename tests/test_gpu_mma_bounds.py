"""The MFMA bounds themselves: for every (query, slot) pair, the f16 tiles'
lower and upper bounds (mrl_scan_mma_bounds) bracket the oracle's full score
(ora_exhaustive_scores: every stage of scan.rs:453-634 run, f32 in the
reference's order), and the bracket is narrow.  The top-K parity tests only
see pairs near the K-th score; this checks all of them, over both prefix
codecs, both depths with an S1 stage, two query chunks with a partial one,
inactive slots, meta beyond the operand range, and queries equal to (or the
negation of) corpus rows, which put scores at the ends of the range.  Each
case checks the full tiles' bounds and those of the final pass that bounds
the S4 stage (mrl_ctx_set_s4_bound ALWAYS: every pair forced through that
pass and made exact at its flush)."""
import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import normalized

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["full-tiles", "s4-bounded"], autouse=True)
def s4_policy(request, device):
    device.set_s4_bound(device.S4_BOUND_NEVER if request.param == "full-tiles" else device.S4_BOUND_ALWAYS)
    yield request.param
    device.set_s4_bound(device.S4_BOUND_AUTO)


def _queries(rows, rng, n_q):
    src = rng.integers(0, rows.shape[0], n_q)
    q = rows[src] + rng.standard_normal((n_q, rows.shape[1])).astype(np.float32) * np.float32(0.1 / np.sqrt(rows.shape[1]))
    q[0] = rows[src[0]]       # a corpus row itself: the top score
    q[1] = -rows[src[1]]      # its negation: the bottom score
    return (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)


def _check(device, blocks, qs, dims, fit, depth=m.StrataDepth.FULL64B, lo=None, hi=None, width=None, what=""):
    """width: the largest bracket allowed.  The prefix term dominates it,
    2 * 2^-8 * max|codebook| * scale * sum|w|: about 0.03 for EDEN's
    codebook (|c| < 2.7) and 0.15 for MinMax4's levels 0..15 on unit
    vectors."""
    eden = fit is not None
    if width is None:
        width = 0.03 if eden else 0.15
    codec = m.PrefixCodec.EDEN_PROD if eden else m.PrefixCodec.MIN_MAX4
    plan = m.QueryPlan.from_query_codec(qs, dims, codec, m.MidCodec.RABITQ, fit, None, device)
    cfg = m.ScanConfig(shortlist_cand=64, strata_depth=depth)
    up, lw = m.scan_mma_bounds(m.DeviceIndex.upload(blocks, device), plan, cfg, lo, hi)
    ofit = ora.Fit(fit.mean, 4, 1, fit.n_observed) if eden else None
    ocfg = ora.scan_config(64, depth=int(depth))
    widths = []
    for qi in range(len(qs)):
        op = ora.plan_build(qs[qi], dims, int(codec), 0, ofit, None)
        sc, valid = ora.exhaustive_scores(blocks, op, ocfg, lo, hi)
        u, l = up[qi], lw[qi]
        # inactive slots are not appended; active ones always are
        assert np.all(np.isnan(u[~valid])) and np.all(np.isnan(l[~valid])), f"{what} q={qi}: inactive slot bounded"
        assert not np.any(np.isnan(u[valid])) and not np.any(np.isnan(l[valid])), f"{what} q={qi}: active slot missing"
        bad = np.nonzero(~((l[valid] <= sc[valid]) & (sc[valid] <= u[valid])))[0]
        assert bad.size == 0, (f"{what} q={qi}: {bad.size} scores outside their bounds, first slot "
                               f"{np.nonzero(valid)[0][bad[0]]}: {l[valid][bad[0]]} <= {sc[valid][bad[0]]} <= "
                               f"{u[valid][bad[0]]}")
        fin = np.isfinite(u[valid]) & np.isfinite(l[valid])
        widths.append((u[valid][fin] - l[valid][fin]).astype(np.float64))
    w = np.concatenate(widths)
    print(f"[mma bounds] {what}: {w.size} pairs, width median {np.median(w):.3g} max {w.max():.3g}", flush=True)
    assert w.max() < width, f"{what}: bound width {w.max()} is not tight"
    return up, lw


def test_eden_full64b_two_chunks(device):
    print("[mma bounds] eden 768, 70 queries", flush=True)
    rng = np.random.default_rng(31)
    rows = normalized(rng, 100 * 64 - 5, 768)
    fit = m.EdenFit.fit_prefix(rows[:4096], 4, 1)
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    _check(device, blocks, _queries(rows, rng, 70), 768, fit, what="eden")


def test_minmax_l1_depth(device):
    print("[mma bounds] minmax 384 L1Rabitq", flush=True)
    rng = np.random.default_rng(32)
    rows = normalized(rng, 80 * 64, 384)
    blocks = m.encode_corpus(rows, 8)
    _check(device, blocks, _queries(rows, rng, 24), 384, None, depth=m.StrataDepth.L1_RABITQ, what="minmax L1")


def test_minmax_full_depth_generic_dims(device):
    print("[mma bounds] minmax 200", flush=True)
    rng = np.random.default_rng(33)
    rows = normalized(rng, 60 * 64 - 31, 200, head_heavy=False)
    blocks = m.encode_corpus(rows, 8)
    _check(device, blocks, _queries(rows, rng, 9), 200, None, what="minmax 200")


def test_inactive_and_out_of_range_slots(device):
    print("[mma bounds] tombstones, time filter, extreme meta", flush=True)
    rng = np.random.default_rng(34)
    rows = normalized(rng, 90 * 64, 768)
    blocks = m.encode_corpus(rows, 8)
    tomb = rng.integers(0, 2**63, size=blocks.shape[0], dtype=np.uint64)
    tomb[::3] = 0
    blocks[:, 16:24] = tomb.view(np.uint8).reshape(-1, 8)
    meta = blocks[:, 64:512].reshape(-1, 64, 7)
    big = np.frombuffer(np.float16(30000.0).tobytes(), dtype=np.uint8)
    meta[0, 7, 0:2] = big      # scale beyond the operand range (block 0: never tombstoned)
    meta[3, 9, 4:6] = big      # tail norm
    blocks[0, 16:24] = 0
    blocks[3, 16:24] = 0
    qs = _queries(rows, rng, 12)
    up, lw = _check(device, blocks, qs, 768, None, what="tombstones")
    assert np.all(np.isposinf(up[:, 7])) and np.all(np.isneginf(lw[:, 7]))
    assert np.all(np.isposinf(up[:, 3 * 64 + 9])) and np.all(np.isneginf(lw[:, 3 * 64 + 9]))
    # timestamps are row indices: keep rows 1000 .. 4000
    _check(device, blocks, qs, 768, None, lo=1000, hi=4000, what="temporal")


@pytest.mark.parametrize("eden", [True, False])
def test_subnormal_operands(device, eden):
    """Slots whose f16 scale, offset and tail norm lie in the f16 subnormal
    range (so the prefix operands cb[l]*scale, the S1 / S4 operands
    +-mid_n/2 and +-hn*w_s4/2, and the error-column entries are subnormal
    f16 values), and MinMax4 queries whose prefix weights span 2^-40 .. 1
    (the smallest become subnormal f16 operands after the query's
    power-of-two scaling).  Every pair's score must stay inside its bounds.
    Were subnormal operands flushed to zero, a slot with a subnormal scale
    would lose its whole prefix term, far more than its error term
    |scale| * eP, and the bracket would break."""
    print(f"[mma bounds] subnormal operands, eden={eden}", flush=True)
    rng = np.random.default_rng(36 + eden)
    rows = normalized(rng, 40 * 64, 768)
    fit = m.EdenFit.fit_prefix(rows[:2048], 4, 1) if eden else None
    blocks = m.encode_corpus(rows, m.source.DOC, fit)
    meta = blocks[:, 64:512].reshape(-1, 64, 7)
    sub = lambda n: rng.integers(1, 0x400, size=n, dtype=np.uint16) | (rng.integers(0, 2, size=n, dtype=np.uint16) << 15)
    for b in range(24):
        for part, sel in ((0, b % 3 != 2), (1, b % 3 != 1), (2, b % 3 != 0)):
            if sel:  # part 0: scale, 1: offset, 2: tail norm (kept positive)
                v = sub(64)
                if part == 2:
                    v &= 0x7FFF
                meta[b, :, 2 * part:2 * part + 2] = v.view(np.uint8).reshape(64, 2)
    meta[:24, :, 6] = rng.integers(0, 256, size=(24, 64), dtype=np.uint8)   # any rho
    qs = _queries(rows, rng, 16)
    if not eden:
        for qi in range(2, 16):
            dims = rng.choice(64, 12, replace=False)
            qs[qi, dims] *= np.float32(2.0) ** -rng.integers(20, 41, size=12).astype(np.float32)
    up, lw = _check(device, blocks, qs, 768, fit, what=f"subnormal eden={eden}")
    assert np.all(np.isfinite(up[:, :24 * 64])) and np.all(np.isfinite(lw[:, :24 * 64]))
