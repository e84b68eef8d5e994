"""Pins the oracle's encoder, EDEN codec and query plan: the reference's own
tests (quantize.rs:375-427, eden.rs:384-424, scan.rs:996-1008) plus closed
forms in float64 (explicit Hadamard matrices), and byte-identity of the
product's host encoder with the oracle."""
import ctypes as C

import numpy as np
import pytest
from scipy.linalg import hadamard

import mrl_index_amd as m
import ora
from helpers import normalized, oracle_encode_corpus, oracle_fit, oracle_fit_mid

L = ora.lib
H64 = hadamard(64).astype(np.float64) / 8.0
H128 = hadamard(128).astype(np.float64) / np.sqrt(128)


def rad(seed, n):
    return np.array([L.ora_rademacher_diag(seed, i) for i in range(n)])


def tail_signs(nb):
    return np.array([[L.ora_tail_rademacher(b, d) for d in range(64)] for b in range(nb)])


def fold64(x, dims):
    nb = min((dims - 192) // 64, 9) if dims > 192 else 0
    S = tail_signs(nb) if nb else np.zeros((0, 64))
    u = np.zeros(64)
    for b in range(nb):
        u += S[b] * x[192 + 64 * b:256 + 64 * b]
    return u


def meta(block, v):
    out = np.zeros(6, dtype=np.float32)
    L.ora_meta_decode(ora.u8p(block), v, ora.fp(out))
    return out  # scale, offset, tail, rho, mid_norm, high_norm


def bits4(block, v):
    out = np.zeros(64, dtype=np.uint8)
    L.ora_extract_bits4(ora.u8p(block), v, ora.u8p(out))
    return out


def plane(block, off, n):
    return block[off:off + 8 * n].view("<u8")


# ---------------------------------------------------------------- encoder
def test_encode_roundtrip_bits_and_crc():
    """quantize.rs:375-398"""
    v = np.array([((i * 0.07) % 2.0) - 1.0 for i in range(256)], dtype=np.float32)
    blk = ora.encode_block(v, 256, [42], [4])
    assert L.ora_verify_crc(ora.u8p(blk)) == 1
    assert blk[0:4].view("<u4")[0] == 42
    tomb = int(blk[16:24].view("<u8")[0])
    assert bin(~tomb & (2 ** 64 - 1)).count("1") == 1 and (tomb >> 1) & 1
    lv = bits4(blk, 0).astype(np.float32)
    mt = meta(blk, 0)
    approx = lv * mt[0] + mt[1]
    assert np.mean(np.abs(approx - v[:64])) < 0.2


def test_encode_768_packs_rho_and_stratum4():
    """quantize.rs:401-427"""
    v = np.array([((i * 0.013) % 2.0) - 1.0 for i in range(768)], dtype=np.float32)
    v /= np.linalg.norm(v)
    blk = ora.encode_block(v, 768, [1], [8])
    assert blk[64 + 6] > 0
    mt = meta(blk, 0)
    assert abs(mt[4] ** 2 + mt[5] ** 2 - mt[2] ** 2) < 1e-3
    ones = sum(int(w) & 1 for w in plane(blk, 3072, 64))
    assert 5 < ones < 60


@pytest.mark.parametrize("dims", [192, 384, 768, 1024])
def test_encoder_fields_match_float64_closed_forms(dims):
    rng = np.random.default_rng(dims)
    x = normalized(rng, 64, dims)
    blk = ora.encode_block(x, dims)
    s1 = plane(blk, 1024, 128)
    s4 = plane(blk, 3072, 64)
    for v in range(64):
        xv = x[v].astype(np.float64)
        # min-max levels reconstruct within half a step
        mt = meta(blk, v)
        lv = bits4(blk, v).astype(np.float64)
        rec = mt[1] + mt[0] * lv
        step = (xv[:64].max() - xv[:64].min()) / 15
        assert np.max(np.abs(rec - xv[:64])) <= step / 2 + 2e-3 * max(1.0, abs(xv[:64]).max())
        # RaBitQ signs of H128 x_mid and folded-tail signs of H64 fold(x)
        rot = H128 @ xv[64:192]
        got = np.array([(int(s1[d]) >> v) & 1 for d in range(128)])
        sure = np.abs(rot) > 1e-5
        assert np.array_equal(got[sure], (rot[sure] >= 0).astype(int))
        if dims > 192:
            tf = H64 @ fold64(xv, dims)
            got4 = np.array([(int(s4[d]) >> v) & 1 for d in range(64)])
            sure = np.abs(tf) > 1e-5
            assert np.array_equal(got4[sure], (tf[sure] >= 0).astype(int))
        # rho = round(255 * |x_tail| / |x_rest|)
        rest = np.linalg.norm(xv[64:])
        high = np.linalg.norm(xv[192:])
        assert abs(int(blk[64 + 7 * v + 6]) - 255 * high / rest) <= 0.5 + 1e-3
        assert abs(mt[2] - rest) <= 1e-3 * rest + 1e-7


def test_eden_levels_are_nearest_centroids_of_the_rotated_unit_vector():
    rng = np.random.default_rng(5)
    rows = normalized(rng, 500, 768)
    fit = oracle_fit(rows)
    p = C.POINTER(C.c_float)()
    L.ora_lloyd_max_normal(4, C.byref(p))
    cb = np.array([p[i] for i in range(16)])
    R = H64 @ np.diag(rad(1, 64))
    for v in range(100):
        lv = np.zeros(64, dtype=np.uint8)
        cn = C.c_float()
        ss = C.c_float()
        L.ora_eden_encode_slice(fit.ref(), ora.fp(rows[v]), ora.u8p(lv), C.byref(cn), C.byref(ss))
        xc = rows[v, :64].astype(np.float64) - fit.mean.astype(np.float64)
        assert abs(cn.value - np.linalg.norm(xc)) < 1e-6
        z = R @ (xc / np.linalg.norm(xc)) * 8.0
        d = np.abs(z[:, None] - cb[None, :])
        best = np.argmin(d, axis=1)
        margin = np.sort(d, axis=1)[:, 1] - np.sort(d, axis=1)[:, 0]
        ok = margin > 1e-4
        assert np.array_equal(lv[ok], best[ok])
        # unbiased scale: S * <u, codeword> = 1
        cw = cb[lv] / 8.0
        u = R @ (xc / np.linalg.norm(xc))
        assert abs(ss.value * float(u @ cw) - 1.0) < 1e-4


def test_eden_unbiased_slope_near_one_on_gaussian():
    """eden.rs:384-424 with the reference's deterministic pseudo-gaussian rows."""
    M = (1 << 64) - 1
    rows = []
    for n in range(128):
        v = np.zeros(64, dtype=np.float32)
        for i in range(64):
            x = ((n * 0x9E37 + i) * 0xBF58) & M
            x ^= x >> 17
            xi = x - (1 << 64) if x >= (1 << 63) else x
            v[i] = np.float32(np.float32(xi) / np.float32(M)) * np.float32(2.0) - np.float32(1.0)
        nrm = max(float(np.sqrt(np.sum(v * v, dtype=np.float32))), 1e-6)
        rows.append((v / np.float32(nrm)).astype(np.float32))
    rows = np.stack(rows)
    fit = oracle_fit(rows, seed=1)
    q = rows[0]
    qr = np.zeros(64, dtype=np.float32)
    L.ora_eden_rotate_query(fit.ref(), ora.fp(q), ora.fp(qr))
    num = den = 0.0
    for r in rows:
        lv = np.zeros(64, dtype=np.uint8)
        cn, ss = C.c_float(), C.c_float()
        L.ora_eden_encode_slice(fit.ref(), ora.fp(r), ora.u8p(lv), C.byref(cn), C.byref(ss))
        est = L.ora_eden_score_ip(fit.ref(), ora.fp(q), ora.fp(qr), ora.u8p(lv), cn.value * ss.value)
        exact = float(np.dot(q, r))
        num += est * exact
        den += exact * exact
    assert abs(num / max(den, 1e-8) - 1.0) < 0.35


def test_eden_fit_is_the_corpus_mean_and_observe_is_welford():
    rng = np.random.default_rng(6)
    rows = normalized(rng, 1000, 384)
    fit = oracle_fit(rows)
    assert np.max(np.abs(fit.mean - rows[:, :64].astype(np.float64).mean(axis=0))) < 1e-6
    mean = np.zeros(64, dtype=np.float32)
    n = C.c_uint64(0)
    for r in rows:
        L.ora_eden_observe(ora.fp(mean), 64, C.byref(n), ora.fp(r))
    assert n.value == 1000
    assert np.max(np.abs(mean - fit.mean)) < 1e-5


# ---------------------------------------------------------------- product encoder
@pytest.mark.parametrize("dims", [192, 384, 768, 1024])
@pytest.mark.parametrize("codec", ["minmax", "eden", "dual"])
def test_product_encoder_is_byte_identical_to_oracle(dims, codec):
    rng = np.random.default_rng(dims + len(codec))
    rows = normalized(rng, 64 * 3 + 11, dims)
    rows[5] = 0.0                     # zero vector
    rows[6, 64:] = 0.0                # no residual
    rows[7, :64] = 0.25               # constant prefix
    rows[8] *= np.float32(3e4)        # large magnitude
    rows[9] *= np.float32(1e-30)      # tiny magnitude
    rows[10, 5] = np.nan              # NaN in the prefix (f32::max keeps 1e-12 for the norm)
    rows[11, 100] = np.nan            # NaN in the mid band
    rows[12, dims - 1] = np.inf       # infinity in the tail
    rows[13, 70] = -np.inf            # infinity in the mid band
    pf = oracle_fit(rows[16:])
    mf = oracle_fit_mid(rows[16:])
    ef, emf = {"minmax": (None, None), "eden": (pf, None), "dual": (pf, mf)}[codec]
    ref = oracle_encode_corpus(rows, dims, ef, emf)
    P = lambda f: m.EdenFit(f.mean.shape[0], f.c.bits, f.c.seed, f.mean, f.c.n_observed) if f else None
    got = m.encode_corpus(rows, 8, P(ef), P(emf), n_threads=4)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- query plan
def test_s4_abs_budget_is_positive_for_768d_query():
    """scan.rs:996-1008"""
    q = np.array([((i * 17) % 101) * 0.01 - 0.5 for i in range(768)], dtype=np.float32)
    q /= np.linalg.norm(q)
    p = ora.plan_build(q, 768)
    assert p.has_tail_fold and p.s4_abs_budget > 0 and p.q_mid_norm > 0 and p.q_tail_norm > 0
    assert p.q_after_s1 == p.q_tail_norm


@pytest.mark.parametrize("dims", [200, 384, 768])
def test_plan_fields_match_float64_closed_forms(dims):
    rng = np.random.default_rng(dims)
    rows = normalized(rng, 300, dims)
    fit = oracle_fit(rows)
    q = normalized(rng, 1, dims)[0]
    p = ora.plan_build(q, dims, ora.PREFIX_EDEN_PROD, ora.MID_RABITQ, fit)
    d = ora.plan_to_dict(p)
    qd = q.astype(np.float64)
    rs = np.sqrt(2 / np.pi) / np.sqrt(128)
    ts = np.sqrt(2 / np.pi) / 8
    rq = H128 @ qd[64:192]
    assert np.max(np.abs(d["rabitq_q"] - rq)) < 1e-6
    assert np.max(np.abs(d["rabitq_weights2"] - 2 * rq * rs)) < 1e-6
    assert abs(d["rabitq_base"] + np.sum(rq * rs)) < 1e-5
    for g in range(32):
        pos = rq[4 * g:4 * g + 4] * rs
        for mask in range(16):
            sgn = np.array([1 if mask >> i & 1 else -1 for i in range(4)])
            assert abs(d["rabitq_lut"][g, mask] - np.sum(sgn * pos)) < 1e-6
    assert abs(d["q_mid_norm"] - np.linalg.norm(qd[64:192])) < 1e-6
    assert abs(d["q_tail_norm"] - np.linalg.norm(qd[192:])) < 1e-6
    assert abs(d["q_after_prefix"] - np.linalg.norm(qd[64:])) < 1e-6
    tf = H64 @ fold64(qd, dims)
    assert np.max(np.abs(d["tail_fold_q"] - tf)) < 1e-5
    assert abs(d["s4_abs_budget"] - np.sum(np.abs(tf * ts))) < 1e-5
    assert abs(d["tail_fold_base"] + np.sum(tf * ts)) < 1e-5
    er = H64 @ (rad(1, 64) * qd[:64])
    assert np.max(np.abs(d["eden_q_rot"] - er)) < 1e-6
    assert abs(d["eden_mean_ip"] - qd[:64] @ fit.mean.astype(np.float64)) < 1e-6
    assert np.max(np.abs(d["prefix_weight"] - er / 8)) < 1e-6
    # q * 2^k is exact in binary floating point
    for kk in range(4):
        assert np.array_equal(d["bit_weights"][:, kk].view(np.uint32), (q[:64] * np.float32(2 ** kk)).view(np.uint32))
    assert abs(d["prefix_sum"] - qd[:64].sum()) < 1e-6 and abs(d["prefix_l1"] - np.abs(qd[:64]).sum()) < 1e-6


def test_plan_rejects_what_the_reference_asserts():
    q = np.zeros(191, dtype=np.float32)
    with pytest.raises(ValueError):
        ora.plan_build(q, 191)
    with pytest.raises(ValueError):
        ora.plan_build(np.zeros(384, dtype=np.float32), 384, ora.PREFIX_EDEN_PROD)
