"""Pins the oracle's primitives against mathematics and independent
implementations: IEEE binary16 (numpy), CRC-32 (zlib), the Walsh-Hadamard
transform (explicit Hadamard matrices), the folded-tail operator structure
(tests/test_operator_folding.rs of the reference) and the Lloyd-Max
codebooks (the N(0,1) centroid condition)."""
import ctypes as C
import zlib

import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.stats import norm

import ora

L = ora.lib


# ---------------------------------------------------------------- binary16
def test_f16_to_f32_all_patterns_match_numpy():
    h = np.arange(65536, dtype=np.uint16)
    out = np.zeros(65536, dtype=np.float32)
    L.ora_f16_to_f32_array(h.ctypes.data_as(C.POINTER(C.c_uint16)), ora.fp(out), 65536)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(100000) * 1e-5).astype(np.float32),     # f16 subnormal range
        (rng.standard_normal(20000) * 1e5).astype(np.float32),       # overflow to inf
        np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32),  # exact halves
    ])
    # exact halfway points between neighbouring halves (ties to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((lo + hi) / 2).astype(np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    out = np.zeros(x.size, dtype=np.uint16)
    L.ora_f32_to_f16_array(ora.fp(x), out.ctypes.data_as(C.POINTER(C.c_uint16)), x.size)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(out, ref)


# ---------------------------------------------------------------- CRC-32
def test_crc32_known_answer_and_zlib():
    kat = np.frombuffer(b"123456789", dtype=np.uint8)
    assert L.ora_crc32(ora.u8p(kat), 9) == 0xCBF43926
    rng = np.random.default_rng(1)
    for n in (0, 1, 7, 4096, 10001):
        buf = rng.integers(0, 256, n, dtype=np.uint8)
        assert L.ora_crc32(ora.u8p(buf), n) == zlib.crc32(buf.tobytes())


def test_block_crc_verifies_and_detects_corruption():
    rng = np.random.default_rng(2)
    v = rng.standard_normal((5, 384)).astype(np.float32)
    blk = ora.encode_block(v, 384)
    assert L.ora_verify_crc(ora.u8p(blk)) == 1
    blk[1000] ^= 1
    assert L.ora_verify_crc(ora.u8p(blk)) == 0


# ---------------------------------------------------------------- FWHT
@pytest.mark.parametrize("n", [64, 128])
def test_fwht_is_the_orthonormal_hadamard_transform(n):
    rng = np.random.default_rng(n)
    H = hadamard(n).astype(np.float64) / np.sqrt(n)
    for _ in range(20):
        x = rng.standard_normal(n).astype(np.float32)
        y = x.copy()
        L.ora_fwht_inplace(ora.fp(y), n)
        assert np.max(np.abs(y - H @ x.astype(np.float64))) < 1e-6
        # rotate.rs:204-210: L2 preserved
        assert abs(np.linalg.norm(y) - np.linalg.norm(x)) < 1e-4
        # involution
        L.ora_fwht_inplace(ora.fp(y), n)
        assert np.max(np.abs(y - x)) < 1e-5


def test_rademacher_would_be_noop_but_fwht_is_not():
    """rotate.rs:212-219"""
    mid = np.zeros(128, dtype=np.float32)
    mid[0] = 1.0
    out = np.zeros(128, dtype=np.float32)
    L.ora_rotate_mid_band(ora.fp(mid), ora.fp(out))
    assert np.any(np.abs(out[1:]) > 1e-6)


def test_fold_tail_768_is_nontrivial():
    """rotate.rs:221-234"""
    v = np.array([((i * 3) % 17) * 0.01 - 0.08 if i >= 192 else 0.0 for i in range(768)], dtype=np.float32)
    folded = np.zeros(64, dtype=np.float32)
    rot = np.zeros(64, dtype=np.float32)
    L.ora_fold_tail(ora.fp(v), 768, ora.fp(folded))
    L.ora_rotate_tail_fold(ora.fp(v), 768, ora.fp(rot))
    assert float(np.sum(folded.astype(np.float64) ** 2)) > 1e-6
    assert abs(np.linalg.norm(folded) - np.linalg.norm(rot)) < 1e-4


def _operator_t():
    """256 x 768 sketch operator built from impulses (test_operator_folding.rs:12-48)."""
    T = np.zeros((256, 768))
    T[:64, :64] = np.eye(64)
    for j in range(128):
        e = np.zeros(128, dtype=np.float32)
        e[j] = 1
        out = np.zeros(128, dtype=np.float32)
        L.ora_rotate_mid_band(ora.fp(e), ora.fp(out))
        T[64:192, 64 + j] = out
    for j in range(576):
        e = np.zeros(768, dtype=np.float32)
        e[192 + j] = 1
        out = np.zeros(64, dtype=np.float32)
        L.ora_rotate_tail_fold(ora.fp(e), 768, ora.fp(out))
        T[192:, 192 + j] = out
    return T


def test_operator_gram_structure_and_fold_amplification():
    """test_operator_folding.rs:224-438: T T^T = diag(I64, I128, 9 I64); the
    fold amplifies by at most sqrt(9) = 3 and is exact on the tail blocks."""
    T = _operator_t()
    G = T @ T.T
    expect = np.diag(np.concatenate([np.ones(192), 9 * np.ones(64)]))
    assert np.max(np.abs(G - expect)) < 1e-5
    s = np.linalg.svd(T[192:, 192:], compute_uv=False)
    assert abs(s.max() - 3.0) < 1e-5 and abs(s.min() - 3.0) < 1e-5
    # the operator reproduces the pipeline functions (test_operator_folding.rs:52-93)
    rng = np.random.default_rng(42)
    for _ in range(20):
        z = rng.uniform(-2, 2, 768).astype(np.float32)
        mid = np.zeros(128, dtype=np.float32)
        tail = np.zeros(64, dtype=np.float32)
        L.ora_rotate_mid_band(ora.fp(np.ascontiguousarray(z[64:192])), ora.fp(mid))
        L.ora_rotate_tail_fold(ora.fp(z), 768, ora.fp(tail))
        exp = np.concatenate([z[:64], mid, tail])
        assert np.max(np.abs(T @ z.astype(np.float64) - exp)) < 2e-5


def test_bit_scales_closed_form():
    assert abs(L.ora_rabitq_bit_scale() - np.sqrt(2 / np.pi) / np.sqrt(128)) < 1e-8
    assert abs(L.ora_tail_fold_bit_scale() - np.sqrt(2 / np.pi) / np.sqrt(64)) < 1e-8


# ---------------------------------------------------------------- EDEN codebooks
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_lloyd_max_codebooks_are_the_normal_centroids(bits):
    """Sorted, symmetric (eden.rs:374-381) and each level is E[Z | Z in its
    Voronoi cell] for Z ~ N(0,1): the Lloyd-Max fixed point, to 1e-6."""
    p = C.POINTER(C.c_float)()
    n = L.ora_lloyd_max_normal(bits, C.byref(p))
    cb = np.array([p[i] for i in range(n)], dtype=np.float64)
    assert n == 2 ** bits
    assert np.all(np.diff(cb) > 0)
    assert np.max(np.abs(cb + cb[::-1])) < 1e-7
    edges = np.concatenate([[-np.inf], (cb[1:] + cb[:-1]) / 2, [np.inf]])
    a, b = edges[:-1], edges[1:]
    centroid = (norm.pdf(a) - norm.pdf(b)) / (norm.cdf(b) - norm.cdf(a))
    assert np.max(np.abs(centroid - cb)) < 2e-6


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_lloyd_max_codebooks_bit_exact_to_reference_literals(bits):
    """Every codebook entry has the binary32 bits of the reference's decimal
    literal (eden.rs:15-44, rounded directly to f32 by
    tests/golden/make_codebooks.py), not just a value within 2e-6."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "eden_codebooks.json")) as f:
        fx = json.load(f)
    want = np.array([int(h, 16) for h in fx[f"B{bits}"]["f32_bits"]], dtype=np.uint32)
    p = C.POINTER(C.c_float)()
    n = L.ora_lloyd_max_normal(bits, C.byref(p))
    got = np.array([p[i] for i in range(n)], dtype=np.float32).view(np.uint32)
    assert np.array_equal(got, want)
    # the fixture's bits are the nearest binary32 of each decimal literal
    from fractions import Fraction
    for lit, h in zip(fx[f"B{bits}"]["decimal"], want):
        v = np.array(h, dtype=np.uint32).view(np.float32)
        up = np.nextafter(v, np.float32(np.inf))
        dn = np.nextafter(v, np.float32(-np.inf))
        e = abs(Fraction(float(v)) - Fraction(lit))
        assert e <= abs(Fraction(float(up)) - Fraction(lit)) and e <= abs(Fraction(float(dn)) - Fraction(lit))


def test_nearest_centroid_matches_brute_force_with_lower_index_ties():
    p = C.POINTER(C.c_float)()
    n = L.ora_lloyd_max_normal(4, C.byref(p))
    cb = np.array([p[i] for i in range(n)], dtype=np.float32)
    rng = np.random.default_rng(3)
    mids = ((cb[1:] + cb[:-1]) / np.float32(2)).astype(np.float32)
    zs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 2, cb, mids,
                         np.array([-10, 10, 0, -0.0], dtype=np.float32)])
    cbp = cb.ctypes.data_as(C.POINTER(C.c_float))
    for z in zs:
        d = np.abs(np.float32(z) - cb)  # eden.rs:58-71: |z - lo| <= |hi - z| keeps the lower
        best = int(np.argmin(d))
        got = L.ora_nearest_centroid(cbp, n, float(z))
        if got != best:
            assert abs(float(d[got]) - float(d[best])) == 0.0 and got < best
