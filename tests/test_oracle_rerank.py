"""Pins the oracle's rerank restatement (src/embed.rs:115-206, src/lowprec.rs:49-121,
src/pipeline.rs:157-169) with checks that do not retype its formulas:
float64 closed forms with error bounds, exact-integer inputs, inputs whose f32
rounding exposes the accumulation order, numpy's IEEE binary16 conversion,
a round-half-away-from-zero quantizer written from the definition, and
Python's stable sort."""
import math

import numpy as np
import pytest

import ora

TWO24 = np.float32(2.0 ** 24)


def _rng(seed):
    return np.random.default_rng(seed)


def test_dot768_is_close_to_the_float64_dot():
    r = _rng(1)
    for _ in range(20):
        a = r.standard_normal(768).astype(np.float32)
        b = r.standard_normal(768).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = 768 * 2.0 ** -24 * float(np.abs(a.astype(np.float64) * b).sum()) * 1.01
        assert abs(ora.dot(a, b) - exact) <= bound


def test_dot768_exact_on_integers():
    r = _rng(2)
    a = r.integers(-20, 21, 768).astype(np.float32)
    b = r.integers(-20, 21, 768).astype(np.float32)
    assert ora.dot(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def test_dot768_accumulator_j_takes_indices_j_mod_8():
    # 2^24 in accumulator 0; two ones in accumulator 1 (indices 1 and 9) add
    # to 2 before meeting 2^24, so 2^24 + 2 survives.  One sequential sum
    # would drop each 1 against 2^24 (ties to even).
    a = np.ones(768, dtype=np.float32)
    b = np.zeros(768, dtype=np.float32)
    b[0], b[1], b[9] = TWO24, 1.0, 1.0
    assert ora.dot(a, b) == float(TWO24) + 2.0


def test_dot768_final_sum_runs_left_to_right():
    # acc0 = 2^24, acc1 = acc2 = acc3 = 1: ((2^24 + 1) + 1) + 1 keeps 2^24
    # at every step; a pairwise tree would give 2^24 + 2.
    a = np.ones(768, dtype=np.float32)
    b = np.zeros(768, dtype=np.float32)
    b[0], b[1], b[2], b[3] = TWO24, 1.0, 1.0, 1.0
    assert ora.dot(a, b) == float(TWO24)


def test_dot768_accumulators_start_at_plus_zero():
    a = np.full(768, -1.0, dtype=np.float32)
    b = np.zeros(768, dtype=np.float32)  # every product is -0.0
    assert math.copysign(1.0, ora.dot(a, b)) == 1.0


def test_generic_dot_is_sequential_from_minus_zero():
    # dims != 768: a.iter().zip(b).map(x*y).sum() -- one chain, so the ones
    # are dropped against 2^24 one at a time.
    a = np.ones(384, dtype=np.float32)
    b = np.zeros(384, dtype=np.float32)
    b[0], b[1], b[9] = TWO24, 1.0, 1.0
    assert ora.dot(a, b) == float(TWO24)
    b[:] = 0.0
    b[3] = 1.0
    b[0] = -TWO24
    assert ora.dot(a, b) == -float(TWO24) + 1.0  # -2^24 + 1 is representable
    neg = ora.dot(np.full(384, -1.0, np.float32), np.zeros(384, np.float32))
    assert math.copysign(1.0, neg) == -1.0  # parity unpinned: Sum's start value


def test_dot_fp16_is_dot768_of_the_binary16_row():
    r = _rng(3)
    for scale in (1.0, 1e-6, 2e3):  # 1e-6: f16 subnormals; 2e3: large but finite
        q = r.standard_normal(768).astype(np.float32)
        v = (r.standard_normal(768) * scale).astype(np.float32)
        v16 = v.astype(np.float16).astype(np.float32)  # numpy: IEEE round to nearest even
        assert ora.dot_fp16_768(q, v) == ora.dot(q, v16)


def _round_half_away(x):
    x = np.asarray(x, dtype=np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def _quantize_from_definition(v):
    v = np.asarray(v, dtype=np.float32)
    absv = np.abs(v)
    max_abs = np.float32(np.max(np.where(np.isnan(absv), 0.0, absv), initial=0.0))
    scale = np.float32(0.0) if max_abs < np.float32(1e-12) else np.float32(max_abs / np.float32(127.0))
    inv = np.float32(1.0) / scale if scale > 0 else np.float32(0.0)
    with np.errstate(invalid="ignore"):
        prod = (v * np.float32(inv)).astype(np.float32)
    q = np.clip(_round_half_away(prod), -127, 127)
    q = np.where(np.isnan(q), 0, q).astype(np.int8)
    return q, np.float16(scale).view(np.uint16)


def test_int8_quantize_matches_the_definition():
    r = _rng(4)
    for scale in (1.0, 1e-3, 50.0):
        v = (r.standard_normal(768) * scale).astype(np.float32)
        codes, s = ora.int8_quantize_768(v)
        want_c, want_s = _quantize_from_definition(v)
        assert np.array_equal(codes, want_c)
        assert s == int(want_s)
        assert np.abs(codes).max() == 127


def test_int8_rounds_half_away_from_zero():
    v = np.zeros(768, dtype=np.float32)
    v[0] = 127.0      # scale exactly 1, inv exactly 1
    v[1], v[2], v[3], v[4] = 2.5, -2.5, 0.5, -1.5
    codes, s = ora.int8_quantize_768(v)
    assert list(codes[:5]) == [127, 3, -3, 1, -2]
    assert np.float16(1.0).view(np.uint16) == s


def test_int8_special_rows():
    zero = np.zeros(768, dtype=np.float32)
    c, s = ora.int8_quantize_768(zero)
    assert not c.any() and s == 0
    tiny = np.full(768, 1e-13, dtype=np.float32)   # below 1e-12: scale 0, codes 0
    c, s = ora.int8_quantize_768(tiny)
    assert not c.any() and s == 0
    v = _rng(5).standard_normal(768).astype(np.float32)
    v[7] = np.nan                                  # ignored by max; code 0
    c, s = ora.int8_quantize_768(v)
    want_c, want_s = _quantize_from_definition(v)
    assert c[7] == 0 and np.array_equal(c, want_c) and s == int(want_s)


def test_int8_dot_is_scaled_dot768_of_the_codes():
    r = _rng(6)
    q = r.standard_normal(768).astype(np.float32)
    v = r.standard_normal(768).astype(np.float32)
    codes, s = ora.int8_quantize_768(v)
    scale = np.array([s], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    want = np.float32(np.float32(ora.dot(q, codes.astype(np.float32))) * scale)
    assert ora.dot_int8_768(q, codes, s) == want
    assert ora.rerank_dot(ora.RERANK_INT8, q, v) == want
    # dequantized with the f32 scale max|v|/127: |v - scale*code| <= scale/2
    s32 = float(np.float32(np.abs(v).max() / np.float32(127.0)))
    deq = codes.astype(np.float64) * s32
    assert np.all(np.abs(v - deq) <= s32 * 0.5 * (1 + 1e-5))
    assert abs(float(scale) - s32) <= s32 * 2.0 ** -11  # f16 rounding of the scale


def test_rerank_dot_dispatch():
    r = _rng(7)
    q = r.standard_normal(768).astype(np.float32)
    v = r.standard_normal(768).astype(np.float32)
    assert ora.rerank_dot(ora.RERANK_FP32, q, v) == ora.dot(q, v)
    assert ora.rerank_dot(ora.RERANK_FP16, q, v) == ora.dot_fp16_768(q, v)


@pytest.mark.parametrize("prec", [ora.RERANK_FP32, ora.RERANK_FP16, ora.RERANK_INT8])
def test_rerank_is_a_stable_descending_sort(prec):
    r = _rng(8 + prec)
    rows = r.standard_normal((300, 768)).astype(np.float32)
    rows[10] = rows[20]            # equal rows -> exactly tied scores
    rows[30] = 0.0
    rows[31] = 0.0                 # +0.0 and -0.0 scores compare equal
    q = r.standard_normal(768).astype(np.float32)
    cand = np.array([20, 5, 31, 10, 30, 7, 20] + list(range(40, 120)), dtype=np.uint64)
    got_rows, got_scores = ora.rerank(prec, q, rows, cand)
    scored = [(int(c), ora.rerank_dot(prec, q, rows[int(c)])) for c in cand]
    want = sorted(scored, key=lambda t: -t[1])  # Python's sort is stable
    assert [w[0] for w in want] == list(got_rows)
    assert np.array_equal(np.array([w[1] for w in want], dtype=np.float32), got_scores)


def test_rerank_nan_is_an_error():
    rows = np.ones((4, 768), dtype=np.float32)
    rows[2, 5] = np.nan
    q = np.ones(768, dtype=np.float32)
    assert ora.rerank(ora.RERANK_FP32, q, rows, np.array([0, 2], dtype=np.uint64)) is None
    assert ora.rerank(ora.RERANK_FP16, q, rows, np.array([2], dtype=np.uint64)) is None
    # int8 maps the NaN element to code 0: a finite score
    assert ora.rerank(ora.RERANK_INT8, q, rows, np.array([2], dtype=np.uint64)) is not None


def test_ring_search_exact_sorts_and_truncates():
    r = _rng(20)
    pending = r.standard_normal((40, 768)).astype(np.float32)
    pending[7] = pending[3]                       # tie: index 3 first
    q = r.standard_normal(768).astype(np.float32)
    loc, sc = ora.ring_search_exact(pending, q, 10)
    scored = sorted([(i, ora.dot(pending[i], q)) for i in range(40)], key=lambda t: -t[1])[:10]
    assert loc.tolist() == [i for i, _ in scored]
    assert np.array_equal(sc, np.array([s for _, s in scored], dtype=np.float32))
    loc, sc = ora.ring_search_exact(pending, q, 100)  # top_k above the pending count
    assert loc.size == 40
    pending[5, 0] = np.nan
    assert ora.ring_search_exact(pending, q, 10) is None


def test_shortlist_push_known_answers():
    ids = np.array([1, 2, 3], dtype=np.uint64)
    # full, equal to the minimum: rejected (push replaces only if strictly greater)
    oi, os_ = ora.shortlist_push_sorted(3, ids, [5.0, 4.0, 3.0], [9], [3.0])
    assert oi.tolist() == [1, 2, 3]
    # below capacity: appended whatever the score
    oi, os_ = ora.shortlist_push_sorted(3, ids[:1], [5.0], [9, 10, 11], [1.0, 0.5, 0.2])
    assert oi.tolist() == [1, 9, 10] and os_.tolist() == [5.0, 1.0, 0.5]
    # first minimum in internal order is replaced: [3a, 5, 3b] + 4 -> 3a goes
    oi, os_ = ora.shortlist_push_sorted(3, ids, [3.0, 5.0, 3.0], [9], [4.0])
    assert oi.tolist() == [2, 9, 3]
    # into_sorted is stable: equal scores keep internal order
    oi, _ = ora.shortlist_push_sorted(4, ids, [2.0, 2.0, 2.0], [9], [2.0])
    assert oi.tolist() == [1, 2, 3, 9]


def test_shortlist_push_keeps_the_top_k_of_the_union():
    r = _rng(21)
    for k, n, m in [(16, 16, 40), (16, 5, 8), (64, 64, 64), (8, 0, 20)]:
        s = np.sort(r.standard_normal(n).astype(np.float32))[::-1]
        p = np.sort(r.standard_normal(m).astype(np.float32))[::-1]
        ids = np.arange(n, dtype=np.uint64)
        pids = np.arange(1000, 1000 + m, dtype=np.uint64)
        oi, os_ = ora.shortlist_push_sorted(k, ids, s, pids, p)
        union = np.concatenate([s, p])
        top = np.sort(union)[::-1][:k]
        assert os_.size == min(k, n + m)
        assert np.array_equal(os_, top)
        assert np.all(np.diff(os_) <= 0)
