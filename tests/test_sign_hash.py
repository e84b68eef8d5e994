"""Pins the ±1 sign hashes rademacher_diag (/root/reference/src/eden.rs:75-88)
and tail_rademacher (/root/reference/src/rotate.rs:53-67) to the reference's
own text: tests/golden/make_sign_hash.py parsed both function bodies into
tests/golden/sign_hash.json (operations + the signs they give).  The oracle,
the host encoder, the GPU encoder and the GPU plan builder each restate the
hash; each is compared with the fixture here, the encoders and the plan
through what they write (a one-hot input exposes one sign)."""
import json
import os
import sys

import numpy as np
import pytest
from scipy.linalg import hadamard

import mrl_index_amd as m
import ora

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_sign_hash as msh  # noqa: E402  (the fixture's interpreter; reads no reference file at import)

FIX = json.load(open(os.path.join(HERE, "golden", "sign_hash.json")))
DIAG = FIX["functions"]["rademacher_diag"]
TAIL = FIX["functions"]["tail_rademacher"]
L = ora.lib
H64 = hadamard(64)
H128 = hadamard(128)


def fixture_diag(seed):
    return np.array([1.0 if c == "+" else -1.0 for c in FIX["values"]["rademacher_diag"][str(seed)]])


def fixture_tail():
    return np.array([[1.0 if c == "+" else -1.0 for c in row] for row in FIX["values"]["tail_rademacher"]])


# ---------------------------------------------------------------- the fixture itself
def test_fixture_operations_give_the_fixture_values():
    for seed in (1, 7):
        got = np.array([msh.evaluate(DIAG, (seed, i)) for i in range(128)])
        assert np.array_equal(got, fixture_diag(seed))
    got = np.array([[msh.evaluate(TAIL, (b, d)) for d in range(64)] for b in range(9)])
    assert np.array_equal(got, fixture_tail())


def test_fixture_parser_refuses_other_statement_shapes():
    ok = ("fn h(seed: u64, i: usize) -> f32 {\n let mut x = seed.wrapping_mul(3).wrapping_add(i as u64);\n"
          " x ^= x >> 5;\n if x & 1 == 0 { 1.0 } else { -1.0 }\n}\n")
    fn = msh.parse_function(ok, "h")
    assert [o["op"] for o in fn["ops"]] == ["load", "mul", "add", "xor_shr"]
    for bad in (ok.replace(">> 5", "<< 5"), ok.replace("wrapping_add", "rotate_left"),
                ok.replace("x & 1 == 0", "x & 1 != 0"), ok.replace(" x ^= x >> 5;\n", " x += 1;\n")):
        with pytest.raises(SystemExit):
            msh.parse_function(bad, "h")


def test_fixture_values_discriminate_plausible_slips():
    """A dropped step, a shift off by one, a flipped sign rule or a swapped
    add/multiply each change many of the fixture's signs, so agreeing with
    the fixture pins the operation sequence."""
    import copy
    ref = fixture_diag(1)

    def run(fn):
        return np.array([msh.evaluate(fn, (1, i)) for i in range(128)])

    muts = []
    for k, op in enumerate(DIAG["ops"]):
        f = copy.deepcopy(DIAG)
        del f["ops"][k]
        muts.append(f)
        if op["op"] == "xor_shr":
            f = copy.deepcopy(DIAG)
            f["ops"][k]["n"] += 1
            muts.append(f)
    f = copy.deepcopy(DIAG)
    f["sign"]["equals"] = 1
    muts.append(f)
    f = copy.deepcopy(DIAG)
    f["ops"][1], f["ops"][2] = f["ops"][2], f["ops"][1]
    muts.append(f)
    for f in muts:
        assert np.sum(run(f) != ref) >= 20


# ---------------------------------------------------------------- oracle
def test_oracle_rademacher_diag_matches_reference_text():
    for seed in (1, 7):
        got = np.array([L.ora_rademacher_diag(seed, i) for i in range(128)])
        assert np.array_equal(got, fixture_diag(seed))
    # beyond the fixture's pairs, through the parsed operations
    for seed in (0, 2, 12345, (1 << 63) + 5, (1 << 64) - 1):
        for i in (0, 1, 63, 64, 127, 1023, 1 << 40):
            assert L.ora_rademacher_diag(seed, i) == msh.evaluate(DIAG, (seed, i))


def test_oracle_tail_rademacher_matches_reference_text():
    got = np.array([[L.ora_tail_rademacher(b, d) for d in range(64)] for b in range(9)])
    assert np.array_equal(got, fixture_tail())
    for b in (9, 100, (1 << 32) + 3):
        for d in (0, 31, 63, 64, 500):
            assert L.ora_tail_rademacher(b, d) == msh.evaluate(TAIL, (b, d))


def test_balance():
    assert abs(fixture_tail().mean()) < 0.15
    assert abs(fixture_diag(1).mean()) < 0.25 and abs(fixture_diag(7).mean()) < 0.25


# ---------------------------------------------------------------- host encoder
def _tail_docs():
    """Row 64b+d is 1 at dim 192+64b+d (768 dims).  The folded tail is then
    s(b,d)·e_d, whose FWHT is s(b,d)·H[:,d]/8: S4 bit k of that slot is set
    iff s(b,d)·H[k][d] >= 0 (quantize.rs:199-213), so bit 0 carries s(b,d)."""
    rows = np.zeros((9 * 64, 768), dtype=np.float32)
    for b in range(9):
        for d in range(64):
            rows[64 * b + d, 192 + 64 * b + d] = 1.0
    return rows


def _prefix_docs(first, n):
    """Row i is 1 at dim first+i: with a zero-mean fit, EDEN rotates e_i to
    s(seed,i)·H[:,i]/√d, so coordinate 0 (level >= half the codebook iff
    positive) carries s(seed,i) (eden.rs:225-269)."""
    rows = np.zeros((n, 768), dtype=np.float32)
    for i in range(n):
        rows[i, first + i] = 1.0
    return rows


def _plane_bits(blocks, off, dim):
    """bit `dim` of the plane at byte `off` for every slot of every block (reference layout)."""
    out = []
    for blk in blocks:
        w = int(blk[off + 8 * dim:off + 8 * dim + 8].view("<u8")[0])
        out.extend((w >> v) & 1 for v in range(64))
    return np.array(out)


def _check_encoder_signs(encode):
    zero_p = m.EdenFit(64, 4, 1, np.zeros(64, np.float32))
    zero_m = m.EdenFit(128, 1, 7, np.zeros(128, np.float32))
    # tail fold: S4 plane @3072, bit 0; every other bit k follows H[k][d]
    blocks = encode(_tail_docs(), None, None)
    for k in (0, 1, 37, 63):
        bits = _plane_bits(blocks, 3072, k).reshape(9, 64)
        want = (fixture_tail() * H64[k][None, :] >= 0).astype(int)
        assert np.array_equal(bits, want), f"S4 bit {k}"
    # EDEN prefix diagonal, seed 1: S0 plane @512 holds level bit 3 (the sign half)
    blocks = encode(_prefix_docs(0, 64), zero_p, None)
    assert np.array_equal(_plane_bits(blocks, 512, 0)[:64], (fixture_diag(1)[:64] > 0).astype(int))
    # EdenB1 mid band diagonal, seed 7: the S1 plane @1024 holds the 1-bit levels
    blocks = encode(_prefix_docs(64, 128), zero_p, zero_m)
    assert np.array_equal(_plane_bits(blocks, 1024, 0)[:128], (fixture_diag(7) > 0).astype(int))


def test_host_encoder_signs_match_reference_text():
    _check_encoder_signs(lambda rows, p, mid: m.encode_corpus(rows, 8, p, mid, n_threads=2))


def test_oracle_encoder_signs_match_reference_text():
    def enc(rows, p, mid):
        pf = ora.Fit(p.mean, p.bits, p.seed, 0) if p else None
        mf = ora.Fit(mid.mean, mid.bits, mid.seed, 0) if mid else None
        n = rows.shape[0]
        return np.stack([ora.encode_block(rows[b:b + 64], 768, np.arange(b, min(b + 64, n)),
                                          np.full(min(64, n - b), 8), pf, mf) for b in range(0, n, 64)])
    _check_encoder_signs(enc)


# ---------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_gpu_encoder_signs_match_reference_text(device):
    def enc(rows, p, mid):
        n = rows.shape[0]
        x = m.DeviceBuffer.from_array(np.ascontiguousarray(rows), device)
        out = m.DeviceBuffer(((n + 63) // 64) * 4096, device)
        m.encode_corpus_device(x.ptr, n, 768, out.ptr, device, 8, p, mid)
        return out.to_array(np.uint8, ((n + 63) // 64, 4096))
    _check_encoder_signs(enc)


@pytest.mark.gpu
def test_gpu_plan_signs_match_reference_text(device):
    """One-hot queries: eden_q_rot = s(1,i)·H[:,i]/8, eden_mid_q_rot =
    s(7,i)·H[:,i]/√128 and tail_fold_q = s(b,d)·H[:,d]/8, exactly."""
    zero_p = m.EdenFit(64, 4, 1, np.zeros(64, np.float32))
    zero_m = m.EdenFit(128, 1, 7, np.zeros(128, np.float32))
    q = np.zeros((64 + 128 + 9 * 64, 768), dtype=np.float32)
    for r in range(q.shape[0]):
        q[r, r] = 1.0
    plan = m.QueryPlan.from_query_codec(q, 768, m.PrefixCodec.EDEN_PROD, m.MidCodec.EDEN_B1, zero_p, zero_m, device)
    got = plan.export()
    s1, s7, st = fixture_diag(1), fixture_diag(7), fixture_tail()
    inv128 = np.float32(1.0) / np.sqrt(np.float32(128.0))
    for i in range(64):
        rot = np.ctypeslib.as_array(got[i].eden_q_rot)
        assert np.array_equal(rot, (s1[i] * H64[:, i] / 8.0).astype(np.float32)), f"prefix dim {i}"
    for i in range(128):
        rot = np.ctypeslib.as_array(got[64 + i].eden_mid_q_rot)
        assert np.array_equal(np.sign(rot), s7[i] * H128[:, i]), f"mid dim {i}"
        assert np.all(np.abs(rot) == inv128), f"mid dim {i}"
    for b in range(9):
        for d in range(64):
            tf = np.ctypeslib.as_array(got[192 + 64 * b + d].tail_fold_q)
            assert np.array_equal(tf, (st[b, d] * H64[:, d] / 8.0).astype(np.float32)), f"tail {b},{d}"
