"""Shared helpers for the parity tests."""
import numpy as np

import ora


def normalized(rng, n, dims, offset=0.05, head_heavy=True):
    x = rng.standard_normal((n, dims)).astype(np.float32)
    if head_heavy:
        x *= (1.0 / np.sqrt(np.arange(1, dims + 1, dtype=np.float32)))[None, :]
    x += np.float32(offset)
    x /= np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)
    return x.astype(np.float32)


def oracle_fit(rows, seed=1):
    m = np.zeros(64, dtype=np.float32)
    r = np.ascontiguousarray(rows, dtype=np.float32)
    rc = ora.lib.ora_eden_fit_band(ora.fp(r), r.shape[0], r.shape[1], 0, 64, ora.fp(m))
    assert rc == 0
    return ora.Fit(m, 4, seed, r.shape[0])


def oracle_fit_mid(rows, seed=7):
    m = np.zeros(128, dtype=np.float32)
    r = np.ascontiguousarray(rows, dtype=np.float32)
    rc = ora.lib.ora_eden_fit_band(ora.fp(r), r.shape[0], r.shape[1], 64, 128, ora.fp(m))
    assert rc == 0
    return ora.Fit(m, 1, seed, r.shape[0])


def oracle_encode_corpus(rows, dims, eden=None, eden_mid=None):
    n = rows.shape[0]
    blocks = []
    for b in range(0, n, 64):
        chunk = rows[b:b + 64]
        blocks.append(ora.encode_block(chunk, dims, np.arange(b, b + chunk.shape[0]), np.full(chunk.shape[0], 8),
                                       eden, eden_mid))
    return np.stack(blocks)


def assert_topk_equal(got_ids, got_scores, ref_ids, ref_scores, k, what=""):
    """Same top-K set except for exact ties at the K-th score; scores bit-exact."""
    got_ids = np.asarray(got_ids, dtype=np.uint64)
    ref_ids = np.asarray(ref_ids, dtype=np.uint64)
    gs = np.asarray(got_scores, dtype=np.float32)
    rs = np.asarray(ref_scores, dtype=np.float32)
    assert len(got_ids) == len(ref_ids), f"{what}: count {len(got_ids)} != {len(ref_ids)}"
    if len(ref_ids) == 0:
        return
    # sorted score multisets identical bit for bit
    g_sorted = np.sort(gs)[::-1]
    r_sorted = np.sort(rs)[::-1]
    assert np.array_equal(g_sorted.view(np.uint32), r_sorted.view(np.uint32)), f"{what}: score multiset differs"
    kth = r_sorted[-1] if len(ref_ids) >= k else -np.inf
    g_strict = set(got_ids[gs > kth].tolist())
    r_strict = set(ref_ids[rs > kth].tolist())
    assert g_strict == r_strict, f"{what}: ids above the K-th score differ"
    # every reported (id, score) pair agrees where both report the id
    rmap = dict(zip(ref_ids.tolist(), rs.view(np.uint32).tolist()))
    for i, s in zip(got_ids.tolist(), gs.view(np.uint32).tolist()):
        if i in rmap:
            assert rmap[i] == s, f"{what}: score of id {i} differs"
