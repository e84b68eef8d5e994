"""Host side of the pipeline seam: Shortlist (scan.rs:310-399) against the
oracle's restatement, EdenFit / manifest JSON (eden.rs:193-202,
engine.rs:38-44,132-192, config.rs serde forms), and the checks open_index
makes before it touches a device."""
import json
import math

import numpy as np
import pytest

import mrl_index_amd as m
import ora
from mrl_index_amd.jsonf32 import f32_from_text, f32_text


def _hits(ids, scores):
    return [m.ScoredHit(m.VectorId.from_u64(int(i)), float(s)) for i, s in zip(ids, scores)]


@pytest.mark.parametrize("seed", range(6))
def test_shortlist_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    for cap in (1, 2, 3, 7, 16):
        n = int(rng.integers(0, 40))
        # few distinct values: many exact ties, and both zeros
        scores = rng.choice(np.array([-1.0, -0.0, 0.0, 0.5, 0.5, 1.0, 2.0, 3.0], dtype=np.float32), n)
        ids = rng.permutation(1000)[:n].astype(np.uint64)
        sl = m.Shortlist(cap)
        for h in _hits(ids, scores):
            sl.push(h)
        got = sl.into_sorted()
        want_i, want_s = ora.shortlist_push_sorted(cap, [], [], ids, scores)
        assert [h.id.as_u64() for h in got] == [int(i) for i in want_i]
        assert np.array_equal(np.array([h.score for h in got], dtype=np.float32).view(np.uint32),
                              want_s.view(np.uint32))


def test_shortlist_floor_threshold_and_nan():
    sl = m.Shortlist.with_floor(2, 0.5)
    assert sl.threshold() == np.float32(0.5)
    for h in _hits([1, 2, 3, 4], [0.25, 0.75, 0.5, 0.9]):
        sl.push(h)
    assert [h.id.as_u64() for h in sl.into_sorted()] == [4, 2]  # 0.25 under the floor; 0.5 replaced
    assert sl.threshold() == np.float32(0.75)
    full = m.Shortlist(2)
    for h in _hits([1, 2, 3], [1.0, 2.0, 1.0]):  # equal to the minimum: rejected
        full.push(h)
    assert [h.id.as_u64() for h in full.into_sorted()] == [2, 1]
    one = m.Shortlist(4)
    one.push(m.ScoredHit(m.VectorId(0, 1), math.nan))
    assert len(one.into_sorted()) == 1  # no comparison, no panic
    two = m.Shortlist(4)
    for h in _hits([1, 2], [math.nan, 1.0]):
        two.push(h)
    with pytest.raises(ValueError):
        two.into_sorted()
    assert m.Shortlist(0).capacity == 1


def test_f32_json_text_is_exact():
    # decimal -> f32 in one rounding: this text lies just above the midpoint
    # of 1 and the next f32, and decimal -> f64 -> f32 would give 1.0
    assert f32_from_text("1.0000000596046448") == np.nextafter(np.float32(1), np.float32(2))
    assert np.float32(float("1.0000000596046448")) == np.float32(1)
    assert f32_from_text("-0.0").view(np.uint32) == np.float32(-0.0).view(np.uint32)
    assert f32_from_text("1e-46") == 0 and f32_from_text("8e-46") == np.float32(1e-45)
    assert np.isinf(f32_from_text("3.5e38"))
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(3000), rng.standard_normal(300) * 1e-38]).astype(np.float32)
    for x in v:
        assert f32_from_text(f32_text(x)).view(np.uint32) == x.view(np.uint32)


def test_eden_fit_json_round_trip_and_serde_defaults(tmp_path):
    rng = np.random.default_rng(5)
    fit = m.EdenFit(64, 4, 7, rng.standard_normal(64).astype(np.float32) * np.float32(0.05), 1234)
    fit.save_json(tmp_path / "e.json")
    back = m.EdenFit.load_json(tmp_path / "e.json")
    assert (back.dim, back.bits, back.seed, back.n_observed) == (64, 4, 7, 1234)
    assert np.array_equal(back.mean.view(np.uint32), fit.mean.view(np.uint32))
    # as serde_json writes it (no n_observed: #[serde(default)] gives 0)
    text = '{\n  "dim": 4,\n  "bits": 4,\n  "seed": 1,\n  "mean": [\n    0.1,\n    -1.5e-7,\n    0,\n    2.0\n  ]\n}'
    f2 = m.EdenFit.from_json(text)
    assert f2.n_observed == 0
    assert np.array_equal(f2.mean, np.array([0.1, -1.5e-7, 0, 2], dtype=np.float32))
    for bad in ('{"dim": 4, "bits": 4, "seed": 1}', '{"dim": -1, "bits": 4, "seed": 1, "mean": []}',
                '{"dim": 1, "bits": 4, "seed": 1, "mean": [true]}'):
        with pytest.raises(ValueError):
            m.EdenFit.from_json(bad)


def test_manifest_round_trip_defaults_and_errors(tmp_path):
    cfg = m.EngineConfig(embed_dims=768, shortlist_cand=256, stratum4_weight=0.3, cs_tolerance=1.1,
                         strata_depth=m.StrataDepth.L1_RABITQ, mid_codec=m.MidCodec.EDEN_B1, eden_seed=9)
    man = m.IndexManifest("3.5.0", cfg, 1000, 16)
    man.save(tmp_path / "manifest.json")
    d = json.load(open(tmp_path / "manifest.json"))
    assert d["config"]["strata_depth"] == "l1_rabitq" and d["config"]["mid_codec"] == "eden_b1"
    assert d["config"]["prefix_codec"] == "eden_prod" and d["config"]["stratum4_weight"] == 0.3
    assert "exhaustive" not in d["config"]
    back = m.IndexManifest.load(tmp_path / "manifest.json")
    assert back == man
    # serde defaults: use_gemma2, prefix_codec (the enum's default MinMax4), eden_seed, mid_codec
    for k in ("use_gemma2", "prefix_codec", "eden_seed", "mid_codec"):
        del d["config"][k]
    d["config"]["unknown_future_field"] = 1
    json.dump(d, open(tmp_path / "m2.json", "w"))
    c2 = m.IndexManifest.load(tmp_path / "m2.json").config
    assert (c2.use_gemma2, c2.prefix_codec, c2.eden_seed, c2.mid_codec) == (False, m.PrefixCodec.MIN_MAX4, 1,
                                                                             m.MidCodec.RABITQ)
    for mutate in (lambda c: c.pop("shortlist_cand"), lambda c: c.update(strata_depth="Full64b"),
                   lambda c: c.update(numa_sharding=1), lambda c: c.update(embed_dims=-5)):
        e = json.load(open(tmp_path / "manifest.json"))
        mutate(e["config"])
        json.dump(e, open(tmp_path / "bad.json", "w"))
        with pytest.raises(ValueError):
            m.IndexManifest.load(tmp_path / "bad.json")


def test_open_index_checks_before_the_device(tmp_path):
    rows = np.random.default_rng(2).standard_normal((130, 384)).astype(np.float32)
    blocks = m.encode_corpus(rows)  # 3 blocks, 130 live slots
    seg = m.SegmentWriter.create(tmp_path / "segments" / "000001.pax")
    for b in blocks:
        seg.append_block(b)
    seg.close()
    assert m.live_slots(tmp_path / "segments" / "000001.pax") == 130
    m.IndexManifest("3.5.0", m.EngineConfig(), 129, 3).save(tmp_path / "manifest.json")
    with pytest.raises(ValueError, match="segment/passage mismatch"):
        m.open_index(tmp_path)
    m.IndexManifest("3.5.0", m.EngineConfig(shortlist_cand=8), 130, 3).save(tmp_path / "manifest.json")
    with pytest.raises(ValueError, match="shortlist_cand"):
        m.open_index(tmp_path)


def test_open_index_reopen_check_uses_the_passage_store(tmp_path):
    """IndexEngine::open (engine.rs:163-168) compares live slots with
    PassageStore::len(), the 24-byte entries of passages.idx
    (passage.rs:152-202); a size that is not a multiple of 24 is corrupt."""
    rows = np.random.default_rng(3).standard_normal((130, 384)).astype(np.float32)
    seg = m.SegmentWriter.create(tmp_path / "segments" / "000001.pax")
    for b in m.encode_corpus(rows):
        seg.append_block(b)
    seg.close()
    # the manifest alone would pass; the passage store holds 129 entries
    m.IndexManifest("3.5.0", m.EngineConfig(), 130, 3).save(tmp_path / "manifest.json")
    (tmp_path / "passages.idx").write_bytes(b"\0" * (24 * 129))
    assert m.passage_count(tmp_path) == 129
    with pytest.raises(ValueError, match="130 live slots vs 129 passages"):
        m.open_index(tmp_path)
    (tmp_path / "passages.idx").write_bytes(b"\0" * (24 * 130 + 5))
    with pytest.raises(ValueError, match="corrupt passage index"):
        m.open_index(tmp_path)
    (tmp_path / "passages.idx").unlink()
    assert m.passage_count(tmp_path) is None
