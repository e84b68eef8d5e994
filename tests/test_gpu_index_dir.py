"""An index directory through the scan path (engine.rs:132-192,
pipeline.rs:104-133): manifest.json's config and eden_prefix.json pick the
codec and fit; segments/000001.pax streams into HBM in pinned chunks of 4096
blocks; QueryPipeline.scan_segments_into pushes into a caller-owned
Shortlist.  The top K is checked against the oracle."""
import os
import shutil

import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import synth
import ora
from helpers import assert_topk_equal

pytestmark = pytest.mark.gpu

N_BLOCKS = 4500  # two staging chunks, the second partial


@pytest.fixture(scope="module")
def index_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("idx")
    w = synth.CONFIGS[2].scaled(64 * N_BLOCKS - 17, 3)  # a partial last block
    fit = synth.eden_fit(w)
    blocks = synth.encode(w, fit, 16)
    seg = m.SegmentWriter.create(d / "segments" / "000001.pax")
    seg.append_block(blocks)
    seg.close()
    cfg = m.EngineConfig(embed_dims=768, shortlist_cand=64, eden_seed=1)
    m.IndexManifest("3.5.0", cfg, w.n_docs, N_BLOCKS).save(d / "manifest.json")
    fit.save_json(d / "eden_prefix.json")
    return d, w, fit, blocks


def test_open_index_streams_the_segment_and_scans(device, index_dir):
    d, w, fit, blocks = index_dir
    print(f"[index_dir] {N_BLOCKS} blocks", flush=True)
    pipe, ix, man = m.open_index(d, device, verify_crc=True)
    assert ix.block_count() == N_BLOCKS and man.blocks_written == N_BLOCKS
    assert np.array_equal(ix.download(), blocks)
    assert np.array_equal(pipe.eden.mean.view(np.uint32), fit.mean.view(np.uint32))
    qs, _ = synth.queries(w)
    k = pipe.cfg.shortlist_cand
    ofit = ora.Fit(fit.mean, 4, 1, fit.n_observed)
    for qi in range(qs.shape[0]):
        plan = pipe.build_plan(qs[qi])
        sl = m.Shortlist(k)
        assert pipe.scan_segments_into(plan, ix, sl) == N_BLOCKS
        hits = sl.into_sorted()
        ids = np.array([h.id.as_u64() for h in hits], dtype=np.uint64)
        sc = np.array([h.score for h in hits], dtype=np.float32)
        op = ora.plan_build(qs[qi], 768, ora.PREFIX_EDEN_PROD, 0, ofit, None)
        rids, rsc = ora.scan_blocks(blocks, op, ora.scan_config(k, sharding=True, threads=16))
        assert_topk_equal(ids, sc, rids, rsc, k, f"index dir q={qi}")
    # a shortlist that already holds hits keeps the best of both (the ring merge's use)
    plan = pipe.build_plan(qs[0])
    top = m.scan_blocks(ix, plan, pipe.cfg)
    sl = m.Shortlist(k)
    extra = m.ScoredHit(m.VectorId(0xFFFFFFFF, 0), float(top[0].score) + 1.0)
    sl.push(extra)
    pipe.scan_segments_into(plan, ix, sl)
    out = sl.into_sorted()
    assert out[0] == extra and [h.id for h in out[1:]] == [h.id for h in top[:k - 1]]


def test_open_index_without_a_fit_file_and_crc_in_a_later_chunk(device, index_dir, tmp_path):
    d, w, fit, blocks = index_dir
    d2 = tmp_path / "copy"
    shutil.copytree(d, d2)
    os.remove(d2 / "eden_prefix.json")
    pipe, ix, _ = m.open_index(d2, device)  # EdenFit::default_prefix(eden_seed)
    assert pipe.eden.n_observed == 0 and not pipe.eden.mean.any() and pipe.eden.seed == 1
    ix.close()
    bad = blocks.copy()
    bad[4321, 3000] ^= 0x10
    with open(d2 / "segments" / "000001.pax", "wb") as f:
        f.write(bad.tobytes())
    with pytest.raises(m.MrlError) as e:
        m.open_index(d2, device, verify_crc=True)
    assert e.value.code == 6 and "4321" in str(e.value)
    ok, _, _ = m.open_index(d2, device, verify_crc=False)  # unchecked, it loads
    assert ok.cfg.shortlist_cand == 64
