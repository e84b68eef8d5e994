"""GPU encoder (mrl_encode_corpus_device): byte-identical records to the host
encoder, itself byte-identical to the oracle's encode_block (quantize.rs:36-96);
device-resident index built from them (mrl_index_from_device)."""
import numpy as np
import pytest

import mrl_index_amd as m
from mrl_index_amd import synth
from helpers import normalized

pytestmark = pytest.mark.gpu


def _gpu_encode(rows, device, source=8, eden=None, eden_mid=None):
    n, dims = rows.shape
    n_blocks = (n + 63) // 64
    x = m.DeviceBuffer.from_array(np.ascontiguousarray(rows, dtype=np.float32), device)
    out = m.DeviceBuffer(n_blocks * 4096, device)
    m.encode_corpus_device(x.ptr, n, dims, out.ptr, device, source, eden, eden_mid)
    return out.to_array(np.uint8, (n_blocks, 4096)), out, x


def _fits(rows, kind):
    if kind == "minmax":
        return None, None
    fit = m.EdenFit.fit_prefix(rows, 4, 1)
    if kind == "eden":
        return fit, None
    mid = m.EdenFit.fit_band(rows, 64, 128, 1, 7)
    return fit, mid


@pytest.mark.parametrize("dims", [192, 200, 384, 768, 1000])
@pytest.mark.parametrize("kind", ["minmax", "eden", "eden_dual"])
def test_gpu_encoder_is_byte_identical_to_host(device, dims, kind):
    rng = np.random.default_rng(dims)
    rows = normalized(rng, 200, dims)
    eden, mid = _fits(rows, kind)
    gpu, _, _ = _gpu_encode(rows, device, 8, eden, mid)
    host = m.encode_corpus(rows, 8, eden, mid)
    assert gpu.shape == host.shape
    bad = np.nonzero((gpu != host).any(axis=1))[0]
    assert bad.size == 0, f"{kind} dims={dims}: blocks {bad[:8]} differ"


@pytest.mark.parametrize("n", [1, 63, 64, 65, 129])
def test_gpu_encoder_partial_blocks(device, n):
    rng = np.random.default_rng(n)
    rows = normalized(rng, n, 384)
    eden, _ = _fits(rows, "eden")
    gpu, _, _ = _gpu_encode(rows, device, 3, eden)
    assert np.array_equal(gpu, m.encode_corpus(rows, 3, eden))


def test_gpu_encoder_special_values(device):
    """Zero rows, huge and tiny magnitudes, NaN and infinity: same bytes as the host."""
    rng = np.random.default_rng(11)
    rows = normalized(rng, 128, 768)
    rows[1] = 0.0
    rows[2] *= np.float32(3e4)
    rows[3] *= np.float32(1e-30)
    rows[4, 5] = np.nan
    rows[5, 300] = np.inf
    rows[6, 70] = -np.inf
    rows[7, :64] = np.float32(0.25)
    for kind in ("minmax", "eden", "eden_dual"):
        eden, mid = _fits(rows[8:], kind)
        gpu, _, _ = _gpu_encode(rows, device, 1, eden, mid)
        assert np.array_equal(gpu, m.encode_corpus(rows, 1, eden, mid)), kind


def test_index_from_device_matches_upload(device):
    rng = np.random.default_rng(5)
    rows = normalized(rng, 64 * 20 + 7, 768)
    eden, _ = _fits(rows, "eden")
    gpu, out, _ = _gpu_encode(rows, device, 8, eden)
    ix = m.DeviceIndex.from_device(out.ptr, gpu.shape[0], device)
    assert np.array_equal(ix.download(), gpu)
    host_ix = m.DeviceIndex.upload(gpu, device, verify_crc=True)  # the GPU-written CRCs verify
    q = rows[[3, 900]] + np.float32(0.01)
    plan = m.QueryPlan.from_query_eden(q, 768, eden, device)
    cfg = m.EngineConfig(embed_dims=768, shortlist_cand=64)
    a, b = m.scan_batch(ix, plan, cfg), m.scan_batch(host_ix, plan, cfg)
    assert np.array_equal(a.ids, b.ids) and np.array_equal(a.scores.view(np.uint32), b.scores.view(np.uint32))


def test_gpu_encoder_benchmark_corpus_slice(device):
    """65,536 rows of the 1M x 768 benchmark corpus: same bytes as the host encoder."""
    w = synth.CONFIGS[2]
    fit = synth.eden_fit(w)
    rows = synth.docs(w, 0, 65536)
    gpu, _, _ = _gpu_encode(rows, device, 0, fit)
    assert np.array_equal(gpu, m.encode_corpus(rows, 0, fit))
