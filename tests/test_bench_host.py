"""bench.py's host-side arithmetic, without a GPU: the refusal of runs on
more than one GPU, the committed traffic figures it quotes, and the
roofline of each path worked out by hand from recorded launch times."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from mrl_index_amd import synth  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("kernel,workload", [("k_scan_mma", "8.8m-768-clustered-b64"), ("k_scan", "1m-768-b1")])
def test_committed_traffic_is_the_profile_figure(kernel, workload):
    path = os.path.join(ROOT, "profiles", f"{kernel}_traffic.txt")
    want = None
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == workload:
            want = float(f[2])
    t = bench.committed_traffic(kernel, workload)
    assert want is not None and t["bytes_per_launch"] == want
    assert t["source"] == f"profiles/{kernel}_traffic.txt"
    # the traffic is the launch's HBM bytes: at least the algorithmic bytes of a standard-layout pass
    # (config 4: 137,500 blocks of 4096 B; config 2's final pass fetches less, only the S1 / S4
    # lines of blocks with survivors)
    assert want > (0.5 * 4096 * 15625 if kernel == "k_scan" else 4096 * 137500)
    assert bench.committed_traffic(kernel, "no-such-workload") is None


def test_mfma_roofline_by_hand():
    """Config 4: every block for each of 64 queries, one S4-bounded launch
    and one with the full tiles per step, 0.25 / 0.30 ms."""
    w = synth.CONFIGS[4]
    n_blocks = 137500
    groups = {
        ("plan+mma_prep", 0): {"ms": [0.011, 0.011], "blocks": [0, 0], "flags": [0, 0]},
        ("scan", 0): {"ms": [0.012, 0.012], "blocks": [538, 538], "flags": [0, 0]},
        ("scan", 1): {"ms": [0.25, 0.30], "blocks": [n_blocks, n_blocks], "flags": [bench.KT_S4_BOUNDED, 0]},
        ("scan", -1): {"ms": [0.004, 0.004], "blocks": [n_blocks, n_blocks], "flags": [0, 0]},
    }
    r = bench.roofline_of(groups, 64, 2, w)
    pairs = 64.0 * n_blocks * 64
    macs = 0.5 * (64 + 5 + 3 + 8) + 0.5 * (64 + 128 + 64 + 5)
    flops = 2.0 * macs * pairs
    # MFMA floor 2 x 170.5 x 563.2M / 2.5 PFLOP/s = 76.8 us against the HBM floor 563.2 MB / 8 TB/s = 70.4 us
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2500.0
    assert r["kernel_avg_ms"] == pytest.approx(0.275)
    assert r["algorithmic_flops_per_launch"] == pytest.approx(flops)
    assert r["achieved"] == pytest.approx(flops / 0.275e-3 / 1e12, rel=1e-4)
    assert r["frac"] == pytest.approx(r["achieved"] / 2500.0, abs=1e-4)
    assert r["mfma_frac"] == r["frac"]
    assert r["launches_per_step"] == 1.0
    # the same launch's HBM figure: 4096 B per block, each block read once for the whole batch
    assert r["hbm_achieved_gb_s"] == pytest.approx(4096.0 * n_blocks / 0.275e-3 / 1e9, rel=1e-4)
    # every launch bounded: 80 MACs per pair, the bytes bind (MFMA floor 36.0 us < HBM floor 70.4 us)
    gb = dict(groups)
    gb[("scan", 1)] = {"ms": [0.2, 0.2], "blocks": [n_blocks, n_blocks], "flags": [bench.KT_S4_BOUNDED] * 2}
    rb = bench.roofline_of(gb, 64, 2, w)
    assert rb["bound"] == "hbm" and rb["unit"] == "GB/s" and rb["peak"] == 8000.0 and rb["macs_per_pair"] == 80
    assert rb["achieved"] == pytest.approx(4096.0 * n_blocks / 0.2e-3 / 1e9, rel=1e-4)
    assert rb["frac"] == rb["hbm_frac"]
    assert rb["mfma_achieved_tflops"] == pytest.approx(2.0 * 80 * pairs / 0.2e-3 / 1e12, rel=1e-4)
    assert r["traffic"] == bench.committed_traffic("k_scan_mma", w.name)["bytes_per_launch"]
    # cold-cache runs quote no traffic; block-listed passes count the pairs they scanned
    assert bench.roofline_of(groups, 64, 2, w, cold=True)["traffic"] is None
    rl = bench.roofline_of(groups, 64, 2, w, scanned=11000 * 64)
    assert rl["algorithmic_flops_per_launch"] == pytest.approx(2.0 * macs * 64.0 * 11000 * 64)
    assert rl["traffic"] is None


def test_one_query_roofline_by_hand():
    """Config 2 over two steps: the final passes (every block) count; the
    sampling pass that builds the plan is its own instantiation ("plan+scan")
    and the safe-floor re-run (pass -1) ends at once, so neither does."""
    w = synth.CONFIGS[2]
    groups = {
        ("plan+scan", 0): {"ms": [0.012, 0.013], "blocks": [245, 245], "flags": [0, 0]},
        ("scan", 1): {"ms": [0.018, 0.020], "blocks": [15625, 15625], "flags": [0, 0]},
        ("scan", -1): {"ms": [0.004, 0.004], "blocks": [15625, 15625], "flags": [0, 0]},
        ("select", 1): {"ms": [0.009, 0.009], "blocks": [0, 0], "flags": [0, 0]},
    }
    r = bench.roofline_of(groups, 1, 2, w)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["kernel_avg_ms"] == pytest.approx(0.019)
    assert r["algorithmic_bytes_per_launch"] == 4096.0 * 15625
    assert r["achieved"] == pytest.approx(4096.0 * 15625 / 0.019e-3 / 1e9, rel=1e-4)
    assert r["frac"] == pytest.approx(r["achieved"] / 8000.0, abs=1e-4)
    assert r["final_pass"]["avg_ms"] == pytest.approx(0.019)
    assert r["launches_per_step"] == 1.0
    assert r["traffic"] == bench.committed_traffic("k_scan", w.name)["bytes_per_launch"]
