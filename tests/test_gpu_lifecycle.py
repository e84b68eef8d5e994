"""Handle lifetimes through the C ABI: objects made on a context keep it
alive, so the context and its objects may be destroyed in any order
(include/mrl_scan.h), and a process that exits with handles still open exits
normally."""
import itertools
import os
import subprocess
import sys

import numpy as np
import pytest

import mrl_index_amd as m
import ora
from helpers import assert_topk_equal, normalized, oracle_encode_corpus

pytestmark = pytest.mark.gpu
L = m._lib.lib
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def small():
    rng = np.random.default_rng(77)
    rows = normalized(rng, 64 * 20 - 3, 256)
    blocks = oracle_encode_corpus(rows, 256)
    q = rows[:3] + np.float32(0.01)
    refs = []
    for i in range(3):
        op = ora.plan_build(q[i], 256, ora.PREFIX_MINMAX4, ora.MID_RABITQ)
        refs.append(ora.scan_blocks(blocks, op, ora.scan_config(32, sharding=False)))
    return blocks, q, refs


def _scan_on_new_ctx(blocks, q):
    dev = m.Device(0)
    ix = m.DeviceIndex.upload(blocks, dev)
    plan = m.QueryPlan.from_query(q, 256, dev)
    res = m.DeviceResults(q.shape[0], 32, dev)
    res.scan(ix, plan, m.ScanConfig(shortlist_cand=32))
    out = res.fetch()
    store = m.RerankStore.create(np.zeros((4, 256), np.float32), device=dev)
    return dev, {"index": ix, "plans": plan, "results": res, "store": store}, out


@pytest.mark.parametrize("order", list(itertools.permutations(["ctx", "index", "plans", "results", "store"]))[::13])
def test_destroy_in_any_order(device, small, order):
    blocks, q, refs = small
    dev, objs, out = _scan_on_new_ctx(blocks, q)
    for i in range(3):
        c = int(out.counts[i])
        assert_topk_equal(out.ids[i, :c], out.scores[i, :c], refs[i][0], refs[i][1], 32, f"q{i}")
    for name in order:
        (dev if name == "ctx" else objs[name]).close()
    # the runtime is healthy afterwards: a fresh context scans again
    dev2, objs2, out2 = _scan_on_new_ctx(blocks, q)
    assert np.array_equal(out2.ids, out.ids) and np.array_equal(out2.scores.view(np.uint32), out.scores.view(np.uint32))
    for o in objs2.values():
        o.close()
    dev2.close()


def test_context_destroyed_first_leaves_objects_usable_for_destroy(device, small):
    """The raw C sequence a Rust Drop order can produce: the context handle
    dropped while its index, plans and results are alive."""
    import ctypes as C
    blocks, q, _ = small
    ctx = C.c_void_p()
    m._lib.check(L.mrl_ctx_create(0, C.byref(ctx)))
    ix = C.c_void_p()
    b = np.ascontiguousarray(blocks)
    m._lib.check(L.mrl_index_upload(ctx, m._lib.vptr(b), b.shape[0], 0, C.byref(ix)))
    res = C.c_void_p()
    m._lib.check(L.mrl_results_create(ctx, 3, 32, C.byref(res)))
    L.mrl_ctx_destroy(ctx)
    L.mrl_results_destroy(res)
    L.mrl_index_destroy(ix)


def test_process_exit_with_open_handles(device, small):
    """A script that never closes its context, index, plans or results (one
    of them a raw handle Python never frees) exits with status 0."""
    script = (
        "import sys, ctypes as C, numpy as np\n"
        f"sys.path.insert(0, {os.path.join(ROOT, 'mrl-index-rust-vector_amd')!r})\n"
        "import mrl_index_amd as m\n"
        "rng = np.random.default_rng(3)\n"
        "rows = rng.standard_normal((64 * 40, 256)).astype(np.float32)\n"
        "rows /= np.linalg.norm(rows, axis=1, keepdims=True)\n"
        "blocks = m.encode_corpus(rows, 8)\n"
        "dev = m.Device(0)\n"
        "ix = m.DeviceIndex.upload(blocks, dev)\n"
        "plan = m.QueryPlan.from_query(rows[:9], 256, dev)\n"
        "raw = C.c_void_p()\n"
        "m._lib.check(m._lib.lib.mrl_results_create(dev.handle, 9, 16, C.byref(raw)))\n"
        "cfg = m.ScanConfig(shortlist_cand=16).to_c()\n"
        "tr = m._lib.TimeRangeC(0, 0, 0, 0)\n"
        "for _ in range(3):\n"
        "    m._lib.check(m._lib.lib.mrl_scan_async(dev.handle, ix.handle, plan.handle, C.byref(cfg), C.byref(tr), raw))\n"
        "dev.synchronize()\n"
        "print('done', flush=True)\n")
    p = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=110)
    assert p.returncode == 0, p.stderr[-2000:]
    assert "done" in p.stdout and "terminate" not in p.stderr
