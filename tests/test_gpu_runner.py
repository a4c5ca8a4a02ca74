"""FlatRunner on the GPU (h3/htrc_flat_runner.py:85-203): the captured HIP graph replays
equal eager launches on every replay (with eager work and syncs in between), head-batched
replays equal per-head calls, sink mode hands over the static output, and a capture
failure degrades to eager with ``graph_error`` recorded.
"""
from __future__ import annotations

import gc
import weakref

import pytest
import torch

from htrc_amd import htrc_flat, htrc_flat_runner, workloads

pytestmark = pytest.mark.gpu

KW = dict(leaf=64, exact_leaves=8)


def _jobs(device, heads=3, n=2048, seed=0):
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=heads, seed=seed)
    return [(h, q[h].float().to(device), k[h].to(device), v[h].to(device)) for h in range(heads)]


def test_graph_replays_equal_eager(device):
    jobs = _jobs(device)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", **KW)
    assert r.graph is not None, r.graph_error
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], **r.cfg) for j in jobs]
    for rep in range(3):
        outs = r.run(jobs)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"
        _ = torch.randn(1 << 20, device=device).sum().item()      # eager work between replays


@pytest.mark.parametrize("store", ["fp8", "bf16"])
def test_16bit_store_graph_replays_equal_eager(device, store):
    """The runner with a 16-bit state store (its stats and route16 launches inside the graph):
    every replay equals the eager call bit for bit."""
    jobs = _jobs(device, heads=2, seed=3)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", store=store, **KW)
    assert r.graph is not None, r.graph_error
    assert r.cfg["store"] == store
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], **r.cfg) for j in jobs]
    for rep in range(3):
        outs = r.run(jobs)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"
        _ = torch.randn(1 << 20, device=device).sum().item()      # eager work between replays


def test_head_batched_runner_matches_per_head(device):
    jobs = _jobs(device, heads=5, seed=1)
    single = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", use_graph=False, **KW)
    batched = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", heads=2, **KW)
    assert batched.graph is not None, batched.graph_error
    a = single.run(jobs)
    b = batched.run(jobs)                      # 2 + 2 + 1 (padded) heads per replay
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    got = {}
    batched.run(jobs, sink=lambda i, o: got.__setitem__(i, o.clone()))
    for i, x in enumerate(a):
        assert torch.equal(got[i], x)


def test_capture_runs_with_the_collector_off_and_runners_free_by_refcount(device, monkeypatch):
    """The recording runs with Python's garbage collector off (a collection inside it could
    destroy another dead runner's graph and pool, which is illegal during a capture), the
    collector is back on afterwards, and a runner with its graph is freed as soon as its last
    reference goes (no runner <-> replay cycle left for the collector)."""
    seen = []
    orig = torch.cuda.graph

    class Spy(orig):
        def __enter__(self):
            seen.append(gc.isenabled())
            return super().__enter__()

    monkeypatch.setattr(torch.cuda, "graph", Spy)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", **KW)
    monkeypatch.setattr(torch.cuda, "graph", orig)
    assert r.graph is not None, r.graph_error
    assert seen == [False] and gc.isenabled()
    gc.disable()
    try:
        ref = weakref.ref(r)
        del r
        assert ref() is None
    finally:
        gc.enable()


def test_capture_failure_falls_back_to_eager(device, monkeypatch):
    orig = torch.cuda.graph

    def broken(*a, **k):
        raise RuntimeError("capture refused for the test")

    monkeypatch.setattr(torch.cuda, "graph", broken)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", **KW)
    monkeypatch.setattr(torch.cuda, "graph", orig)
    assert r.graph is None and "capture refused" in r.graph_error
    jobs = _jobs(device, heads=1)
    out = r.run(jobs)[0]
    ref = htrc_flat.flat_attention(jobs[0][1], jobs[0][2], jobs[0][3], **r.cfg)
    assert torch.equal(out, ref)


def test_tail_rows_graph_equals_eager(device):
    """tail_rows: the captured graph reads the tail from static buffers, refreshed per call
    (h3/htrc_flat_runner.py:136-139, 162-165)."""
    jobs = _jobs(device, heads=3, seed=4)
    g = torch.Generator().manual_seed(4)
    tails = [(torch.randn((7, 128), generator=g).to(device), torch.randn((7, 128), generator=g).to(device))
             for _ in jobs]
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", tail_rows=7, **KW)
    assert r.graph is not None, r.graph_error
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], tail=t, **r.cfg) for j, t in zip(jobs, tails)]
    outs = r.run([(*j, t) for j, t in zip(jobs, tails)])
    torch.cuda.synchronize()
    for o, e in zip(outs, eager):
        assert torch.equal(o, e)
    with pytest.raises(ValueError, match="tail"):
        r.head(jobs[0][1], jobs[0][2], jobs[0][3])
    batched = htrc_flat_runner.FlatRunner(2048, 2048, mode="fast", tail_rows=7, heads=2, **KW)
    assert batched.graph is not None, batched.graph_error
    got = batched.run([(*j, t) for j, t in zip(jobs, tails)])
    torch.cuda.synchronize()
    for o, e in zip(got, eager):
        assert torch.equal(o, e)


def test_accurate_mode_graph_replays_equal_eager(device):
    """mode="accurate" (k-means query order, h3/htrc_flat_runner.py:51): the k-means launches
    are captured with the rest; every replay equals the eager operator call."""
    jobs = _jobs(device, heads=2, seed=4)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="accurate", **KW)
    assert r.cfg["order"] == "kmeans"
    assert r.graph is not None, r.graph_error
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], **r.cfg) for j in jobs]
    for rep in range(3):
        outs = r.run(jobs)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"
        _ = torch.randn(1 << 20, device=device).sum().item()


def test_max_mode_graph_replays_equal_eager(device):
    """mode="max" (32-row tiles with k-means order, h3/htrc_flat_runner.py:52): every replay of
    the captured graph equals the eager operator call, and the tiles are 32 rows."""
    jobs = _jobs(device, heads=2, seed=6)
    r = htrc_flat_runner.FlatRunner(2048, 2048, mode="max", **KW)
    assert r.cfg["tile"] == 32 and r.cfg["order"] == "kmeans"
    assert r.graph is not None, r.graph_error
    st = {}
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], **r.cfg) for j in jobs]
    htrc_flat.flat_attention(jobs[0][1], jobs[0][2], jobs[0][3], state=st, **r.cfg)
    assert st["idx"].shape[1] == 2048 // 32
    for rep in range(3):
        outs = r.run(jobs)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"
        _ = torch.randn(1 << 20, device=device).sum().item()
