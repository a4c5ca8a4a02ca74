"""Tile windows (tile_chunk), sink leaves, long near lists, many leaves and the attend kernel's
reference-max retry on the GPU, against the CPU oracle.

* tile_chunk (h3/htrc_flat.py:236-273): every windowing of a layer gives the one-window result
  bit for bit (tiles are independent; every launch choice depends on the layer's shape).
* sink_leaves (h3/htrc_flat.py:232-233, 262-263): leaves < sink are always near, on the fused
  route and on the stage path, with and without shared centres.
* The reference runner's live H3 shape in mode "accurate" (h3/htrc_flat_runner.py:51;
  tools/sweep_h3_flat_kernels.py:6-8): 40759 queries, 2547 leaves of 16 keys, 220 forced sink
  leaves + 1024 exact leaves = 1244 near leaves per tile, k-means order, 7 tail keys.
* 20000 leaves per head: route_select keeps its top-k keys in global memory, the stage top-k
  reads rows from global memory.
* A query row aligned with a near-field outlier key scores 80 or 362 nats above its far-field
  maximum (or, under a sampled tile reference, every other row scores ~300 nats below it), so the
  fixed softmax reference misses by more than 60 octaves and the tile is redone at every row's
  exact largest score.

Routing is compared with the oracle through the measured SEL error (helpers.routing_report):
a tile's near set may differ only where the oracle's top-k boundary gap is at most twice the
largest |SEL_gpu - SEL_oracle| of that tile.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import bits, rel_l2, routing_report, sel_error
from htrc_amd import htrc_flat, htrc_flat_hip as hip, htrc_flat_runner, workloads
from oracle import flat_i8

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-2
LOGZ_ABS = 1e-3
KW = dict(backend="hip", store="int8", dot="bf16", splits=4, kern={"tile_bn": 64})


def _kw(**over):
    kw = {**KW, **over}
    kw["kern"] = {**KW["kern"], **over.get("kern", {})}
    return kw


def _gpu_sel(st, nb, group, tile, stride=1):
    """SEL from the GPU's own state (the route select computes exactly this, bit for bit)."""
    sel = hip.rowmax_select(g=st["g8"], lz=st["lz"], sg=st.get("sg"), stride=stride, nb=nb,
                            dq8=st.get("dq8", st.get("dq16")), sdq=st.get("sdq"), group=group, tile=tile)
    return sel.cpu().numpy()


def _check_routing(idx_gpu, ref, sel_gpu, nb, sink):
    """routing_report on the leaves past the sinks (the sinks are forced on both sides)."""
    idx_gpu = np.asarray(idx_gpu)
    assert np.array_equal(idx_gpu[:, :sink], np.broadcast_to(np.arange(sink), (idx_gpu.shape[0], sink)))
    osel = ref["sel"][:, sink:nb]
    delta = sel_error(sel_gpu[:, sink:nb], osel, nb - sink)
    return routing_report(idx_gpu[:, sink:] - sink, ref["idx"][:, sink:] - sink, osel, delta)


@pytest.mark.parametrize("fused,group,tile,order,store", [
    (True, 1, 64, "seq", "int8"), (False, 1, 64, "seq", "int8"), (True, 3, 64, "seq", "int8"),
    (False, 2, 32, "seq", "int8"), (True, 1, 32, "kmeans", "int8"), (True, 2, 64, "kmeans", "int8"),
    (True, 2, 64, "seq", "fp8"), (False, 1, 64, "seq", "fp8"), (True, 1, 32, "kmeans", "bf16")])
def test_windows_bit_identical(device, fused, group, tile, order, store):
    n, leaf, ex = 4096, 64, 8
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=2, seed=5 + group + tile)
    q, k, v = q.to(device), k.to(device), v.to(device)
    kw = _kw(leaf=leaf, exact_leaves=ex, tile=tile, order=order, sink_leaves=2, store=store,
             kern={"fused": fused, "group": group})
    st1 = {}
    one, lz1 = htrc_flat.flat_attention(q, k, v, tile_chunk=4096, return_logz=True, state=st1, **kw)
    assert len(st1["windows"]) == 1
    for chunk in (16, 48, 0):
        st = {}
        out, lz = htrc_flat.flat_attention(q, k, v, tile_chunk=chunk, return_logz=True, state=st, **kw)
        torch.cuda.synchronize()
        assert len(st["windows"]) == (1 if chunk == 0 else -(-st1["idx"].shape[1] // max(1, chunk // group)))
        assert torch.equal(out, one) and torch.equal(lz, lz1), f"tile_chunk {chunk}"
        assert torch.equal(st["idx"], st1["idx"])
        assert torch.equal(st["lz"], st1["lz"]) and torch.equal(st["g8"], st1["g8"])
    for nst in (1, 2, 3):            # no state: the windows dealt over nst streams
        out, lz = htrc_flat.flat_attention(q, k, v, tile_chunk=16, return_logz=True,
                                           **{**kw, "kern": {**kw["kern"], "window_streams": nst}})
        torch.cuda.synchronize()
        assert torch.equal(out, one) and torch.equal(lz, lz1), f"{nst} window streams"


@pytest.mark.parametrize("fused,group,store", [(True, 1, "int8"), (False, 1, "int8"), (True, 2, "int8"),
                                              (False, 3, "int8"), (True, 2, "fp8"), (True, 1, "bf16")])
def test_sink_leaves_vs_oracle(device, fused, group, store):
    n, leaf, ex, sink = 4096, 32, 8, 5
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=1, seed=77 + group)
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), leaf=leaf,
                                         exact_leaves=ex, sink_leaves=sink, return_logz=True, state=st,
                                         **_kw(store=store, kern={"fused": fused, "group": group}))
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex, sink_leaves=sink,
                          splits=1 if fused else 4, bn=64, group=group, store=store)
    nb = n // leaf
    assert st["kx"] == ex + sink
    rep = _check_routing(st["idx"][0].cpu().numpy(), ref, _gpu_sel(st, nb, group, 64)[0], nb, sink)
    assert rep["mismatched"] <= rep["tieable"]
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


def test_live_h3_shape_accurate_mode(device):
    """FlatRunner(mode="accurate", sink_leaves=220, leaf=16, tail_rows=7) at the live H3 shape:
    graph replays equal the eager call, and whole tiles match the oracle run on the same rows
    (the GPU's k-means order, bit-exact against the oracle elsewhere) with the head's full key
    set, the sinks and the tail."""
    n, keys, tail_rows, sink = 40759, 40752, 7, 220
    q, k, v, tk, tv = workloads.h3_live(n=n, keys=keys, tail=tail_rows, heads=2, seed=3)
    jobs = [(h, q[h].float().to(device), k[h].to(device), v[h].to(device), (tk[h].to(device), tv[h].to(device)))
            for h in range(2)]
    r = htrc_flat_runner.FlatRunner(n, keys, mode="accurate", sink_leaves=sink, tail_rows=tail_rows, leaf=16)
    assert r.graph is not None, r.graph_error
    assert r.cfg["exact_leaves"] == 1024 and r.cfg["order"] == "kmeans"
    eager = [htrc_flat.flat_attention(j[1], j[2], j[3], tail=j[4], **r.cfg) for j in jobs]
    for rep in range(2):
        outs = r.run(jobs)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"
    h = 1
    st = {}
    out, logz = htrc_flat.flat_attention(jobs[h][1], jobs[h][2], jobs[h][3], tail=jobs[h][4], return_logz=True,
                                         state=st, **r.cfg)
    torch.cuda.synchronize()
    assert torch.equal(out, eager[h])
    nb, kx = keys // 16, 1024 + sink
    assert st["kx"] == kx
    perm = st["perm"][0].cpu().numpy()
    tiles = (0, 1, 318, 636)
    rows = np.concatenate([perm[64 * t: min(n, 64 * t + 64)] for t in tiles])
    qr = q[h].float().numpy()[rows]
    # the runner runs PROD's precision="tf32": the oracle's statistics on TF32 operands too
    ref = flat_i8.flat_i8(qr, bits(k[h]), bits(v[h]), tile=64, leaf=16, exact_leaves=1024, sink_leaves=sink, splits=1,
                          bn=64, prec="tf32")
    ref_out, ref_lz = flat_i8.tail_merge(ref["out"], ref["logz"], qr, tk[h].numpy(), tv[h].numpy(),
                                         1 / math.sqrt(128))
    tix = torch.tensor(tiles, device=device)
    sel = _gpu_sel(st, nb, 1, 64)[0][list(tiles)]
    rep = _check_routing(st["idx"][0, tix].cpu().numpy(), ref, sel, nb, sink)
    assert rep["mismatched"] <= rep["tieable"]
    r_t = torch.from_numpy(rows).to(device)
    assert rel_l2(out[r_t].cpu().numpy(), ref_out) <= OUT_REL_L2
    assert np.abs(logz[r_t].cpu().numpy() - ref_lz).max() <= LOGZ_ABS


@pytest.mark.parametrize("fused", [True, False])
def test_many_leaves_vs_oracle(device, fused):
    """20000 leaves of 16 keys per head, 2048 queries: the fused top-k keys live in global
    memory (keys_ws), the stage top-k reads its rows from global memory."""
    nq, leaf, nb, ex = 2048, 16, 20000, 64
    g = torch.Generator().manual_seed(11)
    c = torch.randn((nb // 8, 128), generator=g) * 1.5
    k = (c.repeat_interleave(8 * leaf, 0) + 0.5 * torch.randn((nb * leaf, 128), generator=g)).to(torch.bfloat16)
    v = torch.randn((nb * leaf, 128), generator=g).to(torch.bfloat16)
    q = (c[torch.randint(0, nb // 8, (nq // 64,), generator=g)].repeat_interleave(64, 0)
         + 0.5 * torch.randn((nq, 128), generator=g)).to(torch.bfloat16)
    st = {}
    out, logz = htrc_flat.flat_attention(q.to(device), k.to(device), v.to(device), leaf=leaf, exact_leaves=ex,
                                         return_logz=True, state=st, **_kw(kern={"fused": fused}))
    torch.cuda.synchronize()
    tiles = (0, 13, 31)
    rows = np.concatenate([np.arange(64 * t, 64 * t + 64) for t in tiles])
    ref = flat_i8.flat_i8(bits(q[rows]), bits(k), bits(v), tile=64, leaf=leaf, exact_leaves=ex, splits=1, bn=64)
    tix = torch.tensor(tiles, device=device)
    sel = _gpu_sel(st, nb, 1, 64)[0][list(tiles)]
    rep = _check_routing(st["idx"][0, tix].cpu().numpy(), ref, sel, nb, 0)
    assert rep["mismatched"] <= rep["tieable"]
    r_t = torch.from_numpy(rows).to(device)
    assert rel_l2(out[r_t].cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz[r_t].cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


@pytest.mark.parametrize("heads,store,mag,stride", [
    (1, "int8", 30, 1), (6, "int8", 30, 1), (8, "int8", 30, 1), (1, "fp8", 30, 1), (2, "bf16", 30, 1),
    (1, "int8", 64, 1), (6, "int8", 64, 1), (8, "int8", 64, 1), (1, "fp8", 64, 1), (2, "bf16", 64, 1),
    (1, "int8", 64, 2), (8, "int8", 64, 2), (1, "fp8", 64, 2), (1, "bf16", 64, 2)])
def test_reference_max_retry(device, heads, store, mag, stride):
    """Row r of tile 0 is mag e_0 and key 3 of leaf 0 (a sink, so always near) is mag e_0: its exact
    score mag^2 / sqrt(128) (80 nats at mag 30, 362 at 64) sits far above the row's far-field
    maximum, the row total at the fixed reference leaves [2^-60, 2^64] (overflows fp32 at 64) and
    the tile is redone at every row's exact largest score.  With sel_stride 2 the row is sampled
    and its far-field maximum (~300 nats at 64) is the reference of the whole tile: every other
    row's total underflows to zero and is redone too.  1, 6 and 8 heads of 64 tiles take the attend
    kernel's four-, two- and one-pair shapes; the 16-bit stores take their own fused route."""
    n, leaf, ex = 4096, 64, 4
    row = 5 if stride == 1 else 4
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=heads, seed=31)
    q = (q.float() * 0.3).to(torch.bfloat16)
    k = (k.float() * 0.3).to(torch.bfloat16)
    q[:, row] = 0
    q[:, row, 0] = mag
    k[:, 3] = 0
    k[:, 3, 0] = mag
    out, logz = htrc_flat.flat_attention(q.to(device), k.to(device), v.to(device), leaf=leaf, exact_leaves=ex,
                                         sink_leaves=1, sel_stride=stride, return_logz=True, **_kw(store=store))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(logz).all())
    h = heads - 1
    ref = flat_i8.flat_i8(bits(q[h, :256]), bits(k[h]), bits(v[h]), tile=64, leaf=leaf, exact_leaves=ex,
                          sink_leaves=1, sel_stride=stride, splits=1, bn=64, store=store)
    assert ref["logz"][row] > 0.9 * mag * mag / math.sqrt(128)      # the outlier dominates its row
    assert rel_l2(out[h, :256].cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz[h, :256].cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


def _ws_bytes(ws) -> int:
    """Device bytes held by a workspace dict (window workspaces nested inside it)."""
    n = 0
    for t in ws.values():
        n += _ws_bytes(t) if isinstance(t, dict) else t.numel() * t.element_size()
    return n


@pytest.mark.parametrize("store,chunk,streams", [("int8", None, 2), ("int8", 4, 2), ("int8", 4, 1), ("int8", 3, 3),
                                                 ("fp8", 4, 2), ("bf16", 5, 2)])
def test_memory_model_equals_the_buffers_a_call_allocates(device, store, chunk, streams):
    """htrc_flat_runner.workspace_bytes (what plan_chunk sizes tile windows against) is the byte
    count of the buffers one operator call leaves in its workspace: the layer's operands, outputs
    and one shared rowmax, plus the state and routing of each window stream's buffers."""
    q, k, v = (x.to(device) for x in workloads.clustered_runs(n=1024, runs=16, heads=2, seed=7))
    ws = {}
    htrc_flat.flat_attention(q, k, v, ws=ws, **_kw(store=store, leaf=64, exact_leaves=3, tile_chunk=chunk,
                                                 kern={"window_streams": streams}))
    torch.cuda.synchronize()
    want = htrc_flat_runner.workspace_bytes(1024, 1024, leaf=64, heads=2, kx=3, tile_chunk=chunk, store=store,
                                            window_streams=streams)
    assert _ws_bytes(ws) == want
