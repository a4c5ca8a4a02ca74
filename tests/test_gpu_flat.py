"""End-to-end GPU parity of flat_attention against the CPU oracle.

Routing: the GPU leaf statistics differ from the oracle's sequential fp32 by rounding
only, so a tile's near-leaf set may differ from the oracle's only where the oracle's
own SEL has a near-tie at the top-k boundary; every other tile must match exactly.
Outputs: rel-L2 <= 1e-2 and |dlogZ| <= 1e-3 (the operator's stated bar).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, check_logz, gpu_sel, record, rel_l2, routing_report, sel_error
from htrc_amd import htrc_flat, htrc_flat_hip as hip, workloads
from oracle import bf16, flat_i8

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-2
LOGZ_ABS = 1e-3


def _routing_check(st, ref, name, stride=1):
    """Near sets against the oracle through the measured SEL error of every tile (group): a set
    may differ only where the oracle's top-k boundary gap is at most twice the tile's largest
    |SEL_gpu - SEL_oracle|; returns the number of differing tiles."""
    nb = st["nb"]
    sel = gpu_sel(st, stride)
    delta = sel_error(sel, ref["sel"], nb)
    rep = routing_report(st["idx"][0].cpu().numpy(), ref["idx"], ref["sel"][:, :nb], delta)
    record(name, rep)
    return rep["mismatched"]


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,leaf,ex", [(16384, 64, 16), (4096, 32, 24), (3000, 64, 8)])
def test_flat_attention_vs_oracle(device, fused, n, leaf, ex):
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + leaf)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="int8", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         kern={"fused": fused, "tile_bn": 64}, return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex,
                          splits=1 if fused else 4, bn=64)
    assert np.array_equal(st["q8"][0].cpu().numpy(), ref["q8"])
    assert np.array_equal(st["k8"][0].cpu().numpy(), ref["k8"])
    _routing_check(st, ref, f"flat fused={fused} n={n} leaf={leaf} ex={ex}")
    err = rel_l2(out.cpu().numpy(), ref["out"])
    record(f"flat fused={fused} n={n} leaf={leaf} ex={ex} errors",
           {"rel_l2": err, "dlogz_max": float(np.abs(logz.cpu().numpy() - ref["logz"]).max())})
    assert err <= OUT_REL_L2
    check_logz(logz.cpu().numpy(), ref, st, LOGZ_ABS)


@pytest.mark.parametrize("store", ["int8", "fp8", "bf16"])
def test_flat_attention_tf32_statistics_vs_oracle(device, store):
    """precision="tf32" (the reference PROD's setting) on the dot="bf16" stores: the leaf
    statistics on TF32 operands, as the reference's leaf_stats takes PREC for every store, against
    the oracle run at TF32; routing up to the oracle's near-ties, outputs within the bar."""
    n, leaf, ex = 4096, 64, 8
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=1, seed=77)
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store=store, dot="bf16", precision="tf32", leaf=leaf, exact_leaves=ex,
                                         return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex, splits=1, bn=64,
                          store=store, prec="tf32")
    if store == "int8":
        _routing_check(st, ref, f"flat tf32 statistics {store}")
    else:
        assert (st["idx"][0].cpu().numpy() != ref["idx"]).any(1).mean() <= 0.05
    err = rel_l2(out.cpu().numpy(), ref["out"])
    dl = float(np.abs(logz.cpu().numpy() - ref["logz"]).max())
    record(f"flat tf32 statistics {store} errors", {"rel_l2": err, "dlogz_max": dl})
    assert err <= OUT_REL_L2 and dl <= LOGZ_ABS, (err, dl)


def test_multihead_equals_per_head(device):
    q, k, v = workloads.clustered_runs(n=2048, runs=32, heads=3, seed=9)
    kw = dict(backend="hip", store="int8", dot="bf16", leaf=64, exact_leaves=8)
    out = htrc_flat.flat_attention(q.to(device), k.to(device), v.to(device), **kw)
    for h in range(3):
        oh = htrc_flat.flat_attention(q[h].to(device), k[h].to(device), v[h].to(device), **kw)
        assert torch.equal(out[h], oh)


def test_route_grid_shapes_agree(device):
    """The attend launch splits a tile's keys over 4, 2 or 1 wave pairs by grid size (at most
    one tile per CU, up to two, more).  One head's data in grids of 128, 384 and 1152 tiles
    (1, 3 and 9 heads, N = 8192) takes each shape on a 256-CU MI355X: the outputs agree to
    fp32 summation order, and sampled whole tiles match the oracle on the head's full key set."""
    n, leaf, ex = 8192, 64, 16
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=9, seed=21)
    q, k, v = q.to(device), k.to(device), v.to(device)
    kw = dict(backend="hip", store="int8", dot="bf16", leaf=leaf, exact_leaves=ex)
    res = [htrc_flat.flat_attention(q[:h], k[:h], v[:h], return_logz=True, **kw) for h in (1, 3, 9)]
    torch.cuda.synchronize()
    o0, l0 = res[0][0][0], res[0][1][0]
    for out, logz in res[1:]:
        assert rel_l2(out[0].cpu().numpy(), o0.cpu().numpy()) <= 1e-5
        assert float((logz[0] - l0).abs().max()) <= 1e-5
    tiles = (0, 1, 64, 127)
    rows = torch.from_numpy(np.concatenate([np.arange(64 * t, 64 * t + 64) for t in tiles])).to(device)
    ref = flat_i8.flat_i8(bits(q[0, rows].cpu()), bits(k[0].cpu()), bits(v[0].cpu()), tile=64, leaf=leaf,
                          exact_leaves=ex, splits=1, bn=64)
    for out, logz in res:
        assert rel_l2(out[0, rows].cpu().numpy(), ref["out"]) <= OUT_REL_L2
        assert np.abs(logz[0, rows].cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


def test_deterministic(device):
    q, k, v = workloads.clustered_runs(n=4096, runs=64, heads=2, seed=1)
    kw = dict(backend="hip", store="int8", dot="bf16", leaf=64, exact_leaves=16)
    a = htrc_flat.flat_attention(q.to(device), k.to(device), v.to(device), **kw).clone()
    b = htrc_flat.flat_attention(q.to(device), k.to(device), v.to(device), **kw)
    assert torch.equal(a, b)


@pytest.mark.parametrize("fused,chunk", [(True, 1024), (False, 1024), (True, 16)])
def test_prof_stage_times(device, fused, chunk):
    """prof={} (h3/htrc_flat.py:32-44): wall times in ms per stage, a device sync at each, summed
    over the tile windows under the reference's stage names; the result is the one without prof."""
    q, k, v = workloads.clustered_runs(n=4096, runs=64, heads=1, seed=5)
    args = (q[0].to(device), k[0].to(device), v[0].to(device))
    kw = dict(backend="hip", store="int8", dot="bf16", leaf=64, exact_leaves=16, tile_chunk=chunk,
              kern={"fused": fused})
    ref = htrc_flat.flat_attention(*args, **kw).clone()
    prof = {}
    out = htrc_flat.flat_attention(*args, prof=prof, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    names = {"prep", "stats", "tile", "finish"} | ({"select"} if not fused else set())
    assert set(prof) == names
    assert all(isinstance(t, float) and t >= 0.0 for t in prof.values())
    prof2 = dict(prof)
    htrc_flat.flat_attention(*args, prof=prof2, **kw)
    assert all(prof2[n] >= prof[n] for n in names)    # accumulates into the caller's dict


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("ntail", [7, 16, 33])
def test_tail_keys_vs_oracle(device, fused, ntail):
    """Keys past the last full leaf (h3/htrc_flat_triton.py:187-207, 381-388): the oracle's
    operator output merged with its tail restatement."""
    n, leaf, ex = 4096, 64, 8
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=1, seed=100 + ntail)
    g = torch.Generator().manual_seed(ntail)
    tk = torch.randn((ntail, 128), generator=g) * 1.5
    tv = torch.randn((ntail, 128), generator=g)
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="int8", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         kern={"fused": fused, "tile_bn": 64}, tail=(tk.to(device), tv.to(device)),
                                         return_logz=True)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex,
                          splits=1 if fused else 4, bn=64)
    want, wz = flat_i8.tail_merge(ref["out"], ref["logz"], bf16.to_f32(bits(q[0])), tk.numpy(), tv.numpy(),
                                  1 / np.sqrt(128))
    assert rel_l2(out.cpu().numpy(), want) <= OUT_REL_L2
    assert np.abs(logz.cpu().numpy() - wz).max() <= LOGZ_ABS


@pytest.mark.parametrize("ntail", [1, 5, 16, 20])
def test_tail_merge_kernel_matches_oracle(device, ntail):
    """The tail kernel alone on arbitrary (out, logz): the oracle's merge to fp32 rounding (a p
    next to a bf16 rounding boundary may round the other way: 2e-3 relative at most)."""
    g = torch.Generator().manual_seed(7 + ntail)
    h, nq = 2, 300
    q = (torch.randn((h, nq, 128), generator=g)).to(torch.bfloat16)
    out0 = torch.randn((h, nq, 128), generator=g)
    lz0 = torch.randn((h, nq), generator=g) * 3
    tk = torch.randn((h, ntail, 128), generator=g)
    tv = torch.randn((h, ntail, 128), generator=g)
    out, lz = out0.clone().to(device), lz0.clone().to(device)
    hip.tail_merge(q.to(device), tk.to(device), tv.to(device), scale=0.0884, out=out, logz=lz)
    torch.cuda.synchronize()
    for i in range(h):
        want, wz = flat_i8.tail_merge(out0[i].numpy(), lz0[i].numpy(), bf16.to_f32(bits(q[i])), tk[i].numpy(),
                                      tv[i].numpy(), 0.0884)
        got = out[i].cpu().numpy()
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()
        assert rel_l2(got, want) <= 1e-5 if ntail > 16 else rel_l2(got, want) <= 2e-4
        assert np.abs(lz[i].cpu().numpy() - wz).max() <= 2e-5 * (1 + np.abs(wz).max())


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,group,stride", [(8192, 2, 1), (5000, 4, 1), (4096, 3, 4)])
def test_group_centres_vs_oracle(device, fused, n, group, stride):
    """kern["group"] (h3/htrc_flat.py:223-231): G tiles share one centre, state and near set.
    The group centres, packed rows and SEL are bit-exact; routing per group as above."""
    leaf, ex = 64, 12
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + group)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="int8", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         sel_stride=stride, kern={"fused": fused, "tile_bn": 64, "group": group},
                                         return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex,
                          splits=1 if fused else 4, bn=64, sel_stride=stride, group=group)
    assert np.array_equal(st["mu"][0].cpu().numpy(), ref["mu"])
    assert np.array_equal(st["dq8"][0].cpu().numpy(), ref["dq8"])
    assert np.array_equal(st["sdq"][0].cpu().numpy(), ref["sdq"])
    if not fused:
        # SEL from the GPU state vs the oracle's select on that same state: bit-exact
        nb = ref["g8"].shape[1]
        g8 = st["g8"][0, :, :nb].cpu().numpy()
        sg = st["sg"][0, :, :nb].cpu().numpy()
        lz = st["lz"][0, :, :nb].cpu().numpy()
        want = flat_i8.select(ref["dq8"], ref["sdq"], 64, g8, sg, lz, stride, group)
        assert np.array_equal(st["sel"][0, :, :nb].cpu().numpy().view(np.uint32), want.view(np.uint32))
    _routing_check(st, ref, f"group fused={fused} n={n} G={group} stride={stride}", stride=stride)
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    check_logz(logz.cpu().numpy(), ref, st, LOGZ_ABS)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,group", [(8192, 1), (5000, 2)])
def test_kmeans_order_vs_oracle(device, fused, n, group):
    """order="kmeans" (h3/htrc_flat.py:146-149, 159-165): tiles cut from the queries regrouped
    by the k-means order, the output back in query order.  The permutation and the packed
    rows are bit-exact; routing and output as above."""
    leaf, ex = 64, 12
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + 7)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    perm = q[0][torch.randperm(n, generator=torch.Generator().manual_seed(n))]   # spatially mixed queries
    st = {}
    out, logz = htrc_flat.flat_attention(perm.to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="int8", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         order="kmeans", kern={"fused": fused, "tile_bn": 64, "group": group},
                                         return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(perm), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex,
                          splits=1 if fused else 4, bn=64, group=group, order="kmeans")
    assert np.array_equal(st["perm"][0].cpu().numpy(), ref["perm"])
    assert np.array_equal(st["dq8"][0].cpu().numpy(), ref["dq8"])
    _routing_check(st, ref, f"kmeans fused={fused} n={n} G={group}")
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    check_logz(logz.cpu().numpy(), ref, st, LOGZ_ABS)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,leaf,ex,group", [(8192, 64, 16, 1), (3000, 32, 8, 2)])
def test_fp8_store_vs_oracle(device, fused, n, leaf, ex, group):
    """store="fp8" (h3/htrc_flat_triton.py:65-72 with FP8 = 1): e4m3 leaf state, fp16 far dots,
    bf16 near dots, on the fused route and in the reference's stage structure; routing and
    output as above."""
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + leaf + 5)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="fp8", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         kern={"tile_bn": 64, "group": group, "fused": fused}, return_logz=True,
                                         state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex, splits=4, bn=64,
                          group=group, store="fp8")
    assert np.array_equal(st["dq16"][0].view(torch.int16).cpu().numpy().view(np.uint16), ref["dq16"])
    assert (st.get("sel") is None) == fused
    _routing_check(st, ref, f"fp8 store fused={fused} n={n} leaf={leaf} G={group}")
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,leaf,ex,group", [(8192, 64, 16, 1), (3000, 32, 8, 2)])
def test_bf16_store_vs_oracle(device, fused, n, leaf, ex, group):
    """store="bf16" (the 16-bit state of h3/htrc_flat_triton.py:132-153, 214-254 with FP8 = 0):
    bf16 leaf state, bf16 far and near dots, on the fused route and in the reference's stage
    structure."""
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + leaf + 7)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="bf16", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         kern={"tile_bn": 64, "group": group, "fused": fused}, return_logz=True,
                                         state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=64, leaf=leaf, exact_leaves=ex, splits=4, bn=64,
                          group=group, store="bf16")
    assert np.array_equal(st["dq16"][0].view(torch.int16).cpu().numpy().view(np.uint16), ref["dq16"])
    assert (st.get("sel") is None) == fused
    _routing_check(st, ref, f"bf16 store fused={fused} n={n} leaf={leaf} G={group}")
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


@pytest.mark.parametrize("store,quant", [("int8", {"q": "int8", "kv": "int8", "group": 32}),
                                         ("int8", {"q": "fp8", "kv": "fp8"}),
                                         ("fp8", {"kv": "int4", "group": 16}),
                                         ("bf16", {"state": "int8"}),
                                         ("bf16", {"q": "int8", "kv": "int8", "state": "fp4"})])
def test_quant_simulation_vs_oracle(device, store, quant):
    """quant= (h3/htrc_flat.py:190-195, 246-248): q and K/V fake-quantised before the operator,
    the bf16 store's g and vb after the statistics; against the oracle run on the oracle's
    fake-quantised inputs (K/V then rounded to bf16, as the operator feeds its kernels)."""
    from oracle.fake_quant import fake_quant as ofq
    n, leaf, ex = 4096, 64, 8
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=1, seed=41)
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store=store, dot="bf16", leaf=leaf, exact_leaves=ex, splits=4,
                                         kern={"tile_bn": 64}, quant=quant, return_logz=True, state=st)
    torch.cuda.synchronize()
    qg = quant.get("group", 0)
    qf, kf, vf = (x[0].float().numpy() for x in (q, k, v))
    if quant.get("q"):
        qf = ofq(qf, quant["q"], qg)
    if quant.get("kv"):
        kf, vf = ofq(kf, quant["kv"], qg), ofq(vf, quant["kv"], qg)
    ref = flat_i8.flat_i8(qf, bf16.from_f32(kf), bf16.from_f32(vf), tile=64, leaf=leaf, exact_leaves=ex, splits=4,
                          bn=64, store=store, state_quant=quant.get("state"), quant_group=qg)
    _routing_check(st, ref, f"quant {store} {quant}")
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    if store == "int8":
        check_logz(logz.cpu().numpy(), ref, st, LOGZ_ABS)
    else:
        assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


@pytest.mark.parametrize("order,group,sink,tile", [("seq", 1, 0, 64), ("kmeans", 2, 3, 64), ("seq", 1, 2, 32)])
def test_bound_select_vs_oracle(device, order, group, sink, tile):
    """select="bound" (h3/htrc_flat.py:255-257), store="bf16": near sets chosen by lz + r ||g||, on
    the stage path; routing, output and logZ against the oracle."""
    n, leaf, ex = 4096, 64, 8
    q, k, v = workloads.clustered_runs(n=n, runs=n // 64, heads=1, seed=53 + group)
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip",
                                         store="bf16", dot="bf16", leaf=leaf, exact_leaves=ex, splits=4, tile=tile,
                                         select="bound", order=order, sink_leaves=sink,
                                         kern={"tile_bn": 64, "group": group}, return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=tile, leaf=leaf, exact_leaves=ex, splits=4, bn=64,
                          group=group, order=order, sink_leaves=sink, store="bf16", select_mode="bound")
    assert st.get("sel") is not None                     # the stage path ran
    nb = st["nb"]
    sel = st["sel"][0].cpu().numpy()
    rep = routing_report(st["idx"][0].cpu().numpy(), ref["idx"], ref["sel"][:, :nb], sel_error(sel, ref["sel"], nb))
    record(f"bound order={order} G={group} sink={sink} tile={tile}", rep)
    assert rep["mismatched"] <= rep["tieable"]
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS


def test_quant_rejections(device):
    q, k, v = workloads.clustered_runs(n=256, runs=4, heads=1, seed=1)
    args = (q[0].to(device), k[0].to(device), v[0].to(device))
    kw = dict(backend="hip", dot="bf16", leaf=64, exact_leaves=2)
    with pytest.raises(ValueError, match="no state fake-quant"):
        htrc_flat.flat_attention(*args, store="int8", quant={"state": "int8"}, **kw)
    with pytest.raises(ValueError, match="unknown quant format"):
        htrc_flat.flat_attention(*args, store="int8", quant={"q": "int3"}, **kw)
    with pytest.raises(ValueError, match="divide"):
        htrc_flat.fake_quant(args[0], "int8", 48)
    with pytest.raises(ValueError, match="HIP device"):
        htrc_flat.fake_quant(q[0], "int8")
    with pytest.raises(ValueError, match="select='max'"):
        htrc_flat.flat_attention(*args, store="int8", select="bound", **kw)
    with pytest.raises(ValueError, match="select must be"):
        htrc_flat.flat_attention(*args, store="bf16", select="mean", **kw)


@pytest.mark.parametrize("store,fused,order", [("int8", True, "seq"), ("int8", False, "seq"), ("int8", True, "kmeans"),
                                               ("fp8", False, "seq"), ("fp8", True, "seq"), ("bf16", True, "kmeans")])
def test_tile32_vs_oracle(device, store, fused, order):
    """tile=32 (the runner's mode "max", h3/htrc_flat_runner.py:52) end to end: 32-row tiles,
    each with its own centre, state and near set; routing and output as above."""
    n, leaf, ex = 6000, 16, 48
    nk = (n // leaf) * leaf
    q, k, v = workloads.clustered_runs(n=n, runs=max(1, n // 64), heads=1, seed=n + 32)
    k, v = k[:, :nk].contiguous(), v[:, :nk].contiguous()
    st = {}
    out, logz = htrc_flat.flat_attention(q[0].to(device), k[0].to(device), v[0].to(device), backend="hip", tile=32,
                                         store=store, dot="bf16", leaf=leaf, exact_leaves=ex, splits=4, order=order,
                                         kern={"tile_bn": 64, "fused": fused}, return_logz=True, state=st)
    torch.cuda.synchronize()
    ref = flat_i8.flat_i8(bits(q[0]), bits(k[0]), bits(v[0]), tile=32, leaf=leaf, exact_leaves=ex,
                          splits=1 if fused else 4, bn=64, order=order, store=store)
    assert st["tile"] == 32 and st["idx"].shape[1] == -(-n // 32)
    _routing_check(st, ref, f"tile32 store={store} fused={fused} order={order}")
    assert rel_l2(out.cpu().numpy(), ref["out"]) <= OUT_REL_L2
    if store == "int8":
        check_logz(logz.cpu().numpy(), ref, st, LOGZ_ABS)
    else:
        assert np.abs(logz.cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS
