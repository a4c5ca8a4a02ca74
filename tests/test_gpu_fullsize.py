"""Full-size layers on the GPU: cfg3 (B=1, H=24, N=64512, d=128, leaf 64, 32 near leaves), cfg4
(N=124992, 1953 leaves per head, all 24 heads) and the runner's 32-row-tile shape at the cfg3 N
(leaf 16, 256 near leaves; 4 heads, whose leaf state is 3 GB each), checked against the oracle:

* tiles are independent given the keys, so whole tiles of the full-size run (first, second,
  middle, last) of two or three heads are compared with the oracle run on just those tiles and
  the head's full key set: pack bit-exact, output rel-L2 <= 1e-2 and |dlogZ| <= 1e-3;
* routing of one whole head of each shape (32-row tiles included): the oracle's leaf state and SEL
  of every tile of the head against the GPU's, the near sets compared through the measured SEL
  error (helpers.routing_report);
* a run in tile windows of 128 tiles (PROD's tile_chunk) gives the one-window result bit for bit,
  and one head run alone gives exactly the head-batched result.

BASELINE configuration 5 (50 sequential cfg2-shape calls and its 18-point ablation grid) runs
whole, every grid point checked against the oracle on sampled tiles.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import bits, gpu_sel, record, rel_l2, routing_report, sel_error
from htrc_amd import htrc_flat, htrc_flat_hip as hip, workloads
from oracle import flat_i8

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-2
LOGZ_ABS = 1e-3
KW = dict(backend="hip", store="int8", dot="bf16", splits=4, kern={"tile_bn": 64})
# (workload, tile, leaf, near leaves, heads, checked tiles, checked heads, whole-head routing head)
SHAPES = {
    "cfg3": ("cfg3", 64, None, None, 24, (0, 1, 503, 1007), (0, 11, 23), 11),
    "tile32": ("cfg3", 32, 16, 256, 4, (0, 1, 1007, 2015), (0, 3), 1),
    "cfg4": ("cfg4", 64, None, None, 24, (0, 1, 976, 1952), (0, 12, 23), 12),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def layer(device, request):
    name = request.param
    cfg, tile, leaf, ex, heads, tiles, hs, hr = SHAPES[name]
    q, k, v, leaf0, ex0 = workloads.make(cfg, heads=heads, device=device)
    leaf, ex = leaf or leaf0, ex or ex0
    st = {}
    out, logz = htrc_flat.flat_attention(q, k, v, tile=tile, leaf=leaf, exact_leaves=ex, tile_chunk=1 << 20,
                                         return_logz=True, state=st, **KW)
    torch.cuda.synchronize()
    yield name, q, k, v, tile, leaf, ex, tiles, hs, hr, st, out, logz
    del st, out, logz
    torch.cuda.empty_cache()


def test_fullsize_tiles_match_the_oracle(layer):
    name, q, k, v, tile, leaf, ex, tiles, hs, hr, st, out, logz = layer
    assert tuple(out.shape) == tuple(q.shape) and len(st["windows"]) == 1
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(logz).all())
    rows = np.concatenate([np.arange(tile * t, tile * t + tile) for t in tiles])
    r = torch.from_numpy(rows).to(q.device)
    tix = torch.tensor(tiles, device=q.device)
    nb = st["nb"]
    for h in hs:
        ref = flat_i8.flat_i8(bits(q[h, r].cpu()), bits(k[h].cpu()), bits(v[h].cpu()), tile=tile, leaf=leaf,
                              exact_leaves=ex, splits=1, bn=64)
        assert np.array_equal(st["mu"][h, tix].cpu().numpy().view(np.uint32), ref["mu"].view(np.uint32))
        for nm in ("q8", "dq8"):
            assert np.array_equal(st[nm][h, r].cpu().numpy(), ref[nm]), f"head {h} {nm}"
        for nm in ("sq", "sdq"):
            assert np.array_equal(st[nm][h, r].cpu().numpy().view(np.uint32), ref[nm].view(np.uint32))
        sel = hip.rowmax_select(g=st["g8"][h:h + 1, tix].contiguous(), lz=st["lz"][h:h + 1, tix].contiguous(),
                                sg=st["sg"][h:h + 1, tix].contiguous(), nb=nb, dq8=st["dq8"][h:h + 1, r].contiguous(),
                                sdq=st["sdq"][h:h + 1, r].contiguous(), tile=tile)[0].cpu().numpy()
        rep = routing_report(st["idx"][h, tix].cpu().numpy(), ref["idx"], ref["sel"], sel_error(sel, ref["sel"], nb))
        rep["rel_l2"] = rel_l2(out[h, r].cpu().numpy(), ref["out"])
        rep["dlogz_max"] = float(np.abs(logz[h, r].cpu().numpy() - ref["logz"]).max())
        record(f"{name} head {h} tiles {tiles}", rep)
        assert rep["rel_l2"] <= OUT_REL_L2, f"head {h}"
        assert rep["dlogz_max"] <= LOGZ_ABS, f"head {h}"


def test_fullsize_whole_head_routing(layer):
    """Every tile of one head: the oracle's leaf state and SEL (IEEE fp32) against the GPU's; the
    g8 codes agree except at fp32-noise ties, and the near sets differ only where the oracle's
    top-k boundary gap is within twice the measured SEL error of the tile."""
    name, q, k, v, tile, leaf, ex, tiles, hs, hr, st, out, logz = layer
    nb = st["nb"]
    mu = st["mu"][hr].cpu().numpy()
    og8, osg, _, olz = flat_i8.stats(mu, bits(k[hr].cpu()), bits(v[hr].cpu()), leaf, 1 / math.sqrt(128))
    g8 = st["g8"][hr, :, :nb].cpu().numpy()
    flips = float((g8 != og8).mean())
    assert np.abs(g8.astype(np.int32) - og8.astype(np.int32)).max() <= 1
    assert flips < 1e-4, f"g8 codes differ on {flips:.2e} of entries"
    osel = flat_i8.select(st["dq8"][hr].cpu().numpy(), st["sdq"][hr].cpu().numpy(), tile, og8, osg, olz)
    oidx, _ = flat_i8.topk(osel, ex)
    sel = hip.rowmax_select(g=st["g8"][hr:hr + 1], lz=st["lz"][hr:hr + 1], sg=st["sg"][hr:hr + 1], nb=nb,
                            dq8=st["dq8"][hr:hr + 1], sdq=st["sdq"][hr:hr + 1], tile=tile)[0].cpu().numpy()
    delta = sel_error(sel, osel, nb)
    rep = routing_report(st["idx"][hr].cpu().numpy(), oidx, osel, delta)
    # a tile whose g8 codes all agree differs in SEL by the fp32 rounding of lz and sg only
    clean = ~(g8 != og8).any(axis=(1, 2))
    rep["g8_flip_frac"] = flips
    rep["tiles_with_flips"] = int((~clean).sum())
    rep["max_delta_clean"] = float(delta[clean].max()) if clean.any() else 0.0
    record(f"{name} whole head {hr}", rep)
    assert rep["max_delta_clean"] <= 2e-6 * max(1.0, float(np.abs(osel[:, :nb]).max()))


def test_fullsize_windows_and_single_head_are_bit_identical(layer):
    name, q, k, v, tile, leaf, ex, tiles, hs, hr, st, out, logz = layer
    out2, logz2 = htrc_flat.flat_attention(q, k, v, tile=tile, leaf=leaf, exact_leaves=ex, tile_chunk=128,
                                           return_logz=True, **KW)
    torch.cuda.synchronize()
    assert torch.equal(out2, out) and torch.equal(logz2, logz)
    del out2, logz2
    h = hs[-1]
    o1, l1 = htrc_flat.flat_attention(q[h], k[h], v[h], tile=tile, leaf=leaf, exact_leaves=ex, tile_chunk=1 << 20,
                                      return_logz=True, **KW)
    torch.cuda.synchronize()
    assert torch.equal(o1, out[h]) and torch.equal(l1, logz[h])


def test_cfg5_sweep_every_grid_point_vs_oracle(device):
    """BASELINE configuration 5 whole: the 50-call sweep (bench.py --config cfg5), and every
    point of the ablation grid leaf {32, 64, 128} x near {16, 32, 64} x Q/K {int8, bf16} at the
    cfg2 shape checked against the oracle (store="int8" / store="bf16") on sampled tiles, plus
    the error against exact softmax that the bench reports."""
    import bench
    total, grid = bench.sweep_cfg5(calls=50, warmup=2, reps=1)
    assert total > 0 and len(grid) == 18
    for g in grid:
        assert 0.0 <= g["logz_err_max"] < 0.5 and 0.0 <= g["out_rel_l2"] < 0.5 and g["ms"] > 0
    q, k, v, _, _ = workloads.make("cfg2", seed=0, device=device)
    tiles = (0, 1, 128, 255)
    rows = np.concatenate([np.arange(64 * t, 64 * t + 64) for t in tiles])
    r = torch.from_numpy(rows).to(device)
    tix = torch.tensor(tiles, device=device)
    qb, kb, vb = bits(q[0].cpu()), bits(k[0].cpu()), bits(v[0].cpu())
    for leaf in (32, 64, 128):
        for near in (16, 32, 64):
            for store in ("int8", "bf16"):
                st = {}
                out, logz = htrc_flat.flat_attention(q[0], k[0], v[0], backend="hip", store=store, dot="bf16",
                                                     leaf=leaf, exact_leaves=near, return_logz=True, state=st,
                                                     splits=4, kern={"tile_bn": 64})
                torch.cuda.synchronize()
                ref = flat_i8.flat_i8(qb[rows], kb, vb, tile=64, leaf=leaf, exact_leaves=near, store=store,
                                      splits=1 if store == "int8" else 4, bn=64)
                sel = gpu_sel(st)[list(tiles)]
                nb = st["nb"]
                rep = routing_report(st["idx"][0, tix].cpu().numpy(), ref["idx"], ref["sel"][:, :nb],
                                     sel_error(sel, ref["sel"], nb))
                record(f"cfg5 leaf={leaf} near={near} {store}", rep)
                assert rel_l2(out[r].cpu().numpy(), ref["out"]) <= OUT_REL_L2, (leaf, near, store)
                assert np.abs(logz[r].cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS, (leaf, near, store)
