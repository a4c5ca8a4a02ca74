"""Full-size layers on the GPU: cfg3 (B=1, H=24, N=64512, d=128, leaf 64, 32 near leaves),
the runner's 32-row-tile shape at the same N (leaf 16, 256 near leaves; 4 heads, whose leaf
state is 3 GB each) and cfg4 (N=124992, 1953 leaves per head; 4 of its 24 heads), checked
through properties that do not need the oracle to run the whole layer:

* tiles are independent given the keys, so whole tiles of the full-size run (first, second,
  middle, last) of two or three heads are compared with the oracle run on just those tiles and the
  head's full key set: pack bit-exact, routing identical up to oracle near-ties, output
  rel-L2 <= 1e-2 and |dlogZ| <= 1e-3;
* a second call gives bit-identical output and logZ (no data-dependent scheduling);
* one head run alone gives exactly the head-batched result.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, rel_l2
from htrc_amd import htrc_flat, workloads
from oracle import flat_i8

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-2
LOGZ_ABS = 1e-3
NEAR_TIE = 1e-4
KW = dict(backend="hip", store="int8", dot="bf16", splits=4, kern={"tile_bn": 64})
# (workload, tile, leaf, near leaves, heads, checked tiles, checked heads)
SHAPES = {
    "cfg3": ("cfg3", 64, None, None, 24, (0, 1, 503, 1007), (0, 11, 23)),
    "tile32": ("cfg3", 32, 16, 256, 4, (0, 1, 1007, 2015), (0, 3)),
    "cfg4": ("cfg4", 64, None, None, 4, (0, 1, 976, 1952), (0, 3)),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def layer(device, request):
    cfg, tile, leaf, ex, heads, tiles, hs = SHAPES[request.param]
    q, k, v, leaf0, ex0 = workloads.make(cfg, heads=heads, device=device)
    leaf, ex = leaf or leaf0, ex or ex0
    st = {}
    out, logz = htrc_flat.flat_attention(q, k, v, tile=tile, leaf=leaf, exact_leaves=ex, return_logz=True, state=st,
                                         **KW)
    torch.cuda.synchronize()
    yield q, k, v, tile, leaf, ex, tiles, hs, st, out, logz
    del st, out, logz
    torch.cuda.empty_cache()


def test_fullsize_tiles_match_the_oracle(layer):
    q, k, v, tile, leaf, ex, tiles, hs, st, out, logz = layer
    assert tuple(out.shape) == tuple(q.shape)
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(logz).all())
    rows = np.concatenate([np.arange(tile * t, tile * t + tile) for t in tiles])
    for h in hs:
        qh = bits(q[h, torch.from_numpy(rows).to(q.device)].cpu())
        ref = flat_i8.flat_i8(qh, bits(k[h].cpu()), bits(v[h].cpu()), tile=tile, leaf=leaf, exact_leaves=ex, splits=1,
                              bn=64)
        tix = torch.tensor(tiles, device=q.device)
        assert np.array_equal(st["mu"][h, tix].cpu().numpy().view(np.uint32), ref["mu"].view(np.uint32))
        r = torch.from_numpy(rows).to(q.device)
        for name in ("q8", "dq8"):
            assert np.array_equal(st[name][h, r].cpu().numpy(), ref[name]), f"head {h} {name}"
        for name in ("sq", "sdq"):
            assert np.array_equal(st[name][h, r].cpu().numpy().view(np.uint32), ref[name].view(np.uint32))
        idx = st["idx"][h, tix].cpu().numpy()
        for j, t in enumerate(tiles):
            if np.array_equal(idx[j], ref["idx"][j]):
                continue
            s = np.sort(ref["sel"][j])[::-1]
            gap = abs(float(s[ex - 1]) - float(s[ex]))
            assert gap <= NEAR_TIE * max(1.0, abs(float(s[ex - 1]))), f"head {h} tile {t}: routing differs, gap {gap:.3e}"
        assert rel_l2(out[h, r].cpu().numpy(), ref["out"]) <= OUT_REL_L2, f"head {h}"
        assert np.abs(logz[h, r].cpu().numpy() - ref["logz"]).max() <= LOGZ_ABS, f"head {h}"


def test_fullsize_repeat_and_single_head_are_bit_identical(layer):
    q, k, v, tile, leaf, ex, tiles, hs, st, out, logz = layer
    out2, logz2 = htrc_flat.flat_attention(q, k, v, tile=tile, leaf=leaf, exact_leaves=ex, return_logz=True, **KW)
    torch.cuda.synchronize()
    assert torch.equal(out2, out) and torch.equal(logz2, logz)
    del out2, logz2
    h = hs[-1]
    o1, l1 = htrc_flat.flat_attention(q[h], k[h], v[h], tile=tile, leaf=leaf, exact_leaves=ex, return_logz=True, **KW)
    torch.cuda.synchronize()
    assert torch.equal(o1, out[h]) and torch.equal(l1, logz[h])


def test_cfg5_sweep_reports_every_grid_point(device):
    """BASELINE configuration 5 (bench.py --config cfg5) on a reduced grid: every point runs,
    errors against exact softmax are finite and small, more near leaves never hurt much, and
    the bf16 Q/K point is at least as close as the int8 one."""
    import bench
    total, grid = bench.sweep_cfg5(calls=3, warmup=1, leaves=(64,), nears=(16, 64), reps=1)
    assert total > 0 and len(grid) == 4
    for g in grid:
        assert 0.0 <= g["logz_err_max"] < 0.5 and 0.0 <= g["out_rel_l2"] < 0.5 and g["ms"] > 0
    by = {(g["near_leaves"], g["qk"]): g for g in grid}
    for qk in ("int8", "bf16"):
        assert by[(64, qk)]["out_rel_l2"] <= by[(16, qk)]["out_rel_l2"] * 1.05
    for near in (16, 64):
        assert by[(near, "bf16")]["out_rel_l2"] <= by[(near, "int8")]["out_rel_l2"] * 1.05
