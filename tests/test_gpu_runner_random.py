"""Seeded random FlatRunner configurations (h3/htrc_flat_runner.py:85-203) on the GPU.

Each case draws the mode, the state store, the heads batched per replay, forced sink leaves,
tail rows, a tile window, the leaf size, the near-leaf count and the query and key counts
from its own seed.  Every replay of the captured graph (two rounds, with eager work between
them) returns, for every head, exactly the eager operator call under the runner's own
configuration.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from htrc_amd import htrc_flat, htrc_flat_runner, workloads

pytestmark = pytest.mark.gpu

CASES = 16


def _case(seed: int) -> dict:
    rng = np.random.default_rng(3000 + seed)
    leaf = int(rng.choice([32, 64]))
    return dict(mode=str(rng.choice(["fast", "balanced", "accurate", "max"])),
                store=("int8", "fp8", "bf16")[seed % 3], batch=int(rng.choice([1, 2, 3])),
                sink=int(rng.choice([0, 0, 3])), tail=int(rng.choice([0, 0, 5])),
                chunk=int(rng.choice([0, 8, 16])), leaf=leaf, ex=int(rng.integers(1, 24)),
                n=int(rng.integers(600, 2600)), m=int(rng.integers(1024 // leaf, 2600 // leaf)) * leaf,
                heads=int(rng.integers(2, 5)))


@pytest.mark.parametrize("seed", range(CASES))
def test_random_runner_replays_equal_eager(device, seed):
    c = _case(seed)
    name = "runner " + " ".join(f"{k}={v}" for k, v in c.items())
    print(name, flush=True)
    q, k, v = workloads.clustered_runs(n=max(c["n"], c["m"]), runs=max(c["n"], c["m"]) // 64, heads=c["heads"],
                                       seed=4000 + seed)
    jobs = [(h, q[h, :c["n"]].float().to(device), k[h, :c["m"]].contiguous().to(device),
             v[h, :c["m"]].contiguous().to(device)) for h in range(c["heads"])]
    g = torch.Generator().manual_seed(seed)
    tails = [(torch.randn((c["tail"], 128), generator=g).to(device),
              torch.randn((c["tail"], 128), generator=g).to(device)) for _ in jobs] if c["tail"] else None
    over = dict(leaf=c["leaf"], exact_leaves=c["ex"], store=c["store"])
    r = htrc_flat_runner.FlatRunner(c["n"], c["m"], mode=c["mode"], heads=c["batch"], sink_leaves=c["sink"],
                                    tail_rows=c["tail"], tile_chunk=c["chunk"] or None, **over)
    try:
        assert r.graph is not None, f"{name}: {r.graph_error}"
        eager = [htrc_flat.flat_attention(j[1], j[2], j[3], tail=(tails[i] if tails else None), **r.cfg)
                 for i, j in enumerate(jobs)]
        run_jobs = [(*j, tails[i]) for i, j in enumerate(jobs)] if tails else jobs
        for rep in range(2):
            outs = r.run(run_jobs)
            torch.cuda.synchronize()
            for h, (o, e) in enumerate(zip(outs, eager)):
                assert torch.equal(o, e), f"{name}: replay {rep}, head {h} differs from eager"
            _ = torch.randn(1 << 20, device=device).sum().item()      # eager work between replays
    finally:
        r.close()
