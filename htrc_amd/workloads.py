"""Seeded synthetic workloads of the flat-HTRC benchmark configurations.

There are no captures or datasets on this machine, so every configuration is
synthetic.  Values are drawn in float32 from a seeded ``torch.Generator`` and
rounded once to bf16 (round to nearest even), so the HIP path and the CPU
oracle see identical bits when the generator runs on the CPU.

* ``clustered_runs`` -- configuration 2: ``runs`` centroids ~ N(0, 1.5^2 I); run r
  (tokens 64r .. 64r+63) uses centroid r; K = C[r] + N(0, 0.5^2 I), Q the same with
  independent noise; V ~ N(0, 1).
* ``video_regions`` -- configurations 3 and 4: N = t*y*x latent patches in raster
  order; region id (t//4, y//8, x//8); region centroid ~ N(0, 1.5^2 I); tokens add
  N(0, 0.5^2 I) for Q and K; V ~ N(0, 1).
"""
from __future__ import annotations

import torch

CONFIGS = {
    # name: (generator, kwargs, leaf, exact_leaves, heads)
    "cfg2": ("clustered_runs", dict(n=16384, runs=256, run=64), 64, 16, 1),
    "cfg3": ("video_regions", dict(t=16, y=48, x=84), 64, 32, 24),
    "cfg4": ("video_regions", dict(t=31, y=48, x=84), 64, 32, 24),
}


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def clustered_runs(n: int = 16384, runs: int = 256, run: int = 64, d: int = 128, heads: int = 1,
                   seed: int = 0, device="cpu"):
    """Configuration 2 generator -> q, k, v bf16 [heads, n, d]."""
    g = torch.Generator(device=device).manual_seed(int(seed))
    qs, ks, vs = [], [], []
    rid = (torch.arange(n, device=device) // run).clamp_max(runs - 1)
    for _ in range(heads):
        c = torch.randn((runs, d), generator=g, device=device) * 1.5
        k = c[rid] + 0.5 * torch.randn((n, d), generator=g, device=device)
        q = c[rid] + 0.5 * torch.randn((n, d), generator=g, device=device)
        v = torch.randn((n, d), generator=g, device=device)
        qs.append(_bf16(q))
        ks.append(_bf16(k))
        vs.append(_bf16(v))
    return torch.stack(qs), torch.stack(ks), torch.stack(vs)


def region_ids(t: int, y: int, x: int, rt: int = 4, ry: int = 8, rx: int = 8, device="cpu"):
    """Region index of every raster-ordered (t, y, x) token -> (ids [t*y*x], regions)."""
    tt = torch.arange(t, device=device) // rt
    yy = torch.arange(y, device=device) // ry
    xx = torch.arange(x, device=device) // rx
    ny, nx = -(-y // ry), -(-x // rx)
    ids = (tt[:, None, None] * ny + yy[None, :, None]) * nx + xx[None, None, :]
    return ids.reshape(-1), (-(-t // rt)) * ny * nx


def video_regions(t: int = 16, y: int = 48, x: int = 84, d: int = 128, heads: int = 24,
                  seed: int = 0, device="cpu"):
    """Configurations 3 / 4 generator -> q, k, v bf16 [heads, t*y*x, d]."""
    g = torch.Generator(device=device).manual_seed(int(seed))
    ids, nreg = region_ids(t, y, x, device=device)
    n = ids.numel()
    qs, ks, vs = [], [], []
    for _ in range(heads):
        c = torch.randn((nreg, d), generator=g, device=device) * 1.5
        k = c[ids] + 0.5 * torch.randn((n, d), generator=g, device=device)
        q = c[ids] + 0.5 * torch.randn((n, d), generator=g, device=device)
        v = torch.randn((n, d), generator=g, device=device)
        qs.append(_bf16(q))
        ks.append(_bf16(k))
        vs.append(_bf16(v))
    return torch.stack(qs), torch.stack(ks), torch.stack(vs)


def h3_live(n: int = 40759, keys: int = 40752, tail: int = 7, d: int = 128, heads: int = 1, rank: int = 24,
            seed: int = 0, device="cpu"):
    """The reference runner's live H3 shape (tools/sweep_h3_flat_kernels.py:6-8: 40759 queries,
    37232 keys plus 3520 sink rows = 40752 leaf keys, 7 tail keys): q and k are low-rank mixtures
    of ``rank`` shared directions (coefficients N(0, 0.45^2)) plus N(0, 0.6^2) noise, v ~ N(0, 1)
    -> q, k, v bf16 [heads, n | keys, d] and the tail keys / values fp32 [heads, tail, d]."""
    g = torch.Generator(device=device).manual_seed(int(seed))
    out = [[], [], [], [], []]
    for _ in range(heads):
        basis = torch.randn((rank, d), generator=g, device=device)

        def mix(rows):
            c = torch.randn((rows, rank), generator=g, device=device) * 0.45
            return c @ basis + 0.6 * torch.randn((rows, d), generator=g, device=device)

        q = _bf16(mix(n))
        k = _bf16(mix(keys + tail))
        v = _bf16(torch.randn((keys + tail, d), generator=g, device=device))
        for lst, x in zip(out, (q, k[:keys], v[:keys], k[keys:].float(), v[keys:].float())):
            lst.append(x)
    return tuple(torch.stack(x) for x in out)


def config1(seed: int = 0, queries: int = 1024, keys: int = 4096, d: int = 64):
    """BASELINE configuration 1's inputs (src/htrc_reference/model.py evaluated on q, k, v ~ N(0, 1)
    from numpy's default_rng(seed), drawn q, then k, then v; the reference scales q by 1 / sqrt(d))
    rounded once to bf16 -> q, k, v bf16 [1, n, d] with q unscaled: the flat operator's default
    scale 1 / sqrt(d) (0.125 at d = 64, a power of two) gives the reference's logits exactly."""
    import numpy as np
    rng = np.random.default_rng(int(seed))
    q = rng.standard_normal((queries, d))
    k = rng.standard_normal((keys, d))
    v = rng.standard_normal((keys, d))
    return tuple(_bf16(torch.from_numpy(x).float()).unsqueeze(0) for x in (q, k, v))


def make(name: str, *, seed: int = 0, heads: int | None = None, device="cpu"):
    """(q, k, v, leaf, exact_leaves) for a named configuration."""
    gen, kw, leaf, ex, h = CONFIGS[name]
    kw = dict(kw)
    h = h if heads is None else heads
    fn = clustered_runs if gen == "clustered_runs" else video_regions
    q, k, v = fn(heads=h, seed=seed, device=device, **kw)
    return q, k, v, leaf, ex
