"""torch-CPU restatement of the reference's torch backend ``_flat`` -- TEST INFRASTRUCTURE ONLY.

The reference's CPU path is ``flat_attention(backend="torch")`` (h3/htrc_flat.py:133-139 ->
``_flat`` :279-388): torch fp32 ops on whatever device the tensors live on.  This module states the
same steps with torch ops on CPU tensors, so bench.py can time the reference's CPU operator as it
runs (torch's own threaded GEMM, exp, max and top-k kernels) rather than a NumPy port of it:

  per window of ``tile_chunk`` tiles (h3/htrc_flat.py:311-380):
    stats       logits mu_t . k_s * scale per leaf -> lz = logsumexp, w = softmax,
                g = (w K) * scale, vb = w V                          (:318-326)
    far logits  (q - mu_t) . g + lz  (+ the iso curvature term)      (:327-336)
    select      row max (or the bound score), top-k leaves, -inf in the far logits (:337-346)
    far apply   exp against the row max, P vb                        (:347-353)
    near        the selected leaves' tokens (and tail keys) exactly,
                merged with the far part under a shared maximum      (:354-380)

``order="seq"`` only (the k-means order of the runner's accurate modes is the GPU operator's).
It is pinned by tests/test_oracle_torch.py: equal to the NumPy restatement ``flat_fp32`` within
fp32 rounding, and the dense limits (all leaves exact; one query per tile).  bench.py times it
over a whole layer as ``cpu_baseline``; ``flat_fp32`` stays the parity oracle.
"""
from __future__ import annotations

import math

import torch


def _leaf_moments(mu_c, k3, v3, scale: float):
    """Exact leaf cumulants at the window's centres: lz [tc, nb], w [tc, nb, L], g and vb
    [nb, tc, d] (h3/htrc_flat.py:318-326)."""
    tc = mu_c.shape[0]
    nb, leaf, d = k3.shape
    logits = torch.matmul(mu_c, k3.reshape(nb * leaf, d).T).mul_(scale).view(tc, nb, leaf)
    lz = torch.logsumexp(logits, dim=-1)
    w = torch.softmax(logits, dim=-1)
    del logits
    wl = w.transpose(0, 1)                                   # [nb, tc, L]: one batch per leaf
    g = torch.bmm(wl, k3).mul_(scale)
    vb = torch.bmm(wl, v3)
    return lz, w, g, vb


@torch.inference_mode()
def flat_torch(q, k, v, *, tile: int = 64, exact_leaves: int = 64, curvature: str = "lin", tile_chunk: int = 32,
               leaf: int = 16, scale: float | None = None, select: str = "max", tiles: slice | None = None,
               return_logz: bool = False):
    """q [N, D], k / v [M, D] (CPU tensors or arrays) -> out [N, D] fp32 torch tensor, the
    reference's ``_flat`` with order="seq" (and logZ [N] with ``return_logz``).  ``tiles``
    restricts the work to a slice of query tiles (rows outside stay zero)."""
    if select not in ("max", "bound"):
        raise ValueError("select must be max or bound")
    if curvature not in ("lin", "iso"):
        raise ValueError("curvature must be lin or iso")
    q, k, v = (torch.as_tensor(x).float().cpu() for x in (q, k, v))
    n, d = (int(x) for x in q.shape)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    nb = int(k.shape[0]) // leaf
    if nb <= 0:
        raise ValueError("flat attention needs at least one full leaf")
    main = nb * leaf
    kf, vf = k[:main].contiguous(), v[:main].contiguous()
    k3, v3 = kf.view(nb, leaf, d), vf.view(nb, leaf, d)
    kt, vt = k[main:], v[main:]                             # tail keys: exact for every query
    ksq = (k3 * k3).sum(-1) if curvature == "iso" else None
    nt = -(-n // tile)
    rows = nt * tile
    # tiles padded by repeating the last query; each centre is the mean of its real rows
    qpad = torch.cat([q, q[-1:].expand(rows - n, d)]) if rows > n else q
    real = (torch.arange(rows) < n).float().view(nt, tile)
    qt = qpad.view(nt, tile, d)
    mu = (qt * real[..., None]).sum(1) / real.sum(1, keepdim=True)
    kx = min(int(exact_leaves), nb)
    out = torch.zeros((rows, d))
    logz = torch.zeros((rows,))
    span = range(nt) if tiles is None else range(*tiles.indices(nt))
    offs = torch.arange(leaf)
    for t0 in range(span.start, span.stop, tile_chunk):
        t1 = min(span.stop, t0 + tile_chunk)
        tc = t1 - t0
        mu_c, q_c = mu[t0:t1], qt[t0:t1]
        lz, w, g, vb = _leaf_moments(mu_c, k3, v3, scale)
        dq = q_c - mu_c[:, None, :]
        far = torch.bmm(dq, g.permute(1, 2, 0)).add_(lz[:, None, :])      # [tc, T, nb]
        if curvature == "iso":
            spread = (w * ksq[None]).sum(-1).mul_(scale * scale) - g.square().sum(-1).T
            far.add_(spread.clamp_min(0.0)[:, None, :] * dq.square().sum(-1)[:, :, None] * (0.5 / d))
        if kx > 0:
            if select == "bound":
                score = lz + dq.norm(dim=-1).amax(1)[:, None] * g.norm(dim=-1).T
            else:
                score = far.amax(1)
            near = torch.topk(score, kx, dim=-1, sorted=False).indices          # [tc, kx]
            far.scatter_(2, near[:, None, :].expand(tc, tile, kx), -math.inf)
        del w, g
        fmax = far.amax(-1)                                  # -inf where every leaf is near
        fref = torch.where(torch.isfinite(fmax), fmax, torch.zeros_like(fmax))
        pf = far.sub_(fref[..., None]).exp_()
        zf = pf.sum(-1)
        of = torch.bmm(pf, vb.transpose(0, 1))
        del pf, far, vb
        keys, vals = [], []
        if kx > 0:
            tok = (near[..., None] * leaf + offs).reshape(-1)
            keys.append(kf.index_select(0, tok).view(tc, kx * leaf, d))
            vals.append(vf.index_select(0, tok).view(tc, kx * leaf, d))
        if kt.shape[0]:
            keys.append(kt[None].expand(tc, -1, -1))
            vals.append(vt[None].expand(tc, -1, -1))
        if keys:
            ke = keys[0] if len(keys) == 1 else torch.cat(keys, 1)
            ve = vals[0] if len(vals) == 1 else torch.cat(vals, 1)
            se = torch.bmm(q_c, ke.transpose(1, 2)).mul_(scale)
            emax = se.amax(-1)
            pe = se.sub_(emax[..., None]).exp_()
            ze = pe.sum(-1)
            oe = torch.bmm(pe, ve)
            both = torch.maximum(fmax, emax)
            af, ae = torch.exp(fmax - both), torch.exp(emax - both)
            num = of * af[..., None] + oe * ae[..., None]
            den = zf * af + ze * ae
        else:
            both, num, den = fref, of, zf
        out[t0 * tile:t1 * tile] = (num / den.clamp_min(1e-30)[..., None]).reshape(tc * tile, d)
        logz[t0 * tile:t1 * tile] = (both + torch.log(den)).reshape(-1)
    if return_logz:
        return out[:n], logz[:n]
    return out[:n]
