"""Seeded random knob combinations of the fp32-dot path (the reference's default triton call:
store="fp32", or "bf16" with dot other than "bf16") against the fp32 oracle (oracle/flat_f32.py).

Each case draws the store, the operand precision (IEEE or TF32), the tile (64 or 32 rows), the
leaf size, ragged query and key counts, the near-leaf count, shared centres, the select row
stride, forced sink leaves, the query order, the split count and a tile window from its own seed.
Bars: every tile group's near set equals the oracle's except where a leaf swapped at the oracle's
top-k boundary within fp32 noise of its k-th score (the output is then checked against the
oracle's attention under the GPU's routing); outputs rel-L2 <= 1e-5 (2e-4 for the bf16 store, whose
state rounding the GPU's sums may tip the other way) and |dlogZ| <= 1e-4 at IEEE precision, 2e-3
and 2e-3 at TF32 (the GPU rounds the softmax weights to TF32 as the reference
does, the oracle does not); the same call in tile windows reproduces the result bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from htrc_amd import htrc_flat, workloads
from oracle import flat_f32
from test_gpu_f32 import _check_operator, _np

pytestmark = pytest.mark.gpu

CASES = 24


def _case(seed: int) -> dict:
    rng = np.random.default_rng(5000 + seed)
    leaf = int(rng.choice([16, 32, 64, 128]))
    nb = int(rng.integers(max(4, 640 // leaf), 3000 // leaf + 1))
    return dict(store=("fp32", "bf16")[seed % 2], precision=str(rng.choice(["fp32", "tf32"])),
                tile=int(rng.choice([64, 32])), leaf=leaf, n=int(rng.integers(500, 2501)), nk=nb * leaf,
                ex=int(rng.integers(0, min(24, nb) + 1)), group=int(rng.choice([1, 1, 2, 3])),
                stride=int(rng.choice([1, 1, 2, 4])), sink=int(rng.choice([0, 0, 2])),
                order=str(rng.choice(["seq", "seq", "kmeans"])), splits=int(rng.choice([1, 2, 4, 8])),
                chunk=int(rng.choice([8, 24, 64])))


@pytest.mark.parametrize("seed", range(CASES))
def test_random_fp32_dots_vs_oracle(device, seed):
    c = _case(seed)
    name = "random_f32 " + " ".join(f"{k}={v}" for k, v in c.items())
    print(name, flush=True)
    q, k, v = workloads.clustered_runs(n=max(c["n"], c["nk"]), runs=max(1, max(c["n"], c["nk"]) // 64), heads=1,
                                       seed=6000 + seed)
    q = q[:, :c["n"]].contiguous()
    k, v = k[:, :c["nk"]].contiguous(), v[:, :c["nk"]].contiguous()
    kw = dict(backend="triton", store=c["store"], dot="tf32", precision=c["precision"], tile=c["tile"],
              leaf=c["leaf"], exact_leaves=c["ex"], sink_leaves=c["sink"], sel_stride=c["stride"], order=c["order"],
              splits=c["splits"], kern={"group": c["group"]}, return_logz=True)
    qd, kd, vd = q[0].to(device), k[0].to(device), v[0].to(device)
    st: dict = {}
    out, logz = htrc_flat.flat_attention(qd, kd, vd, tile_chunk=1 << 20, state=st, **kw)
    out_w, logz_w = htrc_flat.flat_attention(qd, kd, vd, tile_chunk=c["chunk"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(out_w, out) and torch.equal(logz_w, logz), f"{name}: windows differ"
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(logz).all()), name
    prec = "tf32" if c["precision"] == "tf32" else "ieee"
    ref = flat_f32.flat_f32(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(), tile=c["tile"],
                            leaf=c["leaf"], exact_leaves=c["ex"], store=c["store"], prec=prec, group=c["group"],
                            sel_stride=c["stride"], sink_leaves=c["sink"], order=c["order"])
    if ref.get("perm") is not None:
        # compare in operator row order: the routing check recomputes attention in that order
        perm = ref["perm"]
        out_o, logz_o = _np(out)[perm], _np(logz)[perm]
        ref = {**ref, "out": ref["out"][perm], "logz": ref["logz"][perm]}
        qo = q[:, torch.from_numpy(perm)]
    else:
        out_o, logz_o, qo = _np(out), _np(logz), q
    if st.get("idx") is None:                          # no near set: the far field alone
        from helpers import rel_l2
        from test_gpu_f32 import LOGZ, OUT
        bar = max(OUT[prec], 2e-4) if c["store"] == "bf16" else OUT[prec]
        assert rel_l2(out_o, ref["out"]) <= bar and np.abs(logz_o - ref["logz"]).max() <= LOGZ[prec], name
        return
    _check_operator(out_o, logz_o, st, ref, prec, qo, k, v, c["tile"], c["leaf"], c["group"], name, store=c["store"])
