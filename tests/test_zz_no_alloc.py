"""htrc_route_noalloc, the route entry point that allocates nothing (its rowmax, near leaves and
top-k keys live in the library's per-device scratch array), against htrc_route with caller
workspace, through the C ABI: bit-identical outputs on calls in a row with shrinking inputs
(the scratch keeps the previous call's contents), a tile window, and a head of 20000 leaves (top-k
keys in the scratch).  The host-side rejection of calls that need more than the scratch is a CPU
test (tests/test_abi_host.py): it passes pointers that are never dereferenced.
"""
from __future__ import annotations

import math

import pytest
import torch

from htrc_amd import _lib, htrc_flat_hip as hip, workloads
from htrc_amd._lib import call, ptr, stream_handle

pytestmark = pytest.mark.gpu


def _layer(device, q, k, v, leaf, group=1, g0=0, gn=None):
    """Packed operands and the leaf state of the window [g0, g0 + gn) of a layer."""
    q, k, v = q.to(device), k.to(device), v.to(device)
    mu, q8, sq, dq8, sdq = hip.pack_q(q, group=group)
    k8, ks = hip.pack_k(k)
    nb = k.shape[1] // leaf
    g8, lz, vb, sg, _ = hip.leaf_stats(mu, k, v, nb, 1 / math.sqrt(128), leaf=leaf, c0=g0, cn=gn)
    return (q8, sq, dq8, sdq, g8, sg, lz, vb, k8, ks, v), q.shape


def _args(ops):
    return [ptr(t) for t in ops]


def _route_ws(device, ops, shape, nk, leaf, kx, sink, group, g0, gn):
    """htrc_route with torch-allocated workspace -> (out, logz)."""
    h, nq, d = (int(x) for x in shape)
    nt = -(-nq // 64)
    nb = nk // leaf
    kxe = min(kx, nb)
    out = torch.zeros((h, nq, d), device=device)
    logz = torch.zeros((h, nq), device=device)
    idx = torch.empty((h, gn, kxe), dtype=torch.int32, device=device)
    rowmax = torch.empty((h, nt * 64), device=device)
    keys = torch.empty((h, gn, _lib.nb_pad(nb)), dtype=torch.int32, device=device) if nb > 16384 else None
    call("htrc_route", *_args(ops), h, nq, nk, leaf, d, kx, sink, 1, 64, group, g0, gn, None, 1 / math.sqrt(128),
         ptr(out), ptr(logz), ptr(idx), ptr(rowmax), ptr(keys), stream_handle(device))
    return out, logz


def _route_noalloc(device, ops, shape, nk, leaf, kx, sink, group, g0, gn):
    h, nq, d = (int(x) for x in shape)
    out = torch.zeros((h, nq, d), device=device)
    logz = torch.zeros((h, nq), device=device)
    call("htrc_route_noalloc", *_args(ops), h, nq, nk, leaf, d, kx, sink, 1, 64, group, g0, gn, None,
         1 / math.sqrt(128), ptr(out), ptr(logz), stream_handle(device))
    return out, logz


def _case(device, q, k, v, leaf, kx, sink=0, group=1, g0=0, gn=None):
    nt = -(-q.shape[1] // 64)
    ng = -(-nt // group)
    gn = ng - g0 if gn is None else gn
    ops, shape = _layer(device, q, k, v, leaf, group, g0, gn)
    nk = int(k.shape[1])
    a = _route_ws(device, ops, shape, nk, leaf, kx, sink, group, g0, gn)
    b = _route_noalloc(device, ops, shape, nk, leaf, kx, sink, group, g0, gn)
    torch.cuda.synchronize()
    return a, b


def test_noalloc_equals_route_on_calls_in_a_row(device):
    # 1: two heads, the second window of tile groups (groups 10..31 of 32), one sink leaf
    q, k, v = workloads.clustered_runs(n=4096, runs=64, heads=2, seed=3)
    (oa, la), (ob, lb) = _case(device, q, k, v, 64, kx=9, sink=1, g0=10, gn=22)
    rows = slice(10 * 64, 32 * 64)
    assert torch.equal(oa[:, rows], ob[:, rows]) and torch.equal(la[:, rows], lb[:, rows])
    assert bool(torch.isfinite(ob[:, rows]).all())
    # 2: a smaller input: one head of 2048 queries, the whole layer, groups of two tiles
    q, k, v = workloads.clustered_runs(n=2048, runs=32, heads=1, seed=4)
    (oa, la), (ob, lb) = _case(device, q, k, v, 32, kx=6, group=2)
    assert torch.equal(oa, ob) and torch.equal(la, lb)
    # 3: 20000 leaves of 16 keys, 1024 queries: the top-k keys also live in the scratch
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, 320000, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 320000, 128), generator=g).to(torch.bfloat16)
    q = k[:, 64000:65024].clone()
    (oa, la), (ob, lb) = _case(device, q, k, v, 16, kx=40)
    assert torch.equal(oa, ob) and torch.equal(la, lb)

