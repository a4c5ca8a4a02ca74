"""Flat (tree-free) HTRC attention operator on MI355X -- the drop-in for h3/htrc_flat.py.

Same call surface as the reference (``flat_attention``, ``PROD``, ``flat_attention_prod``):
queries are cut into tiles of 64 (or 32) rows with centre mu_t; every (tile, leaf) gets the exact
leaf cumulants at the centre (log-partition lz, tilted key mean g, value mean vb); each
query sees far leaves through lz + (q - mu).g with value vb, and the ``exact_leaves``
leaves of largest row-max far logit exactly; both merge in one online softmax.

One backend: hand-written gfx950 HIP kernels (``htrc_flat_hip``) for the reference's
``dot="bf16"`` state stores: ``store="int8"`` (INT8 Q/K dots, bf16 PV, fp32 accumulation:
the production path), ``"fp8"`` (e4m3 leaf state) and ``"bf16"``.  ``backend="triton"`` (the
reference's GPU backend name) and ``backend="hip"`` select it; any other backend, or knobs
the HIP path does not implement, raise ``ValueError``.

Extensions over the reference: q/k/v may carry a leading head dimension ([H, N, D]) so a
whole layer runs in one set of launches, and ``return_logz=True`` also returns the
per-row log-partition of the approximate attention.  ``tail=(tk, tv)`` ([n, D], or [H, n, D])
are keys past the last full leaf, attended exactly by every query (as the reference's GPU
backend does).
"""
from __future__ import annotations

import contextlib
import math
import threading
import time

import torch

from . import htrc_flat_hip as hip
from ._lib import nb_pad
from .htrc_flat_runner import F32_UNSPLIT_TILES


def fake_quant(x, fmt, group=0):
    """Round-trip x [..., D] through a low-bit format with symmetric per-group scales
    (h3/htrc_flat.py:68-96): group=0 is one scale per row; fmt int8, int4, fp8 (e4m3) or fp4
    (e2m1, default group 16).  A simulation of low-bit operands (their accuracy cost), run by
    the HIP kernel ``htrc_fake_quant`` on the device -> fp32 of x's shape."""
    shape = x.shape
    d = int(shape[-1])
    if fmt == "fp4" and not group:
        group = 16
    gsz = d if not group else int(group)
    if gsz < 1 or d % gsz:
        raise ValueError("quant group must divide the feature size")
    if fmt not in hip.FAKE_QUANT_FMTS:
        raise ValueError(f"unknown quant format {fmt}")
    if not x.is_cuda:
        raise ValueError("fake_quant runs on the HIP device (this build has no CPU path)")
    xin = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
    return hip.fake_quant(xin.contiguous(), gsz, fmt)


def kmeans_order(q, clusters=32, sample=4096, iters=8):
    """Permutation grouping queries by a small k-means (h3/htrc_flat.py:47-61): Lloyd's k-means
    on an even sample, every query to its nearest centre, stable order by centre.  q [N, D]
    (or [H, N, D]) on the device -> int64 [N] (or [H, N]), as ``torch.argsort`` returns."""
    perm = hip.kmeans_order(q, clusters=clusters, sample=sample, iters=iters)
    return perm[0].long() if q.dim() == 2 else perm.long()


class _Tick:
    """Per-stage wall time with a device sync per stage (h3/htrc_flat.py:32-44)."""

    def __init__(self, prof):
        self.prof = prof
        if prof is not None:
            torch.cuda.synchronize()
            self.t = time.perf_counter()

    def __call__(self, name):
        if self.prof is not None:
            torch.cuda.synchronize()
            t = time.perf_counter()
            self.prof[name] = self.prof.get(name, 0.0) + 1e3 * (t - self.t)
            self.t = t


def _store_dtype(store):
    """The state element type of a store name (h3/htrc_flat.py:123: any other name is fp32)."""
    return {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "int8": torch.int8}.get(store, torch.float32)


def _validate(q, k, v, tile, order, curvature, leaf, select, backend, store, dot, quant, tail, kern):
    if backend not in ("hip", "triton"):
        raise ValueError(f"backend {backend!r} is not part of this build: the flat operator runs only as "
                         "HIP kernels (backend='hip', alias 'triton')")
    if curvature != "lin":
        raise ValueError("the HIP backend needs curvature='lin'")
    # h3/htrc_flat.py:123, 196-210: any store other than int8 / fp8 / bf16 is the fp32 state, and
    # any dot other than "bf16" runs fp32 dots (the precision knob picks IEEE or TF32 operands)
    if dot == "bf16" and _store_dtype(store) == torch.float32:
        raise ValueError("dot='bf16' needs store='bf16', 'fp8' or 'int8'")
    if store in ("fp8", "int8") and dot != "bf16":
        raise ValueError(f"store={store!r} needs dot='bf16', select='max' and no state fake-quant")
    if select not in ("max", "bound"):
        raise ValueError("select must be 'max' or 'bound'")
    if select == "bound" and store in ("int8", "fp8"):
        # h3/htrc_flat.py:209-210: the int8 / fp8 stores route by the row-max score only
        raise ValueError(f"store={store!r} needs dot='bf16', select='max' and no state fake-quant")
    if order not in ("seq", "kmeans"):
        raise ValueError("order must be seq or kmeans")
    if quant:
        if not isinstance(quant, dict) or set(quant) - {"q", "kv", "state", "group"}:
            raise ValueError("quant is a dict of 'q', 'kv', 'state' (formats) and 'group'")
        for key in ("q", "kv", "state"):
            if quant.get(key) and quant[key] not in hip.FAKE_QUANT_FMTS:
                raise ValueError(f"unknown quant format {quant[key]}")
        if quant.get("state") and store in ("int8", "fp8"):
            # h3/htrc_flat.py:209-210: the int8 / fp8 stores take no state fake-quant
            raise ValueError(f"store={store!r} needs dot='bf16', select='max' and no state fake-quant")
    if tail is not None:
        if not isinstance(tail, (tuple, list)) or len(tail) != 2:
            raise ValueError("tail must be (tail_keys, tail_values)")
        tk, tv = tail
        want = (q.dim() == 2 and tk.dim() == 2) or (q.dim() == 3 and tk.dim() == 3 and tk.shape[0] == q.shape[0])
        if not want or tuple(tk.shape) != tuple(tv.shape) or tk.shape[-1] != q.shape[-1]:
            raise ValueError("tail keys / values must be [n, D] (or [H, n, D] with q [H, N, D])")
    if int(kern.get("group", 1)) > 1024:
        raise ValueError("kern['group'] must be at most 1024 tiles")
    if int(tile) not in hip.TILES:
        raise ValueError("the HIP backend uses tile=64 or tile=32")
    if leaf not in (16, 32, 64, 128):
        raise ValueError("leaf must be 16, 32, 64 or 128")
    if q.dim() not in (2, 3) or k.dim() != q.dim() or v.shape != k.shape:
        raise ValueError("q [N,D] with k/v [M,D], or q [H,N,D] with k/v [H,M,D]")
    if not 1 <= q.shape[-1] <= hip.D or k.shape[-1] != q.shape[-1]:
        raise ValueError("head dim must be at most 128 and the same for q and k/v")
    if q.dim() == 3 and q.shape[0] != k.shape[0]:
        raise ValueError("q and k/v must have the same number of heads")
    if int(k.shape[-2]) % int(leaf):
        raise ValueError("HIP backend: key count must be a multiple of the leaf size")


class _Collect:
    """Whole-layer copies of the per-window leaf state and routing for ``state=`` checks: one
    window is referenced as is; several are copied window by window into full tensors."""

    def __init__(self, state, h, ng, windows):
        self.state, self.h, self.ng, self.single = state, h, ng, windows == 1
        self.full = {}

    def add(self, g0, gn, **parts):
        if self.state is None:
            return
        for name, t in parts.items():
            if t is None:
                continue
            if self.single:
                self.full[name] = t
                continue
            if name not in self.full:
                self.full[name] = torch.empty((self.h, self.ng, *t.shape[2:]), dtype=t.dtype, device=t.device)
            self.full[name][:, g0:g0 + gn].copy_(t)

    def finish(self, **extra):
        if self.state is not None:
            self.state.update(self.full)
            self.state.update(extra)


_WINDOW_STREAMS = threading.local()


def _window_streams(device, n: int) -> tuple:
    """``n`` side streams of the device (default priority), created once per (device, thread),
    over which the tile windows of a call are dealt in turn.  Each thread owns its streams: a
    graph capture in one thread (``FlatRunner`` records with capture_error_mode="thread_local")
    records its windows on streams no other thread's eager call launches on or waits for."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    per = getattr(_WINDOW_STREAMS, "by_device", None)
    if per is None:
        per = _WINDOW_STREAMS.by_device = {}
    have = per.setdefault(idx, [])
    while len(have) < n:
        have.append(torch.cuda.Stream(device=idx))
    return tuple(have[:n])


def _pad_dims(x, ws, name: str, dtype):
    """x [H, n, d] (d < 128) -> a workspace copy [H, n, 128] of ``dtype`` whose dims past d are
    zero (the pad dims are cleared by a fill kernel on every call, so a reused buffer and a
    graph replay see zeros there)."""
    buf = hip._buf(ws, name, (*x.shape[:-1], hip.D), dtype, x.device)
    d = int(x.shape[-1])
    buf[..., d:].zero_()
    buf[..., :d].copy_(x)
    return buf


def _windows(ng: int, tile_chunk, group: int):
    """Tile-group windows of the chunk loop (h3/htrc_flat.py:236-240): tile_chunk tiles, i.e.
    tile_chunk // group groups, per window; tile_chunk None or < 1 means one window."""
    step = ng if tile_chunk is None or int(tile_chunk) < 1 else max(1, int(tile_chunk) // int(group))
    return [(g0, min(step, ng - g0)) for g0 in range(0, ng, step)]


@torch.inference_mode()
def flat_attention(q, k, v, *, tile=64, exact_leaves=64, order="seq", curvature="lin", tile_chunk=32,
                   precision="fp32", leaf=16, scale=None, prof=None, select="max", backend="torch",
                   store="fp32", splits=8, dot="tf32", sel_stride=1, kern=None, quant=None, sink_leaves=0,
                   tail=None, ws=None, return_logz=False, state=None):
    """q [N,D] (or [H,N,D]), k/v [M,D] (or [H,M,D]), any float dtype -> out fp32 of q's shape
    (h3/htrc_flat.py:99-139).  ``kern['fused']`` (default True) runs select, top-k, far and
    near field as two fused launches per window, for every state store; False runs the
    reference's stage structure (select, top-k, split tile kernel, merge) honouring ``splits``
    and ``kern['tile_bn']``.  Shapes the fused kernels do not hold (more than 8192 near leaves
    per tile, or more than 262144 leaves per head for store="int8" and 16384 for the 16-bit
    stores) take the stage structure automatically.
    ``kern['group']`` = G > 1 makes G consecutive tiles share one expansion centre (the mean
    of their rows), one leaf state and one near set (h3/htrc_flat.py:223-231).
    ``order='kmeans'`` cuts the tiles from the queries regrouped by ``kmeans_order``; the
    output rows come back in query order (:148-149, 159-165).
    ``tile_chunk`` tiles of every head are processed per window (h3/htrc_flat.py:236-273): the
    per-(tile, leaf) state is held for at most S windows at a time (several windows are dealt
    over S = ``kern['window_streams']`` streams, default 2; S = 1 keeps one), and the result does not
    depend on it.  ``dot`` other than "bf16" runs fp32 dots over an fp32 (``store="fp32"``, the
    reference's default) or bf16 state in the reference's stage structure, with IEEE operands or,
    for ``precision="tf32"``, TF32 ones (h3/htrc_flat.py:122-123, 196-212), its tile kernel
    unsplit when a window holds F32_UNSPLIT_TILES (head, tile) pairs or more.  Every store's leaf
    statistics take TF32 operands for ``precision="tf32"`` (PROD's setting), as the reference's
    leaf_stats takes PREC for every store (h3/htrc_flat.py:243-245), and IEEE fp32 ones otherwise.
    ``state``, if a dict, receives the packed operands and the whole layer's leaf state and routing
    (for checks)."""
    kern = dict(kern or {})
    _validate(q, k, v, tile, order, curvature, leaf, select, backend, store, dot, quant, tail, kern)
    squeeze = q.dim() == 2
    qh = q.unsqueeze(0) if squeeze else q
    kh = k.unsqueeze(0) if squeeze else k
    vh = v.unsqueeze(0) if squeeze else v
    tick = _Tick(prof)
    h, nq, d = (int(x) for x in qh.shape)
    nk = int(kh.shape[1])
    nb = nk // int(leaf)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    sink = max(0, min(int(sink_leaves), nb))
    kx = min(int(exact_leaves) + sink, nb)
    if kx < 0:
        raise ValueError("exact_leaves must be >= 0")
    tile = int(tile)
    stride = int(sel_stride)
    if stride < 1 or tile % stride:
        raise ValueError(f"sel_stride must divide the tile ({tile})")
    group = max(1, int(kern.get("group", 1)))           # G consecutive tiles share one centre
    quant = dict(quant or {})
    qg = int(quant.get("group", 0))
    if quant.get("kv"):                                  # h3/htrc_flat.py:190-195
        kh = fake_quant(kh, quant["kv"], qg)
        vh = fake_quant(vh, quant["kv"], qg)
    if quant.get("q"):
        qh = fake_quant(qh, quant["q"], qg)
    if qh.dtype not in (torch.float32, torch.bfloat16):
        qh = qh.float()
    d_in = d
    if d < hip.D:
        # head dims below 128 (the reference takes any power-of-two D, h3/htrc_flat_triton.py:43, 90):
        # zero dims leave every row maximum, int32 dot, state code and softmax as they are, so the
        # kernels run at 128 on copies padded with zeros and the output keeps the first d dims
        qh = _pad_dims(qh, ws, "q_pad", qh.dtype)
        kh = _pad_dims(kh, ws, "k_pad", torch.bfloat16)
        vh = _pad_dims(vh, ws, "v_pad", torch.bfloat16)
        d = hip.D
    perm = hip.kmeans_order(qh, ws=ws) if order == "kmeans" else None   # query rows regrouped by k-means
    qsrc = qh.contiguous()                               # the query rows select="bound" measures
    f32dots = dot != "bf16"
    prec = "tf32" if precision == "tf32" else "ieee"    # h3/htrc_flat.py:122
    if f32dots:
        # fp32 dots (h3/htrc_flat.py:196-212 with dot != "bf16"): centres from pack_q16, q itself
        # read by the select and tile kernels; the reference's stage structure
        mu, _, _ = hip.pack_q16(qh.contiguous(), tile=tile, ws=ws, group=group, perm=perm, dq_fp16=False)
        packed = {"mu": mu}
        sdt = _store_dtype(store)
        fused = False
    elif store in ("fp8", "bf16"):
        mu, q16, dq16 = hip.pack_q16(qh.contiguous(), tile=tile, ws=ws, group=group, perm=perm, dq_fp16=store == "fp8")
        packed = {"q16": q16, "dq16": dq16, "mu": mu}
        sdt = torch.float8_e4m3fn if store == "fp8" else torch.bfloat16
        fused = bool(kern.get("fused", True)) and hip.route16_fits(nb, kx) and select == "max"
    else:
        mu, q8, sq, dq8, sdq = hip.pack_q(qh.contiguous(), tile=tile, ws=ws, group=group, perm=perm)
        packed = {"q8": q8, "sq": sq, "dq8": dq8, "sdq": sdq, "mu": mu}
        sdt = torch.int8
        fused = bool(kern.get("fused", True)) and hip.route_fits(nb, kx)
    kb = kh.to(torch.bfloat16).contiguous()
    vb = vh.to(torch.bfloat16).contiguous()
    packed["k"], packed["v"] = kb, vb
    if sdt == torch.int8:
        packed["k8"], packed["ks"] = hip.pack_k(kb, ws=ws)
    if f32dots:
        packed["q"] = qsrc
    tick("prep")
    ng = int(mu.shape[1])                               # centres: tiles, or tile groups
    out = hip._buf(ws, "out", (h, nq, d), torch.float32, qh.device)
    logz = hip._buf(ws, "logz", (h, nq), torch.float32, qh.device)
    # each row's largest far-field score (the fused route's softmax reference): one layer-wide
    # buffer, every window writing and reading only its own tiles' rows
    rowmax = hip._buf(ws, "rowmax", (h, -(-nq // tile) * tile), torch.float32, qh.device) if fused else None

    def _window(w, g0, gn):
        """Statistics, select / top-k and attention of the tile groups [g0, g0 + gn), the window's
        buffers in workspace w."""
        g, lz, vbs, sg, sv = hip.leaf_stats(mu, kb, vb, nb, scale, leaf=leaf, store=sdt, ws=w, c0=g0, cn=gn,
                                            prec=prec)
        if quant.get("state"):                           # h3/htrc_flat.py:246-248, in place
            sfmt = quant["state"]
            sgsz = hip.D if not qg and sfmt != "fp4" else (qg or 16)
            hip.fake_quant(g, sgsz, sfmt, out=g)
            hip.fake_quant(vbs, sgsz, sfmt, out=vbs)
        lstate = {"g8": g, "sg": sg, "lz": lz, "vb": vbs, "sv": sv}
        tick("stats")
        sel = excl = idx = None
        if fused:
            idx = hip._rows(w, "idx", h, gn, (kx,), torch.int32, qh.device) if kx > 0 else None
            fn = hip.route if sdt == torch.int8 else hip.route16
            fn(packed, lstate, nq=nq, leaf=leaf, kx=kx, scale=scale, sink=sink, stride=stride, ws=w, out=out,
               logz=logz, idx=idx, group=group, perm=perm, tile=tile, g0=g0, rowmax=rowmax)
            tick("tile")
        else:
            if kx > 0 and select == "bound":            # h3/htrc_flat.py:255-257
                sel = hip.bound_select(qsrc, mu, g, lz, nb, leaf=leaf, ws=w, group=group, tile=tile, g0=g0, perm=perm)
            if kx > 0 and select == "max" and f32dots:
                sel = hip.select_f32(qsrc, mu, g, lz, nb, stride=stride, group=group, tile=tile, g0=g0, perm=perm,
                                     prec=prec, ws=w)
            elif kx > 0 and select == "max":
                sel = hip.rowmax_select(g=g, lz=lz, sg=sg, stride=stride, nb=nb, dq8=packed.get("dq8", packed.get("dq16")),
                                        sdq=packed.get("sdq"), ws=w, group=group, tile=tile, g0=g0)
            if kx > 0:
                idx, excl = hip.topk_excl(sel, nb, kx, sink, ws=w)
            else:
                excl = hip._rows(w, "excl", h, gn, (nb_pad(nb),), torch.int8, qh.device)
                excl.zero_()
            tick("select")
            if f32dots:
                # splits is a launch parameter: a window whose tiles alone fill the device runs
                # unsplit, with no merge launch (the result differs by the merge's rounding only)
                ntw = min(-(-nq // tile), (g0 + gn) * group) - g0 * group
                fs = 1 if h * ntw >= F32_UNSPLIT_TILES else splits
                hip.tile_f32(qsrc, mu, lstate, excl, idx, kb, vb, nq=nq, leaf=leaf, scale=scale, splits=fs,
                             bn=int(kern.get("tile_bn", 32)), ws=w, out=out, logz=logz, group=group, perm=perm,
                             tile=tile, g0=g0, prec=prec)
            else:
                hip.tile_attention(packed, lstate, excl, idx, nq=nq, leaf=leaf, scale=scale, splits=splits,
                                   bn=int(kern.get("tile_bn", 32)), ws=w, out=out, logz=logz, group=group, perm=perm,
                                   tile=tile, g0=g0)
            tick("tile")
        keep.add(g0, gn, g8=g, sg=sg, lz=lz, vb=vbs, sv=sv, sel=sel, excl=excl, idx=idx)

    wins = _windows(ng, tile_chunk, group)
    keep = _Collect(state, h, ng, len(wins))
    # Several windows: dealt in turn over S = kern["window_streams"] side streams (default 2),
    # each with its own window buffers, so that a window's statistics run beside the previous
    # window's select and attend (filling the tails of their launches; S windows' state in
    # flight).  One window, stage timing (prof), state checks or S = 1: the caller's stream, in
    # order.
    nst = min(int(kern.get("window_streams", 2)), len(wins))
    pipe = nst > 1 and prof is None and state is None
    if pipe:
        cur = torch.cuda.current_stream(qh.device)
        side = _window_streams(qh.device, nst)
        for s in side:
            s.wait_stream(cur)
        wsw = (None,) * nst if ws is None else tuple(ws.setdefault(f"window_{i}", {}) for i in range(nst))
    for wi, (g0, gn) in enumerate(wins):
        with torch.cuda.stream(side[wi % nst]) if pipe else contextlib.nullcontext():
            _window(wsw[wi % nst] if pipe else ws, g0, gn)
    if pipe:
        for s in side:
            cur.wait_stream(s)
    if state is not None:
        state.update(packed)
        keep.finish(nb=nb, kx=kx, group=group, perm=perm, tile=tile, windows=wins)
        state.setdefault("idx", None)
    if tail is not None and int(tail[0].shape[-2]) > 0:
        # keys past the last full leaf, exact for every query (h3/htrc_flat_triton.py:187-207, 381-388)
        tk, tv = (x.unsqueeze(0) if squeeze else x for x in tail)
        if d_in < d:
            tk, tv = (_pad_dims(x.to(qh.device), ws, n, torch.float32) for x, n in ((tk, "tk_pad"), (tv, "tv_pad")))
        hip.tail_merge(qh, tk.to(qh.device), tv.to(qh.device), scale=scale, out=out, logz=logz, f32dots=f32dots,
                       prec=prec)
        tick("tail")
    if d_in < d:
        out = out[..., :d_in]
    res = out[0] if squeeze else out
    lzr = logz[0] if squeeze else logz
    tick("finish")
    return (res, lzr) if return_logz else res


PROD = dict(tile=64, exact_leaves=256, tile_chunk=128, backend="triton", precision="tf32",
            store="int8", dot="bf16", splits=4, kern=dict(tile_warps=4, tile_bn=64, tile_stages=2))
# The reference's production knob set (h3/htrc_flat.py:391-392); "triton" selects the HIP kernels.


def flat_attention_prod(q, k, v, **over):
    """Production configuration of the flat operator (h3/htrc_flat.py:397-399)."""
    return flat_attention(q, k, v, **{**PROD, **over})
