"""HIP kernel module of the flat operator -- the drop-in for h3/htrc_flat_triton.py.

Every function launches hand-written gfx950 kernels of libhtrc_flat.so through the C ABI
(include/htrc_flat.h) on the current HIP stream.  No function allocates when a workspace
dict ``ws`` is given (buffers are reused, as ``_buf`` does in the reference), none
synchronises, so a whole operator call can be captured in a HIP graph.

Tensors carry a leading head dimension H (2-D inputs are treated as H = 1).  Layouts are
those of the C ABI: the per-(centre, leaf) state is ``g`` int8 ``[H, ng, nbp, 128]`` with row
scales ``sg``, ``lz`` fp32 and ``vb`` bf16 ``[H, ng, nbp, 128]`` (nbp = leaves rounded up to
32; padded leaves have lz = -inf).  ng = nt tiles, or ceil(nt / G) when ``group`` = G tiles
share one centre, one state and one near set (the reference's ``kern["group"]``).

Launch-shape knobs of the reference (bt, bl, warps, stages, prec, sel_bn, rb) are
accepted for call compatibility and ignored: the HIP kernels have fixed MI355X launch
shapes.  ``prec`` is always IEEE fp32 accumulate (there is no TF32 on CDNA4).
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr, stream_handle, nb_pad

TILE = 64
TILES = (64, 32)          # query rows per tile the kernels take (32: the runner's mode "max")
D = 128


def _tile(tile) -> int:
    tile = int(tile)
    if tile not in TILES:
        raise ValueError("the HIP kernels use query tiles of 64 or 32 rows")
    return tile


def _split(n: int, ns: int, bn: int) -> int:
    """Per-split range length (h3/htrc_flat_triton.py:297-299)."""
    per = -(-int(n) // int(ns))
    return max(int(bn), -(-per // int(bn)) * int(bn))


def _buf(ws, name, shape, dtype, device):
    """Workspace buffer reused across calls, sliced to the requested leading size
    (h3/htrc_flat_triton.py:302-312)."""
    if ws is None:
        return torch.empty(shape, device=device, dtype=dtype)
    b = ws.get(name)
    if b is None or b.dtype != dtype or b.shape[1:] != tuple(shape[1:]) or b.shape[0] < shape[0]:
        b = torch.empty(shape, device=device, dtype=dtype)
        ws[name] = b
    return b[: shape[0]]


def _heads(x: torch.Tensor) -> torch.Tensor:
    return x.unsqueeze(0) if x.dim() == 2 else x


def _need(t: torch.Tensor, dtype, name: str):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device (got {t.device})")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def pack_q(q: torch.Tensor, tile: int = TILE, ws=None, group: int = 1, perm=None):
    """Centres and row int8 of q and q - mu -> (mu [H,ng,D], q8, sq, dq8, sdq).  group 1: the
    centre of each tile over its real rows (h3/htrc_flat.py:142-156); group G: the centre of
    each G tiles over their padded rows (:223-229).  perm (int32 [H, nq], optional): row p of
    the packed operands is query perm[p] (order="kmeans", :148-149)."""
    tile = _tile(tile)
    group = int(group)
    if group < 1:
        raise ValueError("group must be >= 1")
    q = _heads(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        q = q.float()
    q = q.contiguous()
    _need(q, None, "q")
    h, nq, d = (int(x) for x in q.shape)
    nt = -(-nq // tile)
    ng = -(-nt // group)
    dev = q.device
    mu = _buf(ws, "mu", (h, ng, d), torch.float32, dev)
    q8 = _buf(ws, "q8", (h, nt * tile, d), torch.int8, dev)
    dq8 = _buf(ws, "dq8", (h, nt * tile, d), torch.int8, dev)
    sq = _buf(ws, "sq", (h, nt * tile), torch.float32, dev)
    sdq = _buf(ws, "sdq", (h, nt * tile), torch.float32, dev)
    if perm is not None:
        _need(perm, torch.int32, "perm")
        if tuple(perm.shape) != (h, nq):
            raise ValueError("perm must be int32 [H, nq]")
    call("htrc_pack_q", ptr(q), int(q.dtype == torch.bfloat16), h, nq, d, tile, group, ptr(perm), ptr(mu), ptr(q8),
         ptr(sq), ptr(dq8), ptr(sdq), stream_handle(dev))
    return mu, q8, sq, dq8, sdq


def pack_q16(q: torch.Tensor, tile: int = TILE, ws=None, group: int = 1, perm=None, dq_fp16: bool = True):
    """Centres and the 16-bit operands of the fp8 (and bf16) state stores -> (mu [H,ng,D],
    q16 bf16 [H,nt*tile,D] = bf16(q), dq16 [H,nt*tile,D] = fp16(q - mu) (bf16 when dq_fp16 is
    False)) over the padded tile rows (h3/htrc_flat_triton.py:104-108)."""
    tile = _tile(tile)
    q = _heads(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        q = q.float()
    q = q.contiguous()
    _need(q, None, "q")
    h, nq, d = (int(x) for x in q.shape)
    nt = -(-nq // tile)
    ng = -(-nt // int(group))
    dev = q.device
    if perm is not None:
        _need(perm, torch.int32, "perm")
    mu = _buf(ws, "mu", (h, ng, d), torch.float32, dev)
    q16 = _buf(ws, "q16", (h, nt * tile, d), torch.bfloat16, dev)
    dq16 = _buf(ws, "dq16" if dq_fp16 else "dqb16", (h, nt * tile, d), torch.float16 if dq_fp16 else torch.bfloat16, dev)
    call("htrc_pack_q16", ptr(q), int(q.dtype == torch.bfloat16), h, nq, d, tile, int(group), ptr(perm),
         int(bool(dq_fp16)), ptr(mu), ptr(q16), ptr(dq16), stream_handle(dev))
    return mu, q16, dq16


def pack_k(k: torch.Tensor, ws=None):
    """K int8 per row (round half to even) -> (k8 [H,nk,D] int8, ks [H,nk] fp32)."""
    k = _heads(k).to(torch.bfloat16).contiguous()
    _need(k, torch.bfloat16, "k")
    h, nk, d = (int(x) for x in k.shape)
    dev = k.device
    k8 = _buf(ws, "k8", (h, nk, d), torch.int8, dev)
    ks = _buf(ws, "ks", (h, nk), torch.float32, dev)
    call("htrc_pack_k", ptr(k), h, nk, d, ptr(k8), ptr(ks), stream_handle(dev))
    return k8, ks


def _rows(ws, name, h, n, tail, dtype, device):
    """Workspace buffer viewed as [h, n, *tail]: reused across calls and windows by its flat
    leading size h * n, so a smaller last window takes the same allocation."""
    return _buf(ws, name, (h * n, *tail), dtype, device).view(h, n, *tail)


def _window(ng: int, g0: int, gn) -> tuple[int, int]:
    g0 = int(g0)
    gn = ng - g0 if gn is None else int(gn)
    if g0 < 0 or gn <= 0 or g0 + gn > ng:
        raise ValueError(f"window [{g0}, {g0 + gn}) must lie in the {ng} centres (tile groups) of a head")
    return g0, gn


MUT_ROW = 2 * D + 8          # one centre's row of htrc_centre_terms (uint16 words)


def leaf_stats(mu, kf, vf, nb, scale, leaf=16, prec="ieee", bt=16, bl=4, warps=4, store=torch.int8, ws=None,
               c0=0, cn=None, terms=True):
    """Leaf statistics at the tile centres (h3/htrc_flat_triton.py:329-345), for the centres
    [c0, c0 + cn) of every head (all by default; the reference passes the chunk's centres).
    mu [H,nt,D] fp32, kf/vf bf16 [H,nk,D] -> (g, lz, vb, sg, sv) in the reference's order, with
    cn state rows per head:
    store=int8: g int8 [H,cn,nbp,D], vb bf16, sv None; store=float8_e4m3fn: g and vb e4m3
    with the row scales sg, sv (h3/htrc_flat_triton.py:65-72); store=bfloat16: g and vb bf16,
    sg and sv None; store=float32: g and vb fp32, sg and sv None.  prec="tf32" (the reference's
    PREC, which its leaf_stats takes for every store) rounds the centres and weights to TF32.
    terms (default): the centres' fp16 operands are made once (htrc_centre_terms) and the
    statistics read them (htrc_leaf_stats_terms); terms=False runs the per-store entries, which
    split the centres themselves (the same state, bit for bit; TF32 there for the bf16 and fp32
    stores only)."""
    if store not in (torch.int8, torch.float8_e4m3fn, torch.bfloat16, torch.float32):
        raise ValueError("the HIP leaf statistics store g as int8, float8_e4m3fn, bfloat16 or float32")
    if prec not in ("ieee", "tf32"):
        raise ValueError("prec must be 'ieee' or 'tf32'")
    mu = _heads(mu).contiguous()
    kf = _heads(kf).contiguous()
    vf = _heads(vf).contiguous()
    _need(mu, torch.float32, "mu")
    _need(kf, torch.bfloat16, "k")
    _need(vf, torch.bfloat16, "v")
    h, nt, d = (int(x) for x in mu.shape)
    c0, cn = _window(nt, c0, cn)
    nk = int(kf.shape[1])
    if int(nb) * int(leaf) != nk or tuple(vf.shape) != tuple(kf.shape):
        raise ValueError("keys and values must be [H, nb * leaf, D]")
    nbp = nb_pad(nb)
    dev = mu.device
    tf32 = prec == "tf32"
    if tf32 and not terms and store in (torch.int8, torch.float8_e4m3fn):
        raise ValueError("TF32 statistics of the int8 and fp8 stores run through the centre terms (terms=True)")
    if terms:
        # the centres' fp16 operands once per window (htrc_centre_terms), then the statistics
        mut = _rows(ws, "mu_terms", h, cn, (MUT_ROW,), torch.int16, dev)
        call("htrc_centre_terms", ptr(mu), h, nt, c0, cn, d, int(tf32), ptr(mut), stream_handle(dev))
        code = {torch.int8: 0, torch.bfloat16: 1, torch.float8_e4m3fn: 2, torch.float32: 3}[store]
        names = {0: ("g", "vb", torch.bfloat16), 1: ("g_bf16", "vb", torch.bfloat16),
                 2: ("g_fp8", "vb_fp8", torch.float8_e4m3fn), 3: ("g_f32", "vb_f32", torch.float32)}[code]
        g = _rows(ws, names[0], h, cn, (nbp, d), store, dev)
        vb = _rows(ws, names[1], h, cn, (nbp, d), names[2], dev)
        lz = _rows(ws, "lz", h, cn, (nbp,), torch.float32, dev)
        sg = _rows(ws, "sg", h, cn, (nbp,), torch.float32, dev) if code in (0, 2) else None
        sv = _rows(ws, "sv", h, cn, (nbp,), torch.float32, dev) if code == 2 else None
        call("htrc_leaf_stats_terms", ptr(mut), ptr(kf), ptr(vf), h, cn, nk, int(leaf), d, float(scale), code,
             int(tf32), ptr(g), ptr(sg), ptr(vb), ptr(sv), ptr(lz), stream_handle(dev))
        return g, lz, vb, sg, sv
    if store in (torch.bfloat16, torch.float32):
        sb = store == torch.bfloat16
        g = _rows(ws, "g_bf16" if sb else "g_f32", h, cn, (nbp, d), store, dev)
        vb = _rows(ws, "vb" if sb else "vb_f32", h, cn, (nbp, d), store, dev)
        lz = _rows(ws, "lz", h, cn, (nbp,), torch.float32, dev)
        if sb and prec == "ieee":
            call("htrc_leaf_stats_bf16", ptr(mu), ptr(kf), ptr(vf), h, nt, c0, cn, nk, int(leaf), d, float(scale),
                 ptr(g), ptr(vb), ptr(lz), stream_handle(dev))
        else:
            call("htrc_leaf_stats_f32", ptr(mu), ptr(kf), ptr(vf), h, nt, c0, cn, nk, int(leaf), d, float(scale),
                 int(sb), int(prec == "tf32"), ptr(g), ptr(vb), ptr(lz), stream_handle(dev))
        return g, lz, vb, None, None
    if store == torch.float8_e4m3fn:
        g = _rows(ws, "g_fp8", h, cn, (nbp, d), torch.float8_e4m3fn, dev)
        vb = _rows(ws, "vb_fp8", h, cn, (nbp, d), torch.float8_e4m3fn, dev)
        sg = _rows(ws, "sg", h, cn, (nbp,), torch.float32, dev)
        sv = _rows(ws, "sv", h, cn, (nbp,), torch.float32, dev)
        lz = _rows(ws, "lz", h, cn, (nbp,), torch.float32, dev)
        call("htrc_leaf_stats_fp8", ptr(mu), ptr(kf), ptr(vf), h, nt, c0, cn, nk, int(leaf), d, float(scale), ptr(g),
             ptr(sg), ptr(vb), ptr(sv), ptr(lz), stream_handle(dev))
        return g, lz, vb, sg, sv
    g8 = _rows(ws, "g", h, cn, (nbp, d), torch.int8, dev)
    sg = _rows(ws, "sg", h, cn, (nbp,), torch.float32, dev)
    lz = _rows(ws, "lz", h, cn, (nbp,), torch.float32, dev)
    vb = _rows(ws, "vb", h, cn, (nbp, d), torch.bfloat16, dev)
    call("htrc_leaf_stats", ptr(mu), ptr(kf), ptr(vf), h, nt, c0, cn, nk, int(leaf), d, float(scale), ptr(g8), ptr(sg),
         ptr(vb), ptr(lz), stream_handle(dev))
    return g8, lz, vb, sg, None


def rowmax_select(q_c=None, mu_c=None, g=None, lz=None, prec="ieee", bn=32, warps=4, splits=8, stride=1, dot=1,
                  ws=None, sg=None, *, nb=None, dq8=None, sdq=None, group=1, tile=TILE, g0=0):
    """SEL [H,gn,nbp] (h3/htrc_flat_triton.py:315-326), the max over the rows of each group of
    ``group`` tiles, for the gn = g.shape[1] groups from g0 (the state's window).  Takes the
    packed rows dq8/sdq (pack_q); when absent they are packed from q_c (fp32 [H,nq,D] rows)."""
    tile = _tile(tile)
    if g.dtype in (torch.float8_e4m3fn, torch.bfloat16):
        return _select16(g, lz, sg, stride, nb, dq8, group, ws, q_c, tile, g0)
    if dq8 is None or sdq is None:
        _, _, _, dq8, sdq = pack_q(q_c, tile=tile, group=group)
    g = _heads(g) if g.dim() == 3 else g
    h, gn, nbp, d = (int(x) for x in g.shape)
    nt = int(_heads(dq8).shape[1]) // tile
    g0, gn = _window(-(-nt // int(group)), g0, gn)
    nb = nbp if nb is None else int(nb)
    dev = g.device
    sel = _rows(ws, "sel", h, gn, (nbp,), torch.float32, dev)
    call("htrc_select", ptr(dq8), ptr(sdq), ptr(g), ptr(sg), ptr(lz), h, nt, nb, int(stride), tile, int(group), g0, gn,
         d, ptr(sel), stream_handle(dev))
    return sel


def _select16(g, lz, sg, stride, nb, dq16, group, ws, q_c, tile, g0):
    """SEL over a 16-bit state: dq16 are the rows of pack_q16 (passed as ``dq8``): fp16 for the
    fp8 state, bf16 for the bf16 state."""
    fp8 = g.dtype == torch.float8_e4m3fn
    if dq16 is None:
        _, _, dq16 = pack_q16(q_c, tile=tile, group=group, dq_fp16=fp8)
    _need(dq16, torch.float16 if fp8 else torch.bfloat16, "dq16")
    h, gn, nbp, d = (int(x) for x in g.shape)
    nt = int(_heads(dq16).shape[1]) // tile
    g0, gn = _window(-(-nt // int(group)), g0, gn)
    nb = nbp if nb is None else int(nb)
    sel = _rows(ws, "sel", h, gn, (nbp,), torch.float32, g.device)
    if fp8:
        call("htrc_select_fp8", ptr(dq16), ptr(g), ptr(sg), ptr(lz), h, nt, nb, int(stride), tile, int(group), g0, gn,
             d, ptr(sel), stream_handle(g.device))
    else:
        call("htrc_select_bf16", ptr(dq16), ptr(g), ptr(lz), h, nt, nb, int(stride), tile, int(group), g0, gn, d,
             ptr(sel), stream_handle(g.device))
    return sel


def topk_excl(sel, nb: int, kx: int, sink: int = 0, ws=None):
    """kx largest SEL per row (leaves < sink forced), idx ascending -> (idx [H,gn,kx] int32,
    excl [H,gn,nbp] int8)  (h3/htrc_flat.py:262-265)."""
    h, gn, nbp = (int(x) for x in sel.shape)
    dev = sel.device
    idx = _rows(ws, "idx", h, gn, (kx,), torch.int32, dev)
    excl = _rows(ws, "excl", h, gn, (nbp,), torch.int8, dev)
    call("htrc_topk", ptr(sel), h * gn, int(nb), int(kx), int(sink), ptr(idx), ptr(excl), stream_handle(dev))
    return idx, excl


def _tile_window(nq: int, tile: int, group: int, g0: int, gn):
    """(g0, gn, first tile, tiles) of the window of tile groups [g0, g0 + gn)."""
    nt = -(-int(nq) // tile)
    g0, gn = _window(-(-nt // int(group)), g0, gn)
    tb = g0 * int(group)
    return g0, gn, tb, min(nt, (g0 + gn) * int(group)) - tb


def tile_attention(packed: dict, state: dict, excl, idx, *, nq: int, leaf: int, scale: float, splits: int = 4,
                   bn: int = 64, ws=None, out=None, logz=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0):
    """Far + near online softmax per (tile, split) and the merge (h3/htrc_flat_triton.py:348-391)
    for the tiles of the gn = state["lz"].shape[1] groups from g0 -> (out [H,nq,D] fp32, logz
    [H,nq] fp32), rows of other tiles left as they were."""
    tile = _tile(tile)
    if state["g8"].dtype in (torch.float8_e4m3fn, torch.bfloat16):
        return _tile16(packed, state, excl, idx, nq=nq, leaf=leaf, scale=scale, splits=splits, bn=bn, ws=ws,
                       out=out, logz=logz, group=group, perm=perm, tile=tile, g0=g0)
    q8, sq, dq8, sdq = packed["q8"], packed["sq"], packed["dq8"], packed["sdq"]
    k8, ks, v = packed["k8"], packed["ks"], packed["v"]
    g8, sg, lz, vb = state["g8"], state["sg"], state["lz"], state["vb"]
    h, nk, d = (int(x) for x in k8.shape)
    g0, gn, tb, ntw = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    kx = int(idx.shape[-1]) if idx is not None else 0
    dev = q8.device
    ns = max(1, int(splits))
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    pm = pl = pacc = None
    if ns > 1:
        pm = _rows(ws, "pm", h, ntw, (ns, tile), torch.float32, dev)
        pl = _rows(ws, "pl", h, ntw, (ns, tile), torch.float32, dev)
        pacc = _rows(ws, "pacc", h, ntw, (ns, tile, d), torch.float32, dev)
    call("htrc_tile", ptr(q8), ptr(sq), ptr(dq8), ptr(sdq), ptr(g8), ptr(sg), ptr(lz), ptr(vb), ptr(excl),
         ptr(idx) if kx else None, ptr(k8), ptr(ks), ptr(v), h, nq, nk, int(leaf), d, kx, tile, int(group), g0, gn,
         ptr(perm), ns, int(bn), float(scale), ptr(pm), ptr(pl), ptr(pacc), ptr(out), ptr(logz), stream_handle(dev))
    if ns > 1:
        call("htrc_merge", ptr(pm), ptr(pl), ptr(pacc), h, nq, tile, tb, ntw, ns, d, ptr(perm), ptr(out), ptr(logz),
             stream_handle(dev))
    return out, logz


def select_f32(q, mu, g, lz, nb: int, *, stride: int = 1, group: int = 1, tile: int = TILE, g0: int = 0, perm=None,
               prec: str = "ieee", ws=None):
    """SEL [H,gn,nbp] with fp32 dots (rowmax_select with dot=0, h3/htrc_flat_triton.py:214-254):
    the max over every stride-th row of each group of (q - mu) . g, plus lz.  q [H,nq,D] fp32 or
    bf16 in query order (perm maps operator rows to queries), mu [H,ng,D] the layer's centres,
    g fp32 or bf16 [H,gn,nbp,D] and lz the window's state; prec "tf32" rounds the operands."""
    q = _heads(q).contiguous()
    tile = _tile(tile)
    h, nq, d = (int(x) for x in q.shape)
    gn, nbp = int(g.shape[1]), int(g.shape[2])
    sel = _rows(ws, "sel", h, gn, (nbp,), torch.float32, g.device)
    call("htrc_select_f32", ptr(q), int(q.dtype == torch.bfloat16), ptr(mu), ptr(g), int(g.dtype == torch.bfloat16),
         ptr(lz), h, nq, int(nb), int(stride), tile, int(group), int(g0), gn, ptr(perm), int(prec == "tf32"), d,
         ptr(sel), stream_handle(g.device))
    return sel


def tile_f32(q, mu, state: dict, excl, idx, k, v, *, nq: int, leaf: int, scale: float, splits: int = 4,
             bn: int = 64, ws=None, out=None, logz=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0,
             prec: str = "ieee"):
    """Far + near softmax per (tile, split) with fp32 dots (tile_attention with dot=0,
    h3/htrc_flat_triton.py:88-211, 348-391) and the merge, for the tiles of the gn =
    state["lz"].shape[1] groups from g0: q [H,nq,D] fp32 or bf16 in query order, mu [H,ng,D],
    state g / vb fp32 or bf16 and lz, k / v bf16 [H,nk,D] -> (out, logz)."""
    q = _heads(q).contiguous()
    tile = _tile(tile)
    g, lz, vb = state["g8"], state["lz"], state["vb"]
    h, nk, d = (int(x) for x in k.shape)
    g0, gn, tb, ntw = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    kx = int(idx.shape[-1]) if idx is not None else 0
    dev = q.device
    ns = max(1, int(splits))
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    pm = pl = pacc = None
    if ns > 1:
        pm = _rows(ws, "pm", h, ntw, (ns, tile), torch.float32, dev)
        pl = _rows(ws, "pl", h, ntw, (ns, tile), torch.float32, dev)
        pacc = _rows(ws, "pacc", h, ntw, (ns, tile, d), torch.float32, dev)
    call("htrc_tile_f32", ptr(q), int(q.dtype == torch.bfloat16), ptr(mu), ptr(g), int(g.dtype == torch.bfloat16),
         ptr(lz), ptr(vb), ptr(excl), ptr(idx) if kx else None, ptr(k), ptr(v), h, nq, nk, int(leaf), d, kx, tile,
         int(group), g0, gn, ptr(perm), ns, int(bn), int(prec == "tf32"), float(scale), ptr(pm), ptr(pl), ptr(pacc),
         ptr(out), ptr(logz), stream_handle(dev))
    if ns > 1:
        call("htrc_merge", ptr(pm), ptr(pl), ptr(pacc), h, nq, tile, tb, ntw, ns, d, ptr(perm), ptr(out), ptr(logz),
             stream_handle(dev))
    return out, logz


def _tile16(packed, state, excl, idx, *, nq, leaf, scale, splits, bn, ws, out, logz, group, perm, tile, g0):
    """Far + near softmax per (tile, split) over a 16-bit state, and the merge: packed holds q16,
    dq16 (pack_q16) and the bf16 k, v; state g8 / vb (e4m3 with sg, sv; or bf16) and lz."""
    q16, dq16, k, v = packed["q16"], packed["dq16"], packed["k"], packed["v"]
    g, sg, lz, vb, sv = state["g8"], state.get("sg"), state["lz"], state["vb"], state.get("sv")
    fp8 = g.dtype == torch.float8_e4m3fn
    h, nk, d = (int(x) for x in k.shape)
    g0, gn, tb, ntw = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    kx = int(idx.shape[-1]) if idx is not None else 0
    dev = q16.device
    ns = max(1, int(splits))
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    pm = pl = pacc = None
    if ns > 1:
        pm = _rows(ws, "pm", h, ntw, (ns, tile), torch.float32, dev)
        pl = _rows(ws, "pl", h, ntw, (ns, tile), torch.float32, dev)
        pacc = _rows(ws, "pacc", h, ntw, (ns, tile, d), torch.float32, dev)
    if fp8:
        call("htrc_tile_fp8", ptr(q16), ptr(dq16), ptr(g), ptr(sg), ptr(lz), ptr(vb), ptr(sv), ptr(excl),
             ptr(idx) if kx else None, ptr(k), ptr(v), h, nq, nk, int(leaf), d, kx, tile, int(group), g0, gn, ptr(perm),
             ns, int(bn), float(scale), ptr(pm), ptr(pl), ptr(pacc), ptr(out), ptr(logz), stream_handle(dev))
    else:
        call("htrc_tile_bf16", ptr(q16), ptr(dq16), ptr(g), ptr(lz), ptr(vb), ptr(excl), ptr(idx) if kx else None,
             ptr(k), ptr(v), h, nq, nk, int(leaf), d, kx, tile, int(group), g0, gn, ptr(perm), ns, int(bn),
             float(scale), ptr(pm), ptr(pl), ptr(pacc), ptr(out), ptr(logz), stream_handle(dev))
    if ns > 1:
        call("htrc_merge", ptr(pm), ptr(pl), ptr(pacc), h, nq, tile, tb, ntw, ns, d, ptr(perm), ptr(out), ptr(logz),
             stream_handle(dev))
    return out, logz


ROUTE_NB_LDS = 16384       # leaves per head whose top-k keys route_select keeps in LDS
ROUTE_MAX_KX = 8192        # near leaves per tile the fused route kernel holds in LDS
ROUTE_MAX_NB = 262144      # leaves per head of the fused route (exclusion bits in LDS)


def route_fits(nb: int, kx: int) -> bool:
    """Whether the fused route takes this shape (else the split tile path runs it)."""
    return int(nb) <= ROUTE_MAX_NB and min(int(kx), int(nb)) <= ROUTE_MAX_KX


def _keys_ws(ws, h, gn, nb, dev):
    """top-k key scratch of route_select for heads of more than ROUTE_NB_LDS leaves (else None)."""
    if int(nb) <= ROUTE_NB_LDS:
        return None
    return _rows(ws, "route_keys", h, gn, (nb_pad(nb),), torch.int32, dev)


def _rowmax(ws, rowmax, h: int, rows: int, dev):
    """Each row's largest far-field score [H, rows] fp32: the caller's buffer, else a workspace one."""
    if rowmax is None:
        return _buf(ws, "rowmax", (h, rows), torch.float32, dev)
    _need(rowmax, torch.float32, "rowmax")
    if tuple(rowmax.shape) != (h, rows):
        raise ValueError(f"rowmax must be fp32 [{h}, {rows}]")
    return rowmax


def route(packed: dict, state: dict, *, nq: int, leaf: int, kx: int, scale: float, sink: int = 0, stride: int = 1,
          ws=None, out=None, logz=None, idx=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0,
          rowmax=None):
    """Fused select -> top-k, then far + near -> normalised output (two launches) for the tiles of
    the gn = state["lz"].shape[1] groups from g0 -> (out [H,nq,D], logz [H,nq]); idx
    [H,gn,min(kx,nb)] int32 receives the window's routing (a workspace buffer when not given).
    rowmax [H, nt * tile] fp32 (a workspace buffer when not given): the window writes and reads
    only its own tiles' rows, so the windows of a layer may share one."""
    q8, sq, dq8, sdq = packed["q8"], packed["sq"], packed["dq8"], packed["sdq"]
    k8, ks, v = packed["k8"], packed["ks"], packed["v"]
    g8, sg, lz, vb = state["g8"], state["sg"], state["lz"], state["vb"]
    h, nk, d = (int(x) for x in k8.shape)
    dev = q8.device
    tile = _tile(tile)
    nt = -(-int(nq) // tile)
    g0, gn, _, _ = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    nb = nk // int(leaf)
    kxe = min(int(kx), nb)
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    if idx is None and kxe > 0:
        idx = _rows(ws, "idx", h, gn, (kxe,), torch.int32, dev)
    rowmax = _rowmax(ws, rowmax, h, nt * tile, dev)
    keys = _keys_ws(ws, h, gn, nb, dev)
    call("htrc_route", ptr(q8), ptr(sq), ptr(dq8), ptr(sdq), ptr(g8), ptr(sg), ptr(lz), ptr(vb), ptr(k8), ptr(ks),
         ptr(v), h, nq, nk, int(leaf), d, int(kx), int(sink), int(stride), tile, int(group), g0, gn, ptr(perm),
         float(scale), ptr(out), ptr(logz), ptr(idx), ptr(rowmax), ptr(keys), stream_handle(dev))
    return out, logz


def route_select(packed: dict, state: dict, *, nq: int, leaf: int, kx: int, sink: int = 0, stride: int = 1,
                 ws=None, idx=None, group: int = 1, tile: int = TILE, g0: int = 0, rowmax=None):
    """First launch of route: select -> top-k per tile group of the window -> (idx
    [H,gn,min(kx,nb)] int32 or None, rowmax [H,nt*tile] fp32, each row's largest far-field
    score)."""
    dq8, sdq = packed["dq8"], packed["sdq"]
    g8, sg, lz = state["g8"], state["sg"], state["lz"]
    h, nk = int(packed["k8"].shape[0]), int(packed["k8"].shape[1])
    dev = dq8.device
    tile = _tile(tile)
    nt = -(-int(nq) // tile)
    g0, gn, _, _ = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    nb = nk // int(leaf)
    kxe = min(int(kx), nb)
    if idx is None and kxe > 0:
        idx = _rows(ws, "idx", h, gn, (kxe,), torch.int32, dev)
    rowmax = _rowmax(ws, rowmax, h, nt * tile, dev)
    keys = _keys_ws(ws, h, gn, nb, dev)
    call("htrc_route_select", ptr(dq8), ptr(sdq), ptr(g8), ptr(sg), ptr(lz), h, nq, nk, int(leaf), D, int(kx),
         int(sink), int(stride), tile, int(group), g0, gn, ptr(idx), ptr(rowmax), ptr(keys), stream_handle(dev))
    return idx, rowmax


def route_attend(packed: dict, state: dict, idx, rowmax, *, nq: int, leaf: int, kx: int, scale: float, ws=None,
                 out=None, logz=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0):
    """Second launch of route: far + near field with the row reference rowmax -> (out, logz)."""
    q8, sq, dq8, sdq = packed["q8"], packed["sq"], packed["dq8"], packed["sdq"]
    k8, ks, v = packed["k8"], packed["ks"], packed["v"]
    g8, sg, lz, vb = state["g8"], state["sg"], state["lz"], state["vb"]
    h, nk, d = (int(x) for x in k8.shape)
    dev = q8.device
    tile = _tile(tile)
    g0, gn, _, _ = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    call("htrc_route_attend", ptr(q8), ptr(sq), ptr(dq8), ptr(sdq), ptr(g8), ptr(sg), ptr(lz), ptr(vb), ptr(k8),
         ptr(ks), ptr(v), ptr(idx), ptr(rowmax), h, nq, nk, int(leaf), d, int(kx), tile, int(group), g0, gn,
         ptr(perm), float(scale), ptr(out), ptr(logz), stream_handle(dev))
    return out, logz


def _r16(packed: dict, state: dict, nq: int, tile: int, group: int, g0: int, leaf: int, kx: int):
    """Shared shapes of the 16-bit route launches."""
    q16, dq16, k, v = packed["q16"], packed["dq16"], packed["k"], packed["v"]
    g, sg, lz, vb, sv = state["g8"], state.get("sg"), state["lz"], state["vb"], state.get("sv")
    fp8 = g.dtype == torch.float8_e4m3fn
    h, nk, d = (int(x) for x in k.shape)
    tile = _tile(tile)
    nt = -(-int(nq) // tile)
    g0, gn, _, _ = _tile_window(nq, tile, group, g0, int(lz.shape[1]))
    kxe = min(int(kx), nk // int(leaf))
    return q16, dq16, k, v, g, sg, lz, vb, sv, fp8, h, nk, d, tile, nt, g0, gn, kxe


def route16_select(packed: dict, state: dict, *, nq: int, leaf: int, kx: int, sink: int = 0, stride: int = 1,
                   ws=None, idx=None, group: int = 1, tile: int = TILE, g0: int = 0, rowmax=None):
    """First launch of route16 (16-bit state stores): select -> top-k per tile group of the
    window -> (idx [H,gn,min(kx,nb)] int32 or None, rowmax [H,nt*tile] fp32, each row's largest
    far-field score, the attend launch's fixed softmax reference)."""
    q16, dq16, k, v, g, sg, lz, vb, sv, fp8, h, nk, d, tile, nt, g0, gn, kxe = _r16(packed, state, nq, tile, group,
                                                                                    g0, leaf, kx)
    dev = dq16.device
    if idx is None and kxe > 0:
        idx = _rows(ws, "idx", h, gn, (kxe,), torch.int32, dev)
    rowmax = _rowmax(ws, rowmax, h, nt * tile, dev)
    call("htrc_route16_select", ptr(dq16), ptr(g), ptr(sg), ptr(lz), h, nq, nk, int(leaf), d, int(kx), int(sink),
         int(stride), tile, int(group), g0, gn, int(fp8), ptr(idx), ptr(rowmax), stream_handle(dev))
    return (idx if kxe > 0 else None), rowmax


def route16_attend(packed: dict, state: dict, idx, rowmax, *, nq: int, leaf: int, kx: int, scale: float, ws=None,
                   out=None, logz=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0):
    """Second launch of route16: far + near field with the row reference rowmax -> (out, logz)."""
    q16, dq16, k, v, g, sg, lz, vb, sv, fp8, h, nk, d, tile, nt, g0, gn, kxe = _r16(packed, state, nq, tile, group,
                                                                                    g0, leaf, kx)
    dev = q16.device
    if out is None:
        out = _buf(ws, "out", (h, nq, d), torch.float32, dev)
    if logz is None:
        logz = _buf(ws, "logz", (h, nq), torch.float32, dev)
    call("htrc_route16_attend", ptr(q16), ptr(dq16), ptr(g), ptr(sg), ptr(lz), ptr(vb), ptr(sv), ptr(k), ptr(v),
         ptr(idx), ptr(rowmax), h, nq, nk, int(leaf), d, int(kx), tile, int(group), g0, gn, ptr(perm), int(fp8),
         float(scale), ptr(out), ptr(logz), stream_handle(dev))
    return out, logz


def route16(packed: dict, state: dict, *, nq: int, leaf: int, kx: int, scale: float, sink: int = 0, stride: int = 1,
            ws=None, out=None, logz=None, idx=None, group: int = 1, perm=None, tile: int = TILE, g0: int = 0,
            rowmax=None):
    """Fused route of the 16-bit state stores (select -> top-k, then far + near in one softmax; two
    launches) for the tiles of the gn = state["lz"].shape[1] groups from g0: packed holds q16,
    dq16 (pack_q16) and the bf16 k, v; state g8 / vb (e4m3 with sg, sv; or bf16) and lz
    -> (out [H,nq,D], logz [H,nq]); idx [H,gn,min(kx,nb)] receives the window's routing."""
    idx, rowmax = route16_select(packed, state, nq=nq, leaf=leaf, kx=kx, sink=sink, stride=stride, ws=ws, idx=idx,
                                 group=group, tile=tile, g0=g0, rowmax=rowmax)
    return route16_attend(packed, state, idx, rowmax, nq=nq, leaf=leaf, kx=kx, scale=scale, ws=ws, out=out,
                          logz=logz, group=group, perm=perm, tile=tile, g0=g0)


def route16_fits(nb: int, kx: int) -> bool:
    """Whether the fused 16-bit route takes this shape (else the split tile path runs it)."""
    return int(nb) <= ROUTE_NB_LDS and min(int(kx), int(nb)) <= ROUTE_MAX_KX


def tail_merge(q, tk, tv, *, scale: float, out, logz, f32dots: bool = False, prec: str = "ieee"):
    """Tail keys tk, tv [H, n, D] (past the last full leaf) attended exactly by every query and
    merged in place into out [H, nq, D] / logz [H, nq] (h3/htrc_flat_triton.py:187-207, 381-388).
    f32dots: the fp32-dot path's operands (IEEE, or TF32 for prec="tf32")."""
    q = _heads(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        q = q.float()
    q = q.contiguous()
    tk = _heads(tk).float().contiguous()
    tv = _heads(tv).float().contiguous()
    _need(q, None, "q")
    _need(tk, torch.float32, "tail keys")
    _need(tv, torch.float32, "tail values")
    h, nq, d = (int(x) for x in q.shape)
    if tk.shape != tv.shape or tk.shape[0] != h or tk.shape[2] != d:
        raise ValueError("tail keys / values must be [H, n, D] matching q")
    _need(out, torch.float32, "out")
    _need(logz, torch.float32, "logz")
    if f32dots:
        call("htrc_tail_f32", ptr(q), int(q.dtype == torch.bfloat16), ptr(tk), ptr(tv), h, nq, int(tk.shape[1]), d,
             int(prec == "tf32"), float(scale), ptr(out), ptr(logz), stream_handle(q.device))
    else:
        call("htrc_tail", ptr(q), int(q.dtype == torch.bfloat16), ptr(tk), ptr(tv), h, nq, int(tk.shape[1]), d,
             float(scale), ptr(out), ptr(logz), stream_handle(q.device))
    return out, logz


def kmeans_order(q: torch.Tensor, clusters: int = 32, sample: int = 4096, iters: int = 8, ws=None):
    """k-means query order (h3/htrc_flat.py:47-61) -> perm int32 [H, nq]: the queries ordered by
    their nearest centre (stable), the centres from ``iters`` Lloyd steps on ``sample`` evenly
    spaced queries."""
    q = _heads(q)
    if q.dtype not in (torch.float32, torch.bfloat16):
        q = q.float()
    q = q.contiguous()
    _need(q, None, "q")
    h, nq, d = (int(x) for x in q.shape)
    dev = q.device
    cen = _buf(ws, "km_centres", (h, int(clusters), d), torch.float32, dev)
    assign = _buf(ws, "km_assign", (h, nq), torch.int32, dev)
    perm = _buf(ws, "perm", (h, nq), torch.int32, dev)
    call("htrc_kmeans_order", ptr(q), int(q.dtype == torch.bfloat16), h, nq, d, int(clusters), int(sample), int(iters),
         ptr(cen), ptr(assign), ptr(perm), stream_handle(dev))
    return perm


def dequant_rows(x8, scale, out, br=64):
    """out[r, :] = x8[r, :] * scale[r] in one pass, fp8 (e4m3fn) -> out's dtype (bf16 or fp32)
    (h3/htrc_flat_triton.py:287-294).  x8 [rows, D] and scale [rows] may be strided head
    views of the per-token cache; out [rows, D] contiguous.  ``br`` is accepted for call
    compatibility."""
    if x8.dtype != torch.float8_e4m3fn:
        raise ValueError("x8 must be float8_e4m3fn")
    if x8.dim() != 2 or x8.stride(1) != 1:
        raise ValueError("x8 must be [rows, D] with unit stride along D")
    rows, d = int(x8.shape[0]), int(x8.shape[1])
    if scale.dim() != 1 or int(scale.shape[0]) != rows:
        raise ValueError("scale must be [rows]")
    if scale.dtype != torch.float32:
        scale = scale.float()
    if out.dtype not in (torch.bfloat16, torch.float32) or tuple(out.shape) != (rows, d) or not out.is_contiguous():
        raise ValueError("out must be a contiguous [rows, D] bf16 or fp32 tensor")
    for t, n in ((x8, "x8"), (scale, "scale"), (out, "out")):
        if t.device.type != "cuda":
            raise ValueError(f"{n} must be on a HIP device (got {t.device})")
    call("htrc_dequant_rows", ptr(x8), int(x8.stride(0)) if rows > 1 else d, ptr(scale), int(scale.stride(0)), rows, d,
         ptr(out), int(out.dtype == torch.bfloat16), stream_handle(out.device))
    return out


def selftest_mfma(ai, bi, af, bf):
    """Run the MFMA convention self-test kernel -> (ci int32 [16,16], cf fp32 [16,16])."""
    dev = ai.device
    ci = torch.empty((16, 16), dtype=torch.int32, device=dev)
    cf = torch.empty((16, 16), dtype=torch.float32, device=dev)
    call("htrc_selftest_mfma", ptr(ai), ptr(bi), ptr(ci), ptr(af), ptr(bf), ptr(cf), stream_handle(dev))
    return ci, cf


def bound_select(q: torch.Tensor, mu: torch.Tensor, g: torch.Tensor, lz: torch.Tensor, nb: int, *, leaf: int,
                 ws=None, group: int = 1, tile: int = TILE, g0: int = 0, perm=None) -> torch.Tensor:
    """select="bound" of the bf16 and fp32 stores (h3/htrc_flat.py:255-257): q [H,N,D] (fp32 or
    bf16, query order), mu [H,ng,D], the window's g bf16 or fp32 [H,gn,nbp,D] and lz -> SEL
    [H,gn,nbp] fp32 = lz + r * ||g||, r the tile group's largest ||q - mu||."""
    q = _heads(q)
    h, nq, d = (int(x) for x in q.shape)
    tile = _tile(tile)
    gn = int(lz.shape[1])
    sel = _rows(ws, "sel", h, gn, (int(lz.shape[2]),), torch.float32, q.device)
    fn = "htrc_bound_select_f32" if g.dtype == torch.float32 else "htrc_bound_select"
    call(fn, ptr(q), int(q.dtype == torch.bfloat16), ptr(mu), ptr(g), ptr(lz), h, nq,
         int(nb) * int(leaf), int(leaf), d, tile, int(group), int(g0), gn, ptr(perm), ptr(sel), stream_handle(q.device))
    return sel


FAKE_QUANT_FMTS = {"int8": 0, "int4": 1, "fp8": 2, "fp4": 3}


def fake_quant(x: torch.Tensor, group: int, fmt: str, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., D] (fp32 or bf16, contiguous) round-tripped through ``fmt`` with one symmetric scale
    per group of ``group`` values -> out (fp32 unless given: a bf16 out, or out = x, is allowed)."""
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    d = int(x.shape[-1])
    rows = x.numel() // d if d else 0
    call("htrc_fake_quant", ptr(x), int(x.dtype == torch.bfloat16), rows, d, int(group), FAKE_QUANT_FMTS[fmt],
         ptr(out), int(out.dtype == torch.bfloat16), stream_handle(x.device))
    return out


def selftest_e4m3(codes):
    """Widen uint8 e4m3 codes (a multiple of 8) to fp16 * 2^-8 bit patterns with the kernels'
    conversion instruction and with the exact field shift -> (cvt int16 [n], bits int16 [n])."""
    dev = codes.device
    n = int(codes.numel())
    cvt = torch.empty((n,), dtype=torch.int16, device=dev)
    bits = torch.empty((n,), dtype=torch.int16, device=dev)
    call("htrc_selftest_e4m3", ptr(codes), n, ptr(cvt), ptr(bits), stream_handle(dev))
    return cvt, bits


def selftest_f32_e4m3(x):
    """e4m3 codes of fp32 values (a multiple of 4) from the stats kernel's conversion instruction
    and from the exact software rounding -> (cvt uint8 [n], soft uint8 [n])."""
    dev = x.device
    n = int(x.numel())
    cvt = torch.empty((n,), dtype=torch.uint8, device=dev)
    soft = torch.empty((n,), dtype=torch.uint8, device=dev)
    call("htrc_selftest_f32_e4m3", ptr(x), n, ptr(cvt), ptr(soft), stream_handle(dev))
    return cvt, soft


def library():
    """The loaded C-ABI library (raises when it is not built)."""
    return _lib.lib()
