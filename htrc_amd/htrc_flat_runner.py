"""Production runner of the flat-HTRC operator -- the drop-in for h3/htrc_flat_runner.py.

Call shape of the reference runner (h3/htrc_flat_runner.py:85-203):

    runner = FlatRunner(queries, keys, free_bytes=free_vram, mode="fast")
    outputs = runner.run([(head, q, k, v), ...])        # q [Q,128], k/v [K,128] on the HIP device
    runner.run(jobs, sink=lambda i, out: block_out[i].copy_(out))   # nothing retained

Design on MI355X:

* ``_Plan`` resolves the quality mode and the caller's knobs into the operator's keyword
  arguments and sizes the tile window (``tile_chunk``) against ``free_bytes`` with an exact
  byte count of this implementation's workspace (``workspace_bytes``).
* ``_Replay`` owns the static input buffers, a workspace filled by one eager warm-up call, and a
  HIP graph (torch.cuda.CUDAGraph) recorded over one operator call on those buffers.  The
  operator never synchronises the host and, with its workspace already allocated, allocates
  nothing, so the recorded call is the whole layer: every tile window's statistics, routing
  and attention launches.  A failed recording leaves the runner eager and keeps the reason in
  ``graph_error``.
* ``heads=H`` (an extension) records H heads per replay (static buffers [H, Q, 128]) and
  ``run`` packs consecutive jobs H at a time, so one replay covers a whole layer on the 256
  CUs instead of one head per replay.

The memory model below imports without torch.
"""
from __future__ import annotations

import gc

try:                                   # the memory model below must stay importable without torch
    import torch
except ImportError:                    # pragma: no cover
    torch = None

# Quality modes and tile-window sizes of the reference runner (h3/htrc_flat_runner.py:48-53, 54):
# interface data, all four modes implemented ("max" runs 32-row tiles).
MODES = {
    "fast": dict(exact_leaves=256, order="seq", tile=64),
    "balanced": dict(exact_leaves=512, order="seq", tile=64),
    "accurate": dict(exact_leaves=1024, order="kmeans", tile=64),
    "max": dict(exact_leaves=1024, order="kmeans", tile=32),
}
SUPPORTED_MODES = tuple(MODES)
CHUNKS = (1024, 512, 256, 128, 64, 32, 16)
TILE = 64
MIB = 2 ** 20

# The static graph copies and the k-means scratch of this implementation at the live H3 shape of
# the reference (one head, 40759 queries and keys, h3/htrc_flat_runner.py:55-56 names the same two
# figures for its own implementation); predicted_peak_mib counts both exactly for any shape.
_H3_ROWS = 40759
STATIC_MIB = (4 * _H3_ROWS * 128 + 2 * 2 * _H3_ROWS * 128) / MIB
KMEANS_MIB = (8 * _H3_ROWS + 4 * 32 * 128) / MIB


def _ceil(a: int, b: int) -> int:
    return -(-int(a) // int(b))


# fp32-dot path: windows of at least this many (head, tile) pairs run the tile kernel unsplit
# (one 4-wave workgroup each; 2048 fill the 256 CUs eight times over), with no split partials or
# merge: cfg3's tile stage 24.4 ms with four splits and their merge, 23.1 ms unsplit.
F32_UNSPLIT_TILES = 2048


def workspace_bytes(queries: int, keys: int, leaf: int = 16, dim: int = 128, heads: int = 1, splits: int = 1,
                    kx: int = 0, group: int = 1, order: str = "seq", tile: int = TILE, tile_chunk: int | None = None,
                    store: str = "int8", fused: bool = True, bf16_inputs: bool = True, window_streams: int = 2,
                    f32dots: bool = False) -> int:
    """Device bytes of one operator call's workspace: the whole layer's packed operands and
    outputs, and the per-(centre, leaf) state, routing and partials of the tile windows of
    ``tile_chunk`` tiles (all tiles when None) in flight: one, or min(S, windows) when there are
    several windows and the operator deals them over S = kern["window_streams"] streams (2 by
    default).  ``f32dots``: the fp32-dot path (always so for store="fp32")."""
    pad = int(dim) < 128                 # head dims below 128 run at 128 on zero-padded copies
    dim = 128 if pad else int(dim)
    nt = _ceil(queries, tile)
    ng = _ceil(nt, max(1, int(group)))
    gw = ng if tile_chunk is None else max(1, min(ng, int(tile_chunk) // max(1, int(group))))
    tw = min(nt, gw * max(1, int(group)))            # tiles of a window
    rows = nt * int(tile)
    nb = int(keys) // int(leaf)
    nbp = _ceil(nb, 32) * 32
    kx = min(int(kx), nb)
    layer = 4 * ng * dim + 4 * queries * (dim + 1)                     # mu, out + logz
    if store == "int8":
        layer += 2 * rows * dim + 8 * rows + keys * dim + 4 * keys      # q8, dq8, sq, sdq, k8, ks
        per_state = 3 * dim + 8                                         # g8, vb bf16, sg, lz
    else:
        layer += 2 * 2 * rows * dim                                     # q16, dq16
        # fp8: g, vb, sg, sv, lz; bf16: g, vb, lz; fp32 (the fp32-dot path): g, vb, lz
        per_state = {"fp8": 2 * dim + 12, "bf16": 4 * dim + 4}.get(store, 8 * dim + 4)
    if pad:
        layer += 4 * queries * dim + 2 * 2 * keys * dim                 # padded copies: q (fp32), k, v (bf16)
    elif not bf16_inputs:
        layer += 2 * 2 * keys * dim                                     # bf16 copies of k and v
    window = gw * nbp * per_state + 4 * gw * kx                         # state, idx
    window += gw * (2 * 2 * dim + 16)                                   # the centres' fp16 terms
    # the fused route takes up to 8192 near leaves, and 262144 leaves per head (int8; its top-k
    # keys past 16384 in workspace) or 16384 (the 16-bit stores); larger layers run the stage path
    fused = fused and kx <= 8192 and nb <= (262144 if store == "int8" else 16384)
    if fused:
        layer += 4 * rows                                               # rowmax, shared by the windows
    if fused and nb > 16384:
        window += 4 * gw * nbp                                          # route_select top-k keys
    if not fused:
        window += gw * nbp * 5                                          # sel, excl
        unsplit = (f32dots or store == "fp32") and int(heads) * tw >= F32_UNSPLIT_TILES
        if splits > 1 and not unsplit:
            window += tw * int(splits) * int(tile) * (dim + 2) * 4      # split partials
    if order == "kmeans":
        layer += 8 * queries + 4 * 32 * dim                             # perm, assignments, centres
    if gw < ng and int(window_streams) > 1:
        window *= min(int(window_streams), _ceil(ng, gw))               # windows in flight
    return int(heads) * (layer + window)


def predicted_peak_mib(keys: int, tile: int, tile_chunk: int, splits: int = 8, leaf: int = 16, dim: int = 128,
                       order: str = "seq", graph: bool = True, queries: int = 0, heads: int = 1, group: int = 1,
                       exact_leaves: int = 256, store: str = "int8", fused: bool = True,
                       window_streams: int = 2) -> float:
    """Peak device MiB above the caller's q/k/v (the signature of h3/htrc_flat_runner.py:61-68,
    extended): the operator's workspace with a window of ``tile_chunk`` tiles, plus the static
    fp32 q and bf16 k/v copies in graph mode.  ``queries`` defaults to ``keys``."""
    q = int(queries) if queries else int(keys)
    b = workspace_bytes(q, keys, leaf, dim, heads, splits=splits, kx=exact_leaves, group=group, order=order,
                        tile=tile, tile_chunk=tile_chunk, store=store, fused=fused, window_streams=window_streams)
    if graph:
        b += int(heads) * (4 * q * dim + 2 * 2 * int(keys) * dim)
    return b / MIB


def plan_chunk(free_bytes: int, keys: int, tile: int, splits: int = 8, order: str = "seq", graph: bool = True,
               queries: int = 0, leaf: int = 16, heads: int = 1, group: int = 1, exact_leaves: int = 256,
               store: str = "int8", fused: bool = True, window_streams: int = 2, dim: int = 128) -> int:
    """The largest of CHUNKS whose predicted peak fits in ``free_bytes`` (fewer windows, fewer
    launches; h3/htrc_flat_runner.py:71-82); MemoryError when not even the smallest fits."""
    need = None
    for c in CHUNKS:
        need = predicted_peak_mib(keys, tile, c, splits, leaf=leaf, dim=dim, order=order, graph=graph,
                                  queries=queries, heads=heads, group=group, exact_leaves=exact_leaves, store=store,
                                  fused=fused, window_streams=window_streams)
        if need * MIB <= int(free_bytes):
            return c
    raise MemoryError(f"flat HTRC needs ~{need:.0f} MiB at the smallest window ({CHUNKS[-1]} tiles), "
                      f"{int(free_bytes) >> 20} MiB free")


class _Plan:
    """Operator keyword arguments of a runner: PROD, then the mode, then the caller's knobs
    (``kern`` merged key by key), then the tile window."""

    def __init__(self, flat, mode, overrides, sink_leaves, queries, keys, heads, free_bytes, tile_chunk, graph,
                 dim=128):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {list(MODES)}")
        over = dict(overrides)
        kern = {**flat.PROD.get("kern", {}), **over.pop("kern", {})}
        cfg = {**flat.PROD, **MODES[mode], **over, "kern": kern, "sink_leaves": int(sink_leaves)}
        nb = int(keys) // int(cfg.get("leaf", 16))
        kx = min(int(cfg["exact_leaves"]) + int(sink_leaves), nb)
        sizing = dict(leaf=int(cfg.get("leaf", 16)), order=cfg["order"], graph=graph, queries=int(queries),
                      heads=int(heads), group=max(1, int(kern.get("group", 1))), exact_leaves=kx,
                      store=cfg.get("store", "int8"), fused=bool(kern.get("fused", True)),
                      window_streams=int(kern.get("window_streams", 2)), dim=int(dim))
        if tile_chunk is None:
            tile_chunk = cfg["tile_chunk"] if free_bytes is None else plan_chunk(
                free_bytes, keys, cfg["tile"], cfg.get("splits", 8), **sizing)
        cfg["tile_chunk"] = int(tile_chunk)
        self.cfg = cfg
        self.mib = predicted_peak_mib(keys, cfg["tile"], cfg["tile_chunk"], cfg.get("splits", 8), **sizing)


class _Replay:
    """Static buffers, a workspace filled by one eager warm-up call, and the HIP graph recorded
    over one operator call on them.  It holds the operator call, not the runner: a runner and
    its replay form no reference cycle, so a dropped runner (its graph and memory pool with
    it) is freed at once rather than by a later garbage-collector pass."""

    def __init__(self, op, device, shape, queries: int, keys: int, tail_rows: int):
        self.op, self.device, self.tail_rows = op, device, int(tail_rows)
        gen = torch.Generator(device=device).manual_seed(0)
        # finite, well-spread warm-up data: the k-means order and the softmax see real numbers
        self.q = torch.randn(shape(queries), generator=gen, device=device, dtype=torch.float32)
        self.k = torch.randn(shape(keys), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
        self.v = torch.randn(shape(keys), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
        self.tail = None
        if tail_rows:
            self.tail = tuple(torch.randn(shape(tail_rows), generator=gen, device=device, dtype=torch.float32)
                              for _ in range(2))
        self.ws = {}
        self.out = None
        self.graph = None

    def record(self):
        """Warm up on a side stream (the workspace is allocated there, outside the recording),
        then record one call; the graph then replays on the static buffers.  The garbage
        collector runs before the recording and is off during it: a collection there could
        destroy some other dead object's graph or free its memory, which is illegal while a
        stream is being captured (torch.cuda.graph collects first only when
        torch.compiler.config.force_cudagraph_gc is set)."""
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.op(self.q, self.k, self.v, self.tail, self.ws)
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        gc.collect()
        was = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(graph, capture_error_mode="thread_local"):
                self.out = self.op(self.q, self.k, self.v, self.tail, self.ws)
        finally:
            if was:
                gc.enable()
        torch.cuda.synchronize(self.device)
        self.graph = graph

    def replay(self, q, k, v, tail):
        """Copy this call's operands into the static buffers and replay; returns the static output."""
        if self.tail is not None:
            if tail is None:
                raise ValueError(f"this runner was recorded with tail_rows={self.tail_rows}: pass tail=(tk, tv)")
            self.tail[0].copy_(tail[0])
            self.tail[1].copy_(tail[1])
        self.q.copy_(q)
        self.k.copy_(k)
        self.v.copy_(v)
        self.graph.replay()
        return self.out


class FlatRunner:
    """Flat-HTRC head runner with the reference's call surface (h3/htrc_flat_runner.py:85-203):
    ``head``, ``run``, ``close`` and the attributes ``cfg``, ``predicted_mib``, ``graph``,
    ``graph_error`` and ``ws``."""

    def __init__(self, queries: int, keys: int, *, free_bytes: int | None = None, mode: str = "balanced",
                 tile_chunk: int | None = None, use_graph: bool = True, device="cuda", dim: int = 128,
                 sink_leaves: int = 0, tail_rows: int = 0, heads: int = 1, **overrides):
        from . import htrc_flat
        self.flat = htrc_flat
        self.mode = mode
        self.heads = max(1, int(heads))
        plan = _Plan(htrc_flat, mode, overrides, sink_leaves, queries, keys, self.heads, free_bytes, tile_chunk,
                     bool(use_graph), dim=dim)
        self.cfg = plan.cfg
        self.predicted_mib = plan.mib
        self.queries, self.keys, self.dim = int(queries), int(keys), int(dim)
        self.tail_rows = int(tail_rows)
        self.device = torch.device(device)
        self.ws = {}                     # workspace of eager calls (a graph keeps its own)
        self.graph_error = None
        self._replay = None
        if use_graph:
            flat, cfg = self.flat, self.cfg
            rep = _Replay(lambda q, k, v, tail, ws: flat.flat_attention(q, k, v, tail=tail, ws=ws, **cfg),
                          self.device, self._shape, self.queries, self.keys, self.tail_rows)
            try:
                rep.record()
                self._replay = rep
            except Exception as exc:  # noqa: BLE001 -- any recording failure: run eagerly, keep the reason
                self.graph_error = f"{type(exc).__name__}: {exc}"[:300]
                del rep
                torch.cuda.empty_cache()

    @property
    def graph(self):
        return None if self._replay is None else self._replay.graph

    def _shape(self, n):
        return (self.heads, n, self.dim) if self.heads > 1 else (n, self.dim)

    def _op(self, q, k, v, tail, ws):
        return self.flat.flat_attention(q, k, v, tail=tail, ws=ws, **self.cfg)

    def _eager(self, q, k, v, tail):
        if self.tail_rows and tail is None:
            raise ValueError(f"this runner takes tail_rows={self.tail_rows}: pass tail=(tk, tv)")
        return self._op(q, k, v, tail, self.ws)

    def head(self, q, k, v, tail=None):
        """One call (one head, or ``heads`` stacked heads) -> a fresh fp32 tensor of q's shape.
        tail=(tk, tv) [tail_rows, D] (or [heads, tail_rows, D])."""
        if self._replay is None:
            return self._eager(q, k, v, tail).clone()      # the eager result lives in the workspace
        return self._replay.replay(q, k, v, tail).clone()

    def _batches(self, jobs):
        """(job indices, q, k, v, tail) per call: one job, or ``heads`` jobs stacked (the last
        batch padded with repeats of its first job, whose outputs are dropped)."""
        step = self.heads
        for s in range(0, len(jobs), step):
            ids = list(range(s, min(len(jobs), s + step)))
            if step == 1:
                j = jobs[ids[0]]
                yield ids, j[1], j[2], j[3], (j[4] if len(j) > 4 else None)
                continue
            src = ids + [ids[0]] * (step - len(ids))
            q, k, v = (torch.stack([jobs[i][n] for i in src]) for n in (1, 2, 3))
            tails = [jobs[i][4] if len(jobs[i]) > 4 else None for i in src]
            if any(t is None for t in tails) and not all(t is None for t in tails):
                raise ValueError("a batch of heads needs a tail for every head or for none")
            tail = None if tails[0] is None else tuple(torch.stack([t[n] for t in tails]) for n in (0, 1))
            yield ids, q, k, v, tail

    def run(self, jobs, sink=None):
        """jobs: list of (head_index, q, k, v[, (tail_k, tail_v)]).  Returns the outputs in job
        order (fresh tensors), or hands each to sink(i, output): there the output is the
        graph's static buffer (or the eager workspace), valid until the next call."""
        results = [None] * len(jobs)
        for ids, q, k, v, tail in self._batches(jobs):
            if sink is None:
                out = self.head(q, k, v, tail=tail)
            elif self._replay is not None:
                out = self._replay.replay(q, k, v, tail)
            else:
                out = self._eager(q, k, v, tail)
            for j, i in enumerate(ids):
                o = out if self.heads == 1 else out[j]
                if sink is None:
                    results[i] = o
                else:
                    sink(i, o)
        return results if sink is None else None

    def close(self):
        """Drop the graph, its static buffers and the eager workspace."""
        self._replay = None
        self.ws = {}
