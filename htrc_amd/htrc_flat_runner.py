"""Production runner of the flat-HTRC operator -- the drop-in for h3/htrc_flat_runner.py.

Same call shape as the reference:

    runner = FlatRunner(queries, keys, free_bytes=free_vram, mode="fast")
    outputs = runner.run([(head, q, k, v), ...])        # q [Q,128], k/v [K,128] on the HIP device
    runner.run(jobs, sink=lambda i, out: block_out[i].copy_(out))   # nothing retained

The operator never synchronises the host, so one HIP graph (torch.cuda.CUDAGraph on ROCm)
is captured once over static q/k/v/out buffers and replayed per call; a capture failure
falls back to eager launches and is recorded in ``graph_error``.

MI355X extension: ``heads=H`` captures H heads per replay (static buffers [H, Q, 128]);
``run`` then packs consecutive jobs H at a time, so one replay covers a whole layer and
fills the 256 CUs, instead of one head per replay as on the reference's GPU.

Memory model: ``predicted_peak_mib`` counts this implementation's workspace exactly
(packed operands, per-(tile, leaf) state, outputs, static graph copies).
"""
from __future__ import annotations

try:                                   # the memory model below must stay importable without torch
    import torch
except ImportError:                    # pragma: no cover
    torch = None

MODES = {
    "fast": dict(exact_leaves=256, order="seq", tile=64),
    "balanced": dict(exact_leaves=512, order="seq", tile=64),
    "accurate": dict(exact_leaves=1024, order="kmeans", tile=64),
    "max": dict(exact_leaves=1024, order="kmeans", tile=32),
}
# The reference's quality modes (h3/htrc_flat_runner.py:48-53), all implemented ("max" runs
# 32-row tiles).
SUPPORTED_MODES = ("fast", "balanced", "accurate", "max")
CHUNKS = (1024, 512, 256, 128, 64, 32, 16)
TILE = 64


def workspace_bytes(queries: int, keys: int, leaf: int = 16, dim: int = 128, heads: int = 1,
                    splits: int = 1, kx: int = 0, group: int = 1, order: str = "seq", tile: int = TILE) -> int:
    """Device bytes the operator's workspace holds for one call (all tiles at once); the leaf
    state and the routing hold one row per centre (ng = ceil(nt / group), nt tiles of ``tile``
    rows); order="kmeans" adds the permutation, the assignments and 32 centres."""
    tile = int(tile)
    nt = -(-int(queries) // tile)
    ng = -(-nt // max(1, int(group)))
    rows = nt * tile
    nb = int(keys) // int(leaf)
    nbp = (nb + 31) // 32 * 32
    per_head = (
        4 * ng * dim                       # mu
        + 2 * rows * dim + 8 * rows        # q8, dq8, sq, sdq
        + keys * dim + 4 * keys            # k8, ks
        + 2 * keys * dim * 2               # bf16 copies of k and v when the inputs are not bf16
        + ng * nbp * (3 * dim + 8)         # g8, vb, sg, lz
        + 4 * queries * (dim + 1)          # out, logz
        + 4 * rows                         # rowmax
        + 4 * ng * kx                      # idx (when recorded)
    )
    if splits > 1:
        per_head += nt * splits * tile * (2 + dim) * 4 + ng * nbp * 5 + 4 * ng * kx   # partials, excl, sel
    if order == "kmeans":
        per_head += 8 * int(queries) + 4 * 32 * dim                                   # perm, assign, centres
    return int(heads) * per_head


def predicted_peak_mib(keys: int, tile: int, tile_chunk: int, splits: int = 8, leaf: int = 16,
                       dim: int = 128, order: str = "seq", graph: bool = True, queries: int = 0,
                       heads: int = 1, group: int = 1) -> float:
    """Peak device MiB above the caller's q/k/v (signature of h3/htrc_flat_runner.py:61-68).
    This implementation processes every tile in one launch, so ``tile_chunk`` does not
    bound the workspace; ``queries`` (default: as many as keys) sizes it.  Graph mode adds
    the static fp32 q and bf16 k/v copies."""
    q = int(queries) if queries else int(keys)
    b = workspace_bytes(q, keys, leaf, dim, heads, splits=1, group=group, order=order, tile=tile)
    if graph:
        b += int(heads) * (4 * q * dim + 2 * 2 * int(keys) * dim)
    return b / 2 ** 20


def plan_chunk(free_bytes: int, keys: int, tile: int, splits: int = 8, order: str = "seq",
               graph: bool = True, queries: int = 0, leaf: int = 16, heads: int = 1, group: int = 1) -> int:
    """Tile chunk for the call (h3/htrc_flat_runner.py:71-82): the largest of CHUNKS when the
    whole workspace fits in ``free_bytes``; MemoryError otherwise."""
    need = predicted_peak_mib(keys, tile, CHUNKS[0], splits, leaf=leaf, order=order, graph=graph,
                              queries=queries, heads=heads, group=group)
    if need * 2 ** 20 <= free_bytes:
        return CHUNKS[0]
    raise MemoryError(f"flat HTRC needs ~{need:.0f} MiB, {int(free_bytes) >> 20} MiB free")


class FlatRunner:
    def __init__(self, queries: int, keys: int, *, free_bytes: int | None = None,
                 mode: str = "balanced", tile_chunk: int | None = None, use_graph: bool = True,
                 device="cuda", dim: int = 128, sink_leaves: int = 0, tail_rows: int = 0, heads: int = 1,
                 **overrides):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {list(MODES)}")
        from . import htrc_flat
        self.flat = htrc_flat
        self.mode = mode
        self.device = torch.device(device)
        base = dict(htrc_flat.PROD)
        base.update(MODES[mode])
        overrides = dict(overrides)
        if "kern" in overrides:                         # merge, do not replace, the kernel knobs
            base["kern"] = {**base.get("kern", {}), **overrides.pop("kern")}
        base.update(overrides)
        base["sink_leaves"] = int(sink_leaves)
        self.heads = max(1, int(heads))
        leaf = int(base.get("leaf", 16))
        group = max(1, int(base.get("kern", {}).get("group", 1)))
        if tile_chunk is None:
            if free_bytes is not None:
                tile_chunk = plan_chunk(free_bytes, keys, base["tile"], base.get("splits", 8), base["order"],
                                        use_graph, queries=int(queries), leaf=leaf, heads=self.heads, group=group)
            else:
                tile_chunk = base["tile_chunk"]
        base["tile_chunk"] = int(tile_chunk)
        self.cfg = base
        self.predicted_mib = predicted_peak_mib(keys, base["tile"], base["tile_chunk"], base.get("splits", 8),
                                                leaf=leaf, order=base["order"], graph=use_graph,
                                                queries=int(queries), heads=self.heads, group=group)
        self.queries, self.keys, self.dim = int(queries), int(keys), int(dim)
        self.tail_rows = int(tail_rows)                  # keys past the last full leaf, exact
        self._tk = self._tv = None
        self.ws = {}                                     # reusable workspace (eager path)
        self.graph = None
        self._capturing = False
        self.graph_error = None
        self._sq = self._sk = self._sv = self._so = None
        if use_graph:
            self._capture()

    def _shape(self, n):
        return (self.heads, n, self.dim) if self.heads > 1 else (n, self.dim)

    def _call(self, q, k, v, tail=None):
        if tail is None and self._tk is not None:
            tail = (self._tk, self._tv)
        ws = self.ws if self.graph is None and not self._capturing else None
        return self.flat.flat_attention(q, k, v, tail=tail, ws=ws, **self.cfg)

    def _capture(self):
        dev = self.device
        with torch.cuda.device(dev):
            self._sq = torch.zeros(self._shape(self.queries), device=dev, dtype=torch.float32)
            self._sk = torch.zeros(self._shape(self.keys), device=dev, dtype=torch.bfloat16)
            self._sv = torch.zeros_like(self._sk)
            self._sq.normal_()
            self._sk.normal_()
            self._sv.normal_()
            if self.tail_rows:
                self._tk = torch.randn(self._shape(self.tail_rows), device=dev, dtype=torch.float32)
                self._tv = torch.randn_like(self._tk)
            self._capturing = True
            try:
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side), torch.inference_mode():
                    for _ in range(2):
                        self._call(self._sq, self._sk, self._sv)
                torch.cuda.current_stream().wait_stream(side)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.inference_mode(), torch.cuda.graph(g, capture_error_mode="thread_local"):
                    self._so = self._call(self._sq, self._sk, self._sv)
                torch.cuda.synchronize()
                self.graph = g
                self._capturing = False
            except Exception as exc:  # noqa: BLE001  (fall back to eager launching)
                self.graph = None
                self._capturing = False
                self.graph_error = f"{type(exc).__name__}: {exc}"[:300]
                self._sq = self._sk = self._sv = self._so = None
                self._tk = self._tv = None
                torch.cuda.empty_cache()

    def _set_tail(self, tail):
        """Copy this call's tail into the captured static buffers (h3/htrc_flat_runner.py:162-165)."""
        if self.tail_rows and self.graph is not None:
            if tail is None:
                raise ValueError(f"this runner was captured with tail_rows={self.tail_rows}: pass tail=(tk, tv)")
            self._tk.copy_(tail[0])
            self._tv.copy_(tail[1])

    def head(self, q, k, v, tail=None):
        """One call (one head, or ``heads`` stacked heads); returns a fresh fp32 tensor.
        tail=(tk, tv) [tail_rows, D] (or [heads, tail_rows, D])."""
        if self.graph is None:      # the eager result is a view of the reused workspace: copy it
            with torch.inference_mode():
                return self._call(q, k, v, tail=tail).clone()
        self._set_tail(tail)
        self._sq.copy_(q)
        self._sk.copy_(k)
        self._sv.copy_(v)
        self.graph.replay()
        return self._so.clone()

    def _batches(self, jobs):
        if self.heads == 1:
            for i, job in enumerate(jobs):
                yield [i], job[1], job[2], job[3], (job[4] if len(job) > 4 else None)
            return
        for s in range(0, len(jobs), self.heads):
            grp = list(range(s, min(len(jobs), s + self.heads)))
            if len(grp) < self.heads:          # pad the last batch by repeating its first job
                grp_src = grp + [grp[0]] * (self.heads - len(grp))
            else:
                grp_src = grp
            q = torch.stack([jobs[i][1] for i in grp_src])
            k = torch.stack([jobs[i][2] for i in grp_src])
            v = torch.stack([jobs[i][3] for i in grp_src])
            tails = [jobs[i][4] if len(jobs[i]) > 4 else None for i in grp_src]
            if all(t is None for t in tails):
                yield grp, q, k, v, None
            elif any(t is None for t in tails):
                raise ValueError("a batch of heads needs a tail for every head or for none")
            else:
                yield grp, q, k, v, (torch.stack([t[0] for t in tails]), torch.stack([t[1] for t in tails]))

    def run(self, jobs, sink=None):
        """jobs: list of (head_index, q, k, v[, (tail_k, tail_v)]).  Outputs in job order, or
        via sink(i, output) (graph mode hands over the static output without a copy)."""
        results = [None] * len(jobs)
        for grp, q, k, v, tail in self._batches(jobs):
            if self.graph is None or sink is None:
                out = self.head(q, k, v, tail=tail)
                outs = [out] if self.heads == 1 else [out[j] for j in range(len(grp))]
            else:
                self._set_tail(tail)
                self._sq.copy_(q)
                self._sk.copy_(k)
                self._sv.copy_(v)
                self.graph.replay()
                outs = [self._so] if self.heads == 1 else [self._so[j] for j in range(len(grp))]
            for i, o in zip(grp, outs):
                if sink is None:
                    results[i] = o
                else:
                    sink(i, o)
        return results if sink is None else None

    def close(self):
        self.graph = None
        self._sq = self._sk = self._sv = self._so = None
