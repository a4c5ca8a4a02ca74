"""Benchmark of the MI355X flat-HTRC layer (BASELINE configuration 3 by default).

One step = one flat-HTRC layer call: B=1, H=24, N=64512, d=128, leaf 64, 32 near leaves,
int8 Q/K + bf16 PV, on synthetic clustered video-region inputs already resident in HBM.
Prints ONE JSON line (the driver's contract) with the layer ms/call, the roofline of the
dominant kernel (HIP events on the launch stream, algorithmic bytes or ops per launch),
per-kernel figures, and the reference's CPU path timed on this host in the same run: the torch
backend _flat (h3/htrc_flat.py:279-388) restated with torch CPU ops over the whole layer, and
BASELINE configuration 1's NumPy htrc_reference (src/htrc_reference/model.py:98-137, restated).

  python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--config cfg3] [--no-cpu-baseline]

--config cfg5 is BASELINE configuration 5 instead: 50 sequential cfg2-shape calls (fresh
seeded inputs, seeds 0..49) reported as the total ms, and the ablation grid leaf
{32, 64, 128} x near leaves {16, 32, 64} x Q/K dtype {int8, bf16} with each point's log-Z
error and output rel-L2 against exact softmax attention (fp32 on the GPU).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "flat-HTRC layer ms/call @B1 H24 N64512 d128; % MFMA peak, HBM GB/s"
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, GB/s
PEAK_I8_TOPS = 5000.0          # dense int8 MFMA, TOP/s
PEAK_BF16_TFLOPS = 2500.0      # dense bf16 MFMA, TFLOP/s
PEAK_F32_TFLOPS = 157.3        # dense fp32 MFMA, TFLOP/s


def algorithmic(h, nq, nk, leaf, kx, d=128, tile=64, store="int8"):
    """Per-launch algorithmic HBM bytes and MFMA ops of every kernel of one layer call.
    Each operand is counted once per launch (near-field K/V once per head: adjacent tiles
    share leaves in L2).  Per (tile, leaf) the state is, for store="int8", g8 d + vb 2d + sg 4
    + lz 4 bytes (select reads g8, sg, lz); "fp8": g d + vb d + sg, sv, lz 12; "bf16": g 2d +
    vb 2d + lz 4 (select reads g and lz).  The int8 path's query rows are int8 + a scale (d + 4
    bytes) and its near field reads k8, ks, v (3d + 4 per token); the 16-bit paths read bf16 /
    fp16 rows (2d) and bf16 k, v (4d), and all their products are 16-bit MFMA flops."""
    nt = -(-nq // tile)
    nb = nk // leaf
    rows = nt * tile
    kx = min(kx, nb)
    i8 = store == "int8"
    per_state = {"int8": 3 * d + 8, "fp8": 2 * d + 12, "bf16": 4 * d + 4}[store]
    per_sel = {"int8": d + 8, "fp8": d + 8, "bf16": 2 * d + 4}[store]
    row = d + 4 if i8 else 2 * d
    tok = 3 * d + 4 if i8 else 4 * d
    state = nt * nb * per_state
    far_ops, near_ops = 2 * rows * nb * d, 2 * rows * kx * leaf * d

    def ops(qk):
        # the PV products match the QK products in count: int8 QK and bf16 PV on the int8
        # path, both 16-bit on the others
        return {"i8_ops": h * qk, "bf16_flops": h * qk} if i8 else {"i8_ops": 0, "bf16_flops": 2 * h * qk}

    f = {}
    f["pack_q"] = {"bytes": h * (2 * nq * d + 2 * rows * row + 4 * nt * d)}
    if i8:
        f["pack_k"] = {"bytes": h * (2 * nk * d + nk * d + 4 * nk)}
    f["stats"] = {"bytes": h * (4 * nk * d + state + 4 * nt * d)}
    f["route_select"] = {"bytes": h * (nt * nb * per_sel + rows * row + nt * kx * 4 + rows * 4),
                         **({"i8_ops": h * far_ops, "bf16_flops": 0} if i8 else {"i8_ops": 0, "bf16_flops": h * far_ops})}
    f["route_attend"] = {"bytes": h * (state + 2 * rows * row + nk * tok + nt * kx * 4 + rows * 4 + 4 * nq * (d + 1)),
                         **ops(far_ops + near_ops)}
    # the attend launch's two fields, each timed as a launch of its own: far (kx = 0: every leaf
    # through its state) and near (heads of kx * leaf keys, all kx leaves near: each tile attends
    # the same kx * leaf exact tokens as in the layer, its far field one excluded 32-leaf block)
    f["far_field"] = {"bytes": h * (state + rows * row + rows * 4 + 4 * nq * (d + 1)), **ops(far_ops)}
    f["near_field"] = {"bytes": h * (nt * kx * per_state + 2 * rows * row + kx * leaf * tok + nt * kx * 4 + rows * 4
                                     + 4 * nq * (d + 1)), **ops(near_ops)}
    return f


def algorithmic_f32(h, nq, nk, leaf, kx, d=128, tile=64, splits=4):
    """Per-launch algorithmic HBM bytes and fp32 MFMA flops of the fp32-dot path's stages (the
    reference's default store="fp32" with fp32 dots): the state per (tile, leaf) is g and vb fp32
    (8d bytes) + lz 4; q rows fp32 (4d), k / v bf16 (4d per token, once per head); the tile
    launch's far field 2 x 2d flops per row and leaf (score, PV), its near field 2 x 2d per row
    and near token; the select 2d per row and leaf."""
    nt = -(-nq // tile)
    nb = nk // leaf
    rows = nt * tile
    kx = min(kx, nb)
    state = nt * nb * (8 * d + 4)
    f = {"stats": {"bytes": h * (4 * nk * d + state + nt * (4 * d + 16))},
         "select": {"bytes": h * (nt * nb * (4 * d + 4) + 4 * nq * d + 4 * nt * d), "f32_flops": h * 2 * rows * nb * d},
         "topk": {"bytes": h * (nt * nb * 5 + nt * kx * 4)},
         "tile": {"bytes": h * (state + 4 * nq * d + 4 * nk * d + nt * nb + nt * kx * 4 + 4 * nq * (d + 1)
                                + 2 * splits * rows * (d + 2) * 4),
                  "f32_flops": h * (4 * rows * nb * d + 4 * rows * kx * leaf * d),
                  "far_flops": h * 4 * rows * nb * d, "near_flops": h * 4 * rows * kx * leaf * d}}
    if splits == 1:                                   # no split partials
        f["tile"]["bytes"] -= h * 2 * rows * (d + 2) * 4
    return f


def calib_copy(dev):
    """One copy-shaped elementwise kernel (bitwise_not over 1 GiB int32: reads 1 GiB once, writes
    1 GiB once), the scale of the FETCH_SIZE / WRITE_SIZE counters in the profiles."""
    import torch
    src = torch.empty(1 << 28, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def main_f32(a):
    """The fp32-dot path (store="fp32": the reference's default triton store, fp32 state and fp32
    dots, IEEE or TF32 operands by --precision): the layer in the reference's stage structure
    (statistics, select, top-k, split tile + merge) timed like the int8 layer, and each stage's
    launches back to back."""
    import torch
    from htrc_amd import htrc_flat, htrc_flat_hip as hip, htrc_flat_runner, workloads
    dev = torch.device("cuda:0")
    q, k, v, leaf, ex = workloads.make(a.config, seed=0, device=dev)
    h, nq, d = (int(x) for x in q.shape)
    nk = int(k.shape[1])
    nb = nk // leaf
    kx = min(ex, nb)
    prec = "tf32" if a.precision == "tf32" else "ieee"
    splits = 4
    chunk = htrc_flat_runner.plan_chunk(torch.cuda.mem_get_info(dev)[0], nk, 64, splits=splits, leaf=leaf, queries=nq,
                                        heads=h, exact_leaves=kx, graph=False, store="fp32", fused=False)
    kw = dict(backend="triton", store="fp32", dot="tf32", precision=a.precision, leaf=leaf, exact_leaves=ex,
              tile_chunk=chunk, splits=splits)
    ws = {}
    scale = 1.0 / math.sqrt(d)
    ms = None
    if not a.kernel:
        for _ in range(a.warmup):
            htrc_flat.flat_attention(q, k, v, ws=ws, **kw)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(a.steps):
            out = htrc_flat.flat_attention(q, k, v, ws=ws, **kw)
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / a.steps
        assert torch.isfinite(out).all().item(), "non-finite output"
        del out
    ws.clear()
    # stages of one window holding the whole layer (when it fits; else the first window's tiles);
    # the tile launch split as the operator splits it (unsplit for windows of many tiles)
    mu, _, _ = hip.pack_q16(q, ws=ws, dq_fp16=False)
    kb, vb = k.contiguous(), v.contiguous()
    ng = int(mu.shape[1])
    gn = min(ng, chunk)
    if h * gn >= htrc_flat_runner.F32_UNSPLIT_TILES:
        splits = 1
    g, lz, vbs, _, _ = hip.leaf_stats(mu, kb, vb, nb, scale, leaf=leaf, store=torch.float32, ws=ws, cn=gn, prec=prec)
    st = {"g8": g, "lz": lz, "vb": vbs, "sg": None, "sv": None}
    sel = hip.select_f32(q, mu, g, lz, nb, prec=prec, ws=ws)
    idx, excl = hip.topk_excl(sel, nb, kx, 0, ws=ws)
    sws = {}
    stages = {
        "stats": lambda: hip.leaf_stats(mu, kb, vb, nb, scale, leaf=leaf, store=torch.float32, ws=sws, cn=gn, prec=prec),
        "select": lambda: hip.select_f32(q, mu, g, lz, nb, prec=prec, ws=sws),
        "topk": lambda: hip.topk_excl(sel, nb, kx, 0, ws=sws),
        "tile": lambda: hip.tile_f32(q, mu, st, excl, idx, kb, vb, nq=nq, leaf=leaf, scale=scale, splits=splits, ws=sws,
                                     prec=prec),
    }
    if a.kernel:
        fn = stages[a.kernel]
        for _ in range(a.kernel_reps):
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"kernel": a.kernel, "launches": a.kernel_reps}), flush=True)
        return
    stream = torch.cuda.current_stream(dev)
    kms = {}
    for name, fn in stages.items():
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(a.kernel_reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        kms[name] = e0.elapsed_time(e1) / a.kernel_reps
    if a.calib_copy:
        calib_copy(dev)
    frac = gn / ng                                    # the stages ran over gn of the ng tiles
    figs = algorithmic_f32(h, nq, nk, leaf, kx, d, splits=splits)
    kernels = {}
    for n, t in kms.items():
        e = {"kernel": n, "ms": round(t, 4)}
        gbs = figs[n]["bytes"] * frac / (t * 1e-3) / 1e9
        e["hbm_GBps"] = round(gbs, 1)
        e["hbm_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        if "f32_flops" in figs[n]:
            tf = figs[n]["f32_flops"] * frac / (t * 1e-3) / 1e12
            e["f32_TFLOPs"] = round(tf, 2)
            e["mfma_frac"] = round(tf / PEAK_F32_TFLOPS, 4)
        kernels[n] = e
    # the tile kernel's matrix work: the far field on the fp32 MFMA; the near field on the bf16
    # MFMA, its scores with the query row in nqt bf16 terms and its PV products with the weights in
    # npt terms (each term one product of the fp32-equivalent count)
    nqt = 1 if q.dtype == torch.bfloat16 else (2 if prec == "tf32" else 3)
    npt = 2 if prec == "tf32" else 3
    ft = figs["tile"]
    ideal_s = frac * (ft["far_flops"] / (PEAK_F32_TFLOPS * 1e12)
                      + ft["near_flops"] / 2 * (nqt + npt) / (PEAK_BF16_TFLOPS * 1e12))
    dom = kernels["tile"]
    peak_eff = ft["f32_flops"] * frac / ideal_s / 1e12
    dom["mfma_frac"] = round(ideal_s / (dom["ms"] * 1e-3), 4)
    roof = {"bound": "mfma", "achieved": dom["f32_TFLOPs"], "peak": round(peak_eff, 1), "unit": "TFLOP/s",
            "frac": dom["mfma_frac"], "traffic": None, "kernel": "tile",
            "note": f"fp32-equivalent flops; peak = the kernel's mix: far field at the fp32 MFMA peak "
                    f"{PEAK_F32_TFLOPS}, near field on the bf16 MFMA ({PEAK_BF16_TFLOPS}) with the query in "
                    f"{nqt} and the weights in {npt} bf16 terms"}
    res = {"metric": f"flat-HTRC layer ms/call @B1 H{h} N{nq} d{d} ({a.config}, store=fp32, {prec} dots)",
           "value": round(ms, 4), "unit": "ms/call", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32" if prec == "ieee" else "tf32 operands, f32 accumulate",
           "data": "synthetic: clustered spatiotemporal regions, seed 0, generated on device",
           "config": {"workload": f"{a.config}: B=1 H={h} N={nq} d={d} leaf={leaf} near={kx} tile=64 store=fp32 "
                                  f"precision={a.precision} splits={splits}", "tile_chunk": chunk,
                      "stage_tiles": gn},
           "roofline": roof, "kernels": kernels}
    print(json.dumps(res), flush=True)


def measured_traffic(config, store="int8"):
    """HBM bytes per launch of each kernel, measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (scaled by a copy kernel of known size) and committed in profiles/flat_kernels_<config>.md
    (profiles/flat_kernels_<config>_<store>.md for the 16-bit stores) as a JSON block; {} when
    there is no such summary."""
    name = config if store == "int8" else f"{config}_{store}"
    path = ROOT / "profiles" / f"flat_kernels_{name}.md"
    try:
        text = path.read_text()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block).get("traffic_bytes", {})
    except (OSError, IndexError, ValueError):
        return {}


def roofline_entry(name, ms, fig):
    s = ms * 1e-3
    e = {"kernel": name, "ms": round(ms, 4)}
    gbs = fig["bytes"] / s / 1e9
    e["hbm_GBps"] = round(gbs, 1)
    e["hbm_frac"] = round(gbs / PEAK_HBM_GBS, 4)
    t_hbm = fig["bytes"] / (PEAK_HBM_GBS * 1e9)
    t_mfma = 0.0
    if "i8_ops" in fig:
        t_mfma = fig["i8_ops"] / (PEAK_I8_TOPS * 1e12) + fig["bf16_flops"] / (PEAK_BF16_TFLOPS * 1e12)
        e["mfma_frac"] = round(t_mfma / s, 4)
    e["bound"] = "mfma" if t_mfma > t_hbm else "hbm"
    e["ideal_ms"] = round(max(t_hbm, t_mfma) * 1e3, 4)
    return e


def measured_peaks(dev, reps=5):
    """Rates torch reaches on this GPU, beside the spec peaks, as tools/profile_flat_kernel.py:43-65
    measures them for the reference: a device copy of 1 GiB (torch's copy_; read + write bytes /
    time), an elementwise pass over 1 GiB (bitwise_not: the same bytes through torch's
    elementwise kernel), a fill of 2 GiB (write only), a bf16 GEMM 8192^3 (torch.matmul,
    hipBLASLt), the skinny batched product of the tile kernel's shape (640 x [64,128] @
    [128,2560], bf16), and an int8 GEMM 8192^3 (torch._int_mm) for this path's QK dtype; None
    for a rate this torch build cannot produce.  stream_GBps, the fastest of the three
    streaming rates, is the measured HBM ceiling the kernels' hbm_frac_measured is taken
    against."""
    import torch

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    res = {}
    src = torch.empty(1 << 28, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    res["copy_GBps"] = round(2 * src.numel() * 4 / timed(lambda: dst.copy_(src)) / 1e9, 1)
    res["elementwise_GBps"] = round(2 * src.numel() * 4 / timed(lambda: torch.bitwise_not(src, out=dst)) / 1e9, 1)
    del src, dst
    big = torch.empty(1 << 29, dtype=torch.int32, device=dev)
    res["fill_GBps"] = round(big.numel() * 4 / timed(lambda: big.fill_(3)) / 1e9, 1)
    del big
    res["stream_GBps"] = max(res["copy_GBps"], res["elementwise_GBps"], res["fill_GBps"])
    n = 8192
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    res["bf16_gemm_TFLOPs"] = round(2 * n ** 3 / timed(lambda: torch.matmul(a, b)) / 1e12, 1)
    del a, b
    qs = torch.randn(640, 64, 128, device=dev, dtype=torch.bfloat16)
    ks = torch.randn(640, 128, 2560, device=dev, dtype=torch.bfloat16)    # contiguous right operand
    res["bmm_64x128x2560_TFLOPs"] = round(2 * 640 * 64 * 128 * 2560 / timed(lambda: torch.bmm(qs, ks)) / 1e12, 1)
    del qs, ks
    try:
        a8 = torch.randint(-127, 128, (n, n), device=dev, dtype=torch.int8)
        b8 = torch.randint(-127, 128, (n, n), device=dev, dtype=torch.int8)
        res["int8_gemm_TOPs"] = round(2 * n ** 3 / timed(lambda: torch._int_mm(a8, b8)) / 1e12, 1)
        del a8, b8
    except (RuntimeError, AttributeError, NotImplementedError) as err:
        res["int8_gemm_TOPs"] = None
        res["int8_gemm_error"] = str(err).splitlines()[0][:200]
    torch.cuda.empty_cache()
    res["cu_count"] = torch.cuda.get_device_properties(dev).multi_processor_count
    return res


def _cpu_info():
    """(BLAS threads, CPU model) of this host."""
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001 -- threadpoolctl absent or failing: report the visible CPUs
        threads = os.cpu_count() or 1
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return int(threads), model


def cpu_flat_layer(name, heads=None):
    """The reference's CPU operator, its torch backend _flat (h3/htrc_flat.py:279-388), restated
    with torch ops on CPU tensors (oracle/flat_torch.py) and run with torch's threads on every
    CPU of this host, over the configuration's heads, one pass -> (ms for the heads, heads,
    torch threads)."""
    import torch
    from htrc_amd import workloads
    from oracle import flat_torch
    gen, kw, leaf, ex, h0 = workloads.CONFIGS[name]
    heads = h0 if heads is None else heads
    torch.set_num_threads(os.cpu_count() or 1)
    elapsed = 0.0
    for h in range(heads):
        q, k, v, _, _ = workloads.make(name, seed=1000 + h, heads=1)
        qf, kf, vf = (x[0].float() for x in (q, k, v))
        if h == 0:          # one warm window (thread pool, page faults) outside the timing
            flat_torch.flat_torch(qf, kf, vf, tile=64, leaf=leaf, exact_leaves=ex, tile_chunk=32, tiles=slice(0, 32))
        t0 = time.perf_counter()
        flat_torch.flat_torch(qf, kf, vf, tile=64, leaf=leaf, exact_leaves=ex, tile_chunk=32)
        elapsed += time.perf_counter() - t0
    return elapsed * 1e3, heads, torch.get_num_threads()


def cpu_reference_cfg1():
    """the NumPy float64 htrc_reference (src/htrc_reference/model.py:98-137,
    restated) over all 1024 queries, 4096 keys, d = 64, leaves of 64, fanout 4 -> (ms, errors)."""
    from oracle import htrc_ref
    t0 = time.perf_counter()
    res = htrc_ref.config1(seed=0)
    return (time.perf_counter() - t0) * 1e3, res


def cpu_baseline(name, heads=None):
    """The reference's CPU path timed on this host in the same run: the flat operator (_flat) over
    the whole layer of configuration ``name`` (all heads unless ``heads`` is given, then scaled
    to the layer), and configuration 1's NumPy htrc_reference."""
    from htrc_amd import workloads
    h_layer = workloads.CONFIGS[name][4]
    threads, model = _cpu_info()
    ms, done, torch_threads = cpu_flat_layer(name, heads)
    layer_ms = ms * h_layer / done
    ref_ms, ref = cpu_reference_cfg1()
    sample = (f"one full pass over all {h_layer} heads" if done == h_layer else
              f"{done} of {h_layer} heads ({ms / 1e3:.1f} s), scaled x{h_layer / done:.2f}")
    return {"value": round(layer_ms, 1), "unit": "ms/call", "cores": torch_threads, "kind": "port",
            "sample": f"{sample}; the torch backend _flat (h3/htrc_flat.py:279-388) restated with torch CPU ops "
                      f"(oracle/flat_torch.py), fp32, tile_chunk 32, torch.get_num_threads() = {torch_threads}",
            "cpu": model, "os_cpu_count": os.cpu_count(), "torch_threads": torch_threads,
            "htrc_reference_cfg1": {"value": round(ref_ms, 1), "unit": "ms (1024 queries)", "cores": threads,
                                    "kind": "port",
                                    "sample": "BASELINE configuration 1 whole: NumPy float64 htrc_reference "
                                              "(src/htrc_reference/model.py:98-137, restated), 1024 queries x "
                                              "4096 keys, d=64, leaves of 64, fanout 4",
                                    "rel_l2_median": round(ref["rel_l2_median"], 4),
                                    "logz_abs_max": round(ref["logz_abs_max"], 4)}}


def near_field_launch(q, k, v, leaf, kx, scale, store):
    """The attend launch whose work is the layer's near field: the same heads and queries against
    heads of the first kx * leaf keys, every one of the kx leaves near, so each tile attends kx *
    leaf exact tokens (int8 QK and bf16 PV on the int8 store) as it does in the layer, with a far
    field of one excluded 32-leaf block -> the launch, its operands prepared."""
    import torch
    from htrc_amd import htrc_flat_hip as hip
    nq = int(q.shape[1])
    kn, vn = (x[:, :kx * leaf].contiguous() for x in (k, v))
    ws = {}
    if store == "int8":
        mu, q8, sq, dq8, sdq = hip.pack_q(q, ws=ws)
        k8, ks = hip.pack_k(kn, ws=ws)
        g8, lz, vbs, sg, _ = hip.leaf_stats(mu, kn, vn, kx, scale, leaf=leaf, ws=ws)
        packed = {"q8": q8, "sq": sq, "dq8": dq8, "sdq": sdq, "k8": k8, "ks": ks, "v": vn}
        lstate = {"g8": g8, "sg": sg, "lz": lz, "vb": vbs}
        sel, att = hip.route_select, hip.route_attend
    else:
        sdt = torch.float8_e4m3fn if store == "fp8" else torch.bfloat16
        mu, q16, dq16 = hip.pack_q16(q, ws=ws, dq_fp16=store == "fp8")
        g, lz, vbs, sg, sv = hip.leaf_stats(mu, kn, vn, kx, scale, leaf=leaf, store=sdt, ws=ws)
        packed = {"q16": q16, "dq16": dq16, "k": kn, "v": vn}
        lstate = {"g8": g, "sg": sg, "lz": lz, "vb": vbs, "sv": sv}
        sel, att = hip.route16_select, hip.route16_attend
    idx, rowmax = sel(packed, lstate, nq=nq, leaf=leaf, kx=kx, ws=ws)
    return lambda: att(packed, lstate, idx, rowmax, nq=nq, leaf=leaf, kx=kx, scale=scale, ws=ws)


def exact_attention(q, k, v, scale, chunk=4096):
    """Exact softmax attention of one head in fp32 on the GPU -> (out [N, d], logZ [N])."""
    import torch
    kt = k.float().t().contiguous()
    vf = v.float().contiguous()
    outs, lzs = [], []
    for r0 in range(0, q.shape[0], chunk):
        s_ = torch.matmul(q[r0:r0 + chunk].float().contiguous(), kt) * scale
        lz = torch.logsumexp(s_, dim=1)
        outs.append(torch.matmul(torch.exp(s_ - lz[:, None]), vf))
        lzs.append(lz)
    return torch.cat(outs), torch.cat(lzs)


def sweep_cfg5(calls=50, warmup=2, leaves=(32, 64, 128), nears=(16, 32, 64), stores=("int8", "bf16"), reps=5):
    """`calls` sequential cfg2-shape layer calls on fresh seeded inputs
    (total ms) and the ablation grid, each point's error against exact softmax attention.  Every
    call runs the layer in one tile window (tile_chunk 1024), as the reference's own sweep sets
    it (tools/sweep_h3_flat_kernels.py:244)."""
    import torch
    from htrc_amd import htrc_flat, workloads
    dev = torch.device("cuda:0")
    data = [workloads.make("cfg2", seed=s, device=dev) for s in range(calls)]
    _, _, _, leaf0, ex0 = data[0]
    kw = dict(backend="hip", store="int8", dot="bf16", leaf=leaf0, exact_leaves=ex0, tile_chunk=1024)
    ws = {}
    for j in range(warmup):
        q, k, v = data[j % calls][:3]
        htrc_flat.flat_attention(q[0], k[0], v[0], ws=ws, **kw)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for q, k, v, _, _ in data:
        htrc_flat.flat_attention(q[0], k[0], v[0], ws=ws, **kw)
    e1.record()
    torch.cuda.synchronize()
    total = e0.elapsed_time(e1)
    q, k, v = (x[0] for x in data[0][:3])
    scale = 1.0 / math.sqrt(q.shape[-1])
    ref_out, ref_lz = exact_attention(q, k, v, scale)
    grid = []
    for leaf in leaves:
        for near in nears:
            for store in stores:
                kwp = dict(backend="hip", store=store, dot="bf16", leaf=leaf, exact_leaves=near, tile_chunk=1024)
                wsp = {}
                out, lz = htrc_flat.flat_attention(q, k, v, ws=wsp, return_logz=True, **kwp)
                a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a0.record()
                for _ in range(reps):
                    htrc_flat.flat_attention(q, k, v, ws=wsp, **kwp)
                a1.record()
                torch.cuda.synchronize()
                err = (lz - ref_lz).abs()
                grid.append({"leaf": leaf, "near_leaves": near, "qk": store, "ms": round(a0.elapsed_time(a1) / reps, 4),
                             "logz_err_max": round(float(err.max()), 6), "logz_err_mean": round(float(err.mean()), 6),
                             "out_rel_l2": round(float((out - ref_out).norm() / ref_out.norm()), 6)})
    return total, grid


def main_cfg5(a):
    total, grid = sweep_cfg5(calls=a.calls)
    res = {"metric": f"cfg5: {a.calls} sequential cfg2-shape flat-HTRC calls (seeds 0..{a.calls - 1}), total ms",
           "value": round(total, 3), "unit": "ms", "n_gpus": 1, "steps": a.calls, "warmup": 2,
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "i8/bf16 (fp32 accumulate)",
           "data": "synthetic: clustered 64-token runs (cfg2 generator), seeds 0..49, generated on device",
           "config": {"workload": f"cfg5: B=1 H=1 N=16384 d=128 leaf=64 near=16 tile=64, {a.calls} calls"},
           "ablation": grid}
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3", choices=["cfg2", "cfg3", "cfg4", "cfg5"])
    ap.add_argument("--store", default="int8", choices=["int8", "fp8", "bf16", "fp32"],
                    help="leaf-state store of the layer (BASELINE's metric is quoted on int8); fp32: the "
                         "reference's default fp32-dot path, timed in its stage structure")
    ap.add_argument("--precision", default="fp32", choices=["fp32", "tf32"],
                    help="--store fp32: IEEE fp32 (the reference's default) or TF32 dot operands")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--calls", type=int, default=50, help="cfg5: sequential layer calls")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=None,
                    help="heads of the CPU baseline pass (default: the whole layer)")
    ap.add_argument("--kernel", default=None,
                    choices=["pack_q", "pack_k", "stats", "route_select", "route_attend", "far_field", "near_field",
                             "select", "topk", "tile"],
                    help="run only this stage's launches (--kernel-reps of them), for rocprofv3 counter passes")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also launch one copy-shaped 1 GiB kernel (the scale of the FETCH_SIZE/WRITE_SIZE counters)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {a.gpus}); heads shard across GPUs "
              "without communication, so multi-GPU figures are not produced", file=sys.stderr)
        sys.exit(2)

    import torch
    from htrc_amd import htrc_flat, htrc_flat_hip as hip, htrc_flat_runner, workloads

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if a.config == "cfg5":
        return main_cfg5(a)
    if a.store == "fp32":
        return main_f32(a)
    dev = torch.device("cuda:0")
    q, k, v, leaf, ex = workloads.make(a.config, seed=0, device=dev)
    h, nq, d = (int(x) for x in q.shape)
    nk = int(k.shape[1])
    nb = nk // leaf
    kx = min(ex, nb)
    ws = {}
    # the tile window the production runner plans for this layer and the free device memory
    # (h3/htrc_flat_runner.py:71-82): the whole layer in one window when it fits
    chunk = htrc_flat_runner.plan_chunk(torch.cuda.mem_get_info(dev)[0], nk, 64, leaf=leaf, queries=nq, heads=h,
                                        exact_leaves=kx, graph=False, store=a.store)
    store = a.store
    kw = dict(backend="hip", store=store, dot="bf16", leaf=leaf, exact_leaves=ex, tile_chunk=chunk,
              kern={"fused": True})

    def layer_ms(kwargs, steps, warmup):
        for _ in range(warmup):
            htrc_flat.flat_attention(q, k, v, ws=ws, **kwargs)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            res = htrc_flat.flat_attention(q, k, v, ws=ws, **kwargs)
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / steps, res

    ms = ms_prod_windows = None
    if not a.kernel:
        ms, out = layer_ms(kw, a.steps, a.warmup)
        assert torch.isfinite(out).all().item(), "non-finite output"
        del out
    # the same layer in the reference PROD's tile windows (tile_chunk 128): the memory-bounded mode
    # (two warm-up calls: the first calls after the window buffers are allocated run slower,
    # measured 8.27 against 8.04 ms at cfg3)
    if not a.kernel:
        ms_prod_windows, _ = layer_ms({**kw, "tile_chunk": htrc_flat.PROD["tile_chunk"]}, max(5, a.steps // 2), 2)
    # the same layer at PROD's precision="tf32": the leaf statistics on TF32 operands, as the
    # reference's PROD computes them (the value above keeps the default IEEE fp32 statistics)
    ms_tf32 = None
    if not a.kernel:
        ms_tf32, _ = layer_ms({**kw, "precision": "tf32"}, max(5, a.steps // 2), 2)
    ws.clear()

    # per-kernel launch durations, HIP events on the stream the kernels are launched on
    scale = 1.0 / math.sqrt(d)
    if store == "int8":
        mu, q8, sq, dq8, sdq = hip.pack_q(q, ws=ws)
        k8, ks = hip.pack_k(k, ws=ws)
        g8, lz, vbs, sg, _ = hip.leaf_stats(mu, k, v, nb, scale, leaf=leaf, ws=ws)
        packed = {"q8": q8, "sq": sq, "dq8": dq8, "sdq": sdq, "k8": k8, "ks": ks, "v": v}
        lstate = {"g8": g8, "sg": sg, "lz": lz, "vb": vbs}
        sel, att = hip.route_select, hip.route_attend
        stages = {"pack_q": lambda: hip.pack_q(q, ws=ws), "pack_k": lambda: hip.pack_k(k, ws=ws),
                  "stats": lambda: hip.leaf_stats(mu, k, v, nb, scale, leaf=leaf, ws=ws)}
    else:
        sdt = torch.float8_e4m3fn if store == "fp8" else torch.bfloat16
        mu, q16, dq16 = hip.pack_q16(q, ws=ws, dq_fp16=store == "fp8")
        g, lz, vbs, sg, sv = hip.leaf_stats(mu, k, v, nb, scale, leaf=leaf, store=sdt, ws=ws)
        packed = {"q16": q16, "dq16": dq16, "k": k, "v": v}
        lstate = {"g8": g, "sg": sg, "lz": lz, "vb": vbs, "sv": sv}
        sel, att = hip.route16_select, hip.route16_attend
        stages = {"pack_q": lambda: hip.pack_q16(q, ws=ws, dq_fp16=store == "fp8"),
                  "stats": lambda: hip.leaf_stats(mu, k, v, nb, scale, leaf=leaf, store=sdt, ws=ws)}
    idx, rowmax = sel(packed, lstate, nq=nq, leaf=leaf, kx=kx, ws=ws)
    near = near_field_launch(q, k, v, leaf, kx, scale, store)
    stages.update({
        "route_select": lambda: sel(packed, lstate, nq=nq, leaf=leaf, kx=kx, ws=ws),
        "route_attend": lambda: att(packed, lstate, idx, rowmax, nq=nq, leaf=leaf, kx=kx, scale=scale, ws=ws),
        # the attend launch with no near leaves: the far field alone
        "far_field": lambda: att(packed, lstate, None, rowmax, nq=nq, leaf=leaf, kx=0, scale=scale, ws=ws),
        # the attend launch on heads of kx * leaf keys, every leaf near: the near field alone
        "near_field": near,
    })
    if a.kernel:
        # profiling passes (rocprofv3 --pmc): one stage's launches only, nothing else timed
        fn = stages[a.kernel]
        for _ in range(a.kernel_reps):
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"kernel": a.kernel, "launches": a.kernel_reps}), flush=True)
        return
    kms = {}
    stream = torch.cuda.current_stream(dev)
    for name, fn in stages.items():
        # --kernel-reps launches back to back between two events, as the launches of a layer
        # call follow each other: one launch between an event and a host sync would also count
        # the host's launch latency and the idle GPU's clock ramp (pack_q: 0.150 against
        # 0.138 ms per launch)
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(a.kernel_reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        kms[name] = e0.elapsed_time(e1) / a.kernel_reps
    if a.calib_copy:
        calib_copy(dev)
    figs = algorithmic(h, nq, nk, leaf, kx, d, store=store)
    kernels = {n: roofline_entry(n, kms[n], figs[n]) for n in stages}
    peaks = measured_peaks(dev)
    for n, e in kernels.items():        # the same figures against the measured rates
        e["hbm_frac_measured"] = round(e["hbm_GBps"] / peaks["stream_GBps"], 4)
        if "mfma_frac" in e and peaks.get("int8_gemm_TOPs"):
            t = figs[n]["i8_ops"] / (peaks["int8_gemm_TOPs"] * 1e12) + figs[n]["bf16_flops"] / (
                peaks["bf16_gemm_TFLOPs"] * 1e12)
            e["mfma_frac_measured"] = round(t / (e["ms"] * 1e-3), 4)
    traffic = measured_traffic(a.config, store)
    for n, e in kernels.items():
        e["traffic"] = traffic.get(n)
    dom = max((e for n, e in kernels.items() if n not in ("far_field", "near_field")), key=lambda e: e["ms"])
    fig = figs[dom["kernel"]]
    if dom["bound"] == "hbm":
        ach = fig["bytes"] / (dom["ms"] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic.get(dom["kernel"]), "kernel": dom["kernel"],
                "algorithmic_bytes": fig["bytes"]}
    else:
        # bf16-equivalent rate: an int8 op costs half a bf16 flop at the MI355X dense peaks
        ach = (fig["bf16_flops"] + fig["i8_ops"] * PEAK_BF16_TFLOPS / PEAK_I8_TOPS) / (dom["ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic.get(dom["kernel"]),
                "kernel": dom["kernel"], "note": "bf16-equivalent: int8 ops weighted by 2.5/5.0"}
    if roof["bound"] == "hbm":
        roof["measured_peak"] = peaks["stream_GBps"]
        roof["frac_measured"] = dom["hbm_frac_measured"]
    elif "mfma_frac_measured" in dom:
        roof["frac_measured"] = dom["mfma_frac_measured"]
    # BASELINE's metric is quoted on cfg3; the other layer configurations carry their own shape
    tag = a.config if store == "int8" else f"{a.config}, store={store}"
    metric = (METRIC if tag == "cfg3" else
              f"flat-HTRC layer ms/call @B1 H{h} N{nq} d{d} ({tag}); % MFMA peak, HBM GB/s")
    dtype = {"int8": "i8/bf16 (fp32 accumulate)", "fp8": "e4m3 state, fp16/bf16 MFMA (fp32 accumulate)",
             "bf16": "bf16 (fp32 accumulate)"}[store]
    res = {"metric": metric, "value": round(ms, 4), "unit": "ms/call", "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype,
           "data": "synthetic: clustered spatiotemporal regions, seed 0, generated on device",
           "config": {"workload": f"{a.config}: B=1 H={h} N={nq} d={d} leaf={leaf} near={kx} tile=64 store={store}",
                      "heads": h, "queries": nq, "keys": nk, "leaf": leaf, "near_leaves": kx, "tile_chunk": chunk,
                      "store": store},
           "ms_tile_chunk_128": round(ms_prod_windows, 4),
           "ms_precision_tf32": round(ms_tf32, 4),
           "roofline": roof, "kernels": kernels, "measured_peaks": peaks}
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(a.config, a.cpu_heads)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
