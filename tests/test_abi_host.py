"""CPU checks of the drop-in boundary: the C-ABI library loads and exports every entry point
include/htrc_flat.h declares, its launchers reject bad arguments on the host (without
touching a GPU), and the Python surface mirrors the reference's knobs, errors and memory
planning (h3/htrc_flat.py:99-139, h3/htrc_flat_runner.py:48-203).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from htrc_amd import _lib, htrc_flat, htrc_flat_hip, htrc_flat_runner
from oracle import flat_i8

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "htrc_flat.h"


def _declared():
    text = HEADER.read_text()
    names = re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(htrc_\w+)\s*\(", text, flags=re.M)
    return names, text


def test_library_exports_every_declared_symbol():
    names, text = _declared()
    assert len(names) >= 11
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), f"{n} declared in {HEADER.name} but not exported"
        assert n in _lib.signatures(), f"{n} has no ctypes signature"
    ver = int(re.search(r"#define HTRC_ABI_VERSION (\d+)", text).group(1))
    assert lib.htrc_abi_version() == ver == _lib.ABI_VERSION


def test_nb_pad():
    lib = _lib.lib()
    for nb, want in ((1, 32), (32, 32), (33, 64), (1008, 1024), (1953, 1984)):
        assert lib.htrc_nb_pad(nb) == want == _lib.nb_pad(nb)


_FAKE = ctypes.c_void_p(256)   # never dereferenced: validation fails before any launch


@pytest.mark.parametrize("case", ["null", "dim", "leaf", "block", "leaves", "near", "group", "tile", "stride",
                                  "window", "centres", "keys_ws", "merge", "route16_leaves", "route16_null"])
def test_launchers_reject_bad_arguments_on_host(case):
    lib = _lib.lib()
    f = _FAKE
    if case == "null":
        rc = lib.htrc_pack_q(None, 1, 1, 64, 128, 64, 1, None, f, f, f, f, f, None)
        msg = "null"
    elif case == "dim":
        rc = lib.htrc_pack_k(f, 1, 64, 64, f, f, None)
        msg = "128"
    elif case == "leaf":
        rc = lib.htrc_leaf_stats(f, f, f, 1, 1, 0, 1, 96, 48, 128, 0.1, f, f, f, f, None)
        msg = "leaf"
    elif case == "block":
        rc = lib.htrc_tile(*([f] * 13), 1, 64, 128, 64, 128, 1, 64, 1, 0, 1, None, 4, 48, 0.1, f, f, f, f, f, None)
        msg = "multiple of 32"
    elif case == "leaves":                        # exclusion bits of more than 262144 leaves exceed the LDS
        rc = lib.htrc_route(*([f] * 11), 1, 64, 64 * 300000, 64, 128, 4, 0, 1, 64, 1, 0, 1, None, 0.1, f, f, f, f, f,
                            None)
        msg = "262144"
    elif case == "near":                          # the fused route holds at most 8192 near leaves per tile
        rc = lib.htrc_route(*([f] * 11), 1, 64, 16 * 20000, 16, 128, 9000, 0, 1, 64, 1, 0, 1, None, 0.1, f, f, f, f,
                            f, None)
        msg = "8192 near"
    elif case == "group":
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 640, 64, 128, 4, 0, 1, 64, 0, 0, 1, f, f, None, None)
        msg = "group"
    elif case == "tile":
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 640, 64, 128, 4, 0, 1, 48, 1, 0, 1, f, f, None, None)
        msg = "32 or 64"
    elif case == "stride":                        # stride must divide a 32-row tile
        rc = lib.htrc_select(*([f] * 5), 1, 10, 20, 64, 32, 1, 0, 10, 128, f, None)
        msg = "divide"
    elif case == "window":                        # groups [5, 15) of a head of 10 tiles
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 640, 64, 128, 4, 0, 1, 64, 1, 5, 10, f, f, None, None)
        msg = "window"
    elif case == "centres":                       # centres [2, 4) of 3
        rc = lib.htrc_leaf_stats(f, f, f, 1, 3, 2, 2, 128, 64, 128, 0.1, f, f, f, f, None)
        msg = "window"
    elif case == "keys_ws":                       # above 16384 leaves per head the top-k keys need keys_ws
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 16 * 20000, 16, 128, 4, 0, 1, 64, 1, 0, 10, f, f, None, None)
        msg = "keys_ws"
    elif case == "route16_leaves":                # the 16-bit route keeps its top-k keys in LDS
        rc = lib.htrc_route16(*([f] * 9), 1, 640, 16 * 20000, 16, 128, 4, 0, 1, 64, 1, 0, 10, None, 1, 0.1, f, f, f,
                              f, None)
        msg = "16384"
    elif case == "route16_null":                  # the fp8 store needs its row scales
        rc = lib.htrc_route16(f, f, f, None, f, f, None, f, f, 1, 640, 640, 64, 128, 4, 0, 1, 64, 1, 0, 10, None, 1,
                              0.1, f, f, f, f, None)
        msg = "null"
    else:                                         # tiles [8, 12) of a head of 10
        rc = lib.htrc_merge(f, f, f, 1, 640, 64, 8, 4, 4, 128, None, f, f, None)
        msg = "window"
    assert rc == 1
    assert msg in lib.htrc_last_error().decode()


def test_header_signatures_parse():
    """The ctypes binding is read from the header: pointers, int64_t, int and float parameters."""
    sig = _lib.parse_header("""/* c */ int htrc_x(const float* a, int64_t n, int k, float s, void* st);
                               const char* htrc_y(void);""")
    assert sig["htrc_x"][0] == [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
    assert sig["htrc_y"] == ([], ctypes.c_char_p)
    assert len(_lib.signatures()["htrc_route"][0]) == 31
    assert len(_lib.signatures()["htrc_route16"][0]) == 29


def test_call_maps_errors_to_value_error():
    with pytest.raises(ValueError, match="null"):
        _lib.call("htrc_pack_q", None, 1, 1, 64, 128, 64, 1, None, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, None)


def test_split_and_buf_match_reference_semantics():
    for n in (0, 1, 37, 1008, 2048, 4096):
        for ns in (1, 2, 3, 4, 8):
            for bn in (32, 64, 128):
                assert htrc_flat_hip._split(n, ns, bn) == flat_i8.split(n, ns, bn)
    ws = {}
    a = htrc_flat_hip._buf(ws, "x", (8, 4), torch.float32, "cpu")
    b = htrc_flat_hip._buf(ws, "x", (5, 4), torch.float32, "cpu")
    assert b.data_ptr() == a.data_ptr() and b.shape == (5, 4)
    c = htrc_flat_hip._buf(ws, "x", (9, 4), torch.float32, "cpu")
    assert c.shape == (9, 4) and ws["x"].data_ptr() == c.data_ptr() and ws["x"].shape == (9, 4)


def _qkv(n=128, m=128, d=128):
    return torch.randn(n, d), torch.randn(m, d), torch.randn(m, d)


@pytest.mark.parametrize("over,match", [
    ({"backend": "torch"}, "not part of this build"),
    ({"store": "fp32"}, "int8"),
    ({"dot": "tf32"}, "int8"),
    ({"curvature": "iso"}, "curvature"),
    ({"select": "bound"}, "select"),
    ({"order": "hilbert"}, "order"),
    ({"tile": 16}, "tile=64 or tile=32"),
    ({"tile": 32, "sel_stride": 64}, "divide the tile"),
    ({"leaf": 48}, "leaf"),
    ({"quant": {"q": "int8"}}, "quant"),
    ({"kern": {"group": 2000}}, "group"),
])
def test_flat_attention_rejects_unimplemented_knobs(over, match):
    q, k, v = _qkv()
    kw = dict(htrc_flat.PROD, leaf=16)
    kw.update(over)
    with pytest.raises(ValueError, match=match):
        htrc_flat.flat_attention(q, k, v, **kw)


def test_flat_attention_shape_errors_and_no_cpu_fallback():
    q, k, v = _qkv(m=100)
    with pytest.raises(ValueError, match="multiple of the leaf"):
        htrc_flat.flat_attention_prod(q, k, v, leaf=16)
    q, k, v = _qkv(d=256)
    with pytest.raises(ValueError, match="at most 128"):
        htrc_flat.flat_attention_prod(q, k, v)
    q, k, v = _qkv(d=64)
    with pytest.raises(ValueError, match="same for q and k"):
        htrc_flat.flat_attention_prod(q[:, :32], k, v)
    q, k, v = _qkv()
    with pytest.raises(ValueError, match="HIP device"):      # CPU tensors never fall back to a CPU path
        htrc_flat.flat_attention_prod(q, k, v, leaf=16, exact_leaves=2)


def test_missing_library_raises_instead_of_falling_back(monkeypatch, tmp_path):
    """Without the built library every launcher raises: there is no CPU or torch path to take."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIBPATH", tmp_path / "libhtrc_flat.so")
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()
    with pytest.raises(RuntimeError, match="not built"):
        _lib.call("htrc_abi_version")


def test_prod_knobs_match_reference():
    assert htrc_flat.PROD == dict(tile=64, exact_leaves=256, tile_chunk=128, backend="triton", precision="tf32",
                                  store="int8", dot="bf16", splits=4,
                                  kern=dict(tile_warps=4, tile_bn=64, tile_stages=2))


def test_runner_modes_and_memory_model():
    assert set(htrc_flat_runner.MODES) == {"fast", "balanced", "accurate", "max"}
    assert htrc_flat_runner.CHUNKS == (1024, 512, 256, 128, 64, 32, 16)
    mib = htrc_flat_runner.predicted_peak_mib(64512, 64, 1024, leaf=64, queries=64512, heads=24, exact_leaves=32)
    # cfg3 layer in one window: per-(tile, leaf) state dominates: 24 * 1008 * 1024 * 392 B = 9252 MiB
    assert 9252 < mib < 16000
    assert htrc_flat_runner.plan_chunk(64 << 30, 64512, 64, leaf=64, queries=64512, heads=24) == 1024
    # windows bound the state, two windows of it in flight (the operator alternates them over two
    # streams): 3.5 GiB takes windows of 32 tiles (~3.4 GiB), 64 tiles need ~4.0 GiB; with one in
    # flight (kern["window_streams"] = 1) 64 tiles fit
    c = htrc_flat_runner.plan_chunk(3584 << 20, 64512, 64, leaf=64, queries=64512, heads=24, exact_leaves=32)
    assert c == 32
    assert htrc_flat_runner.predicted_peak_mib(64512, 64, 64, leaf=64, queries=64512, heads=24,
                                               exact_leaves=32) > 3584
    assert htrc_flat_runner.plan_chunk(3584 << 20, 64512, 64, leaf=64, queries=64512, heads=24, exact_leaves=32,
                                       window_streams=1) == 64
    with pytest.raises(MemoryError):             # the layer's operands and outputs alone need ~3 GiB
        htrc_flat_runner.plan_chunk(1 << 30, 64512, 64, leaf=64, queries=64512, heads=24)
    # the window state scales with the window: 1024 tiles (1008 real, one window) against two
    # windows of 128 in flight at cfg3
    m128 = htrc_flat_runner.predicted_peak_mib(64512, 64, 128, leaf=64, queries=64512, heads=24, exact_leaves=32)
    assert mib - m128 == pytest.approx(24 * (1008 - 2 * 128) * (1024 * 392 + 4 * 32 + 528) / 2 ** 20, rel=1e-6)
    # S window streams keep min(S, windows) windows in flight: three of 128 tiles, and no more
    # than the two windows of 512 tiles there are
    per = 24 * 128 * (1024 * 392 + 4 * 32 + 528) / 2 ** 20
    m3 = htrc_flat_runner.predicted_peak_mib(64512, 64, 128, leaf=64, queries=64512, heads=24, exact_leaves=32,
                                             window_streams=3)
    assert m3 - m128 == pytest.approx(per, rel=1e-6)
    kw512 = dict(leaf=64, queries=64512, heads=24, exact_leaves=32)
    assert htrc_flat_runner.predicted_peak_mib(64512, 64, 512, window_streams=3, **kw512) == \
        htrc_flat_runner.predicted_peak_mib(64512, 64, 512, window_streams=2, **kw512)
    with pytest.raises(ValueError, match="mode"):
        htrc_flat_runner.FlatRunner(64, 64, mode="nope")
    assert htrc_flat_runner.SUPPORTED_MODES == ("fast", "balanced", "accurate", "max")
    # 32-row tiles double the centres: the per-(tile, leaf) state doubles
    m32 = htrc_flat_runner.predicted_peak_mib(64512, 32, 4096, leaf=64, queries=64512, heads=24, exact_leaves=32)
    assert m32 - mib == pytest.approx(24 * 1008 * (1024 * 392 + 4 * 32 + 528) / 2 ** 20, rel=0.02)
    km = htrc_flat_runner.predicted_peak_mib(64512, 64, 1024, leaf=64, queries=64512, heads=24, order="kmeans",
                                             exact_leaves=32)
    assert km - mib == pytest.approx(24 * (8 * 64512 + 4 * 32 * 128) / 2 ** 20)
    assert htrc_flat_runner.STATIC_MIB == pytest.approx(39.8, abs=0.05)


def test_runner_and_its_replay_form_no_reference_cycle(monkeypatch):
    """A dropped runner, graph replay included, is freed by reference counting at once, not by a
    later collector pass (which could fall inside another runner's capture, where destroying a
    graph or freeing its pool is illegal).  The recording itself is stubbed: no GPU here."""
    import gc
    import weakref
    monkeypatch.setattr(htrc_flat_runner._Replay, "record", lambda self: None)
    r = htrc_flat_runner.FlatRunner(256, 256, mode="fast", device="cpu", free_bytes=8 << 30, tail_rows=3, leaf=64,
                                    exact_leaves=2)
    assert r._replay is not None and r._replay.tail[0].shape == (3, 128)
    with pytest.raises(ValueError, match="tail_rows=3"):
        r._replay.replay(torch.zeros(256, 128), torch.zeros(256, 128), torch.zeros(256, 128), None)
    gc.disable()
    try:
        ref, rref = weakref.ref(r), weakref.ref(r._replay)
        del r
        assert ref() is None and rref() is None
    finally:
        gc.enable()


def test_memory_model_follows_the_route_limits():
    """Layers the fused route does not take run the stage path; the model counts its SEL / excl
    buffers then (and the int8 route's top-k key workspace past 16384 leaves)."""
    wb = htrc_flat_runner.workspace_bytes
    for store in ("fp8", "bf16"):
        # 20000 leaves of 16 keys: over the 16-bit route's 16384, so fused=True sizes the stage path
        assert wb(2048, 320000, leaf=16, kx=64, store=store, fused=True) == \
            wb(2048, 320000, leaf=16, kx=64, store=store, fused=False, splits=1)
        assert wb(2048, 4096, leaf=16, kx=64, store=store, fused=True) < \
            wb(2048, 4096, leaf=16, kx=64, store=store, fused=False, splits=1)
    # int8 at 20000 leaves stays fused: 32 centres x 20000 leaves of 4-byte top-k keys and the
    # layer's rowmax (2048 rows x 4 bytes), against the stage path's 5 bytes of SEL and excl
    assert wb(2048, 320000, leaf=16, kx=64, store="int8", fused=False, splits=1) - \
        wb(2048, 320000, leaf=16, kx=64, store="int8", fused=True) == 32 * 20000 * (5 - 4) - 4 * 2048


def test_runner_plan_merges_knobs():
    """PROD, then the mode, then the caller's knobs with kern merged key by key; the window from
    free_bytes steps down through CHUNKS."""
    plan = htrc_flat_runner._Plan(htrc_flat, "fast", {"leaf": 64, "kern": {"group": 2}}, 3, 64512, 64512, 24,
                                  6 << 30, None, True)
    assert plan.cfg["exact_leaves"] == 256 and plan.cfg["leaf"] == 64 and plan.cfg["sink_leaves"] == 3
    assert plan.cfg["kern"] == {**htrc_flat.PROD["kern"], "group": 2}
    assert plan.cfg["tile_chunk"] in htrc_flat_runner.CHUNKS[1:] and plan.mib * 2 ** 20 <= 6 << 30
    plan = htrc_flat_runner._Plan(htrc_flat, "max", {}, 0, 4096, 4096, 1, None, None, False)
    assert plan.cfg["tile"] == 32 and plan.cfg["order"] == "kmeans" and plan.cfg["tile_chunk"] == 128


def test_windows_cover_every_group_once():
    for ng in (1, 7, 16, 1008):
        for chunk, group in ((1, 1), (16, 1), (32, 4), (128, 3), (1024, 1), (None, 1), (0, 2)):
            wins = htrc_flat._windows(ng, chunk, group)
            cover = [g for g0, gn in wins for g in range(g0, g0 + gn)]
            assert cover == list(range(ng))
            step = ng if not chunk else max(1, chunk // group)
            assert all(gn == min(step, ng - g0) for g0, gn in wins)


def test_noalloc_rejects_calls_beyond_the_scratch():
    """24 heads of 200000 queries need 24 * 200000 * 4 bytes of rowmax alone (19.2 MB) plus the
    near leaves of 3125 tiles x 200 near leaves x 24 heads (60 MB): more than the 32 MiB scratch of
    htrc_route_noalloc, refused on the host before the scratch is resolved or any launch (the
    pointers are never dereferenced, so this needs no device)."""
    f = _FAKE
    rc = _lib.lib().htrc_route_noalloc(*([f] * 11), 24, 200000, 200000 * 64, 64, 128, 200, 0, 1, 64, 1, 0, 3125,
                                       None, 0.088, f, f, None)
    assert rc == 1
    assert "bytes of scratch" in _lib.lib().htrc_last_error().decode()


def test_window_streams_are_owned_per_thread(monkeypatch):
    """Each host thread deals its tile windows over side streams of its own (a capture in one
    thread must not see another thread's eager launches on them); one thread reuses its streams.
    Streams are stubbed: no GPU here."""
    import threading
    made = []

    def stream(device=None):
        made.append(object())
        return made[-1]

    monkeypatch.setattr(htrc_flat.torch.cuda, "Stream", stream)
    monkeypatch.setattr(htrc_flat, "_WINDOW_STREAMS", threading.local())     # the stubs stay in this test
    dev = torch.device("cuda:0")
    mine = htrc_flat._window_streams(dev, 2)
    assert htrc_flat._window_streams(dev, 2) == mine and len(mine) == 2
    got = {}
    t = threading.Thread(target=lambda: got.setdefault("other", htrc_flat._window_streams(dev, 2)))
    t.start()
    t.join()
    assert len(got["other"]) == 2 and not set(map(id, got["other"])) & set(map(id, mine))
    assert htrc_flat._window_streams(dev, 3)[:2] == mine and len(made) == 5
