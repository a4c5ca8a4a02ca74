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
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    ver = int(re.search(r"#define HTRC_ABI_VERSION (\d+)", text).group(1))
    assert lib.htrc_abi_version() == ver == _lib.ABI_VERSION


def test_nb_pad():
    lib = _lib.lib()
    for nb, want in ((1, 32), (32, 32), (33, 64), (1008, 1024), (1953, 1984)):
        assert lib.htrc_nb_pad(nb) == want == _lib.nb_pad(nb)


_FAKE = ctypes.c_void_p(256)   # never dereferenced: validation fails before any launch


@pytest.mark.parametrize("case", ["null", "dim", "leaf", "block", "leaves", "group", "tile", "stride"])
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
        rc = lib.htrc_leaf_stats(f, f, f, 1, 1, 96, 48, 128, 0.1, f, f, f, f, None)
        msg = "leaf"
    elif case == "block":
        rc = lib.htrc_tile(*([f] * 13), 1, 64, 128, 64, 128, 1, 64, 1, None, 4, 48, 0.1, f, f, f, f, f, None)
        msg = "multiple of 32"
    elif case == "leaves":
        rc = lib.htrc_route(*([f] * 11), 1, 64, 64 * 9000, 64, 128, 4, 0, 1, 64, 1, None, 0.1, f, f, None, f, None)
        msg = "8192"
    elif case == "group":
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 640, 64, 128, 4, 0, 1, 64, 0, f, f, None)
        msg = "group"
    elif case == "tile":
        rc = lib.htrc_route_select(*([f] * 5), 1, 640, 640, 64, 128, 4, 0, 1, 48, 1, f, f, None)
        msg = "32 or 64"
    else:                                          # stride must divide a 32-row tile
        rc = lib.htrc_select(*([f] * 5), 1, 10, 20, 64, 32, 1, 128, f, None)
        msg = "divide"
    assert rc == 1
    assert msg in lib.htrc_last_error().decode()


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
    q, k, v = _qkv(d=64)
    with pytest.raises(ValueError, match="128"):
        htrc_flat.flat_attention_prod(q, k, v)
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
    mib = htrc_flat_runner.predicted_peak_mib(64512, 64, 128, leaf=64, queries=64512, heads=24)
    # cfg3 layer: per-(tile, leaf) state dominates: 24 * 1008 * 1024 * 392 B = 9252 MiB
    assert 9252 < mib < 16000
    assert htrc_flat_runner.plan_chunk(64 << 30, 64512, 64, leaf=64, queries=64512, heads=24) == 1024
    with pytest.raises(MemoryError):
        htrc_flat_runner.plan_chunk(1 << 30, 64512, 64, leaf=64, queries=64512, heads=24)
    with pytest.raises(ValueError, match="mode"):
        htrc_flat_runner.FlatRunner(64, 64, mode="nope")
    assert htrc_flat_runner.SUPPORTED_MODES == ("fast", "balanced", "accurate", "max")
    # 32-row tiles double the centres: the per-(tile, leaf) state doubles
    m32 = htrc_flat_runner.predicted_peak_mib(64512, 32, 128, leaf=64, queries=64512, heads=24)
    assert m32 - mib == pytest.approx(24 * 1008 * 1024 * 392 / 2 ** 20, rel=0.02)
    km = htrc_flat_runner.predicted_peak_mib(64512, 64, 128, leaf=64, queries=64512, heads=24, order="kmeans")
    assert km - mib == pytest.approx(24 * (8 * 64512 + 4 * 32 * 128) / 2 ** 20)
