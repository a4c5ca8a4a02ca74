"""ctypes binding of libhtrc_flat.so (C ABI: include/htrc_flat.h).

torch is imported first so that the library's HIP runtime dependency resolves to the
runtime torch already loaded (one HIP runtime per process).  There is no fallback:
if the library is missing every operator raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBPATH = HERE / "libhtrc_flat.so"
ABI_VERSION = 11

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float

# name -> argument types (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "htrc_abi_version": [],
    "htrc_last_error": [],
    "htrc_nb_pad": [_i64],
    "htrc_pack_q": [_vp, _int, _i64, _i64, _int, _int, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "htrc_pack_k": [_vp, _i64, _i64, _int, _vp, _vp, _vp],
    "htrc_leaf_stats": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _flt, _vp, _vp, _vp, _vp, _vp],
    "htrc_select": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int, _vp, _vp],
    "htrc_topk": [_vp, _i64, _i64, _int, _int, _vp, _vp, _vp],
    "htrc_tile": [_vp] * 13 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _vp, _int, _int, _flt] + [_vp] * 6,
    "htrc_merge": [_vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp, _vp, _vp, _vp],
    "htrc_route_select": [_vp] * 5 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _int, _int, _vp, _vp, _vp],
    "htrc_route_attend": [_vp] * 13 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _vp, _flt, _vp, _vp, _vp],
    "htrc_route": [_vp] * 11 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _int, _int, _vp, _flt, _vp, _vp, _vp, _vp,
                                 _vp],
    "htrc_tail": [_vp, _int, _vp, _vp, _i64, _i64, _i64, _int, _flt, _vp, _vp, _vp],
    "htrc_pack_q16": [_vp, _int, _i64, _i64, _int, _int, _int, _vp, _int, _vp, _vp, _vp, _vp],
    "htrc_leaf_stats_fp8": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _flt, _vp, _vp, _vp, _vp, _vp, _vp],
    "htrc_select_fp8": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int, _vp, _vp],
    "htrc_tile_fp8": [_vp] * 11 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _vp, _int, _int, _flt] + [_vp] * 6,
    "htrc_leaf_stats_bf16": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _flt, _vp, _vp, _vp, _vp],
    "htrc_select_bf16": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int, _vp, _vp],
    "htrc_tile_bf16": [_vp] * 9 + [_i64, _i64, _i64, _int, _int, _int, _int, _int, _vp, _int, _int, _flt] + [_vp] * 6,
    "htrc_kmeans_order": [_vp, _int, _i64, _i64, _int, _int, _int, _int, _vp, _vp, _vp, _vp],
    "htrc_dequant_rows": [_vp, _i64, _vp, _i64, _i64, _int, _vp, _int, _vp],
    "htrc_selftest_mfma": [_vp] * 7,
}
_RESTYPES = {"htrc_last_error": ctypes.c_char_p}

_lib = None


class HTRCLaunchError(RuntimeError):
    """The HIP runtime rejected a kernel launch."""


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIBPATH.exists():
            raise RuntimeError(
                f"{LIBPATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the flat-HTRC operator has no fallback path)")
        L = ctypes.CDLL(str(LIBPATH))
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _int)
        if L.htrc_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libhtrc_flat ABI {L.htrc_abi_version()} != expected {ABI_VERSION}; rebuild")
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call a launcher; map HTRC_ERR_ARG to ValueError and HTRC_ERR_HIP to HTRCLaunchError."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().htrc_last_error().decode()
        if rc == 1:
            raise ValueError(msg)
        raise HTRCLaunchError(msg)


def ptr(t) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def nb_pad(nb: int) -> int:
    return (int(nb) + 31) // 32 * 32
