"""ctypes binding of libhtrc_flat.so (C ABI: include/htrc_flat.h).

torch is imported first so that the library's HIP runtime dependency resolves to the
runtime torch already loaded (one HIP runtime per process).  There is no fallback:
if the library is missing every operator raises.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBPATH = HERE / "libhtrc_flat.so"
HEADER = HERE.parent / "include" / "htrc_flat.h"
ABI_VERSION = 15

_CTYPES = {"int64_t": ctypes.c_int64, "int": ctypes.c_int, "float": ctypes.c_float}


def _c_arg(decl: str):
    """ctypes type of one C parameter declaration: pointers are c_void_p, scalars by type."""
    decl = decl.strip()
    if "*" in decl:
        return ctypes.c_void_p
    base = decl.replace("const ", "").split()[0]
    if base not in _CTYPES:
        raise RuntimeError(f"{HEADER.name}: no ctypes mapping for parameter {decl!r}")
    return _CTYPES[base]


def parse_header(text: str) -> dict:
    """name -> (argument ctypes, restype) of every entry point the header declares."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    sigs = {}
    for ret, name, args in re.findall(r"\b(int|const char\s*\*)\s*(htrc_\w+)\s*\(([^)]*)\)\s*;", text):
        args = args.strip()
        argt = [] if args in ("", "void") else [_c_arg(a) for a in args.split(",")]
        sigs[name] = (argt, ctypes.c_char_p if "char" in ret else ctypes.c_int)
    return sigs


def signatures() -> dict:
    if not HEADER.exists():
        raise RuntimeError(f"{HEADER} is missing: the C-ABI binding is read from it")
    return parse_header(HEADER.read_text())


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
        for name, (args, res) in signatures().items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.htrc_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libhtrc_flat ABI {L.htrc_abi_version()} != expected {ABI_VERSION}; rebuild")
        _fns.clear()
        _lib = L
    return _lib


_fns: dict = {}


def call(name: str, *args) -> None:
    """Call a launcher; map HTRC_ERR_ARG to ValueError and HTRC_ERR_HIP to HTRCLaunchError."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().htrc_last_error().decode()
        if rc == 1:
            raise ValueError(msg)
        raise HTRCLaunchError(msg)


def ptr(t) -> int | None:
    """Device address of a tensor (ctypes takes the int for a void* parameter), None for None."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    """The current HIP stream of the device (torch's), as a void* for the launchers.  Small
    layers are bound by host time per call, so this takes torch's raw-stream query directly
    when the build has it."""
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        if isinstance(device, torch.device) and device.index is not None:
            return raw(device.index)
        if isinstance(device, int):
            return raw(device)
    return torch.cuda.current_stream(device).cuda_stream


def nb_pad(nb: int) -> int:
    return (int(nb) + 31) // 32 * 32
