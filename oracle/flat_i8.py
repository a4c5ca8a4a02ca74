"""ctypes front end of the C oracle ``flat_i8.c`` -- TEST INFRASTRUCTURE ONLY.

Each function wraps one stage of the reference INT8 path and works on one head
(NumPy arrays, bf16 as uint16 bits).  ``flat_i8`` chains the stages the way
``_flat_triton`` does (h3/htrc_flat.py:181-276) with the PROD knobs
(h3/htrc_flat.py:391-392): store="int8", dot="bf16", curvature="lin",
order="seq", and ``group`` tiles per shared centre (kern["group"], :223-231; 1 by default).
Tiles are independent, so ``tile_chunk`` does not enter.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

from . import bf16

_HERE = Path(__file__).resolve().parent
_LIBNAME = "liboracle_flat.so"
_lib = None

_F32 = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_I8 = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_U16 = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_I32 = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> Path:
    """Compile the oracle with its Makefile (gcc, IEEE fp32, no contraction)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE), "-B", _LIBNAME], check=True)
    return _HERE / _LIBNAME


def lib():
    global _lib
    if _lib is None:
        path = _HERE / _LIBNAME
        if not path.exists():
            raise RuntimeError(f"oracle library {path} is not built: run `make -C {_HERE}`")
        L = ctypes.CDLL(str(path))
        L.oracle_abi_version.restype = _int
        L.oracle_r127.restype = _flt
        L.oracle_f2bf.restype = ctypes.c_uint16
        L.oracle_f2bf.argtypes = [_flt]
        L.oracle_split.restype = _i64
        L.oracle_split.argtypes = [_i64, _i64, _i64]
        L.oracle_pack_k.argtypes = [_U16, _i64, _int, _I8, _F32]
        L.oracle_tile_centres.argtypes = [_F32, _i64, _int, _int, _F32]
        L.oracle_group_centres.argtypes = [_F32, _i64, _int, _int, _int, _F32]
        L.oracle_pack_q.argtypes = [_F32, _i64, _int, _int, _int, _F32, _I8, _F32, _I8, _F32]
        L.oracle_stats.argtypes = [_F32, _i64, _U16, _U16, _i64, _int, _int, _flt, _int,
                                   _I8, _F32, _U16, _F32]
        L.oracle_select.argtypes = [_I8, _F32, _int, _int, _int, _i64, _I8, _F32, _F32, _i64, _i64, _int, _F32]
        L.oracle_topk.argtypes = [_F32, _i64, _i64, _int, _int, _I32, _I8]
        L.oracle_tile.argtypes = [_i64, _int, _int, _i64, _int, _int, _int, _I32, _I8,
                                  _I8, _F32, _I8, _F32, _I8, _F32, _F32, _U16,
                                  _I8, _F32, _U16, _flt, _int, _int, _F32, _F32, _F32]
        L.oracle_merge.argtypes = [_F32, _F32, _F32, _i64, _int, _int, _int, _F32, _F32]
        L.oracle_linspace_round.restype = _i64
        L.oracle_linspace_round.argtypes = [_i64, _i64, _i64]
        L.oracle_kmeans_order.argtypes = [_F32, _i64, _int, _int, _int, _int, _I32]
        L.oracle_f32_to_e4m3.restype = ctypes.c_uint8
        L.oracle_f32_to_e4m3.argtypes = [_flt]
        L.oracle_e4m3_to_f32.restype = _flt
        L.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [_flt]
        _U8 = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        L.oracle_stats_fp8.argtypes = [_F32, _i64, _U16, _U16, _i64, _int, _int, _flt, _int, _U8, _F32, _U8, _F32,
                                       _F32]
        L.oracle_select_fp8.argtypes = [_U16, _int, _int, _int, _i64, _U8, _F32, _F32, _i64, _i64, _int, _F32]
        L.oracle_tile_fp8.argtypes = [_i64, _int, _int, _i64, _int, _int, _int, _I32, _I8, _U16, _U16,
                                      _U8, _F32, _F32, _U8, _F32, _U16, _U16, _flt, _int, _int, _F32, _F32, _F32]
        L.oracle_stats_bf16.argtypes = [_F32, _i64, _U16, _U16, _i64, _int, _int, _flt, _int, _U16, _U16, _F32]
        L.oracle_select_bf16.argtypes = [_U16, _int, _int, _int, _i64, _U16, _F32, _i64, _i64, _int, _F32]
        L.oracle_tile_bf16.argtypes = [_i64, _int, _int, _i64, _int, _int, _int, _I32, _I8, _U16, _U16,
                                       _U16, _F32, _U16, _U16, _U16, _flt, _int, _int, _F32, _F32, _F32]
        if L.oracle_abi_version() != 6:
            raise RuntimeError(f"{path} is stale (oracle ABI {L.oracle_abi_version()}): rebuild it")
        _lib = L
    return _lib


def _c(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


def r127() -> float:
    return float(lib().oracle_r127())


def split(n: int, ns: int, bn: int) -> int:
    """_split (h3/htrc_flat_triton.py:297-299)."""
    return int(lib().oracle_split(n, ns, bn))


def pack_k(k_bits: np.ndarray):
    """K int8 pack (h3/htrc_flat.py:216-218) -> (k8 int8 [nk,d], ks f32 [nk])."""
    k_bits = _c(k_bits, np.uint16)
    nk, d = k_bits.shape
    k8 = np.empty((nk, d), np.int8)
    ks = np.empty((nk,), np.float32)
    lib().oracle_pack_k(k_bits, nk, d, k8, ks)
    return k8, ks


def tile_centres(q: np.ndarray, tile: int) -> np.ndarray:
    """mu [nt, d] over the real rows of every tile (h3/htrc_flat.py:142-156)."""
    q = _c(q, np.float32)
    n, d = q.shape
    nt = -(-n // tile)
    mu = np.empty((nt, d), np.float32)
    lib().oracle_tile_centres(q, n, d, tile, mu)
    return mu


def linspace_round(hi: int, steps: int, i: int) -> int:
    """round(torch.linspace(0, hi, steps, dtype=float32)[i]) (round half to even)."""
    return int(lib().oracle_linspace_round(int(hi), int(steps), int(i)))


def kmeans_order(q: np.ndarray, clusters: int = 32, sample: int = 4096, iters: int = 8) -> np.ndarray:
    """k-means query order (h3/htrc_flat.py:47-61) -> perm int32 [n]."""
    q = _c(q, np.float32)
    n, d = q.shape
    perm = np.empty((n,), np.int32)
    lib().oracle_kmeans_order(q, n, d, int(clusters), int(sample), int(iters), perm)
    return perm


def group_centres(q: np.ndarray, tile: int, group: int) -> np.ndarray:
    """mu [ng, d], the mean of the padded rows of every group of ``group`` tiles
    (h3/htrc_flat.py:223-229)."""
    q = _c(q, np.float32)
    n, d = q.shape
    nt = -(-n // tile)
    ng = -(-nt // group)
    mu = np.empty((ng, d), np.float32)
    lib().oracle_group_centres(q, n, d, tile, int(group), mu)
    return mu


def pack_q(q: np.ndarray, tile: int, mu: np.ndarray, group: int = 1):
    """Row int8 of q and q - mu over the padded tile rows (h3/htrc_flat_triton.py:104-117);
    tile t uses centre mu[t // group]."""
    q = _c(q, np.float32)
    n, d = q.shape
    nt = -(-n // tile)
    rows = nt * tile
    q8 = np.empty((rows, d), np.int8)
    dq8 = np.empty((rows, d), np.int8)
    sq = np.empty((rows,), np.float32)
    sdq = np.empty((rows,), np.float32)
    lib().oracle_pack_q(q, n, d, tile, int(group), _c(mu, np.float32), q8, sq, dq8, sdq)
    return q8, sq, dq8, sdq


def _tf32(prec: str) -> int:
    if prec not in ("ieee", "tf32"):
        raise ValueError("prec must be 'ieee' or 'tf32'")
    return int(prec == "tf32")


def stats(mu: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, leaf: int, scale: float, prec: str = "ieee"):
    """Leaf statistics (h3/htrc_flat_triton.py:41-85, I8 store)
    -> g8 int8 [nt,nb,d], sg f32 [nt,nb], vb bf16 bits [nt,nb,d], lz f32 [nt,nb].
    prec="tf32": the dots' fp32 operands (the centre, the normalised weights) rounded to TF32
    first, as PREC "tf32" makes them (the reference's leaf_stats takes prec for every store)."""
    mu = _c(mu, np.float32)
    k_bits, v_bits = _c(k_bits, np.uint16), _c(v_bits, np.uint16)
    nt, d = mu.shape
    nb = k_bits.shape[0] // leaf
    g8 = np.empty((nt, nb, d), np.int8)
    vb = np.empty((nt, nb, d), np.uint16)
    sg = np.empty((nt, nb), np.float32)
    lz = np.empty((nt, nb), np.float32)
    lib().oracle_stats(mu, nt, k_bits, v_bits, nb, leaf, d, float(scale), _tf32(prec), g8, sg, vb, lz)
    return g8, sg, vb, lz


def select(dq8, sdq, tile: int, g8, sg, lz, stride: int = 1, group: int = 1) -> np.ndarray:
    """SEL [ng, nb] (h3/htrc_flat_triton.py:214-254, I8), the max over the rows of each group."""
    g8 = _c(g8, np.int8)
    ng, nb, d = g8.shape
    nt = dq8.shape[0] // tile
    sel = np.empty((ng, nb), np.float32)
    lib().oracle_select(_c(dq8, np.int8), _c(sdq, np.float32), tile, stride, int(group), nt, g8,
                        _c(sg, np.float32), _c(lz, np.float32), ng, nb, d, sel)
    return sel


def topk(sel: np.ndarray, kx: int, sink: int = 0):
    """Near leaves (h3/htrc_flat.py:262-265) -> idx int32 [nt,kx] ascending, excl int8 [nt,nb]."""
    sel = _c(sel, np.float32)
    nt, nb = sel.shape
    idx = np.empty((nt, max(kx, 0)), np.int32)
    excl = np.zeros((nt, nb), np.int8)
    if kx > 0:
        lib().oracle_topk(sel, nt, nb, kx, sink, idx, excl)
    return idx, excl


def tile_partials(st: dict, *, tile: int, leaf: int, scale: float, splits: int, bn: int, group: int = 1):
    """Split partials (pm, pl, pacc) of the tile kernel (h3/htrc_flat_triton.py:88-211); tile t
    uses the state and near set of its group t // group."""
    g8 = st["g8"]
    ng, nb, d = g8.shape
    nt = st["dq8"].shape[0] // tile
    kx = st["idx"].shape[1]
    idx = st["idx"] if kx else np.zeros((ng, 1), np.int32)
    ns = max(1, int(splits))
    pm = np.empty((nt, ns, tile), np.float32)
    pl = np.empty((nt, ns, tile), np.float32)
    pacc = np.empty((nt, ns, tile, d), np.float32)
    lib().oracle_tile(nt, tile, d, nb, leaf, kx, int(group), _c(idx, np.int32), _c(st["excl"], np.int8),
                      _c(st["q8"], np.int8), _c(st["sq"], np.float32),
                      _c(st["dq8"], np.int8), _c(st["sdq"], np.float32),
                      _c(g8, np.int8), _c(st["sg"], np.float32), _c(st["lz"], np.float32),
                      _c(st["vb"], np.uint16), _c(st["k8"], np.int8), _c(st["ks"], np.float32),
                      _c(st["v"], np.uint16), float(scale), ns, int(bn), pm, pl, pacc)
    return pm, pl, pacc


def merge(pm, pl, pacc):
    """Merge of split partials (h3/htrc_flat_triton.py:257-273) -> out [nt*T,d], logz [nt*T]."""
    pm, pl, pacc = _c(pm, np.float32), _c(pl, np.float32), _c(pacc, np.float32)
    nt, ns, tile, d = pacc.shape
    out = np.empty((nt * tile, d), np.float32)
    logz = np.empty((nt * tile,), np.float32)
    lib().oracle_merge(pm, pl, pacc, nt, ns, tile, d, out, logz)
    return out, logz


def f32_to_e4m3(x) -> np.ndarray:
    """e4m3fn codes of float32 values (round to nearest even, |x| saturated at 448)."""
    f = lib().oracle_f32_to_e4m3
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint8).reshape(np.shape(x))


def e4m3_to_f32(b) -> np.ndarray:
    f = lib().oracle_e4m3_to_f32
    return np.array([f(int(v)) for v in np.asarray(b, np.uint8).ravel()], np.float32).reshape(np.shape(b))


def f32_to_f16(x) -> np.ndarray:
    """fp16 bits of float32 values (round to nearest even)."""
    f = lib().oracle_f32_to_f16
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint16).reshape(np.shape(x))


def pack_q16(q: np.ndarray, tile: int, mu: np.ndarray, group: int = 1, dq_fp16: bool = True):
    """16-bit operands of the bf16 / fp8 state stores (h3/htrc_flat_triton.py:104-108) over the
    padded tile rows: q16 = bf16(q) bits, dq16 = fp16(q - mu) (or bf16) bits."""
    q = _c(q, np.float32)
    n, d = q.shape
    nt = -(-n // tile)
    p = np.arange(nt * tile)
    rows = q[np.minimum(p, n - 1)]
    dq = (rows - _c(mu, np.float32)[p // tile // group]).astype(np.float32)
    q16 = bf16.from_f32(rows)
    dq16 = dq.astype(np.float16).view(np.uint16) if dq_fp16 else bf16.from_f32(dq)
    return q16, dq16


def stats_fp8(mu: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, leaf: int, scale: float, prec: str = "ieee"):
    """Leaf statistics with the fp8 state store (h3/htrc_flat_triton.py:65-72)
    -> g8 e4m3 [nt,nb,d], sg [nt,nb], vb8 e4m3 [nt,nb,d], sv [nt,nb], lz [nt,nb]."""
    mu = _c(mu, np.float32)
    k_bits, v_bits = _c(k_bits, np.uint16), _c(v_bits, np.uint16)
    nt, d = mu.shape
    nb = k_bits.shape[0] // leaf
    g8 = np.empty((nt, nb, d), np.uint8)
    vb8 = np.empty((nt, nb, d), np.uint8)
    sg = np.empty((nt, nb), np.float32)
    sv = np.empty((nt, nb), np.float32)
    lz = np.empty((nt, nb), np.float32)
    lib().oracle_stats_fp8(mu, nt, k_bits, v_bits, nb, leaf, d, float(scale), _tf32(prec), g8, sg, vb8, sv, lz)
    return g8, sg, vb8, sv, lz


def stats_bf16(mu: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, leaf: int, scale: float, prec: str = "ieee"):
    """Leaf statistics with the bf16 state store -> g bf16 bits [nt,nb,d], vb bf16 bits, lz [nt,nb]."""
    mu = _c(mu, np.float32)
    k_bits, v_bits = _c(k_bits, np.uint16), _c(v_bits, np.uint16)
    nt, d = mu.shape
    nb = k_bits.shape[0] // leaf
    g16 = np.empty((nt, nb, d), np.uint16)
    vb16 = np.empty((nt, nb, d), np.uint16)
    lz = np.empty((nt, nb), np.float32)
    lib().oracle_stats_bf16(mu, nt, k_bits, v_bits, nb, leaf, d, float(scale), _tf32(prec), g16, vb16, lz)
    return g16, vb16, lz


def select_bf16(dq16, tile: int, g16, lz, stride: int = 1, group: int = 1) -> np.ndarray:
    """SEL [ng, nb] with the bf16 state store (bf16 dq . g + lz)."""
    g16 = _c(g16, np.uint16)
    ng, nb, d = g16.shape
    nt = dq16.shape[0] // tile
    sel = np.empty((ng, nb), np.float32)
    lib().oracle_select_bf16(_c(dq16, np.uint16), tile, stride, int(group), nt, g16, _c(lz, np.float32), ng, nb, d, sel)
    return sel


def tile_partials_bf16(st: dict, *, tile: int, leaf: int, scale: float, splits: int, bn: int, group: int = 1):
    """Split partials of the tile kernel with the bf16 state store."""
    g16 = st["g16"]
    ng, nb, d = g16.shape
    nt = st["dq16"].shape[0] // tile
    kx = st["idx"].shape[1]
    idx = st["idx"] if kx else np.zeros((ng, 1), np.int32)
    ns = max(1, int(splits))
    pm = np.empty((nt, ns, tile), np.float32)
    pl = np.empty((nt, ns, tile), np.float32)
    pacc = np.empty((nt, ns, tile, d), np.float32)
    lib().oracle_tile_bf16(nt, tile, d, nb, leaf, kx, int(group), _c(idx, np.int32), _c(st["excl"], np.int8),
                           _c(st["q16"], np.uint16), _c(st["dq16"], np.uint16), g16, _c(st["lz"], np.float32),
                           _c(st["vb16"], np.uint16), _c(st["k"], np.uint16), _c(st["v"], np.uint16), float(scale),
                           ns, int(bn), pm, pl, pacc)
    return pm, pl, pacc


def select_fp8(dq16, tile: int, g8, sg, lz, stride: int = 1, group: int = 1) -> np.ndarray:
    """SEL [ng, nb] with the fp8 state store (h3/htrc_flat_triton.py:214-254, FP8 = 1)."""
    g8 = _c(g8, np.uint8)
    ng, nb, d = g8.shape
    nt = dq16.shape[0] // tile
    sel = np.empty((ng, nb), np.float32)
    lib().oracle_select_fp8(_c(dq16, np.uint16), tile, stride, int(group), nt, g8, _c(sg, np.float32),
                            _c(lz, np.float32), ng, nb, d, sel)
    return sel


def tile_partials_fp8(st: dict, *, tile: int, leaf: int, scale: float, splits: int, bn: int, group: int = 1):
    """Split partials of the tile kernel with the fp8 state store (h3/htrc_flat_triton.py:88-211)."""
    g8 = st["g8"]
    ng, nb, d = g8.shape
    nt = st["dq16"].shape[0] // tile
    kx = st["idx"].shape[1]
    idx = st["idx"] if kx else np.zeros((ng, 1), np.int32)
    ns = max(1, int(splits))
    pm = np.empty((nt, ns, tile), np.float32)
    pl = np.empty((nt, ns, tile), np.float32)
    pacc = np.empty((nt, ns, tile, d), np.float32)
    lib().oracle_tile_fp8(nt, tile, d, nb, leaf, kx, int(group), _c(idx, np.int32), _c(st["excl"], np.int8),
                          _c(st["q16"], np.uint16), _c(st["dq16"], np.uint16), _c(g8, np.uint8),
                          _c(st["sg"], np.float32), _c(st["lz"], np.float32), _c(st["vb8"], np.uint8),
                          _c(st["sv"], np.float32), _c(st["k"], np.uint16), _c(st["v"], np.uint16), float(scale),
                          ns, int(bn), pm, pl, pacc)
    return pm, pl, pacc


def bound_select(qf: np.ndarray, tile: int, mu: np.ndarray, g16: np.ndarray, lz: np.ndarray,
                 group: int = 1) -> np.ndarray:
    """select="bound" (h3/htrc_flat.py:255-257) of the bf16 store: SEL[t, l] = lz + r_t * ||g_tl||,
    r_t the largest ||q_row - mu_t|| over the tile group's rows, padded as the reference pads its
    tiles (rows past the last query and tiles past the last tile repeat the last).  Norms are
    sequential fp32 sums of squares over the dims and one IEEE square root."""
    n, d = qf.shape
    nt = -(-n // tile)
    ng = mu.shape[0]
    sel = np.empty(lz.shape, np.float32)
    gf = bf16.to_f32(g16)                                           # [ng, nb, d]
    gs = np.zeros(gf.shape[:2], np.float32)
    for c in range(d):
        gs = (gs + gf[:, :, c] * gf[:, :, c]).astype(np.float32)
    gnorm = np.sqrt(gs).astype(np.float32)
    for gi in range(ng):
        rows = []
        for j in range(group):
            t = min(gi * group + j, nt - 1)
            rows.extend(min(t * tile + r, n - 1) for r in range(tile))
        x = (qf[rows] - mu[gi][None, :]).astype(np.float32)
        s = np.zeros(len(rows), np.float32)
        for c in range(d):
            s = (s + x[:, c] * x[:, c]).astype(np.float32)
        r = np.float32(np.sqrt(s).astype(np.float32).max())
        sel[gi] = (lz[gi] + (r * gnorm[gi]).astype(np.float32)).astype(np.float32)
    return sel


def tail_merge(out, logz, q, tk, tv, scale: float):
    """Keys past the last full leaf, attended exactly by every query, merged into a finished
    (out [n,d], logz [n]).  Up to 16 tail keys: q, k, v and p rounded to bf16, fp32
    accumulation, as the tile kernel's tail block (h3/htrc_flat_triton.py:187-207); more:
    fp32 throughout, as the host-side partial (h3/htrc_flat_triton.py:381-388).  Either way the
    result is one softmax over all keys: the split-merge algebra (:257-273) on the partials
    (logz, out) and (lse_tail, mean_tail).  q float32 [n,d]; tk, tv float32 [m,d]."""
    out = _c(out, np.float32)
    logz = _c(logz, np.float32)
    qf, kf, vf = (_c(x, np.float32) for x in (q, tk, tv))
    bfr = kf.shape[0] <= 16
    if bfr:
        qf, kf, vf = bf16.round_f32(qf), bf16.round_f32(kf), bf16.round_f32(vf)
    s = ((qf.astype(np.float64) @ kf.T.astype(np.float64)).astype(np.float32) * np.float32(scale)).astype(np.float32)
    m = s.max(axis=1)
    p = np.exp(s - m[:, None]).astype(np.float32)
    l = p.sum(axis=1, dtype=np.float64).astype(np.float32)
    pv = bf16.round_f32(p) if bfr else p
    mean = ((pv.astype(np.float64) @ vf.astype(np.float64)) / l[:, None].astype(np.float64))
    lse = m.astype(np.float64) + np.log(l.astype(np.float64))
    z = np.logaddexp(logz.astype(np.float64), lse)
    res = out.astype(np.float64) * np.exp(logz - z)[:, None] + mean * np.exp(lse - z)[:, None]
    return res.astype(np.float32), z.astype(np.float32)


def flat_i8(q, k_bits, v_bits, *, tile: int = 64, leaf: int = 64, exact_leaves: int = 64,
            splits: int = 4, bn: int = 64, sel_stride: int = 1, sink_leaves: int = 0,
            scale: float | None = None, keep: bool = True, group: int = 1, order: str = "seq",
            store: str = "int8", state_quant: str | None = None, quant_group: int = 0,
            select_mode: str = "max", prec: str = "ieee") -> dict:
    """The INT8 flat operator for one head: q float32 (or bf16 bits) [n,d], k/v bf16 bits
    [nk,d] with nk % leaf == 0.  Returns every intermediate plus out [n,d] and logz [n].
    order="kmeans": the tiles are cut from q[perm] (perm = kmeans_order(q)) and out / logz
    are returned in query order (h3/htrc_flat.py:146-149, 159-165).  store="fp8": the fp8
    state store (e4m3 g / vb with row scales, fp16 far dots, bf16 near dots).  state_quant (store
    "bf16" only): g and vb fake-quantised in place after the statistics, as quant["state"] does
    (h3/htrc_flat.py:246-248), with quant_group.  select_mode "bound" (store "bf16" only): the
    bound routing score (bound_select) in place of the row-max SEL.  prec="tf32": the leaf
    statistics on TF32 operands (the operator's precision="tf32", h3/htrc_flat.py:122, 243)."""
    q = np.asarray(q)
    qf = bf16.to_f32(q) if q.dtype == np.uint16 else _c(q, np.float32)
    n, d = qf.shape
    nk = k_bits.shape[0]
    if nk % leaf:
        raise ValueError("key count must be a multiple of the leaf size")
    nb = nk // leaf
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    sink = max(0, min(int(sink_leaves), nb))
    kx = min(int(exact_leaves) + sink, nb)
    st: dict = {"v": _c(v_bits, np.uint16)}
    if order == "kmeans":
        st["perm"] = kmeans_order(qf)
        qf = qf[st["perm"]]
    elif order != "seq":
        raise ValueError("order must be seq or kmeans")
    st["k8"], st["ks"] = pack_k(k_bits)
    st["mu"] = tile_centres(qf, tile) if group == 1 else group_centres(qf, tile, group)
    if store == "fp8":
        st["k"] = _c(k_bits, np.uint16)
        st["q16"], st["dq16"] = pack_q16(qf, tile, st["mu"], group, dq_fp16=True)
        st["g8"], st["sg"], st["vb8"], st["sv"], st["lz"] = stats_fp8(st["mu"], k_bits, v_bits, leaf, scale, prec)
    elif store == "bf16":
        st["k"] = _c(k_bits, np.uint16)
        st["q16"], st["dq16"] = pack_q16(qf, tile, st["mu"], group, dq_fp16=False)
        st["g16"], st["vb16"], st["lz"] = stats_bf16(st["mu"], k_bits, v_bits, leaf, scale, prec)
        if state_quant:
            from .fake_quant import fake_quant
            for nm in ("g16", "vb16"):
                st[nm] = bf16.from_f32(fake_quant(bf16.to_f32(st[nm]), state_quant, quant_group))
    elif store == "int8":
        st["q8"], st["sq"], st["dq8"], st["sdq"] = pack_q(qf, tile, st["mu"], group)
        st["g8"], st["sg"], st["vb"], st["lz"] = stats(st["mu"], k_bits, v_bits, leaf, scale, prec)
    else:
        raise ValueError("store must be int8, fp8 or bf16")
    if (state_quant or select_mode != "max") and store != "bf16":
        raise ValueError("state fake-quant and select='bound' need store='bf16'")
    if kx > 0:
        if store == "fp8":
            st["sel"] = select_fp8(st["dq16"], tile, st["g8"], st["sg"], st["lz"], sel_stride, group)
        elif store == "bf16" and select_mode == "bound":
            st["sel"] = bound_select(qf, tile, st["mu"], st["g16"], st["lz"], group)
        elif store == "bf16":
            st["sel"] = select_bf16(st["dq16"], tile, st["g16"], st["lz"], sel_stride, group)
        else:
            st["sel"] = select(st["dq8"], st["sdq"], tile, st["g8"], st["sg"], st["lz"], sel_stride, group)
        st["idx"], st["excl"] = topk(st["sel"], kx, sink)
    else:
        nt = st["mu"].shape[0]
        st["idx"] = np.zeros((nt, 0), np.int32)
        st["excl"] = np.zeros((nt, nb), np.int8)
    tp = {"fp8": tile_partials_fp8, "bf16": tile_partials_bf16}.get(store, tile_partials)
    pm, pl, pacc = tp(st, tile=tile, leaf=leaf, scale=scale, splits=splits, bn=bn, group=group)
    out, logz = merge(pm, pl, pacc)
    st["out"], st["logz"] = out[:n], logz[:n]
    if order == "kmeans":
        st["out_perm"], st["logz_perm"] = st["out"], st["logz"]
        st["out"], st["logz"] = np.empty_like(out[:n]), np.empty_like(logz[:n])
        st["out"][st["perm"]] = st["out_perm"]
        st["logz"][st["perm"]] = st["logz_perm"]
    if keep:
        st["pm"], st["pl"], st["pacc"] = pm, pl, pacc
    return st
