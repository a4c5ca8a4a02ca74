"""Float64 NumPy restatement of the HTRC teaching reference -- TEST INFRASTRUCTURE ONLY.

Follows src/htrc_reference/model.py:29-137: exact softmax leaf statistics
(log-mass L, gradient g, Hessian H, value u, value Jacobian J), their exact
parent merge, contiguous forests, the Taylor-2 log-mass / Taylor-1 value
prediction and the threshold-opening evaluation.  It is BASELINE configuration 1
and the closed-form cross-check of the flat operator's leaf statistics: with the
query centre c = scale * mu, ``leaf_stats(K, V, c)`` gives lz = L, g = scale * grad,
vb = value (h3/htrc_flat_triton.py:55-63).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def _lse_softmax(x: np.ndarray) -> tuple[float, np.ndarray]:
    """(log-sum-exp, softmax) of a logit vector (model.py:29-33)."""
    top = float(np.max(x))
    e = np.exp(x - top)
    s = float(e.sum())
    return top + float(np.log(s)), e / s


@dataclass(frozen=True)
class LeafStats:
    log_mass: float
    gradient: np.ndarray
    hessian: np.ndarray
    value: np.ndarray
    value_jacobian: np.ndarray


@dataclass(frozen=True)
class Node:
    stats: LeafStats
    children: tuple = ()
    keys: np.ndarray = field(default_factory=lambda: np.zeros(0, dtype=np.int64))


def leaf_stats(keys, values, centre) -> LeafStats:
    """Derivatives of a block's log-partition and conditional value at a scaled centre
    (model.py:35-49)."""
    K = np.asarray(keys, dtype=np.float64)
    V = np.asarray(values, dtype=np.float64)
    c = np.asarray(centre, dtype=np.float64)
    if K.ndim != 2 or V.ndim != 2 or K.shape[0] != V.shape[0] or K.shape[0] == 0:
        raise ValueError("keys/values must be matching nonempty matrices")
    if c.shape != (K.shape[1],):
        raise ValueError("scaled query dimension mismatch")
    lm, w = _lse_softmax(K @ c)
    g = w @ K
    u = w @ V
    dk = K - g
    dv = V - u
    H = dk.T @ (dk * w[:, None])
    J = dv.T @ (dk * w[:, None])
    return LeafStats(lm, g, H, u, J)


def merge(children) -> LeafStats:
    """Exact parent statistics from children (model.py:51-66)."""
    children = list(children)
    if not children:
        raise ValueError("cannot merge an empty set")
    lm, w = _lse_softmax(np.array([c.log_mass for c in children], dtype=np.float64))
    G = np.stack([c.gradient for c in children])
    U = np.stack([c.value for c in children])
    g = w @ G
    u = w @ U
    dg = G - g
    du = U - u
    H = np.einsum("c,cij->ij", w, np.stack([c.hessian for c in children])) + dg.T @ (dg * w[:, None])
    J = np.einsum("c,cij->ij", w, np.stack([c.value_jacobian for c in children])) + du.T @ (dg * w[:, None])
    return LeafStats(lm, g, H, u, J)


def forest(keys, values, centre, *, leaf_size: int = 16, fanout: int = 4) -> tuple:
    """Contiguous leaves merged fanout at a time until at most fanout roots remain
    (model.py:68-84)."""
    if leaf_size < 1 or fanout < 2:
        raise ValueError("leaf_size must be positive and fanout >= 2")
    K = np.asarray(keys, dtype=np.float64)
    V = np.asarray(values, dtype=np.float64)
    c = np.asarray(centre, dtype=np.float64)
    level = []
    for a in range(0, len(K), leaf_size):
        b = min(a + leaf_size, len(K))
        level.append(Node(leaf_stats(K[a:b], V[a:b], c), (), np.arange(a, b)))
    while len(level) > fanout:
        level = [Node(merge([n.stats for n in level[i:i + fanout]]), tuple(level[i:i + fanout]))
                 for i in range(0, len(level), fanout)]
    return tuple(level)


def exact_attention(keys, values, query) -> np.ndarray:
    """Softmax attention for an already scaled query (model.py:86-89)."""
    _, w = _lse_softmax(np.asarray(keys, dtype=np.float64) @ np.asarray(query, dtype=np.float64))
    return w @ np.asarray(values, dtype=np.float64)


def exact_log_partition(keys, query) -> float:
    lm, _ = _lse_softmax(np.asarray(keys, dtype=np.float64) @ np.asarray(query, dtype=np.float64))
    return lm


def predict(node: Node, delta: np.ndarray) -> tuple[float, np.ndarray, float]:
    """Taylor-2 log-mass, Taylor-1 value and the quadratic form (model.py:91-96)."""
    s = node.stats
    quad = float(delta @ s.hessian @ delta)
    return s.log_mass + float(s.gradient @ delta) + 0.5 * quad, s.value + s.value_jacobian @ delta, quad


def evaluate(keys, values, query, centre, roots, *, opening_threshold: float = 0.01):
    """Approximate attention with exact fallback at opened leaves (model.py:98-137).
    Returns (output, info) with info = visited_nodes, accepted_nodes, exact_leaves and
    log_norm (the root-level log-partition estimate used for the opening score)."""
    if opening_threshold < 0:
        raise ValueError("opening_threshold must be nonnegative")
    K = np.asarray(keys, dtype=np.float64)
    V = np.asarray(values, dtype=np.float64)
    q = np.asarray(query, dtype=np.float64)
    delta = q - np.asarray(centre, dtype=np.float64)
    norm = float(np.logaddexp.reduce([predict(r, delta)[0] for r in roots]))
    parts: list[tuple[float, np.ndarray]] = []
    info = {"visited_nodes": 0, "accepted_nodes": 0, "exact_leaves": 0, "log_norm": norm}
    stack = list(reversed(roots))
    while stack:                                  # depth-first, children in order
        node = stack.pop()
        info["visited_nodes"] += 1
        lm, val, quad = predict(node, delta)
        score = float(np.exp(min(0.0, lm - norm))) * float(np.expm1(min(0.5 * abs(quad), 80.0)))
        opened = score > opening_threshold
        if opened and node.children:
            stack.extend(reversed(node.children))
        elif opened:
            lme, w = _lse_softmax(K[node.keys] @ q)
            parts.append((lme, w @ V[node.keys]))
            info["exact_leaves"] += 1
        else:
            parts.append((lm, val))
    info["accepted_nodes"] = len(parts)
    _, w = _lse_softmax(np.array([p[0] for p in parts]))
    out = sum(wi * p[1] for wi, p in zip(w, parts))
    info["log_partition"] = float(np.logaddexp.reduce([p[0] for p in parts]))
    return out, info


def config1(seed: int = 0, queries: int = 1024, keys: int = 4096, dim: int = 64,
            leaf: int = 64, fanout: int = 4, opening_threshold: float = 0.01,
            query_limit: int | None = None) -> dict:
    """float64, q/k/v ~ N(0,1), q scaled by 1/sqrt(d), leaves of
    64 contiguous keys, fanout 4, centre = mean of the scaled queries.  Reports the
    log-partition error of the root estimate and of the accepted parts, and the output
    error against exact softmax attention, over the first ``query_limit`` queries."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((queries, dim)) / np.sqrt(dim)
    k = rng.standard_normal((keys, dim))
    v = rng.standard_normal((keys, dim))
    c = q.mean(0)
    roots = forest(k, v, c, leaf_size=leaf, fanout=fanout)
    nq = queries if query_limit is None else min(queries, query_limit)
    err_out, err_norm, err_lz, opened = [], [], [], []
    for i in range(nq):
        approx, info = evaluate(k, v, q[i], c, roots, opening_threshold=opening_threshold)
        dense = exact_attention(k, v, q[i])
        lz = exact_log_partition(k, q[i])
        err_out.append(float(np.linalg.norm(approx - dense) / np.linalg.norm(dense)))
        err_norm.append(abs(info["log_norm"] - lz))
        err_lz.append(abs(info["log_partition"] - lz))
        opened.append(info["exact_leaves"])
    return {"queries": nq, "rel_l2_median": float(np.median(err_out)),
            "rel_l2_max": float(np.max(err_out)),
            "logz_root_abs_max": float(np.max(err_norm)),
            "logz_abs_max": float(np.max(err_lz)),
            "exact_leaves_mean": float(np.mean(opened))}
