"""Shared test helpers: bf16 bit views and tolerance metrics."""
from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 numpy bits (CPU copy)."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(b: np.ndarray, device=None) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def vb_to_quads(vb_bits: np.ndarray, nbp: int) -> np.ndarray:
    """Natural vb bits [nt, nb, d] -> leaf-quad layout [nt, nbp/4, d, 4] (zero padded)."""
    nt, nb, d = vb_bits.shape
    pad = np.zeros((nt, nbp, d), np.uint16)
    pad[:, :nb] = vb_bits
    return np.ascontiguousarray(pad.reshape(nt, nbp // 4, 4, d).transpose(0, 1, 3, 2))


def key_quads(x_bits: np.ndarray) -> np.ndarray:
    """[n, d] bf16 bits -> key-quad layout [n/4, d, 4]."""
    n, d = x_bits.shape
    return np.ascontiguousarray(x_bits.reshape(n // 4, 4, d).transpose(0, 2, 1))
