"""Seeded orthogonal rotation (rotation.py:17-110 of the reference).

The matrix is generated once on the host (numpy RandomState + QR, as the
reference does) and kept on the GPU; the compress / attention kernels apply it.
"""

from __future__ import annotations

import numpy as np
import torch

DEFAULT_SEED = 42  # rotation.py:14

_rotation_cache: dict[tuple[int, int], np.ndarray] = {}
_device_cache: dict[tuple[int, int, str], torch.Tensor] = {}


def generate_rotation_matrix(d: int, seed: int = DEFAULT_SEED) -> np.ndarray:
    """``Q`` of ``QR(RandomState(seed).randn(d, d).astype(f32))`` with columns
    sign-fixed by ``sign(diag(R))`` (zero signs -> +1). float32 (d, d).
    (rotation.py:17-36)"""
    rng = np.random.RandomState(seed)
    g = rng.randn(d, d).astype(np.float32)
    q, r = np.linalg.qr(g)
    signs = np.sign(np.diag(r))
    signs[signs == 0] = 1
    return np.ascontiguousarray((q * signs[np.newaxis, :]).astype(np.float32))


def get_rotation_matrix(d: int, seed: int = DEFAULT_SEED, device=None) -> torch.Tensor:
    """Cached rotation as a float32 tensor on ``device`` (default: current GPU).
    (rotation.py:39-52)"""
    key = (d, seed)
    if key not in _rotation_cache:
        _rotation_cache[key] = generate_rotation_matrix(d, seed)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    dkey = (d, seed, str(dev))
    if dkey not in _device_cache:
        _device_cache[dkey] = torch.from_numpy(_rotation_cache[key]).to(dev)
    return _device_cache[dkey]


def rotate(x: torch.Tensor, rotation: torch.Tensor) -> torch.Tensor:
    """``x @ R.T`` (rotation.py:55-65)."""
    return x.to(torch.float32) @ rotation.T


def inverse_rotate(y: torch.Tensor, rotation: torch.Tensor) -> torch.Tensor:
    """``y @ R`` (rotation.py:68-78)."""
    return y.to(torch.float32) @ rotation


def pre_rotate_query(query: torch.Tensor, rotation: torch.Tensor) -> torch.Tensor:
    """``Q @ R.T``: the query rotation used by attention over packed keys
    (rotation.py:81-110)."""
    return query.to(torch.float32) @ rotation.T
