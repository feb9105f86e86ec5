"""QJL 1-bit sign sketch (qjl.py of the reference).

The projection S (m, d) is generated on the host from RandomState(12345)
(qjl.py:23-36). The cache computes the sketch inside the compress kernel and
applies it inside the dequantize / attention kernels; the tensor-level helpers
below mirror the reference functions for users of the low-level API.
"""

from __future__ import annotations

import math

import numpy as np
import torch

DEFAULT_SEED = 12345  # qjl.py:20

_projection_cache: dict[tuple[int, int, int], np.ndarray] = {}
_device_cache: dict[tuple[int, int, int, str], torch.Tensor] = {}


def generate_projection_matrix(d: int, m: int, seed: int = DEFAULT_SEED) -> np.ndarray:
    """i.i.d. N(0,1) float32 (m, d) (qjl.py:23-36)."""
    rng = np.random.RandomState(seed)
    return np.ascontiguousarray(rng.randn(m, d).astype(np.float32))


def get_projection_matrix(d: int, m: int, seed: int = DEFAULT_SEED, device=None) -> torch.Tensor:
    key = (d, m, seed)
    if key not in _projection_cache:
        _projection_cache[key] = generate_projection_matrix(d, m, seed)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    dkey = (d, m, seed, str(dev))
    if dkey not in _device_cache:
        _device_cache[dkey] = torch.from_numpy(_projection_cache[key]).to(dev)
    return _device_cache[dkey]


def qjl_quantize(residual: torch.Tensor, projection: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(signs = r @ S.T >= 0, norms = ||r||) (qjl.py:47-67)."""
    r = residual.to(torch.float32)
    return (r @ projection.T) >= 0, torch.linalg.vector_norm(r, dim=-1)


def qjl_dequantize(signs: torch.Tensor, norms: torch.Tensor, projection: torch.Tensor, d: int) -> torch.Tensor:
    """(sqrt(pi/2)/d) * gamma * (z @ S), z = +-1 (qjl.py:70-94)."""
    z = torch.where(signs, 1.0, -1.0).to(torch.float32)
    return (math.sqrt(math.pi / 2) / d) * norms[..., None].to(torch.float32) * (z @ projection)
