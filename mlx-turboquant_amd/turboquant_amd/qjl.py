"""QJL 1-bit sign sketch (qjl.py of the reference).

The projection S (m, d) is generated on the host from RandomState(seed),
12345 by default (qjl.py:23-36). The cache computes the sketch inside the
compress kernel and applies it inside the dequantize / attention kernels; the
tensor-level helpers below mirror the reference functions for users of the
low-level API.

Any m in [1, MAX_PROJ] is accepted. The kernels work on whole 32-projection
words, so a codec holds S padded with zero rows to padded_count(m): a zero row
projects every residual to 0, whose sign (>= 0) is +1, and it adds 0 to every
correction sum z @ S and S q, so the padded sketch gives the same corrected
values and scores as the (m, d) one; only the stored sign rows carry the
extra (constant) bits.
"""

from __future__ import annotations

import math

import numpy as np
import torch

DEFAULT_SEED = 12345  # qjl.py:20
MAX_PROJ = 256       # projections the attention kernels hold per query head


def padded_count(m: int) -> int:
    """m rounded up to whole 32-projection words (the kernels' unit)."""
    return (m + 31) // 32 * 32


def check_count(m: int, what: str = "qjl_n_proj") -> None:
    if not (isinstance(m, (int, np.integer)) and 1 <= m <= MAX_PROJ):
        raise ValueError(f"{what} {m} must be an integer in [1, {MAX_PROJ}]")

_projection_cache: dict[tuple[int, int, int], np.ndarray] = {}
_device_cache: dict[tuple[int, int, int, str], torch.Tensor] = {}


def generate_projection_matrix(d: int, m: int, seed: int = DEFAULT_SEED) -> np.ndarray:
    """i.i.d. N(0,1) float32 (m, d) (qjl.py:23-36)."""
    rng = np.random.RandomState(seed)
    return np.ascontiguousarray(rng.randn(m, d).astype(np.float32))


def get_projection_matrix(d: int, m: int, seed: int = DEFAULT_SEED, device=None,
                          padded: bool = False) -> torch.Tensor:
    """S (m, d) on ``device``; with ``padded`` the (padded_count(m), d) codec
    form whose rows past m are zero."""
    key = (d, m, seed)
    if key not in _projection_cache:
        _projection_cache[key] = generate_projection_matrix(d, m, seed)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    dkey = (d, m, seed, str(dev), padded)
    if dkey not in _device_cache:
        s = _projection_cache[key]
        if padded and padded_count(m) != m:
            s = np.concatenate([s, np.zeros((padded_count(m) - m, d), np.float32)])
        _device_cache[dkey] = torch.from_numpy(np.ascontiguousarray(s)).to(dev)
    return _device_cache[dkey]


def qjl_quantize(residual: torch.Tensor, projection: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(signs = r @ S.T >= 0, norms = ||r||) (qjl.py:47-67)."""
    r = residual.to(torch.float32)
    return (r @ projection.T) >= 0, torch.linalg.vector_norm(r, dim=-1)


def qjl_dequantize(signs: torch.Tensor, norms: torch.Tensor, projection: torch.Tensor, d: int) -> torch.Tensor:
    """(sqrt(pi/2)/d) * gamma * (z @ S), z = +-1 (qjl.py:70-94)."""
    z = torch.where(signs, 1.0, -1.0).to(torch.float32)
    return (math.sqrt(math.pi / 2) / d) * norms[..., None].to(torch.float32) * (z @ projection)
