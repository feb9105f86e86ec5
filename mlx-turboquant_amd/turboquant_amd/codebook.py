"""Lloyd-Max codebooks and the scalar quantizer (codebook.py of the reference).

The shipped tables ``codebooks/codebook_d{d}_b{bits}.npz`` are the reference's
own data (codebook.py:146-174 loads them first). Tables that do not ship are
computed by :func:`lloyd_max` on the host and cached under the user cache
directory, following codebook.py:19-28 and 55-116.
"""

from __future__ import annotations

import math
import os
from pathlib import Path

import numpy as np
import torch

from . import _lib

CODEBOOK_DIR = Path(__file__).parent / "codebooks"

_codebook_cache: dict[tuple[int, int], tuple[np.ndarray, np.ndarray]] = {}
_device_cache: dict[tuple[int, int, str], tuple[torch.Tensor, torch.Tensor]] = {}


def _user_cache_dir() -> Path:
    """$XDG_CACHE_HOME or $MLX_TURBOQUANT_CACHE, else ~/.cache (codebook.py:19-28)."""
    base = os.environ.get("XDG_CACHE_HOME") or os.environ.get("MLX_TURBOQUANT_CACHE")
    if base:
        return Path(base) / "mlx_turboquant"
    return Path.home() / ".cache" / "mlx_turboquant"


def _gaussian_pdf(x: np.ndarray, d: int) -> np.ndarray:
    var = 1.0 / d
    return np.exp(-0.5 * x * x / var) / math.sqrt(2 * math.pi * var)


def _beta_pdf(x: np.ndarray, d: int) -> np.ndarray:
    from scipy import special

    alpha = (d - 1) / 2.0
    log_norm = special.gammaln(2 * alpha) - 2 * special.gammaln(alpha) - (2 * alpha - 1) * math.log(2)
    return np.exp(log_norm + (alpha - 1) * np.log(np.maximum(1 - x * x, 1e-300)))


def lloyd_max(d: int, bits: int, num_iter: int = 500, grid_size: int = 10000) -> tuple[np.ndarray, np.ndarray]:
    """Lloyd-Max quantizer of one rotated unit-vector coordinate.

    Density: N(0, 1/d) for d >= 32, else the Beta((d-1)/2, (d-1)/2) law on
    [-1, 1]; support +-6/sqrt(d) on a uniform grid; quantile initialisation;
    boundaries at centroid midpoints; stop when a step moves no centroid by 1e-12
    (codebook.py:55-116), keeping the centroids from before the step that
    moved none by 1e-12. Returns float32 (centroids, boundaries).
    """
    levels = 1 << bits
    sigma = 1.0 / math.sqrt(d)
    lo, hi = -6 * sigma, 6 * sigma
    x = np.linspace(lo, hi, grid_size)
    dx = x[1] - x[0]
    pdf = _gaussian_pdf(x, d) if d >= 32 else _beta_pdf(x, d)
    pdf = pdf / (np.sum(pdf) * dx)
    cdf = np.cumsum(pdf) * dx
    cdf = cdf / cdf[-1]
    c = np.interp(np.linspace(0.5 / levels, 1 - 0.5 / levels, levels), cdf, x)
    for _ in range(num_iter):
        edges = np.concatenate([[lo], (c[:-1] + c[1:]) / 2.0, [hi]])
        new = np.empty(levels)
        for i in range(levels):
            upper = x <= edges[i + 1] if i == levels - 1 else x < edges[i + 1]
            sel = (x >= edges[i]) & upper
            wsum = pdf[sel].sum()
            new[i] = np.sum(x[sel] * pdf[sel]) / wsum if wsum > 0 else c[i]
        if np.max(np.abs(new - c)) < 1e-12:  # converged: the centroids before this step are kept
            break
        c = new
    b = (c[:-1] + c[1:]) / 2.0
    return c.astype(np.float32), b.astype(np.float32)


def codebook_arrays(d: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Host (centroids, boundaries): shipped file, then user cache, then computed."""
    key = (d, bits)
    if key not in _codebook_cache:
        name = f"codebook_d{d}_b{bits}.npz"
        for path in (CODEBOOK_DIR / name, _user_cache_dir() / name):
            if path.exists():
                with np.load(path, allow_pickle=False) as z:
                    _codebook_cache[key] = (z["centroids"].astype(np.float32),
                                            z["boundaries"].astype(np.float32))
                break
        else:
            c, b = lloyd_max(d, bits)
            _codebook_cache[key] = (c, b)
            try:
                path = _user_cache_dir() / name
                path.parent.mkdir(parents=True, exist_ok=True)
                np.savez(path, centroids=c, boundaries=b)
            except OSError:
                pass
    return _codebook_cache[key]


def get_codebook(d: int, bits: int, device=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(centroids, boundaries) as float32 GPU tensors (codebook.py:146-174)."""
    c, b = codebook_arrays(d, bits)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    key = (d, bits, str(dev))
    if key not in _device_cache:
        _device_cache[key] = (torch.from_numpy(c).to(dev), torch.from_numpy(b).to(dev))
    return _device_cache[key]


def precompute_codebooks(dims=(64, 96, 128, 256), bits_range=(2, 3, 4), target_dir: Path | None = None) -> None:
    """Write missing tables to ``target_dir`` (default: user cache) (codebook.py:177-200)."""
    out = Path(target_dir) if target_dir is not None else _user_cache_dir()
    out.mkdir(parents=True, exist_ok=True)
    for d in dims:
        for b in bits_range:
            path = out / f"codebook_d{d}_b{b}.npz"
            if not path.exists():
                c, bb = lloyd_max(d, b)
                np.savez(path, centroids=c, boundaries=bb)


def quantize_scalar(x: torch.Tensor, centroids: torch.Tensor, boundaries: torch.Tensor) -> torch.Tensor:
    """``idx = #{k : x > b_k}`` as uint8, same shape as x (codebook.py:203-225)."""
    _lib.require_device(x)
    y = x.to(torch.float32).contiguous()
    b = boundaries.to(device=y.device, dtype=torch.float32).contiguous()
    out = torch.empty(y.shape, dtype=torch.uint8, device=y.device)
    lib = _lib.load()
    _lib.check(lib.tq_quantize_scalar(y.data_ptr(), y.numel(), b.data_ptr(), b.numel(),
                                      out.data_ptr(), _lib.stream_ptr(y.device)), "quantize_scalar")
    return out


def dequantize_scalar(indices: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """``centroids[indices]`` (codebook.py:228-238)."""
    return centroids[indices.long()]
