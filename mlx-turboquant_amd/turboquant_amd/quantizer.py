"""Tensor-level TurboQuant quantizers (quantizer.py of the reference).

Both classes run the fused compress / dequantize HIP kernels over a flat set
of vectors; they share the numerics of the cache.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _codec
from .qjl import check_count as check_qjl_count
from .rotation import DEFAULT_SEED


@dataclass
class QuantizedTensor:
    """Compressed vectors (quantizer.py:21-31)."""
    packed_indices: torch.Tensor          # (..., d*bits/8) uint8
    norms: torch.Tensor                   # (...) float32
    bits: int
    d: int
    qjl_signs: torch.Tensor | None = None  # (..., m) bool
    qjl_norms: torch.Tensor | None = None  # (...) float32


def _flat(x: torch.Tensor, d: int) -> tuple[torch.Tensor, tuple]:
    if x.shape[-1] != d:
        raise ValueError(f"last dimension {x.shape[-1]} != d={d}")
    lead = tuple(x.shape[:-1])
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    return x.reshape(1, 1, -1, d).contiguous(), lead


def _unpack_signs(bits_u8: torch.Tensor, m: int) -> torch.Tensor:
    """The first m sign bits of LSB-first rows (the rows may hold padding)."""
    shifts = torch.arange(8, device=bits_u8.device, dtype=torch.uint8)
    bits = ((bits_u8[..., :, None] >> shifts) & 1).reshape(*bits_u8.shape[:-1], bits_u8.shape[-1] * 8)
    return bits[..., :m].bool()


def _pack_signs(signs: torch.Tensor, mp: int) -> torch.Tensor:
    """LSB-first rows of mp bits from (..., m) signs, m <= mp (the projections
    past m are zero rows of S: their bits are never used)."""
    m = signs.shape[-1]
    if mp > m:
        signs = torch.cat([signs, torch.zeros(*signs.shape[:-1], mp - m, dtype=signs.dtype, device=signs.device)], -1)
    w = (1 << torch.arange(8, device=signs.device, dtype=torch.int32))
    s = signs.reshape(*signs.shape[:-1], mp // 8, 8).to(torch.int32)
    return (s * w).sum(-1).to(torch.uint8)


class TurboQuantMSE:
    """Algorithm 1: rotate -> normalise -> Lloyd-Max quantize -> pack, storing
    codes and the float32 norm (quantizer.py:33-109)."""

    def __init__(self, d: int, bits: int = 4, seed: int = DEFAULT_SEED, device=None):
        self.d, self.bits, self.seed = d, bits, seed
        self._device = device
        self._codec_cache: dict[str, _codec.DeviceCodec] = {}
        _codec.split_bits(bits, d)

    def _codec(self, device, qjl_m: int = 0, qjl_seed: int = 12345) -> _codec.DeviceCodec:
        return _codec.get_codec(self.d, self.bits, self.seed, qjl_m, device, qjl_seed)

    @property
    def rotation(self) -> torch.Tensor:
        return self._codec(self._device or "cuda").rotation

    @property
    def centroids(self) -> torch.Tensor:
        return self._codec(self._device or "cuda").c_hi

    @property
    def boundaries(self) -> torch.Tensor:
        return self._codec(self._device or "cuda").b_hi

    def _compress(self, x: torch.Tensor, qjl_m: int = 0, qjl_seed: int = 12345):
        codec = self._codec(x.device, qjl_m, qjl_seed)
        if codec.fractional:
            raise ValueError("TurboQuantMSE takes integer bit-widths (1, 2, 3, 4)")
        flat, lead = _flat(x, self.d)
        n = flat.shape[2]
        store = _codec.PackedStore(codec, 1, 1, qjl=qjl_m > 0)
        store.reserve(max(n, 1), 0)
        _codec.compress_into(codec, flat, 0, n, store, 0)
        return codec, store, lead, n

    def quantize(self, x: torch.Tensor) -> QuantizedTensor:
        _, store, lead, n = self._compress(x)
        return QuantizedTensor(packed_indices=store.codes_hi[0, 0, :n].reshape(*lead, -1),
                               norms=store.norms[0, 0, :n].reshape(lead), bits=self.bits, d=self.d)

    def dequantize(self, qt: QuantizedTensor) -> torch.Tensor:
        codec = self._codec(qt.packed_indices.device)
        lead = tuple(qt.norms.shape)
        n = qt.norms.numel()
        store = _codec.PackedStore(codec, 1, 1, qjl=False)
        store.cap = max(n, 1)
        store.codes_hi = qt.packed_indices.reshape(1, 1, n, codec.row_hi).to(torch.uint8).contiguous()
        store.norms = qt.norms.reshape(1, 1, n).to(torch.float32).contiguous()
        out = torch.empty(1, 1, max(n, 1), self.d, dtype=torch.float32, device=qt.norms.device)
        _codec.dequantize_into(codec, store, 0, n, out, 0, apply_qjl=False)
        return out[0, 0, :n].reshape(*lead, self.d)


class TurboQuantProd:
    """Algorithm 2: (bits-1)-bit MSE stage plus a 1-bit QJL sketch of the
    residual (quantizer.py:112-195): any ``qjl_dim`` in [1, 256] and any
    ``qjl_seed`` (the projection is RandomState(qjl_seed).randn(qjl_dim, d),
    qjl.py:23-36)."""

    def __init__(self, d: int, bits: int = 4, qjl_dim: int | None = None, seed: int = DEFAULT_SEED,
                 qjl_seed: int = 12345, device=None):
        self.d, self.bits = d, bits
        self.qjl_dim = qjl_dim or d
        check_qjl_count(self.qjl_dim, "qjl_dim")
        self.qjl_seed = int(qjl_seed)
        self.mse = TurboQuantMSE(d, bits=bits - 1, seed=seed, device=device)

    def quantize(self, x: torch.Tensor) -> QuantizedTensor:
        codec, store, lead, n = self.mse._compress(x, qjl_m=self.qjl_dim, qjl_seed=self.qjl_seed)
        return QuantizedTensor(
            packed_indices=store.codes_hi[0, 0, :n].reshape(*lead, -1),
            norms=store.norms[0, 0, :n].reshape(lead), bits=self.bits, d=self.d,
            qjl_signs=_unpack_signs(store.signs[0, 0, :n], self.qjl_dim).reshape(*lead, self.qjl_dim),
            qjl_norms=store.gamma[0, 0, :n].reshape(lead))

    def dequantize(self, qt: QuantizedTensor) -> torch.Tensor:
        if qt.qjl_signs is None or qt.qjl_norms is None:
            return self.mse.dequantize(QuantizedTensor(qt.packed_indices, qt.norms, self.bits - 1, self.d))
        dev = qt.packed_indices.device
        codec = self.mse._codec(dev, self.qjl_dim, self.qjl_seed)
        lead = tuple(qt.norms.shape)
        n = qt.norms.numel()
        store = _codec.PackedStore(codec, 1, 1, qjl=True)
        store.cap = max(n, 1)
        store.codes_hi = qt.packed_indices.reshape(1, 1, n, codec.row_hi).to(torch.uint8).contiguous()
        store.norms = qt.norms.reshape(1, 1, n).to(torch.float32).contiguous()
        store.signs = _pack_signs(qt.qjl_signs.reshape(1, 1, n, self.qjl_dim), codec.qjl_mp).contiguous()
        store.gamma = qt.qjl_norms.reshape(1, 1, n).to(torch.float32).contiguous()
        out = torch.empty(1, 1, max(n, 1), self.d, dtype=torch.float32, device=dev)
        _codec.dequantize_into(codec, store, 0, n, out, 0, apply_qjl=True)
        return out[0, 0, :n].reshape(*lead, self.d)
