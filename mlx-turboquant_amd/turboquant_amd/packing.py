"""Sub-byte code packing (packing.py of the reference).

Codes of a row form a little-endian, LSB-first bitstream: code j occupies bits
[bits*j, bits*j + bits). This is the byte layout of pack_2bit / pack_3bit /
pack_4bit / pack_1bit (packing.py:9-208); the GPU kernels pack and unpack it.
"""

from __future__ import annotations

import torch

from . import _lib


def _check_bits(bits: int) -> None:
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"Unsupported bit-width: {bits}. Use 1, 2, 3, or 4.")


def pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """(..., d) uint8 codes -> (..., d*bits/8) uint8 (packing.py:211-222)."""
    _check_bits(bits)
    _lib.require_device(indices)
    d = indices.shape[-1]
    assert (d * bits) % 8 == 0, f"Last dimension {d} must be divisible by {8 // _gcd8(bits)} for {bits}-bit packing"
    idx = indices.to(torch.uint8).contiguous()
    rows = idx.numel() // d if d else 0
    out = torch.empty(*idx.shape[:-1], d * bits // 8, dtype=torch.uint8, device=idx.device)
    lib = _lib.load()
    _lib.check(lib.tq_pack_codes(idx.data_ptr(), rows, d, bits, out.data_ptr(), _lib.stream_ptr(idx.device)),
               "pack_indices")
    return out


def unpack_indices(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """(..., d*bits/8) uint8 -> (..., d) uint8 codes (packing.py:225-236)."""
    _check_bits(bits)
    _lib.require_device(packed)
    p = packed.to(torch.uint8).contiguous()
    if p.shape[-1] * 8 != d * bits:
        raise ValueError(f"packed row of {p.shape[-1]} bytes does not hold {d} codes of {bits} bits")
    rows = p.numel() // p.shape[-1] if p.shape[-1] else 0
    out = torch.empty(*p.shape[:-1], d, dtype=torch.uint8, device=p.device)
    lib = _lib.load()
    _lib.check(lib.tq_unpack_codes(p.data_ptr(), rows, d, bits, out.data_ptr(), _lib.stream_ptr(p.device)),
               "unpack_indices")
    return out


def _gcd8(bits: int) -> int:
    import math
    return math.gcd(8, bits)


def pack_1bit(indices):
    return pack_indices(indices, 1)


def pack_2bit(indices):
    return pack_indices(indices, 2)


def pack_3bit(indices):
    return pack_indices(indices, 3)


def pack_4bit(indices):
    return pack_indices(indices, 4)


def unpack_1bit(packed, d):
    return unpack_indices(packed, 1, d)


def unpack_2bit(packed, d):
    return unpack_indices(packed, 2, d)


def unpack_3bit(packed, d):
    return unpack_indices(packed, 3, d)


def unpack_4bit(packed, d):
    return unpack_indices(packed, 4, d)
