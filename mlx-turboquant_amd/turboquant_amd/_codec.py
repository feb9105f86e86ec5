"""Device-side codec (rotation + codebooks + QJL projection) and packed stores.

A :class:`DeviceCodec` owns the GPU tensors a ``tq_codec`` points at and is
shared by every cache / quantizer with the same (d, bits, seed, qjl_m, device).
A :class:`PackedStore` holds one side (keys or values) of a compressed cache
as (batch, heads, capacity, row_bytes) uint8 codes plus float32 norms and the
optional QJL sketch, grown in large steps instead of re-concatenated per drain
(the reference concatenates per drain, cache.py:463-495).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .codebook import get_codebook
from .qjl import DEFAULT_SEED as QJL_SEED, get_projection_matrix, padded_count
from .rotation import get_rotation_matrix


def split_bits(bits: float, d: int) -> tuple[int, int, int]:
    """(bits_hi, bits_lo, split): fractional widths quantise rotated dims
    [0, d/2) at ceil(bits) and [d/2, d) at floor(bits) (cache.py:63-84, 253-274)."""
    if bits != int(bits):
        return int(bits) + 1, int(bits), d // 2
    return int(bits), int(bits), d


class DeviceCodec:
    def __init__(self, d: int, bits: float, seed: int, qjl_m: int, device: torch.device, qjl_seed: int = QJL_SEED):
        self.d = d
        self.bits = bits
        self.bits_hi, self.bits_lo, self.split = split_bits(bits, d)
        if self.bits_hi not in (1, 2, 3, 4) or self.bits_lo not in (1, 2, 3, 4):
            raise ValueError(f"Unsupported bit-width: {bits}. Use 1, 2, 3, or 4.")
        self.device = device
        self.rotation = get_rotation_matrix(d, seed, device)
        # MFMA operands of the K4/V2 decode kernels' query rotation: fp16
        # high part and remainder of R, as 16-bit words
        hi = self.rotation.half()
        self.rotation_parts = torch.stack([
            hi.view(torch.int16), (self.rotation - hi.float()).half().view(torch.int16)]).contiguous()
        self.c_hi, self.b_hi = get_codebook(d, self.bits_hi, device)
        self.c_lo, self.b_lo = get_codebook(d, self.bits_lo, device)
        # the sketch's m projections, held as qjl_mp rows (zero rows past m)
        self.qjl_m = qjl_m
        self.qjl_mp = padded_count(qjl_m) if qjl_m else 0
        self.qjl_seed = qjl_seed
        self.proj = get_projection_matrix(d, qjl_m, qjl_seed, device=device, padded=True) if qjl_m else None
        self.row_hi = self.split * self.bits_hi // 8
        self.row_lo = (d - self.split) * self.bits_lo // 8
        self.row_sign = self.qjl_mp // 8
        self.struct = _lib.Codec(
            d=d, bits_hi=self.bits_hi, bits_lo=self.bits_lo, split=self.split,
            rotation=self.rotation.data_ptr(), centroids_hi=self.c_hi.data_ptr(),
            boundaries_hi=self.b_hi.data_ptr(), centroids_lo=self.c_lo.data_ptr(),
            boundaries_lo=self.b_lo.data_ptr(),
            qjl_proj=self.proj.data_ptr() if self.proj is not None else None,
            qjl_m=self.qjl_mp, flags=0, rotation_parts=self.rotation_parts.data_ptr())
        # host-side tables: the codebook by value and, for 2-bit codebooks,
        # its exact fp16 copy (the K4/V2 decode kernels' value table)
        cen = self.c_hi.detach().cpu().numpy().astype("float32")
        lib = _lib.load()
        _lib.check(lib.tq_codec_prepare(ctypes.byref(self.struct), cen.ctypes.data, len(cen)), "tq_codec_prepare")
        # decode table of the K4/V2 kernels (4-bit keys / 2-bit values), in device memory
        self.decode_table = None
        if len(cen) in (4, 16):
            import numpy as np
            tab = np.zeros(256, np.uint64)
            _lib.check(lib.tq_codec_decode_table(ctypes.byref(self.struct), tab.ctypes.data), "tq_codec_decode_table")
            self.decode_table = torch.from_numpy(tab.view(np.int64)).to(device)
            self.struct.decode_table = self.decode_table.data_ptr()
        self._cen_host = cen

    @property
    def fractional(self) -> bool:
        return self.split < self.d

    def ref(self, general_compress: bool = False):
        """``tq_codec*`` of this codec; ``general_compress`` routes tq_compress
        through the general kernel (a copy of the struct with the flag set)."""
        if not general_compress:
            return ctypes.byref(self.struct)
        c = _lib.Codec.from_buffer_copy(self.struct)
        c.flags |= _lib.TQ_CODEC_GENERAL_COMPRESS
        return ctypes.byref(c)


_codecs: dict[tuple, DeviceCodec] = {}


_supported: dict[str, bool] = {}


def _require_gfx950(dev: torch.device) -> None:
    """The library holds gfx950 code objects only; refuse other devices."""
    if dev.type != "cuda":
        raise RuntimeError("turboquant_amd runs on the GPU only; got device " + str(dev))
    if str(dev) not in _supported:
        with torch.cuda.device(dev):
            _supported[str(dev)] = bool(_lib.load().tq_device_supported())
    if not _supported[str(dev)]:
        raise RuntimeError(f"turboquant_amd: {dev} is not a gfx950 (MI355X) device")


def get_codec(d: int, bits: float, seed: int, qjl_m: int, device, qjl_seed: int = QJL_SEED) -> DeviceCodec:
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    key = (d, float(bits), seed, qjl_m, qjl_seed if qjl_m else None, str(dev))
    if key not in _codecs:
        _require_gfx950(dev)
        _codecs[key] = DeviceCodec(d, bits, seed, qjl_m, dev, qjl_seed)
    return _codecs[key]


class PackedStore:
    """One side of a compressed cache: (B, H, cap, ...) tensors."""

    GROW = 4096  # tokens

    def __init__(self, codec: DeviceCodec, batch: int, heads: int, qjl: bool):
        self.codec = codec
        self.batch, self.heads = batch, heads
        self.qjl = qjl
        self.cap = 0
        self.codes_hi = self.codes_lo = self.norms = self.signs = self.gamma = None

    def _alloc(self, cap: int):
        c, dev, B, H = self.codec, self.codec.device, self.batch, self.heads
        u8 = dict(dtype=torch.uint8, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        new = {
            "codes_hi": torch.zeros(B, H, cap, c.row_hi, **u8),
            "codes_lo": torch.zeros(B, H, cap, c.row_lo, **u8) if c.fractional else None,
            "norms": torch.zeros(B, H, cap, **f32),
            "signs": torch.zeros(B, H, cap, c.row_sign, **u8) if self.qjl else None,
            "gamma": torch.zeros(B, H, cap, **f32) if self.qjl else None,
        }
        return new

    def reserve(self, n_tokens: int, keep: int) -> None:
        """Ensure capacity for ``n_tokens``; copies the first ``keep`` tokens."""
        if n_tokens <= self.cap:
            return
        cap = max(n_tokens, self.cap + self.cap // 2, self.GROW)
        cap = (cap + self.GROW - 1) // self.GROW * self.GROW
        new = self._alloc(cap)
        for name, t in new.items():
            old = getattr(self, name)
            if t is not None and old is not None and keep > 0:
                t[:, :, :keep].copy_(old[:, :, :keep])
            setattr(self, name, t)
        self.cap = cap

    def struct(self, tok0: int = 0) -> _lib.Store:
        """``tq_store`` whose token 0 is token ``tok0`` of this store."""
        c = self.codec

        def at(t, row):
            return None if t is None else t.data_ptr() + tok0 * row

        return _lib.Store(
            codes_hi=at(self.codes_hi, c.row_hi), hi_head_stride=self.cap * c.row_hi,
            codes_lo=at(self.codes_lo, c.row_lo), lo_head_stride=self.cap * c.row_lo,
            norms=at(self.norms, 4), norm_head_stride=self.cap,
            signs=at(self.signs, c.row_sign), sign_head_stride=self.cap * c.row_sign,
            gamma=at(self.gamma, 4), gamma_head_stride=self.cap)


def compress_into(codec: DeviceCodec, x: torch.Tensor, x_tok0: int, n_tok: int,
                  store: PackedStore, dst_tok0: int, general: bool = False) -> None:
    """Compress tokens [x_tok0, x_tok0 + n_tok) of x (B, H, T, D), contiguous in
    its last two dims with head stride x.stride(1), into store tokens
    [dst_tok0, dst_tok0 + n_tok). ``general`` selects the general compress
    kernel (tests compare it with the MFMA kernel)."""
    if n_tok <= 0:
        return
    B, H, T, D = x.shape
    assert x.stride(3) == 1 and x.stride(2) == D and x.stride(0) == H * x.stride(1)
    span = _lib.Span(rows=B * H, heads=H, n_tok=n_tok, reserved=0, n_tok_b=None, src_tok0_b=None, dst_tok0_b=None)
    st = store.struct(dst_tok0)
    xp = x.data_ptr() + x_tok0 * D * x.element_size()
    lib = _lib.load()
    _lib.check(lib.tq_compress(codec.ref(general), xp, _lib.dtype_code(x.dtype), x.stride(1), ctypes.byref(span),
                               ctypes.byref(st), _lib.stream_ptr(x.device)), "tq_compress")


def dequantize_into(codec: DeviceCodec, store: PackedStore, src_tok0: int, n_tok: int,
                    out: torch.Tensor, out_tok0: int, apply_qjl: bool) -> None:
    """Dequantize store tokens [src_tok0, +n_tok) into out (B, H, T, D) float32
    tokens [out_tok0, +n_tok)."""
    if n_tok <= 0:
        return
    B, H, T, D = out.shape
    assert out.dtype == torch.float32 and out.stride(3) == 1 and out.stride(2) == D
    span = _lib.Span(rows=B * H, heads=H, n_tok=n_tok, reserved=0, n_tok_b=None, src_tok0_b=None, dst_tok0_b=None)
    st = store.struct(src_tok0)
    op = out.data_ptr() + out_tok0 * D * 4
    lib = _lib.load()
    _lib.check(lib.tq_dequantize(codec.ref(), ctypes.byref(st), ctypes.byref(span), op, out.stride(1),
                                 1 if apply_qjl else 0, _lib.stream_ptr(out.device)), "tq_dequantize")
