"""TurboQuant KV cache for PyTorch decode loops (cache.py of the reference).

Same constructor, drain policy and duck-typed protocol as the reference's
``TurboQuantKVCache`` (cache.py:19-724): ``update_and_fetch``, ``offset``,
``state`` / ``meta_state``, ``make_mask``, ``empty``, ``is_trimmable``,
``size``, ``nbytes``. Storage is laid out for the GPU:

* compressed tokens live in a pre-allocated packed store grown in 4096-token
  steps (the reference concatenates per drain, cache.py:463-495);
* the fp16 residual window is a ring buffer (the reference shifts its buffer
  on every drain, cache.py:547-551);
* drained tokens are compressed straight from wherever they sit (ring or the
  incoming tensor) by one fused kernel per contiguous piece;
* ``update_and_fetch`` keeps the reference's dense float32 contract through an
  incrementally dequantised buffer, while ``attend`` runs fused decode
  attention over the packed codes and never materialises dense keys/values.
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch

from . import _codec, _lib
from .qjl import check_count as check_qjl_count
from .rotation import DEFAULT_SEED

_workspaces: dict[tuple[str, int], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Per (device, stream) attention workspace: scratch for the partials of
    one call, reused by every later call ordered on the same stream (the
    current stream unless its handle is given)."""
    key = (str(device), _lib.stream_ptr(device) if stream is None else stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


# query heads per kv head of the dense fp16 / bf16 decode kernel (the packed
# route, TurboQuantKVCache.attend, takes any integer ratio)
ATTEND_GROUPS = (1, 2, 4, 8)


def dense_attention(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                    scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of one query token per head over uncompressed K/V
    through ``tq_dense_decode_attention``: the attention of the layers kept
    on an fp16 cache (the reference's outlier / skipped layers, patch.py:337-338).

    ``queries`` (B, Hq, 1, D) or (B, Hq, D); ``keys`` / ``values`` (B, Hkv, T, D)
    fp16 or bf16 with D = 128, Hq a multiple (1, 2, 4, 8) of Hkv, rows
    contiguous (a view of a larger (B, Hkv, T_cap, D) buffer is fine).
    Returns float32 (B, Hq, 1, D) = softmax(scale q K^T) V (default scale
    D**-0.5)."""
    _lib.require_device(keys)
    q = queries[:, :, 0] if queries.dim() == 4 else queries
    q = q.contiguous()
    if q.data_ptr() % 16:
        q = q.clone()  # the kernel reads 16-byte pieces of the query rows
    B, hkv, T, D = keys.shape
    if values.shape != keys.shape or values.dtype != keys.dtype or values.stride() != keys.stride():
        raise ValueError("keys and values must have one shape, dtype and layout")
    if q.dim() != 3 or q.shape[0] != B or q.shape[2] != D:
        raise ValueError(f"query shape {tuple(queries.shape)} does not match keys {tuple(keys.shape)}")
    st = keys.stride()
    if st[3] != 1 or st[2] != D or st[0] != hkv * st[1]:
        raise ValueError("keys / values need contiguous rows and heads laid out (B, Hkv) in order")
    if out is None:
        out = torch.empty(B, q.shape[1], 1, D, dtype=torch.float32, device=q.device)
    desc = _lib.AttnDesc(
        batch=B, hq=q.shape[1], hkv=hkv, qjl=0, scale=D ** -0.5 if scale is None else scale,
        max_comp=0, max_sink=T, max_res=0, q_dtype=_lib.dtype_code(q.dtype), kv_dtype=_lib.dtype_code(keys.dtype),
        q=q.data_ptr(), out=out.data_ptr(), comp_len=None, sink_k=keys.data_ptr(), sink_v=values.data_ptr(),
        sink_head_stride=st[1], sink_len=None, res_k=None, res_v=None, res_head_stride=0, res_cap=0,
        res_start0=0, res_start=None, res_len=None, flags=0)
    lib = _lib.load()
    ws = _workspace(q.device, lib.tq_dense_decode_workspace_bytes(ctypes.byref(desc), D))
    _lib.check(lib.tq_dense_decode_attention(ctypes.byref(desc), D, ws.data_ptr(), ws.numel(),
                                             _lib.stream_ptr(q.device)), "tq_dense_decode_attention")
    return out


def drain_schedule(fp16_len: int, window: int, chunk_size: int) -> list[int]:
    """Sizes of the drains the reference performs on an fp16 buffer of
    ``fp16_len`` tokens (cache.py:497-533)."""
    if chunk_size <= 0:
        return [fp16_len - window] if fp16_len > 2 * window else []
    k = max(0, (fp16_len - window) // chunk_size) if fp16_len >= window + chunk_size else 0
    return [chunk_size] * k


class TurboQuantKVCache:
    """TurboQuant-compressed KV cache (cache.py:19-116)."""

    step = 256
    @staticmethod
    def attend_head_dim(head_dim: int) -> bool:
        """head_dims the codecs and the attention kernels take: multiples of 16
        in [16, 256] (the MFMA kernels at 128, the general kernels at all)."""
        return 16 <= head_dim <= 256 and head_dim % 16 == 0

    def __init__(self, head_dim: int = 128, num_kv_heads: int = 1, key_bits: float = 4,
                 value_bits: float = 2, residual_window: int = 128, rotation_seed: int = DEFAULT_SEED,
                 fp16_sink_size: int = 0, chunk_size: int = 0, qjl_correction: bool = False,
                 qjl_n_proj: int = 32, device=None):
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.residual_window = residual_window
        self.rotation_seed = rotation_seed
        self.fp16_sink_size = fp16_sink_size
        self.chunk_size = chunk_size
        self.qjl_correction = qjl_correction
        self.qjl_n_proj = qjl_n_proj
        if qjl_correction:
            check_qjl_count(qjl_n_proj)
        if not self.attend_head_dim(head_dim):
            raise ValueError(f"head_dim {head_dim} not supported: a multiple of 16 in [16, 256]")
        for bits in (key_bits, value_bits):
            if _codec.split_bits(bits, head_dim)[2] % 16:
                raise ValueError(f"fractional bits {bits} need head_dim a multiple of 32 (the two halves of "
                                 f"head_dim {head_dim} must be multiples of 16)")
        self._k_fractional = key_bits != int(key_bits)
        self._v_fractional = value_bits != int(value_bits)
        self._device = torch.device(device) if device is not None else None
        self._kc = self._vc = None
        # sink (cache.py:86-92)
        self.sink_keys: torch.Tensor | None = None
        self.sink_values: torch.Tensor | None = None
        self._sink_len = 0
        # fp16 residual ring
        self._res_k: torch.Tensor | None = None
        self._res_v: torch.Tensor | None = None
        self._res_start = 0
        self._fp16_len = 0
        # compressed stores
        self._kstore: _codec.PackedStore | None = None
        self._vstore: _codec.PackedStore | None = None
        self._compressed_len = 0
        # dense float32 view for update_and_fetch (lazy)
        self._dense_k: torch.Tensor | None = None
        self._dense_v: torch.Tensor | None = None
        self._dense_comp = 0     # compressed tokens already dequantised into the view
        self._dense_sink = 0     # sink tokens already copied into the view
        self._B = self._H = None
        self._dtype = None
        self.offset = 0
        self.drains: list[int] = []
        self._pending_meta: dict | None = None  # meta_state set before state

    # ------------------------------------------------------------------ setup
    def _setup(self, keys: torch.Tensor) -> None:
        if self._B is not None:
            return
        B, H, _, D = keys.shape
        if D != self.head_dim:
            raise ValueError(f"head_dim {D} != cache head_dim {self.head_dim}")
        _lib.require_device(keys)
        self._device = keys.device
        self._B, self._H, self._dtype = B, H, keys.dtype
        m = self.qjl_n_proj if self.qjl_correction else 0
        self._kc = _codec.get_codec(D, self.key_bits, self.rotation_seed, m, keys.device)
        self._vc = _codec.get_codec(D, self.value_bits, self.rotation_seed, m, keys.device)
        self._kstore = _codec.PackedStore(self._kc, B, H, qjl=m > 0)
        self._vstore = _codec.PackedStore(self._vc, B, H, qjl=m > 0)

    @property
    def rotation(self) -> torch.Tensor:
        return self._kc.rotation if self._kc is not None else None

    @property
    def _res_cap(self) -> int:
        return 0 if self._res_k is None else self._res_k.shape[2]

    def _ring_capacity(self) -> int:
        w = self.residual_window
        cap = 2 * w if self.chunk_size <= 0 else w + self.chunk_size
        return max(cap, 1)

    def _ring_pieces(self, start: int, n: int) -> list[tuple[int, int, int]]:
        """Contiguous (ring_pos, logical_offset, length) pieces of n ring tokens
        beginning ``start`` tokens after the ring start."""
        cap = self._res_cap
        out = []
        pos = (self._res_start + start) % cap
        done = 0
        while done < n:
            ln = min(n - done, cap - pos)
            out.append((pos, done, ln))
            done += ln
            pos = 0
        return out

    # ----------------------------------------------------------------- update
    def _route_sink(self, keys, values):
        """First ``fp16_sink_size`` absolute positions go to a permanent sink
        (cache.py:577-618)."""
        if self.fp16_sink_size <= 0 or self.offset >= self.fp16_sink_size:
            return keys, values
        T = keys.shape[2]
        n = min(self.fp16_sink_size - self.offset, T)
        if n <= 0:
            return keys, values
        if self.sink_keys is None:
            B, H, _, D = keys.shape
            self.sink_keys = torch.zeros(B, H, self.fp16_sink_size, D, dtype=keys.dtype, device=keys.device)
            self.sink_values = torch.zeros(B, H, self.fp16_sink_size, D, dtype=values.dtype, device=values.device)
        self.sink_keys[:, :, self.offset:self.offset + n] = keys[:, :, :n]
        self.sink_values[:, :, self.offset:self.offset + n] = values[:, :, :n]
        self._sink_len = self.offset + n
        return keys[:, :, n:], values[:, :, n:]

    def update(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append keys/values (B, H, T, D) and drain old tokens into the
        compressed store, without building dense outputs."""
        if keys.shape != values.shape:
            raise ValueError("keys and values must have the same shape")
        T_total = keys.shape[2]
        if T_total == 0:
            return
        self._setup(keys)
        if keys.dtype != self._dtype:
            keys, values = keys.to(self._dtype), values.to(self._dtype)
        keys, values = self._route_sink(keys, values)
        self.offset += T_total
        T_new = keys.shape[2]
        if T_new == 0:
            return
        keys, values = keys.contiguous(), values.contiguous()
        L = self._fp16_len
        drains = drain_schedule(L + T_new, self.residual_window, self.chunk_size)
        n_drain = sum(drains)
        if n_drain:
            self._compress(keys, values, L, n_drain)
            self.drains.extend(drains)
        # append the surviving new tokens to the ring
        from_ring = min(n_drain, L)
        self._res_start = (self._res_start + from_ring) % max(self._res_cap, 1)
        self._fp16_len = L - from_ring
        first_new = n_drain - from_ring
        n_keep = T_new - first_new
        if n_keep > 0:
            if self._res_k is None:
                B, H, _, D = keys.shape
                cap = max(self._ring_capacity(), n_keep)
                self._res_k = torch.zeros(B, H, cap, D, dtype=self._dtype, device=keys.device)
                self._res_v = torch.zeros_like(self._res_k)
                self._res_start = 0
            for pos, off, ln in self._ring_pieces(self._fp16_len, n_keep):
                self._res_k[:, :, pos:pos + ln] = keys[:, :, first_new + off:first_new + off + ln]
                self._res_v[:, :, pos:pos + ln] = values[:, :, first_new + off:first_new + off + ln]
            self._fp16_len += n_keep

    def _compress(self, keys, values, L, n_drain):
        """Compress logical tokens [0, n_drain) of [ring (L) ++ new] into the
        store at [compressed_len, compressed_len + n_drain)."""
        c0 = self._compressed_len
        self._kstore.reserve(c0 + n_drain, c0)
        self._vstore.reserve(c0 + n_drain, c0)
        n_ring = min(n_drain, L)
        if n_ring:
            for pos, off, ln in self._ring_pieces(0, n_ring):
                _codec.compress_into(self._kc, self._res_k, pos, ln, self._kstore, c0 + off)
                _codec.compress_into(self._vc, self._res_v, pos, ln, self._vstore, c0 + off)
        n_new = n_drain - n_ring
        if n_new:
            _codec.compress_into(self._kc, keys, 0, n_new, self._kstore, c0 + n_ring)
            _codec.compress_into(self._vc, values, 0, n_new, self._vstore, c0 + n_ring)
        self._compressed_len = c0 + n_drain

    # ------------------------------------------------------------ dense fetch
    def _residual_linear(self, out_dtype=None) -> tuple[torch.Tensor, torch.Tensor]:
        n = self._fp16_len
        if n == 0:
            e = self._res_k[:, :, :0] if self._res_k is not None else None
            return e, e
        pieces = self._ring_pieces(0, n)
        if len(pieces) == 1:
            pos, _, ln = pieces[0]
            k, v = self._res_k[:, :, pos:pos + ln], self._res_v[:, :, pos:pos + ln]
        else:
            k = torch.cat([self._res_k[:, :, p:p + ln] for p, _, ln in pieces], dim=2)
            v = torch.cat([self._res_v[:, :, p:p + ln] for p, _, ln in pieces], dim=2)
        if out_dtype is not None:
            k, v = k.to(out_dtype), v.to(out_dtype)
        return k, v

    def _ensure_dense(self, total: int) -> None:
        B, H, D = self._B, self._H, self.head_dim
        cap = 0 if self._dense_k is None else self._dense_k.shape[2]
        if total <= cap:
            return
        new_cap = max(total, cap + cap // 2, 4096)
        new_cap = (new_cap + 4095) // 4096 * 4096
        nk = torch.empty(B, H, new_cap, D, dtype=torch.float32, device=self._device)
        nv = torch.empty_like(nk)
        keep = self._sink_len + self._dense_comp if self._dense_k is not None else 0
        if keep:
            nk[:, :, :keep].copy_(self._dense_k[:, :, :keep])
            nv[:, :, :keep].copy_(self._dense_v[:, :, :keep])
        self._dense_k, self._dense_v = nk, nv

    def fetch(self) -> tuple[torch.Tensor, torch.Tensor]:
        """[sink | dequantised compressed | residual] (cache.py:674-706)."""
        if self._compressed_len == 0:
            parts_k, parts_v = [], []
            if self._sink_len > 0:
                parts_k.append(self.sink_keys[:, :, :self._sink_len])
                parts_v.append(self.sink_values[:, :, :self._sink_len])
            if self._fp16_len > 0:
                k, v = self._residual_linear()
                parts_k.append(k)
                parts_v.append(v)
            if not parts_k:
                return None, None
            if len(parts_k) == 1:
                return parts_k[0], parts_v[0]
            return torch.cat(parts_k, dim=2), torch.cat(parts_v, dim=2)
        S, C, R = self._sink_len, self._compressed_len, self._fp16_len
        self._ensure_dense(S + C + R)
        dk, dv = self._dense_k, self._dense_v
        if self._dense_sink < S:
            dk[:, :, self._dense_sink:S] = self.sink_keys[:, :, self._dense_sink:S]
            dv[:, :, self._dense_sink:S] = self.sink_values[:, :, self._dense_sink:S]
            self._dense_sink = S
        if self._dense_comp < C:
            n = C - self._dense_comp
            apply = self.qjl_correction
            _codec.dequantize_into(self._kc, self._kstore, self._dense_comp, n, dk, S + self._dense_comp, apply)
            _codec.dequantize_into(self._vc, self._vstore, self._dense_comp, n, dv, S + self._dense_comp, apply)
            self._dense_comp = C
        if R:
            for pos, off, ln in self._ring_pieces(0, R):
                dk[:, :, S + C + off:S + C + off + ln] = self._res_k[:, :, pos:pos + ln]
                dv[:, :, S + C + off:S + C + off + ln] = self._res_v[:, :, pos:pos + ln]
        return dk[:, :, :S + C + R], dv[:, :, :S + C + R]

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append and return all keys/values for attention (cache.py:620-706).

        float32 once anything is compressed, the input dtype before. The
        returned tensors are views of internal buffers, valid until the next
        update."""
        self.update(keys, values)
        k, v = self.fetch()
        if k is None:
            return keys[:, :, :0], values[:, :, :0]
        return k, v

    # ------------------------------------------------------- fused attention
    def attention_descriptor(self, q: torch.Tensor, out: torch.Tensor, scale: float,
                             general: bool = False) -> _lib.AttnDesc:
        B, H = self._B, self._H
        hq = q.shape[1]
        empty = _lib.Store()
        ks = self._kstore.struct(0) if self._compressed_len else empty
        vs = self._vstore.struct(0) if self._compressed_len else empty
        return _lib.AttnDesc(
            batch=B, hq=hq, hkv=H, qjl=1 if self.qjl_correction else 0,
            scale=scale, max_comp=self._compressed_len, max_sink=self._sink_len, max_res=self._fp16_len,
            q_dtype=_lib.dtype_code(q.dtype), kv_dtype=_lib.dtype_code(self._dtype),
            q=q.data_ptr(), out=out.data_ptr(), kstore=ks, vstore=vs, comp_len=None,
            sink_k=_lib.ptr(self.sink_keys), sink_v=_lib.ptr(self.sink_values),
            sink_head_stride=self.fp16_sink_size * self.head_dim, sink_len=None,
            res_k=_lib.ptr(self._res_k), res_v=_lib.ptr(self._res_v),
            res_head_stride=self._res_cap * self.head_dim, res_cap=self._res_cap,
            res_start0=self._res_start, res_start=None, res_len=None,
            flags=_lib.TQ_ATTN_GENERAL if general else 0)

    def attend(self, queries: torch.Tensor, scale: float | None = None,
               out: torch.Tensor | None = None, general_kernel: bool = False) -> torch.Tensor:
        """Attention of the query tokens over the whole cache, scoring
        compressed tokens directly from packed codes.

        ``queries``: (B, Hq, T_q, D) or (B, Hq, D) (T_q = 1); Hq any multiple
        of the kv heads, query head h reads kv head h // (Hq / Hkv). With T_q
        > 1 the queries are the cache's last T_q tokens and attend causally:
        query i sees the first offset - T_q + i + 1 tokens (the reference's
        "causal" prefill mask, cache.py:722-724). Returns float32
        (B, Hq, T_q, D): softmax(scale * q K^T) V over the same tokens
        update_and_fetch would return (default scale D**-0.5).
        ``general_kernel`` forces the general kernel where the K4/V2 fast
        kernels would run (used to cross-check the two)."""
        if self._B is None or self.offset == 0:
            raise ValueError("attend() on an empty cache")
        q = queries if queries.dim() == 4 else queries[:, :, None]
        q = q.contiguous()
        B, hq, tq, D = q.shape
        if B != self._B or D != self.head_dim:
            raise ValueError(f"query shape {tuple(queries.shape)} does not match the cache")
        if tq > self.offset:
            raise ValueError(f"{tq} query tokens > the {self.offset} cached tokens")
        if scale is None:
            scale = D ** -0.5
        if out is None:
            out = torch.empty(B, hq, tq, D, dtype=torch.float32, device=q.device)
        desc = self.attention_descriptor(q, out, scale, general_kernel)
        desc.n_q = tq
        lib = _lib.load()
        need = lib.tq_attention_workspace_bytes(self._kc.ref(), self._vc.ref(), ctypes.byref(desc))
        ws = _workspace(q.device, need)
        _lib.check(lib.tq_decode_attention(self._kc.ref(), self._vc.ref(), ctypes.byref(desc), ws.data_ptr(),
                                           ws.numel(), _lib.stream_ptr(q.device)), "tq_decode_attention")
        return out

    # ------------------------------------------------------------- protocol
    @property
    def keys(self):
        return self._residual_linear()[0] if self._res_k is not None else None

    @property
    def values(self):
        return self._residual_linear()[1] if self._res_k is not None else None

    # ------------------------------------------------------- saved state
    @property
    def state(self) -> tuple:
        """The reference's 10-tuple (cache.py:118-131): (keys, values,
        compressed_keys, compressed_key_norms, compressed_values,
        compressed_value_norms, sink_keys, sink_values, compressed_keys_lo,
        compressed_values_lo), as torch tensors on the cache's device.

        keys / values hold the residual window in order, (B, H, fp16_len, D),
        so meta_state's fp16_capacity equals fp16_len. Packed codes are
        (B, H, compressed_len, row bytes) uint8 and norms (B, H,
        compressed_len) float32, the reference's layouts; the lo parts are
        None for integer widths. With qjl_correction four more entries follow
        (key signs, key gamma, value signs, value gamma), so a reload keeps
        the correction; the reference stores no sketch."""
        if self._B is None:
            return (None,) * 10
        keys, values = self._residual_linear() if self._res_k is not None and self._fp16_len else (None, None)
        if keys is not None:
            keys, values = keys.contiguous().clone(), values.contiguous().clone()
        sk = self.sink_keys.clone() if self.sink_keys is not None else None
        sv = self.sink_values.clone() if self.sink_values is not None else None
        kh, kl, kn = self.packed("k")
        vh, vl, vn = self.packed("v")
        out = (keys, values, kh, kn, vh, vn, sk, sv, kl, vl)
        if self.qjl_correction:
            ks, vs = self.sketch("k"), self.sketch("v")
            out += (ks[0] if ks else None, ks[1] if ks else None, vs[0] if vs else None, vs[1] if vs else None)
        return out

    @state.setter
    def state(self, v) -> None:
        """Load a saved tuple (cache.py:133-173): 6 entries (no sink, no lo
        parts), 8 (with sink), 10 (with sink and lo parts) or 14 (this build's
        tuple with the QJL sketch). Entries may be torch tensors on any device
        or numpy arrays. Lengths come from a meta_state set before or after
        (mlx-lm sets state first), else from the array shapes. Compressed
        tokens loaded without a sketch get gamma = 0, so QJL corrects only the
        tokens compressed after the reload, as in the reference."""
        n = len(v)
        if n not in (6, 8, 10, 14):
            raise ValueError(f"state tuple of {n} entries; expected 6, 8, 10 or 14")
        v = list(v) + [None] * (14 - n)
        keys, values, kh, kn, vh, vn, sk, sv, kl, vl, ks, kg, vs, vg = v
        dev = self._device
        if dev is None:
            if torch.cuda.is_available():
                dev = torch.device("cuda", torch.cuda.current_device())
            else:  # host-only use (tests): the tensors' own device
                dev = next((t.device for t in v if isinstance(t, torch.Tensor)), torch.device("cpu"))

        def dev_t(a):
            if a is None:
                return None
            t = a if isinstance(a, torch.Tensor) else torch.as_tensor(np.asarray(a))
            return t.to(dev)

        keys, values, kh, kn, vh, vn, sk, sv, kl, vl, ks, kg, vs, vg = map(
            dev_t, (keys, values, kh, kn, vh, vn, sk, sv, kl, vl, ks, kg, vs, vg))
        shape_src = next((t for t in (keys, sk) if t is not None), None)
        if shape_src is not None:
            B, H, D, dtype = shape_src.shape[0], shape_src.shape[1], shape_src.shape[3], shape_src.dtype
        elif kh is not None:
            B, H, D, dtype = kh.shape[0], kh.shape[1], self.head_dim, torch.float16
        else:
            self.__init__(**self._ctor_args())
            return
        if D != self.head_dim:
            raise ValueError(f"state head_dim {D} != cache head_dim {self.head_dim}")
        meta = self._pending_meta
        self.__init__(**self._ctor_args())
        self._setup(torch.empty(B, H, 0, D, dtype=dtype, device=dev))
        C = kh.shape[2] if kh is not None else 0
        R = keys.shape[2] if keys is not None else 0
        S = sk.shape[2] if sk is not None else 0
        if meta is not None:
            C = min(C, meta.get("compressed_len", C))
            R = min(R, meta.get("fp16_len", R))
            S = min(S, meta.get("sink_len", S))
        if sk is not None:
            cap_s = max(self.fp16_sink_size, sk.shape[2])
            self.sink_keys = torch.zeros(B, H, cap_s, D, dtype=dtype, device=dev)
            self.sink_values = torch.zeros_like(self.sink_keys)
            self.sink_keys[:, :, :S] = sk[:, :, :S].to(dtype)
            self.sink_values[:, :, :S] = sv[:, :, :S].to(dtype)
            self._sink_len = S
        if C:
            for st, codes_hi, codes_lo, norms, signs, gamma, side in (
                    (self._kstore, kh, kl, kn, ks, kg, "key"), (self._vstore, vh, vl, vn, vs, vg, "value")):
                c = st.codec
                if codes_hi.shape[-1] != c.row_hi or (c.fractional and (codes_lo is None or codes_lo.shape[-1] != c.row_lo)):
                    raise ValueError(f"saved {side} codes do not match {side} bits of this cache")
                st.reserve(C, 0)
                st.codes_hi[:, :, :C] = codes_hi[:, :, :C].to(torch.uint8)
                if c.fractional:
                    st.codes_lo[:, :, :C] = codes_lo[:, :, :C].to(torch.uint8)
                st.norms[:, :, :C] = norms.reshape(B, H, -1)[:, :, :C].float()
                if st.signs is not None and signs is not None and gamma is not None:
                    st.signs[:, :, :C] = signs[:, :, :C].to(torch.uint8)
                    st.gamma[:, :, :C] = gamma.reshape(B, H, -1)[:, :, :C].float()
            self._compressed_len = C
        if R:
            cap = max(self._ring_capacity(), R)
            self._res_k = torch.zeros(B, H, cap, D, dtype=dtype, device=dev)
            self._res_v = torch.zeros_like(self._res_k)
            self._res_k[:, :, :R] = keys[:, :, :R].to(dtype)
            self._res_v[:, :, :R] = values[:, :, :R].to(dtype)
            self._res_start = 0
            self._fp16_len = R
        self.offset = meta["offset"] if meta is not None and "offset" in meta else S + C + R
        self._pending_meta = None

    @property
    def meta_state(self) -> dict:
        """The reference's string dict (cache.py:175-187)."""
        return {
            "offset": str(self.offset),
            "compressed_len": str(self._compressed_len),
            "head_dim": str(self.head_dim),
            "key_bits": str(self.key_bits),
            "value_bits": str(self.value_bits),
            "fp16_sink_size": str(self.fp16_sink_size),
            "sink_len": str(self._sink_len),
            "fp16_len": str(self._fp16_len),
            "fp16_capacity": str(self._fp16_len),
        }

    @meta_state.setter
    def meta_state(self, v) -> None:
        """Lengths of a saved cache (cache.py:189-200). Applied to a state
        already loaded, or kept for the state setter when it comes first."""
        meta = {"offset": int(v["offset"]), "compressed_len": int(v["compressed_len"])}
        for key in ("sink_len", "fp16_len"):
            if key in v:
                meta[key] = int(v[key])
        if "fp16_sink_size" in v:
            self.fp16_sink_size = int(v["fp16_sink_size"])
        if self._B is None:
            self._pending_meta = meta
            self.offset = meta["offset"]
            return
        for key, attr in (("compressed_len", "_compressed_len"), ("sink_len", "_sink_len"), ("fp16_len", "_fp16_len")):
            if key in meta:
                if meta[key] > getattr(self, attr):
                    raise ValueError(f"meta_state {key} {meta[key]} exceeds the loaded state's {getattr(self, attr)}")
                setattr(self, attr, meta[key])
        self._dense_comp = min(self._dense_comp, self._compressed_len)
        self._dense_sink = min(self._dense_sink, self._sink_len)
        self.offset = meta["offset"]

    def _ctor_args(self) -> dict:
        return dict(head_dim=self.head_dim, num_kv_heads=self.num_kv_heads, key_bits=self.key_bits,
                    value_bits=self.value_bits, residual_window=self.residual_window,
                    rotation_seed=self.rotation_seed, fp16_sink_size=self.fp16_sink_size,
                    chunk_size=self.chunk_size, qjl_correction=self.qjl_correction,
                    qjl_n_proj=self.qjl_n_proj, device=self._device)

    def empty(self) -> bool:
        return self._fp16_len == 0 and self._compressed_len == 0 and self._sink_len == 0

    def is_trimmable(self) -> bool:
        return False

    def size(self) -> int:
        return self.offset

    @property
    def nbytes(self) -> int:
        """Bytes held, counted as the reference does (cache.py:211-230):
        fp16 buffers at 4 bytes per element, packed arrays at their size."""
        total = 0
        D = self.head_dim
        if self._fp16_len > 0:
            total += 2 * self._B * self._H * self._fp16_len * D * 4
        if self._sink_len > 0:
            total += 2 * self._B * self._H * self._sink_len * D * 4
        if self._compressed_len > 0:
            n = self._B * self._H * self._compressed_len
            for c in (self._kc, self._vc):
                total += n * (c.row_hi + c.row_lo) + n * 4
        return total

    def make_mask(self, N: int, offset: int = 0, return_array: bool = False,
                  window_size: int | None = None) -> Any | None:
        """None for single-token decode, "causal" otherwise (cache.py:708-724)."""
        if window_size is not None:
            raise NotImplementedError(
                "TurboQuantKVCache does not support sliding-window attention "
                f"(window_size={window_size}). Use the model's default cache "
                "for sliding-window layers.")
        if N == 1 and not return_array:
            return None
        return "causal"

    # ----------------------------------------------------- packed accessors
    def packed(self, side: str = "k") -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
        """(codes_hi, codes_lo, norms) views of the valid compressed tokens."""
        st = self._kstore if side == "k" else self._vstore
        C = self._compressed_len
        if st is None or C == 0:
            return None, None, None
        lo = st.codes_lo[:, :, :C] if st.codes_lo is not None else None
        return st.codes_hi[:, :, :C], lo, st.norms[:, :, :C]

    def sketch(self, side: str = "k") -> tuple[torch.Tensor, torch.Tensor] | None:
        st = self._kstore if side == "k" else self._vstore
        C = self._compressed_len
        if st is None or st.signs is None or C == 0:
            return None
        return st.signs[:, :, :C], st.gamma[:, :, :C]
