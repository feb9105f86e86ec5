"""Ragged decode batches: B sequences of different lengths served by one
compress launch and one attention launch per step.

The reference's cache holds one length for the whole batch (cache.py:19-116).
Serving sequences of different lengths together needs per-sequence lengths,
which the C ABI takes as arrays: ``tq_span`` n_tok_b / src_tok0_b /
dst_tok0_b for the drain (tq_compress), ``tq_attn_desc`` comp_len / sink_len /
res_len / res_start for attention (tq_decode_attention).

Each sequence keeps the layout of ``TurboQuantKVCache``: [fp16 sink |
compressed | fp16 residual window]. The batch shares one packed store per
side (rows of every sequence at their own lengths), one fp16 sink buffer and
one residual ring of window + 1 slots per sequence. A step appends one token
per sequence; a sequence whose window is full drains its oldest residual
token into the store in the same launch as the others (the reference's
chunk_size = 1 policy, cache.py:529-533). The first ``fp16_sink_size``
tokens of a sequence go to the sink (cache.py:577-618).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _codec, _lib
from .cache import _workspace
from .rotation import DEFAULT_SEED

# per-sequence ints of a tq_ragged_step call carried in its kernel arguments
# (more travel by an asynchronous copy)
_STEP_INLINE_INTS = 512


class _IntStage:
    """Host int32 arrays to the device in one asynchronous copy per call,
    through two pinned slots; a slot's host side is rewritten only after its
    previous copy has completed, and its device side is overwritten by a copy
    ordered (on the same stream) after the launches that read it."""

    def __init__(self, n: int, dev: torch.device):
        self.host = [torch.empty(n, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.host_np = [h.numpy() for h in self.host]
        self.dev = [torch.empty(n, dtype=torch.int32, device=dev) for _ in range(2)]
        self.events = [torch.cuda.Event(), torch.cuda.Event()]
        self.used = [False, False]
        self.k = 0

    def _stage(self, arrays) -> torch.Tensor:
        k = self.k
        self.k ^= 1
        if self.used[k]:
            self.events[k].synchronize()
        h = self.host_np[k]
        n = 0
        for x in arrays:
            h[n:n + len(x)] = x
            n += len(x)
        d = self.dev[k]
        if n == len(h):
            d.copy_(self.host[k], non_blocking=True)
        else:
            d[:n].copy_(self.host[k][:n], non_blocking=True)
        self.events[k].record()
        self.used[k] = True
        return d

    def put(self, *arrays) -> list[torch.Tensor]:
        """Device views of the staged arrays (valid until the call after next)."""
        d = self._stage(arrays)
        views, n = [], 0
        for x in arrays:
            views.append(d[n:n + len(x)])
            n += len(x)
        return views

    def put_ptrs(self, *arrays) -> tuple[torch.Tensor, list[int]]:
        """The staging tensor and the device address of each staged array."""
        d = self._stage(arrays)
        base, ptrs, n = d.data_ptr(), [], 0
        for x in arrays:
            ptrs.append(base + 4 * n)
            n += len(x)
        return d, ptrs


class RaggedKVBatch:
    """``batch`` sequences of one layer, ``num_kv_heads`` kv heads each. The
    per-sequence length arrays (sink_len, comp_len, res_len, res_start,
    offset) belong to the batch: load() and step() update them (and the
    device copy the next attention call reads); other code reads them only."""

    def __init__(self, batch: int, num_kv_heads: int, head_dim: int = 128, key_bits: float = 4,
                 value_bits: float = 2, residual_window: int = 128, fp16_sink_size: int = 0,
                 qjl_n_proj: int = 0, rotation_seed: int = DEFAULT_SEED, device=None):
        if residual_window < 1:
            raise ValueError("residual_window must be >= 1")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.B, self.H, self.D = batch, num_kv_heads, head_dim
        self.window, self.sink = residual_window, fp16_sink_size
        self.cap = residual_window + 1  # ring slots
        self.qjl = qjl_n_proj > 0
        self.kc = _codec.get_codec(head_dim, key_bits, rotation_seed, qjl_n_proj, dev)
        self.vc = _codec.get_codec(head_dim, value_bits, rotation_seed, qjl_n_proj, dev)
        self.kstore = _codec.PackedStore(self.kc, batch, num_kv_heads, qjl=self.qjl)
        self.vstore = _codec.PackedStore(self.vc, batch, num_kv_heads, qjl=self.qjl)
        f16 = dict(dtype=torch.float16, device=dev)
        self.sink_k = torch.zeros(batch, num_kv_heads, max(fp16_sink_size, 1), head_dim, **f16)
        self.sink_v = torch.zeros_like(self.sink_k)
        self.ring_k = torch.zeros(batch, num_kv_heads, self.cap, head_dim, **f16)
        self.ring_v = torch.zeros_like(self.ring_k)
        z = lambda: np.zeros(batch, dtype=np.int64)
        self.sink_len, self.comp_len, self.res_len, self.res_start, self.offset = z(), z(), z(), z(), z()
        self._step_ints = _IntStage(8 * batch, dev)   # ring slots / drain arrays / post-step lengths of a step
        # tq_ragged_step (one launch per step at head_dim 128): the
        # per-sequence ints of a step from host arrays, two slots
        # (pinned, and guarded by an event, when they travel by an
        # asynchronous copy rather than in the kernel arguments)
        self._fused = True
        self._seq_async = 8 * batch > _STEP_INLINE_INTS
        self._seq_host = [torch.empty(8 * batch, dtype=torch.int32, pin_memory=self._seq_async).numpy()
                          for _ in range(2)]
        self._seq_dev = [torch.empty(8 * batch, dtype=torch.int32, device=dev) for _ in range(2)]
        self._seq_events = [torch.cuda.Event(), torch.cuda.Event()] if self._seq_async else None
        self._seq_used = [False, False]
        self._seq_k = 0
        self._attn_ints = _IntStage(4 * batch, dev)   # per-sequence lengths of an attention call
        self._desc = None        # the attention descriptor, refreshed per call
        self._structs = None     # (store capacities, tq_store of kstore, of vstore)
        # the lengths change only in load() and step(): a step stages the
        # post-step lengths with its own arrays, and the next attention call
        # uses them while the version still matches
        self._lens_ver = 0
        self._lens_staged = None  # (version, device addresses, staging tensor)

    # ------------------------------------------------------------------ fill
    def load(self, b: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Fill the empty sequence ``b`` from its (H, T, D) keys / values: the
        first fp16_sink_size tokens to the sink, the last residual_window of the
        rest to the ring, the tokens between compressed (the state one-token
        drains leave after T tokens)."""
        if self.offset[b]:
            raise ValueError(f"sequence {b} is not empty")
        H, T, D = keys.shape
        if (H, D) != (self.H, self.D) or values.shape != keys.shape:
            raise ValueError("keys / values must be (num_kv_heads, T, head_dim)")
        k, v = keys.to(self.device, torch.float16), values.to(self.device, torch.float16)
        s = min(T, self.sink)
        r = min(T - s, self.window)
        c = T - s - r
        self.sink_k[b, :, :s] = k[:, :s]
        self.sink_v[b, :, :s] = v[:, :s]
        if c > 0:
            self.kstore.reserve(c, int(self.comp_len.max()))
            self.vstore.reserve(c, int(self.comp_len.max()))
            for codec, x, store in ((self.kc, k, self.kstore), (self.vc, v, self.vstore)):
                _codec.compress_into(codec, x[None, :, s:s + c].contiguous(), 0, c, self._row_view(store, b), 0)
        self.ring_k[b, :, :r] = k[:, s + c:]
        self.ring_v[b, :, :r] = v[:, s + c:]
        self.sink_len[b], self.comp_len[b], self.res_len[b], self.res_start[b] = s, c, r, 0
        self.offset[b] = T
        self._lens_ver += 1

    @staticmethod
    def _row_view(store: _codec.PackedStore, b: int) -> _codec.PackedStore:
        """Store view of batch row b only (same capacity and strides)."""
        view = object.__new__(_codec.PackedStore)
        view.__dict__.update(store.__dict__)
        view.batch = 1
        for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
            t = getattr(store, name)
            setattr(view, name, None if t is None else t[b:b + 1])
        return view

    # ------------------------------------------------------------------ step
    def step(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append one token per sequence ((B, H, D) keys / values). Sequences
        still filling their sink write there; the others append to their ring,
        and a sequence whose ring then holds residual_window + 1 tokens drains
        its oldest one into the store: at head_dim 128 the appends and both
        sides' drains are one tq_ragged_step launch, else tq_ring_append and
        one ragged tq_compress per side."""
        B, H, D, dev = self.B, self.H, self.D, self.device
        if keys.shape != (B, H, D) or values.shape != keys.shape:
            raise ValueError("keys / values must be (batch, num_kv_heads, head_dim)")
        keys, values = keys.to(dev, torch.float16), values.to(dev, torch.float16)
        to_sink = self.offset < self.sink
        # token b goes to sink position sink_len[b] or ring slot (start + len) % cap
        ring_slot = (self.res_start + self.res_len) % self.cap
        res_after = self.res_len + ~to_sink
        drain = res_after > self.window
        if to_sink.any():
            bi = np.nonzero(to_sink)[0]
            bt, pt = self._step_ints.put(bi, self.sink_len[bi])
            self.sink_k[bt, :, pt] = keys[bt]
            self.sink_v[bt, :, pt] = values[bt]
            self.sink_len[bi] += 1
        comp_after = self.comp_len + drain
        start_after = np.where(drain, (self.res_start + 1) % self.cap, self.res_start)
        # the step's ints: ring slots (-1: the token went to the sink), the drain
        # arrays (count, ring start, store position), then the lengths after
        # this step for the next attention call
        ints = (np.where(to_sink, -1, ring_slot), drain, self.res_start, self.comp_len, comp_after, self.sink_len,
                res_after - drain, start_after)
        lib = _lib.load()
        stream = _lib.stream_ptr(dev)
        if drain.any():
            need = int(comp_after.max())
            if need > self.kstore.cap or need > self.vstore.cap:
                keep = int(self.comp_len.max())
                self.kstore.reserve(need, keep)
                self.vstore.reserve(need, keep)
        if self._fused and self._step_fused(lib, keys, values, ints, stream):
            self.comp_len, self.res_start, self.res_len = comp_after, start_after, res_after - drain
            self.offset += 1
            self._lens_ver += 1
            return
        staged, ptrs = self._step_ints.put_ptrs(*ints)
        n_b, src_b, dst_b = ptrs[1:4]
        if not to_sink.all():
            keys, values = keys.contiguous(), values.contiguous()
            _lib.check(lib.tq_ring_append(keys.data_ptr(), values.data_ptr(), _lib.TQ_F16, self.ring_k.data_ptr(),
                                          self.ring_v.data_ptr(), self.cap * D, self.cap, B, H, D, ptrs[0], stream),
                       "tq_ring_append")
        self.res_len = res_after
        if drain.any():
            span = _lib.Span(rows=B * H, heads=H, n_tok=1, reserved=0, n_tok_b=n_b, src_tok0_b=src_b, dst_tok0_b=dst_b)
            for codec, ring, st in zip((self.kc, self.vc), (self.ring_k, self.ring_v), self._store_structs()):
                _lib.check(lib.tq_compress(codec.ref(), ring.data_ptr(), _lib.TQ_F16, self.cap * D,
                                           ctypes.byref(span), ctypes.byref(st), stream), "tq_compress")
            self.comp_len = comp_after
            self.res_start = start_after
            self.res_len -= drain
        self.offset += 1
        self._lens_ver += 1
        self._lens_staged = (self._lens_ver, ptrs[4:8], staged)

    def _step_fused(self, lib, keys: torch.Tensor, values: torch.Tensor, ints, stream: int) -> bool:
        """The step's appends and drains in one tq_ragged_step launch; False
        (and the two-call path from then on) when the codecs have no such
        launch."""
        B = self.B
        k = self._seq_k
        self._seq_k ^= 1
        if self._seq_async and self._seq_used[k]:
            self._seq_events[k].synchronize()  # the copy from this slot has completed
        h = self._seq_host[k]
        for i, x in enumerate(ints):
            h[i * B:(i + 1) * B] = x
        keys, values = keys.contiguous(), values.contiguous()
        d = self._seq_dev[k]
        kst, vst = self._store_structs()
        rc = lib.tq_ragged_step(self.kc.ref(), self.vc.ref(), keys.data_ptr(), values.data_ptr(), _lib.TQ_F16,
                                self.ring_k.data_ptr(), self.ring_v.data_ptr(), self.cap * self.D, self.cap,
                                ctypes.byref(kst), ctypes.byref(vst), B, self.H, h.ctypes.data, 8 * B, d.data_ptr(),
                                stream)
        if rc == _lib.TQ_ERR_UNSUPPORTED:
            self._fused = False
            return False
        _lib.check(rc, "tq_ragged_step")
        if self._seq_async:
            self._seq_events[k].record()
            self._seq_used[k] = True
        base = d.data_ptr()
        self._lens_staged = (self._lens_ver + 1, [base + 4 * i * B for i in range(4, 8)], d)
        return True

    # ------------------------------------------------------------- attention
    def _store_structs(self) -> tuple[_lib.Store, _lib.Store]:
        """``tq_store`` of the key and value stores, rebuilt only when a
        reserve has reallocated them (their capacities then grow)."""
        caps = (self.kstore.cap, self.vstore.cap)
        if self._structs is None or self._structs[0] != caps:
            self._structs = (caps, self.kstore.struct(0), self.vstore.struct(0))
        return self._structs[1], self._structs[2]

    def descriptor(self, q: torch.Tensor, out: torch.Tensor, scale: float, general: bool = False):
        """``tq_attn_desc`` of a (B, Hq, D) query against every sequence; the
        per-sequence arrays are device arrays valid until the call after next.
        One descriptor object is kept and refreshed per call (the fields that
        never change are set once): the host path of a decode step stays
        short, since the GPU waits for it in a step-by-step loop."""
        ls = self._lens_staged
        if ls is not None and ls[0] == self._lens_ver:
            (comp, sink, res, start), staged = ls[1], ls[2]
        else:
            staged, (comp, sink, res, start) = self._attn_ints.put_ptrs(
                self.comp_len, self.sink_len, self.res_len, self.res_start)
        d = self._desc
        if d is None:
            d = self._desc = _lib.AttnDesc(
                batch=self.B, hkv=self.H, qjl=1 if self.qjl else 0, kv_dtype=_lib.dtype_code(self.sink_k.dtype),
                sink_k=self.sink_k.data_ptr(), sink_v=self.sink_v.data_ptr(),
                sink_head_stride=self.sink_k.shape[2] * self.D,
                res_k=self.ring_k.data_ptr(), res_v=self.ring_v.data_ptr(), res_head_stride=self.cap * self.D,
                res_cap=self.cap, res_start0=0, n_q=0)
        d.kstore, d.vstore = self._store_structs()
        d.hq, d.scale, d.q_dtype = q.shape[1], scale, _lib.dtype_code(q.dtype)
        d.max_comp, d.max_sink, d.max_res = int(self.comp_len.max()), int(self.sink_len.max()), int(self.res_len.max())
        d.q, d.out = q.data_ptr(), out.data_ptr()
        d.comp_len, d.sink_len, d.res_len, d.res_start = comp, sink, res, start
        d.flags = _lib.TQ_ATTN_GENERAL if general else 0
        return d, [staged]

    def attend(self, q: torch.Tensor, scale: float | None = None, out: torch.Tensor | None = None,
               general: bool = False) -> torch.Tensor:
        """Decode attention of one query per head and sequence: q (B, Hq, D),
        Hq a multiple of the kv heads; returns float32 (B, Hq, D) over each
        sequence's own [sink | compressed | residual] tokens."""
        if q.dim() != 3 or q.shape[0] != self.B or q.shape[2] != self.D:
            raise ValueError(f"query shape {tuple(q.shape)} does not match the batch")
        if (self.offset == 0).any():
            raise ValueError("attend() with an empty sequence in the batch")
        q = q.contiguous()
        if out is None:
            out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        d, arrays = self.descriptor(q, out, scale if scale is not None else self.D ** -0.5, general)
        lib = _lib.load()
        stream = _lib.stream_ptr(q.device)
        ws = _workspace(q.device, lib.tq_attention_workspace_bytes(self.kc.ref(), self.vc.ref(), ctypes.byref(d)), stream)
        _lib.check(lib.tq_decode_attention(self.kc.ref(), self.vc.ref(), ctypes.byref(d), ws.data_ptr(), ws.numel(),
                                           stream), "tq_decode_attention")
        self._attn_keep = arrays
        return out
