"""Ragged batches through the C ABI (batched ragged decode
with QJL correction).

The reference's cache holds one length per batch (cache.py:19-116); a ragged
batch is served here by one packed store, one fp16 sink and one residual ring
shared by all sequences, with per-sequence lengths:
- tq_compress drains one ring token per sequence per step in one launch
  (tq_span n_tok_b / src_tok0_b / dst_tok0_b);
- tq_decode_attention takes comp_len / sink_len / res_len / res_start arrays.

Checks: the batched call equals one call per sequence (same descriptor
fields, that sequence's rows), and float64 attention over the
oracle-dequantised stored codes (with the stored QJL sketch) within the
attention bar (1e-3 relative, cosine >= 0.9999).
"""

import copy
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err

pytestmark = pytest.mark.gpu

D = 128
HQ_PER_KV = 4
REL_TOL = 1e-3
COS_TOL = 0.9999


def _sub(store, b):
    """Store view holding only sequence b's rows (same capacity and strides)."""
    v = copy.copy(store)
    v.batch = 1
    for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
        t = getattr(store, name)
        setattr(v, name, None if t is None else t[b:b + 1])
    return v


def _i32(xs, dev):
    return torch.tensor(np.asarray(xs, np.int32), dtype=torch.int32, device=dev)


class Ragged:
    """B sequences of lengths ``lens``: [sink | compressed | residual window]
    each, the residual held in a ring of window + 1 slots starting at a
    seeded offset per sequence."""

    def __init__(self, lens, H=8, kb=4, vb=2, qjl_m=0, sink=128, window=128, seed=0, extra=512):
        from turboquant_amd import _codec
        self.dev = dev = torch.device("cuda", 0)
        self.B, self.H = B, H = len(lens), H
        self.kc = _codec.get_codec(D, kb, 42, qjl_m, dev)
        self.vc = _codec.get_codec(D, vb, 42, qjl_m, dev)
        self.kb, self.vb, self.qjl = kb, vb, qjl_m > 0
        self.sink, self.window, self.cap = sink, window, window + 1
        self.comp = np.array([T - sink - window for T in lens], dtype=np.int64)
        assert (self.comp >= 0).all()
        self.ks = _codec.PackedStore(self.kc, B, H, qjl=self.qjl)
        self.vs = _codec.PackedStore(self.vc, B, H, qjl=self.qjl)
        self.ks.reserve(int(self.comp.max()) + extra, 0)
        self.vs.reserve(int(self.comp.max()) + extra, 0)
        self.g = g = torch.Generator(device=dev).manual_seed(seed)
        self.sink_k = torch.randn(B, H, sink, D, generator=g, device=dev).half()
        self.sink_v = torch.randn(B, H, sink, D, generator=g, device=dev).half()
        self.ring_k = torch.zeros(B, H, self.cap, D, dtype=torch.float16, device=dev)
        self.ring_v = torch.zeros_like(self.ring_k)
        self.start = np.random.RandomState(seed).randint(0, self.cap, size=B)
        for b in range(B):
            n = int(self.comp[b])
            xk = torch.randn(1, H, n, D, generator=g, device=dev).half()
            xv = torch.randn(1, H, n, D, generator=g, device=dev).half()
            _codec.compress_into(self.kc, xk, 0, n, _sub(self.ks, b), 0)
            _codec.compress_into(self.vc, xv, 0, n, _sub(self.vs, b), 0)
            slots = torch.as_tensor((self.start[b] + np.arange(window)) % self.cap, device=dev)
            self.ring_k[b][:, slots] = torch.randn(H, window, D, generator=g, device=dev).half()
            self.ring_v[b][:, slots] = torch.randn(H, window, D, generator=g, device=dev).half()

    def step(self):
        """Append one N(0,1) token per sequence; drain each sequence's oldest
        ring token into its store (chunk_size = 1) with one ragged launch per
        side."""
        from turboquant_amd import _lib
        B, H, dev = self.B, self.H, self.dev
        bi = torch.arange(B, device=dev)
        slot = _i32((self.start + self.window) % self.cap, dev).long()
        self.ring_k[bi, :, slot] = torch.randn(B, H, D, generator=self.g, device=dev).half()
        self.ring_v[bi, :, slot] = torch.randn(B, H, D, generator=self.g, device=dev).half()
        n_b, src_b, dst_b = _i32(np.ones(B), dev), _i32(self.start, dev), _i32(self.comp, dev)
        span = _lib.Span(rows=B * H, heads=H, n_tok=1, reserved=0, n_tok_b=n_b.data_ptr(),
                         src_tok0_b=src_b.data_ptr(), dst_tok0_b=dst_b.data_ptr())
        lib = _lib.load()
        for codec, ring, store in ((self.kc, self.ring_k, self.ks), (self.vc, self.ring_v, self.vs)):
            st = store.struct(0)
            _lib.check(lib.tq_compress(codec.ref(), ring.data_ptr(), _lib.dtype_code(ring.dtype), self.cap * D,
                                       ctypes.byref(span), ctypes.byref(st), _lib.stream_ptr(dev)), "tq_compress")
        torch.cuda.synchronize()  # the length arrays above are freed on return
        self.start = (self.start + 1) % self.cap
        self.comp += 1

    def attend(self, q, b=None, general=False):
        """out (B or 1, Hq, D) float32: every sequence in one call, or sequence
        b alone (its rows, the same length hints)."""
        from turboquant_amd import _lib
        from turboquant_amd.cache import _workspace
        dev = self.dev
        rows = slice(None) if b is None else slice(b, b + 1)
        nb = self.B if b is None else 1
        ks = self.ks if b is None else _sub(self.ks, b)
        vs = self.vs if b is None else _sub(self.vs, b)
        qq = q[rows].contiguous()
        out = torch.empty(nb, qq.shape[1], D, dtype=torch.float32, device=dev)
        comp = _i32(self.comp[rows], dev)
        sink_len = _i32(np.full(nb, self.sink), dev)
        res_len = _i32(np.full(nb, self.window), dev)
        start = _i32(self.start[rows], dev)
        sk, sv = self.sink_k[rows], self.sink_v[rows]
        rk, rv = self.ring_k[rows], self.ring_v[rows]
        desc = _lib.AttnDesc(
            batch=nb, hq=qq.shape[1], hkv=self.H, qjl=1 if self.qjl else 0, scale=D ** -0.5,
            max_comp=int(self.comp.max()), max_sink=self.sink, max_res=self.window,
            q_dtype=_lib.dtype_code(qq.dtype), kv_dtype=_lib.dtype_code(sk.dtype),
            q=qq.data_ptr(), out=out.data_ptr(), kstore=ks.struct(0), vstore=vs.struct(0),
            comp_len=comp.data_ptr(), sink_k=sk.data_ptr(), sink_v=sv.data_ptr(),
            sink_head_stride=self.sink * D, sink_len=sink_len.data_ptr(),
            res_k=rk.data_ptr(), res_v=rv.data_ptr(), res_head_stride=self.cap * D, res_cap=self.cap,
            res_start0=0, res_start=start.data_ptr(), res_len=res_len.data_ptr(),
            flags=_lib.TQ_ATTN_GENERAL if general else 0)
        lib = _lib.load()
        need = lib.tq_decode_workspace_bytes(self.kc.ref(), ctypes.byref(desc))
        ws = _workspace(dev, need)
        _lib.check(lib.tq_decode_attention(self.kc.ref(), self.vc.ref(), ctypes.byref(desc), ws.data_ptr(),
                                           ws.numel(), _lib.stream_ptr(dev)), "tq_decode_attention")
        torch.cuda.synchronize()
        return out

    def dense64(self, b):
        """float64 [sink | oracle-dequantised stored codes (+ stored sketch) |
        ring in order] of sequence b, (1, H, T, D) keys and values."""
        R = O.rotation_matrix(D)
        S = self.kc.proj.cpu().numpy() if self.qjl else None
        C = int(self.comp[b])
        parts = []
        for store, bits, sink, ring in ((self.ks, self.kb, self.sink_k, self.ring_k),
                                        (self.vs, self.vb, self.sink_v, self.ring_v)):
            hi = store.codes_hi[b:b + 1, :, :C].cpu().numpy()
            lo = None if store.codes_lo is None else store.codes_lo[b:b + 1, :, :C].cpu().numpy()
            x = O.dequantize(hi, lo, store.norms[b:b + 1, :, :C].cpu().numpy(), R, bits, D)
            if self.qjl:
                signs = np.unpackbits(store.signs[b:b + 1, :, :C].cpu().numpy(), axis=-1,
                                      bitorder="little").astype(bool)
                x = x + O.qjl_correction(signs, store.gamma[b:b + 1, :, :C].cpu().numpy(), S, D)
            slots = torch.as_tensor((self.start[b] + np.arange(self.window)) % self.cap, device=ring.device)
            res = ring[b:b + 1][:, :, slots].cpu().numpy().astype(np.float64)
            parts.append(np.concatenate([sink[b:b + 1].cpu().numpy().astype(np.float64), x, res], axis=2))
        return parts


def check_batch(rg, q, oracle_rows=(), general=False, label=""):
    out = rg.attend(q, general=general)
    for b in range(rg.B):
        one = rg.attend(q, b=b, general=general)
        e = rel_err(out[b:b + 1].cpu().numpy(), one.cpu().numpy())
        assert e < 1e-5, f"{label} sequence {b}: batched vs single {e:.3e}"
    for b in oracle_rows:
        kk, vv = rg.dense64(b)
        ref = O.attention(q[b:b + 1, :, None].cpu().numpy(), kk, vv)[:, :, 0]
        got = out[b:b + 1].cpu().numpy()
        e, cs = rel_err(got, ref), min_cos(got, ref)
        print(f"{label} sequence {b} (T={rg.sink + int(rg.comp[b]) + rg.window}): rel {e:.3e} min cos {cs:.7f}")
        assert e < REL_TOL and cs >= COS_TOL
    return out


@pytest.mark.parametrize("qjl_m", [0, 64], ids=["k4v2", "k4v2_qjl"])
def test_ragged_small(qjl_m):
    lens = [300, 1000, 164, 2000, 700]
    rg = Ragged(lens, H=2, qjl_m=qjl_m, sink=16, window=32, seed=3)
    q = torch.randn(rg.B, 2 * HQ_PER_KV, D, generator=rg.g, device=rg.dev).half()
    check_batch(rg, q, oracle_rows=range(rg.B), label=f"small m={qjl_m}")
    if not qjl_m:  # the K4/V2 kernels against the general kernel on the same batch
        a = rg.attend(q).cpu().numpy()
        b = rg.attend(q, general=True).cpu().numpy()
        assert rel_err(a, b) < 1e-4
    for _ in range(40):
        rg.step()
    check_batch(rg, q, oracle_rows=range(rg.B), label=f"small m={qjl_m} +40")


@pytest.mark.parametrize("qjl_m", [0, 128], ids=["k4v2", "k4v2_qjl"])
def test_config4_ragged_decode(qjl_m):
    """configs[4] at size: 16 Llama-3.1-8B-shaped sequences (H_kv = 8,
    H_q = 32), lengths ~ Uniform[4096, 32768] (seeded), K4/V2 (with the QJL
    sketch through a 128 x 128 projection), 256 decode steps of one new token
    per sequence, each draining one token per sequence into the store."""
    lens = np.random.RandomState(4).randint(4096, 32769, size=16)
    rg = Ragged(lens, H=8, qjl_m=qjl_m, seed=5)
    q = torch.randn(rg.B, 8 * HQ_PER_KV, D, generator=rg.g, device=rg.dev).half()
    short = [int(i) for i in np.argsort(lens)[:2]]
    check_batch(rg, q, oracle_rows=short, label=f"config4 m={qjl_m} step 0")
    for _ in range(256):
        rg.step()
    assert (rg.comp == lens - rg.sink - rg.window + 256).all()
    q = torch.randn(rg.B, 8 * HQ_PER_KV, D, generator=rg.g, device=rg.dev).half()
    check_batch(rg, q, oracle_rows=short, label=f"config4 m={qjl_m} step 256")
