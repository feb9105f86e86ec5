"""Dense decode attention (uncompressed fp16 / bf16 K/V) through the C ABI:
tq_dense_decode_attention, and tq_decode_attention's route for caches with
nothing compressed yet.

The reference attends its uncompressed layers (outlier / skipped layers on a
plain KVCache, patch.py:337-338) with mlx SDPA over the fp16 K/V. Checks:
float64 attention (oracle.attention) over the same stored fp16 / bf16 values
within the attention bar (1e-3 relative, cosine >= 0.9999) for
- every query-group size, both K/V dtypes, fp16 and fp32 queries, lengths
  around the 32-token block (1, 31, 32, 33, ...);
- ragged batches of [sink | residual ring] with per-sequence lengths and ring
  wrap (the three contiguous pieces the kernel splits a sequence into);
- TurboQuantKVCache.attend before the first drain (routed to the dense
  kernel) against the general kernel on the same cache;
- FP16KVCache growing across its 256-token storage steps;
and at the full configs[3] layer shape (65536 tokens, H_kv = 8, H_q = 32)
against float64 torch attention on the GPU.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err

pytestmark = pytest.mark.gpu

D = 128
REL_TOL = 1e-3
COS_TOL = 0.9999
DEV = torch.device("cuda", 0)


def check(got, ref, label):
    got = np.asarray(got, np.float64)
    e, cs = rel_err(got, ref), min_cos(got, ref)
    print(f"{label}: rel {e:.3e} min cos {cs:.7f}")
    assert e < REL_TOL and cs >= COS_TOL, label


def run_desc(q, out, B, hkv, sink_k=None, sink_v=None, sink_len=None, max_sink=0, sink_hs=0,
             res_k=None, res_v=None, res_len=None, res_start=None, max_res=0, cap=0, kv_dtype=None, scale=None):
    from turboquant_amd import _lib
    from turboquant_amd.cache import _workspace
    ptr = lambda t: None if t is None else t.data_ptr()
    desc = _lib.AttnDesc(
        batch=B, hq=q.shape[1], hkv=hkv, qjl=0, scale=D ** -0.5 if scale is None else scale, max_comp=0,
        max_sink=max_sink, max_res=max_res, q_dtype=_lib.dtype_code(q.dtype), kv_dtype=_lib.dtype_code(kv_dtype),
        q=q.data_ptr(), out=out.data_ptr(), comp_len=None, sink_k=ptr(sink_k), sink_v=ptr(sink_v),
        sink_head_stride=sink_hs, sink_len=ptr(sink_len), res_k=ptr(res_k), res_v=ptr(res_v),
        res_head_stride=cap * D, res_cap=cap, res_start0=0, res_start=ptr(res_start), res_len=ptr(res_len), flags=0)
    lib = _lib.load()
    ws = _workspace(DEV, lib.tq_dense_decode_workspace_bytes(ctypes.byref(desc), D))
    _lib.check(lib.tq_dense_decode_attention(ctypes.byref(desc), D, ws.data_ptr(), ws.numel(), _lib.stream_ptr(DEV)),
               "tq_dense_decode_attention")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("T", [1, 31, 32, 33, 100, 1000, 5000])
def test_dense_matches_oracle(T, G, kv_dtype):
    from turboquant_amd.cache import dense_attention
    H = 2
    g = torch.Generator(device=DEV).manual_seed(1000 * T + 10 * G + (kv_dtype == torch.bfloat16))
    k = (torch.randn(2, H, T, D, generator=g, device=DEV) * 1.5).to(kv_dtype)
    v = torch.randn(2, H, T, D, generator=g, device=DEV).to(kv_dtype)
    q_dtype = torch.float32 if T % 2 else torch.float16
    q = torch.randn(2, H * G, D, generator=g, device=DEV).to(q_dtype)
    scale = 0.11 if T == 100 else None
    out = dense_attention(q, k, v, scale=scale)
    torch.cuda.synchronize()
    ref = O.attention(q.double().cpu().numpy()[:, :, None], k.double().cpu().numpy(), v.double().cpu().numpy(),
                      scale=scale)
    check(out.cpu().numpy(), ref, f"T={T} G={G} {kv_dtype}")


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_dense_sink_ring_ragged(kv_dtype):
    """Per-sequence sink lengths, ring starts and ring lengths (wrapping and
    not, empty sink, empty ring)."""
    H, G, cap, scap = 3, 4, 70, 48
    sink_len = [0, 5, 40, 48, 17, 0]
    res_start = [60, 3, 0, 69, 10, 5]
    res_len = [50, 70, 0, 33, 1, 0]   # the last sequence is empty: its output is zero
    B = len(sink_len)
    g = torch.Generator(device=DEV).manual_seed(7)
    sk = torch.randn(B, H, scap, D, generator=g, device=DEV).to(kv_dtype)
    sv = torch.randn(B, H, scap, D, generator=g, device=DEV).to(kv_dtype)
    rk = torch.randn(B, H, cap, D, generator=g, device=DEV).to(kv_dtype)
    rv = torch.randn(B, H, cap, D, generator=g, device=DEV).to(kv_dtype)
    q = torch.randn(B, H * G, D, generator=g, device=DEV).half()
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H * G, D, dtype=torch.float32, device=DEV)
    run_desc(q, out, B, H, sink_k=sk, sink_v=sv, sink_len=i32(sink_len), max_sink=max(sink_len), sink_hs=scap * D,
             res_k=rk, res_v=rv, res_len=i32(res_len), res_start=i32(res_start), max_res=max(res_len), cap=cap,
             kv_dtype=kv_dtype)
    assert (out[B - 1] == 0).all()
    for b in range(B - 1):
        slots = (res_start[b] + np.arange(res_len[b])) % cap
        kk = np.concatenate([sk[b, :, :sink_len[b]].double().cpu().numpy(),
                             rk[b][:, torch.as_tensor(slots, device=DEV)].double().cpu().numpy()], axis=1)
        vv = np.concatenate([sv[b, :, :sink_len[b]].double().cpu().numpy(),
                             rv[b][:, torch.as_tensor(slots, device=DEV)].double().cpu().numpy()], axis=1)
        ref = O.attention(q[b:b + 1, :, None].double().cpu().numpy(), kk[None], vv[None])[:, :, 0]
        check(out[b:b + 1].cpu().numpy(), ref, f"sequence {b} S={sink_len[b]} R={res_len[b]} start={res_start[b]}")


@pytest.mark.parametrize("T,window,sink", [(7, 32, 0), (60, 32, 16), (200, 128, 4)])
def test_turboquant_cache_before_first_drain(T, window, sink):
    """A TurboQuantKVCache with nothing compressed goes to the dense kernel;
    the general kernel on the same cache and the oracle agree."""
    from turboquant_amd import TurboQuantKVCache
    c = TurboQuantKVCache(head_dim=D, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=window,
                          fp16_sink_size=sink)
    g = torch.Generator(device=DEV).manual_seed(T)
    k = torch.randn(1, 2, T, D, generator=g, device=DEV).half()
    v = torch.randn(1, 2, T, D, generator=g, device=DEV).half()
    c.update_and_fetch(k, v)
    assert c._compressed_len == 0
    q = torch.randn(1, 8, 1, D, generator=g, device=DEV).half()
    a = c.attend(q)
    b = c.attend(q, general_kernel=True)
    torch.cuda.synchronize()
    assert rel_err(a.cpu().numpy(), b.cpu().numpy()) < 1e-4
    ref = O.attention(q.double().cpu().numpy(), k.double().cpu().numpy(), v.double().cpu().numpy())
    check(a.cpu().numpy(), ref, f"turboquant cache T={T}")


def test_fp16_cache_attend_grows():
    from turboquant_amd.patch import FP16KVCache
    c = FP16KVCache()
    g = torch.Generator(device=DEV).manual_seed(5)
    ks, vs = [], []
    for n in (300, 1, 211, 1, 1):  # 300 -> 512 slots, 512 -> 513 reallocates
        k = torch.randn(2, 4, n, D, generator=g, device=DEV).bfloat16()
        v = torch.randn(2, 4, n, D, generator=g, device=DEV).bfloat16()
        c.update_and_fetch(k, v)
        ks.append(k)
        vs.append(v)
        q = torch.randn(2, 16, 1, D, generator=g, device=DEV).bfloat16()
        out = c.attend(q)
        torch.cuda.synchronize()
        kk = torch.cat(ks, 2).double().cpu().numpy()
        vv = torch.cat(vs, 2).double().cpu().numpy()
        check(out.cpu().numpy(), O.attention(q.double().cpu().numpy(), kk, vv), f"fp16 cache T={c.offset}")
    assert c._k.shape[2] == 768 and c.offset == 514


def test_dense_errors():
    from turboquant_amd.cache import dense_attention
    k = torch.zeros(1, 2, 10, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError):
        dense_attention(torch.zeros(1, 4, 64, dtype=torch.float16, device=DEV), k, k)  # head_dim 64
    k = torch.zeros(1, 2, 10, D, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        dense_attention(torch.zeros(1, 4, D, device=DEV), k, k)  # fp32 K/V
    k = torch.zeros(1, 2, 10, D, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError):
        dense_attention(torch.zeros(1, 6, D, dtype=torch.float16, device=DEV), k, k)  # 3 query heads per kv head


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_config3_fp16_layer(kv_dtype):
    """configs[3]'s uncompressed layers at size: 65536 tokens, H_kv = 8,
    H_q = 32, keys with 4 channels scaled x25 (the outlier pattern), against
    float64 attention computed with torch on the GPU."""
    T, H, G = 65536, 8, 4
    g = torch.Generator(device=DEV).manual_seed(3)
    k = torch.randn(1, H, T, D, generator=g, device=DEV)
    k[..., torch.randperm(D, generator=torch.Generator().manual_seed(3))[:4].to(DEV)] *= 25
    k = k.to(kv_dtype)
    v = torch.randn(1, H, T, D, generator=g, device=DEV).to(kv_dtype)
    q = torch.randn(1, H * G, D, generator=g, device=DEV).to(kv_dtype)
    from turboquant_amd.cache import dense_attention
    out = dense_attention(q, k, v)
    torch.cuda.synchronize()
    qd = q.double().view(H, G, D)
    s = torch.matmul(qd, k[0].double().transpose(1, 2).contiguous()) * D ** -0.5  # (H, G, T)
    p = torch.softmax(s, dim=-1)
    ref = torch.matmul(p, v[0].double()).reshape(1, H * G, 1, D)
    check(out.cpu().numpy(), ref.cpu().numpy(), f"config3 fp16 layer {kv_dtype}")
