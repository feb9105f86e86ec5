"""Attention of several query tokens over packed codes with the causal
offset of a prefill chunk (the reference's fused QK over a (T_kv, T_q) grid,
kernels.py:558-629, tested at T_q in {1, 4, 32} in
tests/test_fused_attention.py:147-288; prefill uses the "causal" mask,
cache.py:722-724).

The cache holds T_kv tokens; the query tokens are its last T_q, and query i
sees positions <= T_kv - T_q + i. The GPU result is held to 1e-3 / cos
0.9999 against float64 attention (O.attention with causal_offset) over the
codes the cache stores, at 2 / 3 / 4 bits, T_kv in {128, 4000}, T_q in
{1, 4, 32}, plus the QJL sketch, head_dim 96, a ratio of 3 query heads per
kv head and a batch of two. Each query row equals a one-token call over the
cache truncated to its position.

Integer widths at head_dim 128 without a sketch take the query-tiled MFMA
kernels (route 6 of the library's test hook: fp16 query and p * n_v
operands, centroids and uncompressed tokens as fp16 high part + remainder);
the other calls the general kernel (route 0). The route is asserted, and
the query-tiled result is also compared with the general kernel's.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err, to_dev
from test_gpu_attention import build, dense_from_gpu_codes

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
COS_TOL = 0.9999


def _kv(B, H, T, D, seed):
    rng = np.random.RandomState(seed)
    s = np.exp(rng.randn(D) * 0.5)
    return (rng.randn(B, H, T, D) * s).astype(np.float16), rng.randn(B, H, T, D).astype(np.float16)


def prefill_route(c, q):
    """tq_debug_decode_route (a test hook of the library) for c.attend(q)
    with q (B, Hq, T_q, D): 6 the query-tiled prefill kernels, 0 the general
    kernel."""
    from turboquant_amd import _lib
    fn = _lib.load().tq_debug_decode_route
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p] * 3
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    desc = c.attention_descriptor(q, out, q.shape[-1] ** -0.5)
    desc.n_q = q.shape[2]
    return fn(ctypes.addressof(c._kc.struct), ctypes.addressof(c._vc.struct), ctypes.addressof(desc))


def _tiled(kw):
    return (kw["head_dim"] == 128 and not kw.get("qjl_correction") and float(kw["key_bits"]).is_integer()
            and float(kw["value_bits"]).is_integer())


def _prefill(kw, T, tq, G, seed, B=1, q_dtype=np.float16, qmul=1.0):
    k, v = _kv(B, kw["num_kv_heads"], T, kw["head_dim"], seed)
    c, o = build(kw, k, v)
    q = (np.random.RandomState(seed + 1).randn(B, kw["num_kv_heads"] * G, tq, kw["head_dim"]) * qmul).astype(q_dtype)
    qd = to_dev(q)
    if tq > 1:
        assert prefill_route(c, qd) == (6 if _tiled(kw) else 0)
    out = c.attend(qd).cpu().numpy()
    assert out.shape == q.shape
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv, causal_offset=T - tq)
    e, cs = rel_err(out, ref), min_cos(out, ref)
    print(f"T_kv={T} T_q={tq} {kw.get('key_bits')}/{kw.get('value_bits')} G={G}: rel {e:.3e} min cos {cs:.7f} "
          f"(compressed {c._compressed_len})")
    assert np.isfinite(out).all()
    assert e < REL_TOL and cs >= COS_TOL
    if tq > 1 and _tiled(kw):
        gen = c.attend(qd, general_kernel=True).cpu().numpy()
        assert rel_err(out, gen) < REL_TOL
    return c, o, q, out, kk, vv


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("T", [128, 4000])
@pytest.mark.parametrize("tq", [1, 4, 32])
def test_prefill_causal(bits, T, tq):
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=bits, value_bits=bits, residual_window=32, fp16_sink_size=8)
    c, _, _, _, _, _ = _prefill(kw, T, tq, 4, seed=bits * 100 + tq)
    assert c._compressed_len > 0


def test_prefill_rows_match_masked_full_attention():
    """Query i of the chunk equals float64 attention of that query alone over
    the first T_kv - T_q + i + 1 tokens (the causal mask row by row)."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, fp16_sink_size=8)
    _, _, q, out, kk, vv = _prefill(kw, 700, 32, 4, seed=11)
    for i in (0, 13, 31):
        lim = 700 - 32 + i + 1
        ref = O.attention(q[:, :, i:i + 1], kk[:, :, :lim], vv[:, :, :lim])
        assert rel_err(out[:, :, i:i + 1], ref) < REL_TOL


def test_prefill_qjl_d96_gqa3_batch2():
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, fp16_sink_size=8,
              qjl_correction=True, qjl_n_proj=64)
    _prefill(kw, 1000, 16, 4, seed=21)
    kw = dict(head_dim=96, num_kv_heads=2, key_bits=3.5, value_bits=3, residual_window=32, fp16_sink_size=0)
    _prefill(kw, 600, 8, 3, seed=31, B=2)


def test_prefill_d96_k25():
    """head_dim 96 at K2.5 (an 18-byte 3-bit hi segment, the 2-bit lo segment
    staged at the next dword column) with several query tokens."""
    kw = dict(head_dim=96, num_kv_heads=2, key_bits=2.5, value_bits=2.5, residual_window=32, fp16_sink_size=8)
    _prefill(kw, 900, 16, 3, seed=51)


def test_prefill_whole_residual_window():
    """Every query in the fp16 residual window and the sink: nothing of the
    chunk is compressed yet (T_kv below the window)."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=256, fp16_sink_size=16)
    c, _, _, _, _, _ = _prefill(kw, 100, 32, 4, seed=41)
    assert c._compressed_len == 0


@pytest.mark.parametrize("kb,vb", [(4, 2), (2, 4), (3, 3), (4, 4), (2, 2), (3, 4)])
def test_prefill_tiled_widths(kb, vb):
    """The query-tiled kernels at every width pair family, 40 query tokens of
    4 heads per kv head (160 rows: three waves, the last partly filled), a
    window of 32 so the queries reach back into the compressed tokens."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=kb, value_bits=vb, residual_window=32, fp16_sink_size=16)
    c, _, _, _, _, _ = _prefill(kw, 3000, 40, 4, seed=kb * 10 + vb)
    assert c._compressed_len > 40


@pytest.mark.parametrize("T,tq,G", [(9000, 128, 4), (5000, 300, 1), (2000, 7, 3), (600, 600, 2)])
def test_prefill_tiled_shapes(T, tq, G):
    """Several row groups and key-range splits (T = 9000, 128 tokens x 4
    heads), rows not a multiple of a wave (7 x 3), G = 1 and 3, and the whole
    cache as the chunk (every query sees a prefix: the first chunk of a
    prompt)."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=64, fp16_sink_size=8)
    _prefill(kw, T, tq, G, seed=T + tq)


def test_prefill_tiled_query_ranges():
    """float32 queries of norm ~1e-4 and ~1e3 (the per-wave query exponent)."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, fp16_sink_size=8)
    _prefill(kw, 2500, 24, 4, seed=61, q_dtype=np.float32, qmul=1e-5)
    _prefill(kw, 2500, 24, 4, seed=62, q_dtype=np.float32, qmul=100.0)


@pytest.mark.parametrize("kmul,vmul", [(1.0, 1.0), (300.0, 3e4)])
def test_prefill_tiled_bf16_kv(kmul, vmul):
    """bf16 sink / residual tokens (entries past the fp16 range in the second
    case): the preparation kernel reads them as bf16."""
    from turboquant_amd import TurboQuantKVCache
    k, v = _kv(1, 2, 2500, 128, seed=63)
    kt = (torch.from_numpy(k.astype(np.float32)) * kmul).to(torch.bfloat16)
    vt = (torch.from_numpy(v.astype(np.float32)) * vmul).to(torch.bfloat16)
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=64, fp16_sink_size=16)
    c = TurboQuantKVCache(**kw)
    c.update(kt.cuda(), vt.cuda())
    o = O.CacheOracle(**kw)
    o.update(kt.float().numpy(), vt.float().numpy())
    q = (np.random.RandomState(64).randn(1, 8, 48, 128) / kmul).astype(np.float16)
    qd = to_dev(q)
    assert prefill_route(c, qd) == 6
    out = c.attend(qd).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv, causal_offset=2500 - 48)
    print(f"bf16 kv x{kmul}/{vmul}: rel {rel_err(out, ref):.3e}")
    assert np.isfinite(out).all() and rel_err(out, ref) < REL_TOL and min_cos(out, ref) >= COS_TOL


def test_prefill_tiled_large_values():
    """Value norms ~1e5 (p * n_v needs the per-wave power of two)."""
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=3, value_bits=3, residual_window=32, fp16_sink_size=8)
    rng = np.random.RandomState(71)
    k = rng.randn(1, 2, 1500, 128).astype(np.float16)
    v = np.clip(rng.randn(1, 2, 1500, 128) * 1.2e4, -6e4, 6e4).astype(np.float16)
    c, o = build(kw, k, v)
    q = rng.randn(1, 8, 20, 128).astype(np.float16)
    qd = to_dev(q)
    assert prefill_route(c, qd) == 6
    out = c.attend(qd).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv, causal_offset=1500 - 20)
    print(f"large values: rel {rel_err(out, ref):.3e}")
    assert np.isfinite(out).all() and rel_err(out, ref) < REL_TOL and min_cos(out, ref) >= COS_TOL
