"""GPU parity of the uniform-batch MFMA kernels for fractional widths
(tq_decode_split.h): both codecs split at dim 64 into ceil(bits) / floor(bits)
codebooks (cache.py:63-84, 253-300), K3.5 / K2.5 keys with V3.5 / V2.5
values. The route is asserted through the library's test hook (5), and the
output is held to the K4/V2 kernels' bound against float64 attention over the
codes the cache stores (sink and residual exact) and to 1e-4 against the
general kernel on the same cache.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err, to_dev
from test_gpu_attention import build, decode_route, dense_from_gpu_codes

pytestmark = pytest.mark.gpu

FAST_REL_TOL = 5e-6
COS_TOL = 0.9999
SPLITS = [(3.5, 3.5), (2.5, 2.5), (3.5, 2.5), (2.5, 3.5)]


def _kv(B, H, T, D, seed, vmul=1.0):
    rng = np.random.RandomState(seed)
    s = np.exp(rng.randn(D) * 0.5)
    k = (rng.randn(B, H, T, D) * s).astype(np.float16)
    v = np.clip(rng.randn(B, H, T, D) * vmul, -6e4, 6e4).astype(np.float16)
    return k, v


def _check(c, o, q, label, route=5):
    qd = to_dev(q)
    assert decode_route(c, qd) == route
    fast = c.attend(qd).cpu().numpy()
    gen = c.attend(qd, general_kernel=True).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv)
    e_f = rel_err(fast, ref)
    print(f"{label}: rel {e_f:.3e} vs general {rel_err(fast, gen):.3e} min cos {min_cos(fast, ref):.8f}")
    assert np.isfinite(fast).all()
    assert e_f < FAST_REL_TOL and min_cos(fast, ref) >= COS_TOL
    assert rel_err(fast, gen) < 1e-4


@pytest.mark.parametrize("G,T,sink,window", [
    (4, 3000, 128, 128),   # one block per wave, a workgroup's fp16 tokens
    (1, 700, 16, 64),      # partial last block
    (8, 1500, 0, 32),      # G = 8 (one tile per MFMA column set)
    (2, 5000, 300, 300),   # more fp16 tokens than one workgroup stages
])
@pytest.mark.parametrize("kb,vb", SPLITS, ids=[f"K{k}V{v}" for k, v in SPLITS])
def test_split_widths_match_oracle(kb, vb, G, T, sink, window):
    k, v = _kv(1, 2, T, 128, seed=int(T + 10 * kb + vb + G))
    c, o = build(dict(head_dim=128, num_kv_heads=2, key_bits=kb, value_bits=vb, residual_window=window,
                      fp16_sink_size=sink), k, v)
    q = np.random.RandomState(int(kb * 8 + vb + G)).randn(1, 2 * G, 1, 128).astype(np.float16)
    _check(c, o, q, f"K{kb}/V{vb} G={G} T={T}")


def test_split_decode_steps_ring_wrap():
    """Token-by-token decode with chunked drains (a wrapped residual ring)."""
    k, v = _kv(1, 2, 400, 128, seed=9)
    rng = np.random.RandomState(10)
    steps = [(rng.randn(1, 2, 1, 128).astype(np.float16), rng.randn(1, 2, 1, 128).astype(np.float16))
             for _ in range(45)]
    c, o = build(dict(head_dim=128, num_kv_heads=2, key_bits=3.5, value_bits=3.5, residual_window=32,
                      chunk_size=8, fp16_sink_size=8), k, v, steps)
    q = rng.randn(1, 8, 1, 128).astype(np.float16)
    _check(c, o, q, "K3.5/V3.5 ring")


def test_split_large_values_and_small_queries():
    """Values of norm ~1e5 (the P^T operand's exponent) and queries of norm
    ~1e-4 (scaled up per head): the uniform kernel's range handling."""
    k, v = _kv(1, 2, 3000, 128, seed=95, vmul=1.5e4)
    c, o = build(dict(head_dim=128, num_kv_heads=2, key_bits=3.5, value_bits=3.5, residual_window=64,
                      fp16_sink_size=16), k, v)
    q = (np.random.RandomState(96).randn(1, 8, 1, 128) * 1e-4).astype(np.float16)
    _check(c, o, q, "K3.5/V3.5 large values, small queries")
    q = (np.random.RandomState(97).randn(1, 8, 1, 128).astype(np.float32)).astype(np.float32)
    qd = to_dev(q)
    assert decode_route(c, qd) == 5  # float32 queries take the route too
    fast = c.attend(qd).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    assert rel_err(fast, O.attention(q, kk, vv)) < FAST_REL_TOL


MIXED = [(3.5, 2), (3.5, 3), (3.5, 4), (2.5, 2), (2.5, 4), (4, 3.5), (3, 3.5), (2, 3.5), (4, 2.5), (2, 2.5)]


@pytest.mark.parametrize("kb,vb", MIXED, ids=[f"K{k}V{v}" for k, v in MIXED])
@pytest.mark.parametrize("G,T", [(4, 3000), (1, 700), (8, 1500)])
def test_split_mixed_integer_side(kb, vb, G, T):
    """A fractional width on one side, an integer width (one codebook, one
    row per token, the lo segment from byte 8 W) on the other."""
    k, v = _kv(1, 2, T, 128, seed=int(T + 10 * kb + vb + G))
    c, o = build(dict(head_dim=128, num_kv_heads=2, key_bits=kb, value_bits=vb, residual_window=64,
                      fp16_sink_size=16), k, v)
    q = np.random.RandomState(int(kb * 8 + vb + G)).randn(1, 2 * G, 1, 128).astype(np.float16)
    _check(c, o, q, f"K{kb}/V{vb} G={G} T={T}")


def test_split_route_limits():
    """Integer widths on both sides keep their kernels; a sketch takes the
    general kernel."""
    k, v = _kv(1, 2, 900, 128, seed=5)
    q = to_dev(np.random.RandomState(6).randn(1, 8, 1, 128).astype(np.float16))
    for kw, route in ((dict(key_bits=3.5, value_bits=3.5), 5), (dict(key_bits=3, value_bits=3), 4),
                      (dict(key_bits=3.5, value_bits=2), 5), (dict(key_bits=4, value_bits=2.5), 5),
                      (dict(key_bits=4, value_bits=2), 2),
                      (dict(key_bits=3.5, value_bits=3.5, qjl_correction=True, qjl_n_proj=64), 0)):
        c, _ = build(dict(head_dim=128, num_kv_heads=2, residual_window=64, fp16_sink_size=16, **kw), k, v)
        assert decode_route(c, q) == route, kw


def _geometry(c, q):
    from turboquant_amd import _lib
    qq = q[:, :, 0].contiguous()
    out = torch.empty(qq.shape, dtype=torch.float32, device=qq.device)
    desc = c.attention_descriptor(qq, out, 128 ** -0.5)
    fn = _lib.load().tq_debug_uniform_geometry
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p] * 4
    geo = (ctypes.c_int32 * 4)()
    assert fn(ctypes.addressof(c._kc.struct), ctypes.addressof(c._vc.struct), ctypes.addressof(desc),
              ctypes.addressof(geo)) == 0
    return tuple(geo)


@pytest.mark.parametrize("T,geometry", [(32768, (32, 32, 8, 4)), (40000, (32, 39, 8, 8))])
def test_split_configs1_layer_shape(T, geometry):
    """K3.5/V3.5 at configs[1]'s layer shape (Hkv 8, Hq 32, sink 128, window
    128; 4 blocks per wave) and at 40,000 tokens (the NPW = 8 kernel), against
    float64 over the stored codes."""
    from test_gpu_headline_geometry import _dense_reference
    from turboquant_amd import TurboQuantKVCache
    k, v = _kv(1, 8, T, 128, seed=T)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=3.5, value_bits=3.5, residual_window=128,
                          fp16_sink_size=128)
    c.update(to_dev(k), to_dev(v))
    q = np.random.RandomState(T + 1).randn(1, 32, 1, 128).astype(np.float16)
    qd = to_dev(q)
    assert decode_route(c, qd) == 5
    assert _geometry(c, qd) == geometry
    fast = c.attend(qd).cpu().numpy()
    gen = c.attend(qd, general_kernel=True).cpu().numpy()
    kk, vv = _dense_reference(c, k, v)
    ref = O.attention(q, kk, vv)
    print(f"K3.5/V3.5 T={T}: rel {rel_err(fast, ref):.3e} vs general {rel_err(fast, gen):.3e}")
    assert rel_err(fast, ref) < FAST_REL_TOL and min_cos(fast, ref) >= COS_TOL
    assert rel_err(fast, gen) < 1e-4
