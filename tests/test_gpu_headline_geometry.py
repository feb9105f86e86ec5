"""GPU parity of the uniform-batch decode kernels at the launch geometries the
benchmark runs.

configs[1] (B 1, Hkv 8, Hq 32, T 32,768 = 128 sink + 32,512 packed + 128
residual) gives 32 workgroups per kv head with 32 compressed blocks each, i.e.
4 blocks per wave (block slots 0-3 and their two-ahead prefetch), on the
NPW = 4 instantiation. A context of 40,000 tokens over 8 kv heads gives 39
blocks per workgroup, which selects the NPW = 8 instantiations. The launch
geometry is asserted through the library's test hook, and the outputs are
held to the K4/V2 kernels' bound against float64 attention over the codes the
cache stores (sink and residual tokens exact) and to 1e-4 against the general
kernel on the same cache.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err, to_dev

pytestmark = pytest.mark.gpu

FAST_REL_TOL = 5e-6
COS_TOL = 0.9999


def _kv(H, T, seed):
    """configs[1]-style inputs: keys N(0,1) x per-channel LogNormal(0, 0.5),
    values N(0,1), fp16."""
    rng = np.random.RandomState(seed)
    s = np.exp(rng.randn(128) * 0.5)
    k = (rng.randn(1, H, T, 128) * s).astype(np.float16)
    v = rng.randn(1, H, T, 128).astype(np.float16)
    return k, v


def _hook(c, q, name):
    from turboquant_amd import _lib
    qq = q[:, :, 0].contiguous()
    out = torch.empty(qq.shape, dtype=torch.float32, device=qq.device)
    desc = c.attention_descriptor(qq, out, 128 ** -0.5)
    fn = getattr(_lib.load(), name)
    fn.restype = ctypes.c_int32
    if name == "tq_debug_uniform_geometry":
        geo = (ctypes.c_int32 * 4)()
        fn.argtypes = [ctypes.c_void_p] * 4
        rc = fn(ctypes.addressof(c._kc.struct), ctypes.addressof(c._vc.struct), ctypes.addressof(desc),
                ctypes.addressof(geo))
        assert rc == 0, "the uniform-batch grid does not take the call"
        return tuple(geo)
    fn.argtypes = [ctypes.c_void_p] * 3
    return fn(ctypes.addressof(c._kc.struct), ctypes.addressof(c._vc.struct), ctypes.addressof(desc))


def _dense_reference(c, k, v):
    """float64 [sink | stored codes dequantised by the oracle | residual] for a
    cache filled by one update (no drain steps): the fp16 segments are the
    inputs' first sink_len and last fp16_len tokens."""
    S, C, F = c._sink_len, c._compressed_len, c._fp16_len
    assert S + C + F == k.shape[2]
    R = O.rotation_matrix(128)
    ks, vs = [k[:, :, :S].astype(np.float64)], [v[:, :, :S].astype(np.float64)]
    for side, bits, acc in (("k", c.key_bits, ks), ("v", c.value_bits, vs)):
        hi, lo, n = c.packed(side)
        acc.append(O.dequantize(hi.cpu().numpy(), None if lo is None else lo.cpu().numpy(), n.cpu().numpy(), R,
                                bits, 128))
    ks.append(k[:, :, S + C:].astype(np.float64))
    vs.append(v[:, :, S + C:].astype(np.float64))
    return np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)


def _run(kb, vb, H, G, T, seed, geometry, route):
    from turboquant_amd import TurboQuantKVCache
    k, v = _kv(H, T, seed)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=H, key_bits=kb, value_bits=vb, residual_window=128,
                          fp16_sink_size=128)
    c.update(to_dev(k), to_dev(v))
    q = np.random.RandomState(seed + 1).randn(1, H * G, 1, 128).astype(np.float16)
    qd = to_dev(q)
    assert _hook(c, qd, "tq_debug_decode_route") == route
    geo = _hook(c, qd, "tq_debug_uniform_geometry")
    print(f"K{kb}/V{vb} Hkv={H} G={G} T={T}: nwg {geo[0]} blocks/workgroup {geo[1]} fp16/workgroup {geo[2]} "
          f"NPW {geo[3]}", flush=True)
    assert geo == geometry, geo
    fast = c.attend(qd).cpu().numpy()
    gen = c.attend(qd, general_kernel=True).cpu().numpy()
    kk, vv = _dense_reference(c, k, v)
    ref = O.attention(q, kk, vv)
    e_f, e_g = rel_err(fast, ref), rel_err(fast, gen)
    print(f"  rel vs float64 {e_f:.3e}, vs general kernel {e_g:.3e}, min cos {min_cos(fast, ref):.8f}", flush=True)
    assert e_f < FAST_REL_TOL and min_cos(fast, ref) >= COS_TOL
    assert e_g < 1e-4


@pytest.mark.parametrize("kb,vb,route", [(4, 2, 2), (3, 2, 4)], ids=["K4V2", "K3V2"])
def test_configs1_layer_geometry(kb, vb, route):
    """configs[1]'s layer: 32 workgroups per kv head, 32 blocks each (4 per
    wave), 8 fp16 tokens per workgroup, NPW = 4."""
    _run(kb, vb, 8, 4, 32768, 1000 + 10 * kb + vb, (32, 32, 8, 4), route)


WIDTHS = [(2, 2), (2, 3), (2, 4), (3, 2), (3, 3), (3, 4), (4, 3), (4, 4)]


@pytest.mark.parametrize("kb,vb", WIDTHS, ids=[f"K{k}V{v}" for k, v in WIDTHS])
def test_widths_npw8_geometry(kb, vb):
    """The NPW = 8 instantiations of the other integer widths: 8 kv heads x
    40,000 tokens give 32 workgroups per kv head with 39 blocks each."""
    _run(kb, vb, 8, 4, 40000, 2000 + 10 * kb + vb, (32, 39, 8, 8), 4)


@pytest.mark.parametrize("kb,vb,G", [(4, 2, 1), (4, 2, 8), (3, 3, 8), (2, 4, 2)])
def test_npw8_query_groups(kb, vb, G):
    """NPW = 8 at the other query-group sizes (K4/V2 included)."""
    _run(kb, vb, 8, G, 40000, 3000 + 10 * kb + vb + G, (32, 39, 8, 8), 2 if (kb, vb) == (4, 2) else 4)
