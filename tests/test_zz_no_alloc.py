"""tq_decode_attention_noalloc (scratch held by the library) against
tq_decode_attention (caller's workspace): same kernels, so the outputs must be
bit-identical. Two calls in a row per route, the second on a smaller cache, so
the second call runs over scratch contents the first one left."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# (key_bits, value_bits, qjl): the K4/V2 kernels, the general kernel, the QJL route
ROUTES = [(4, 2, False), (3, 2, False), (4, 2, True)]


def _cache(T, kb, vb, qjl, seed):
    from turboquant_amd import TurboQuantKVCache
    rng = np.random.RandomState(seed)
    k = torch.from_numpy(rng.randn(1, 4, T, 128).astype(np.float16)).cuda()
    v = torch.from_numpy(rng.randn(1, 4, T, 128).astype(np.float16)).cuda()
    q = torch.from_numpy(rng.randn(1, 16, 128).astype(np.float16)).cuda()
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=4, key_bits=kb, value_bits=vb, residual_window=64,
                          fp16_sink_size=32, qjl_correction=qjl, qjl_n_proj=128)
    c.update(k, v)
    return c, q


@pytest.mark.parametrize("kb,vb,qjl", ROUTES)
def test_noalloc_matches_workspace_entry(kb, vb, qjl):
    from turboquant_amd import _lib
    lib = _lib.load()
    assert lib.tq_decode_noalloc_scratch_bytes() == 64 << 20
    for T, seed in ((3000, 1), (700, 2)):  # the second call is smaller
        cache, q = _cache(T, kb, vb, qjl, seed)
        ref = cache.attend(q)
        out = torch.full_like(ref, float("nan"))
        desc = cache.attention_descriptor(q, out, 128 ** -0.5)
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        rc = lib.tq_decode_attention_noalloc(cache._kc.ref(), cache._vc.ref(), ctypes.byref(desc),
                                             _lib.stream_ptr(q.device))
        _lib.check(rc, "tq_decode_attention_noalloc")
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.equal(out, ref), (T, float((out - ref).abs().max()))


def test_noalloc_rejects_calls_beyond_the_scratch():
    """A call whose workspace exceeds the scratch fails with TQ_ERR_WORKSPACE."""
    from turboquant_amd import _lib
    cache, q = _cache(3000, 4, 2, False, 3)
    out = torch.empty(1, 16, 1, 128, dtype=torch.float32, device=q.device)
    desc = cache.attention_descriptor(q, out, 128 ** -0.5, general=True)
    desc.batch, desc.max_comp = 64, 1 << 20  # host bounds only: fails before any launch
    lib = _lib.load()
    rc = lib.tq_decode_attention_noalloc(cache._kc.ref(), cache._vc.ref(), ctypes.byref(desc), None)
    assert rc == _lib.TQ_ERR_WORKSPACE
    assert b"no-allocation" in lib.tq_last_error()
