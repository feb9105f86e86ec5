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


def _noalloc(lib, cache, q, out):
    from turboquant_amd import _lib
    desc = cache.attention_descriptor(q, out, 128 ** -0.5)
    rc = lib.tq_decode_attention_noalloc(cache._kc.ref(), cache._vc.ref(), ctypes.byref(desc),
                                         _lib.stream_ptr(q.device))
    _lib.check(rc, "tq_decode_attention_noalloc")
    return desc


def test_noalloc_takes_no_device_memory_per_call():
    """hipMemGetInfo's free bytes (torch.cuda.mem_get_info) do not move across
    no-allocation calls of different sizes and routes, once the library's
    code object (which holds the scratch array) is resident."""
    from turboquant_amd import _lib
    lib = _lib.load()
    cases = [_cache(T, kb, vb, qjl, seed) for T, kb, vb, qjl, seed in
             ((3000, 4, 2, False, 11), (700, 3, 2, False, 12), (1500, 4, 2, True, 13))]
    outs = [torch.empty(1, 16, 1, 128, dtype=torch.float32, device="cuda") for _ in cases]
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    descs = [_noalloc(lib, c, q, o) for (c, q), o in zip(cases, outs)]  # first calls: the scratch lookup
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    # the first call on the device may bring the code object (and so the
    # 64 MiB array) in; nothing more
    assert free0 - free1 <= (64 << 20) + (32 << 20), (free0, free1)
    for _ in range(3):
        for (c, q), o in zip(cases, outs):
            _noalloc(lib, c, q, o)
    torch.cuda.synchronize()
    free2, _ = torch.cuda.mem_get_info()
    assert free2 == free1, (free1, free2)
    del descs


@pytest.mark.parametrize("kb,vb,qjl", ROUTES)
def test_noalloc_under_graph_capture(kb, vb, qjl):
    """The no-allocation entry point captured in a HIP graph: every replay
    (with eager library work and synchronisations between the replays)
    matches the workspace entry point's output bit for bit."""
    from turboquant_amd import _lib
    lib = _lib.load()
    cache, q = _cache(2500, kb, vb, qjl, 21)
    other, q2 = _cache(900, kb, vb, qjl, 22)
    ref = cache.attend(q)
    ref2 = other.attend(q2)
    out = torch.full_like(ref, float("nan"))
    _noalloc(lib, cache, q, out)  # warm-up outside the capture (the scratch address lookup)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        _noalloc(lib, cache, q, out)
    for i in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (i, float((out - ref).nan_to_num(1e30).abs().max()))
        # eager work on the same scratch between replays
        out2 = torch.full_like(ref2, float("nan"))
        _noalloc(lib, other, q2, out2)
        torch.cuda.synchronize()
        assert torch.equal(out2, ref2)


def test_noalloc_rejects_a_malformed_descriptor_first():
    """A malformed descriptor (here a negative compressed length) is rejected
    as invalid before any scratch sizing."""
    from turboquant_amd import _lib
    cache, q = _cache(3000, 4, 2, False, 3)
    out = torch.empty(1, 16, 1, 128, dtype=torch.float32, device=q.device)
    desc = cache.attention_descriptor(q, out, 128 ** -0.5)
    desc.max_comp = -5
    lib = _lib.load()
    rc = lib.tq_decode_attention_noalloc(cache._kc.ref(), cache._vc.ref(), ctypes.byref(desc), None)
    assert rc == _lib.TQ_ERR_INVALID, rc
