"""GPU tests of the cache's saved state: ``state`` / ``meta_state`` get and set
(the reference's cache.py:118-200, used by mlx-lm's prompt-cache save/load).

A reloaded cache must hold exactly the saved tokens: its dense fetch and its
fused attention equal the original's bit for bit, and both caches stay equal
through further updates that drain into the compressed store.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import to_dev

pytestmark = pytest.mark.gpu

D = 128


def make(kw, T, seed, steps=0):
    from turboquant_amd import TurboQuantKVCache
    rng = np.random.RandomState(seed)
    c = TurboQuantKVCache(**kw)
    c.update(to_dev(rng.randn(1, kw["num_kv_heads"], T, D).astype(np.float16)),
             to_dev(rng.randn(1, kw["num_kv_heads"], T, D).astype(np.float16)))
    for _ in range(steps):
        c.update(to_dev(rng.randn(1, kw["num_kv_heads"], 1, D).astype(np.float16)),
                 to_dev(rng.randn(1, kw["num_kv_heads"], 1, D).astype(np.float16)))
    return c


def same_cache(a, b, seed):
    """Dense fetch and fused attention of a and b are identical."""
    ka, va = a.fetch()
    kb, vb = b.fetch()
    assert ka.shape == kb.shape and torch.equal(ka, kb) and torch.equal(va, vb)
    assert a.offset == b.offset and a.meta_state == b.meta_state
    H = a.num_kv_heads
    q = to_dev(np.random.RandomState(seed).randn(1, 4 * H, 1, D).astype(np.float16))
    assert torch.equal(a.attend(q), b.attend(q))


def feed_both(a, b, n, seed):
    rng = np.random.RandomState(seed)
    H = a.num_kv_heads
    for t in range(n):
        k = to_dev(rng.randn(1, H, 1 if t % 3 else 5, D).astype(np.float16))
        v = to_dev(rng.randn(*k.shape).astype(np.float16))
        a.update(k, v)
        b.update(k, v)


KW = [
    dict(head_dim=D, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=64, fp16_sink_size=16),
    dict(head_dim=D, num_kv_heads=2, key_bits=3.5, value_bits=2.5, residual_window=32, fp16_sink_size=8),
    dict(head_dim=D, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, chunk_size=16),
    dict(head_dim=D, num_kv_heads=1, key_bits=3, value_bits=3, residual_window=16, fp16_sink_size=4,
         qjl_correction=True, qjl_n_proj=64),
]


@pytest.mark.parametrize("kw", KW, ids=["k4v2_sink", "k3.5v2.5", "chunked", "qjl"])
def test_state_round_trip(kw):
    from turboquant_amd import TurboQuantKVCache
    a = make(kw, 700, seed=1, steps=9)
    st, meta = a.state, a.meta_state
    assert len(st) == (14 if kw.get("qjl_correction") else 10)
    assert (st[8] is not None) == (kw["key_bits"] != int(kw["key_bits"]))
    b = TurboQuantKVCache(**kw)
    b.state = st        # mlx-lm's order: state, then meta_state
    b.meta_state = meta
    same_cache(a, b, seed=2)
    feed_both(a, b, 120, seed=3)  # drains into the store on both
    same_cache(a, b, seed=4)


def test_state_meta_first():
    from turboquant_amd import TurboQuantKVCache
    kw = KW[0]
    a = make(kw, 300, seed=5)
    b = TurboQuantKVCache(**kw)
    b.meta_state = a.meta_state
    b.state = a.state
    same_cache(a, b, seed=6)


def test_state_reference_layout():
    """A tuple laid out as the reference saves it: the residual buffer at its
    pre-allocated capacity (valid prefix fp16_len), the sink buffer at
    fp16_sink_size, exact-length compressed arrays, numpy arrays on the host;
    meta_state carries the lengths."""
    from turboquant_amd import TurboQuantKVCache
    kw = KW[0]
    a = make(kw, 500, seed=7, steps=4)
    keys, values, kh, kn, vh, vn, sk, sv, kl, vl = a.state
    R = keys.shape[2]
    cap = R + 256
    kbuf = torch.zeros(1, 2, cap, D, dtype=keys.dtype, device=keys.device)
    vbuf = torch.zeros_like(kbuf)
    kbuf[:, :, :R] = keys
    vbuf[:, :, :R] = values
    np_tuple = tuple(None if t is None else t.cpu().numpy() for t in (kbuf, vbuf, kh, kn, vh, vn, sk, sv, kl, vl))
    meta = dict(a.meta_state, fp16_capacity=str(cap))
    b = TurboQuantKVCache(**kw)
    b.state = np_tuple
    b.meta_state = meta
    same_cache(a, b, seed=8)
    feed_both(a, b, 80, seed=9)
    same_cache(a, b, seed=10)


def test_state_legacy_tuples():
    """6 entries (pre-sink format) and 8 entries (sink, no lo parts)."""
    from turboquant_amd import TurboQuantKVCache
    kw6 = dict(KW[0], fp16_sink_size=0)
    a = make(kw6, 400, seed=11)
    b = TurboQuantKVCache(**kw6)
    b.state = a.state[:6]
    b.meta_state = a.meta_state
    same_cache(a, b, seed=12)
    a8 = make(KW[0], 400, seed=13)
    b8 = TurboQuantKVCache(**KW[0])
    b8.state = a8.state[:8]
    b8.meta_state = a8.meta_state
    same_cache(a8, b8, seed=14)


def test_state_without_sketch_drops_old_corrections():
    """A 10-entry tuple of a QJL cache carries no sketch, as the reference's:
    the reloaded tokens are served uncorrected (their gamma is zero), tokens
    compressed after the reload are corrected."""
    from turboquant_amd import TurboQuantKVCache, _codec
    kw = KW[3]
    a = make(kw, 300, seed=15)
    b = TurboQuantKVCache(**kw)
    b.state = a.state[:10]
    b.meta_state = a.meta_state
    C = b._compressed_len
    assert C > 0
    assert torch.count_nonzero(b.sketch("k")[1]) == 0 and torch.count_nonzero(b.sketch("v")[1]) == 0
    # b's dense compressed part = a's codes dequantised without the correction
    S = b._sink_len
    kb, _ = b.fetch()
    plain = torch.zeros(1, 1, C, D, dtype=torch.float32, device=kb.device)
    _codec.dequantize_into(a._kc, a._kstore, 0, C, plain, 0, False)
    assert torch.equal(kb[:, :, S:S + C], plain)
    # new drains on b carry a sketch again
    feed_both(a, b, 60, seed=16)
    g = b.sketch("k")[1]
    assert torch.count_nonzero(g[:, :, :C]) == 0 and torch.count_nonzero(g[:, :, C:b._compressed_len]) > 0


def test_state_errors():
    from turboquant_amd import TurboQuantKVCache
    a = make(KW[0], 300, seed=17)
    other_bits = TurboQuantKVCache(**dict(KW[0], key_bits=3))
    with pytest.raises(ValueError):
        other_bits.state = a.state
    b = TurboQuantKVCache(**KW[0])
    b.state = a.state
    bad = dict(a.meta_state, compressed_len=str(a._compressed_len + 1))
    with pytest.raises(ValueError):
        b.meta_state = bad
