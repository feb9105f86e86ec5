"""Host-side logic of TurboQuantKVCache on the CPU (no GPU).

The two device calls (compress_into / dequantize_into) are replaced by
oracle-backed stand-ins writing into CPU tensors, so the drain schedule, the
residual ring, sink routing, store growth and dense assembly of the real host
code are checked against the oracle's state machine (cache.py:497-706).
"""

import numpy as np
import pytest
import torch

import oracle as O


@pytest.fixture
def cpu_cache(monkeypatch):
    from turboquant_amd import _codec, _lib, cache as cache_mod

    def fake_compress(codec, x, x_tok0, n_tok, store, dst_tok0):
        if n_tok <= 0:
            return
        xs = x[:, :, x_tok0:x_tok0 + n_tok].cpu().numpy()
        r = O.compress(xs, codec.rotation.cpu().numpy(), codec.bits)
        store.codes_hi[:, :, dst_tok0:dst_tok0 + n_tok] = torch.from_numpy(r.codes_hi)
        if r.codes_lo is not None:
            store.codes_lo[:, :, dst_tok0:dst_tok0 + n_tok] = torch.from_numpy(r.codes_lo)
        store.norms[:, :, dst_tok0:dst_tok0 + n_tok] = torch.from_numpy(r.norms)
        if store.signs is not None:
            deq = O.dequantize(r.codes_hi, r.codes_lo, r.norms, codec.rotation.cpu().numpy(), codec.bits, codec.d)
            s, g, _ = O.qjl_sketch((xs.astype(np.float64) - deq).reshape(-1, codec.d), codec.proj.cpu().numpy())
            packed = np.packbits(s.reshape(-1, codec.qjl_m // 8, 8), axis=-1, bitorder="little")
            store.signs[:, :, dst_tok0:dst_tok0 + n_tok] = torch.from_numpy(packed.reshape(*xs.shape[:3], -1))
            store.gamma[:, :, dst_tok0:dst_tok0 + n_tok] = torch.from_numpy(g.reshape(xs.shape[:3]).astype(np.float32))

    def fake_dequant(codec, store, src_tok0, n_tok, out, out_tok0, apply_qjl):
        if n_tok <= 0:
            return
        sl = slice(src_tok0, src_tok0 + n_tok)
        lo = None if store.codes_lo is None else store.codes_lo[:, :, sl].numpy()
        x = O.dequantize(store.codes_hi[:, :, sl].numpy(), lo, store.norms[:, :, sl].numpy(),
                         codec.rotation.cpu().numpy(), codec.bits, codec.d)
        if apply_qjl:
            signs = np.unpackbits(store.signs[:, :, sl].numpy(), axis=-1, bitorder="little").astype(bool)
            x = x + O.qjl_correction(signs, store.gamma[:, :, sl].numpy(), codec.proj.cpu().numpy(), codec.d)
        out[:, :, out_tok0:out_tok0 + n_tok] = torch.from_numpy(x.astype(np.float32))

    monkeypatch.setattr(_codec, "compress_into", fake_compress)
    monkeypatch.setattr(_codec, "dequantize_into", fake_dequant)
    monkeypatch.setattr(_lib, "require_device", lambda t: None)
    monkeypatch.setattr(_codec, "_require_gfx950", lambda dev: None)
    return cache_mod.TurboQuantKVCache


def _run(cls, kw, chunks, seed=0):
    rng = np.random.RandomState(seed)
    c = cls(**kw)
    o = O.CacheOracle(**kw)
    for T in chunks:
        k = rng.randn(1, 2, T, kw.get("head_dim", 128)).astype(np.float16)
        v = rng.randn(1, 2, T, kw.get("head_dim", 128)).astype(np.float16)
        c.update(torch.from_numpy(k), torch.from_numpy(v))
        o.update(k, v)
        assert c.offset == o.offset
        assert c._compressed_len == o.compressed_len
        assert c._fp16_len == o.fp16_len
        assert c._sink_len == o.sink_len
        assert c.drains == o.drains
    return c, o


def _assert_state_equal(c, o):
    if o.fp16_len:
        rk, rv = c._residual_linear()
        assert np.array_equal(rk.numpy(), o.buf_k) and np.array_equal(rv.numpy(), o.buf_v)
    if o.compressed_len:
        for side in ("k", "v"):
            hi, lo, n = c.packed(side)
            ohi, olo, on = o.packed(side)
            assert np.array_equal(hi.numpy(), ohi)
            assert np.array_equal(n.numpy(), on)
            if olo is not None:
                assert np.array_equal(lo.numpy(), olo)
    kd, vd = c.fetch()
    ko, vo = o.dense()
    assert kd.shape == ko.shape
    assert np.allclose(kd.numpy().astype(np.float64), ko, atol=1e-5)
    assert np.allclose(vd.numpy().astype(np.float64), vo, atol=1e-5)


@pytest.mark.parametrize("kw,chunks", [
    (dict(residual_window=32), [100] + [1] * 80),
    (dict(residual_window=32, chunk_size=8, fp16_sink_size=8), [200] + [1] * 77),
    (dict(residual_window=16, chunk_size=5), [3, 50, 1, 1, 7, 40] + [1] * 30),
    (dict(residual_window=0), [10, 1, 1, 5]),
    (dict(residual_window=8, fp16_sink_size=20), [5, 5, 5, 30, 1, 1]),
    (dict(residual_window=128, fp16_sink_size=128, key_bits=3.5, value_bits=2.5), [1024]),
    (dict(residual_window=4, chunk_size=1, qjl_correction=True, qjl_n_proj=32), [40] + [1] * 12),
])
def test_host_logic_matches_oracle(cpu_cache, kw, chunks):
    kw = dict(head_dim=128, num_kv_heads=2, **kw)
    c, o = _run(cpu_cache, kw, chunks)
    _assert_state_equal(c, o)


def test_fixed_size_chunks(cpu_cache):
    """Mirrors test_phase2.py:405-457."""
    c, o = _run(cpu_cache, dict(head_dim=128, num_kv_heads=2, residual_window=16, chunk_size=32), [100])
    assert c.drains == [32, 32] and c._fp16_len == 36


def test_drain_schedule():
    from turboquant_amd.cache import drain_schedule
    assert drain_schedule(256, 128, 0) == []
    assert drain_schedule(257, 128, 0) == [129]
    assert drain_schedule(32640, 128, 0) == [32512]
    assert drain_schedule(131072 - 128, 128, 4096) == [4096] * 31
    assert drain_schedule(129, 128, 1) == [1]
    assert drain_schedule(10, 0, 0) == [10]
    assert drain_schedule(0, 0, 0) == []


@pytest.mark.parametrize("kw,chunks,more", [
    (dict(residual_window=32, chunk_size=8, fp16_sink_size=8), [200] + [1] * 7, [1] * 40),
    (dict(residual_window=16, key_bits=3.5, value_bits=2.5, fp16_sink_size=4), [90, 3], [1] * 50),
    (dict(residual_window=4, chunk_size=1, qjl_correction=True, qjl_n_proj=32), [40], [1] * 12),
])
def test_state_round_trip_host(cpu_cache, kw, chunks, more):
    """state / meta_state (cache.py:118-200): a reloaded cache holds the same
    tokens as the oracle and keeps following it through later drains."""
    kw = dict(head_dim=128, num_kv_heads=2, **kw)
    c, o = _run(cpu_cache, kw, chunks)
    st, meta = c.state, c.meta_state
    assert len(st) == (14 if kw.get("qjl_correction") else 10)
    assert meta == {k: str(x) for k, x in dict(
        offset=o.offset, compressed_len=o.compressed_len, head_dim=128, key_bits=kw.get("key_bits", 4),
        value_bits=kw.get("value_bits", 2), fp16_sink_size=kw.get("fp16_sink_size", 0), sink_len=o.sink_len,
        fp16_len=o.fp16_len, fp16_capacity=o.fp16_len).items()}
    r = cpu_cache(**kw)
    r.state = st
    r.meta_state = meta
    _assert_state_equal(r, o)
    rng = np.random.RandomState(1)
    for T in more:
        k = rng.randn(1, 2, T, 128).astype(np.float16)
        v = rng.randn(1, 2, T, 128).astype(np.float16)
        r.update(torch.from_numpy(k), torch.from_numpy(v))
        o.update(k, v)
    assert (r.offset, r._compressed_len, r._fp16_len, r._sink_len) == (o.offset, o.compressed_len, o.fp16_len, o.sink_len)
    _assert_state_equal(r, o)


def test_state_reference_layout_host(cpu_cache):
    """The reference's layout: residual buffer at capacity with a valid
    prefix, lengths in meta_state set after the arrays (mlx-lm's order)."""
    kw = dict(head_dim=128, num_kv_heads=2, residual_window=32, fp16_sink_size=8)
    c, o = _run(cpu_cache, kw, [150, 1, 1])
    keys, values, *rest = c.state
    cap = keys.shape[2] + 256
    kbuf = torch.zeros(1, 2, cap, 128, dtype=keys.dtype)
    vbuf = torch.zeros_like(kbuf)
    kbuf[:, :, :keys.shape[2]] = keys
    vbuf[:, :, :keys.shape[2]] = values
    r = cpu_cache(**kw)
    r.state = tuple(t.numpy() if t is not None else None for t in (kbuf, vbuf, *rest))
    assert r._fp16_len == cap  # lengths from shapes until meta_state arrives
    r.meta_state = dict(c.meta_state, fp16_capacity=str(cap))
    _assert_state_equal(r, o)


def test_state_shapes_and_errors():
    from turboquant_amd import TurboQuantKVCache
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=2)
    assert c.state == (None,) * 10
    assert c.meta_state["offset"] == "0" and c.meta_state["fp16_capacity"] == "0"
    for n in (5, 7, 9, 11):
        with pytest.raises(ValueError):
            c.state = (None,) * n


def test_qjl_projection_any_count_and_seed():
    """Any projection count in [1, 256] and any seed: the codec's S is the
    reference's RandomState(seed).randn(m, d) (qjl.py:23-36) padded with zero
    rows to whole 32-projection words; a zero row contributes nothing to the
    correction (its sign is +1 but it multiplies a zero row) nor to S q."""
    from turboquant_amd import TurboQuantKVCache, qjl
    rng = np.random.RandomState(3)
    for m, seed in ((1, 12345), (17, 7), (32, 12345), (48, 12345), (100, 2024), (256, 12345)):
        S = qjl.get_projection_matrix(128, m, seed, device="cpu", padded=True).numpy()
        mp = qjl.padded_count(m)
        assert S.shape == (mp, 128) and mp % 32 == 0 and mp - m < 32
        assert np.array_equal(S[:m], O.projection_matrix(128, m, seed))
        assert not S[m:].any()
        r = rng.randn(5, 128)
        s_pad, g_pad, _ = O.qjl_sketch(r, S)
        s_ref, g_ref, _ = O.qjl_sketch(r, S[:m])
        assert np.array_equal(s_pad[:, :m], s_ref) and s_pad[:, m:].all() and np.array_equal(g_pad, g_ref)
        assert np.allclose(O.qjl_correction(s_pad, g_pad, S, 128), O.qjl_correction(s_ref, g_ref, S[:m], 128),
                           rtol=0, atol=1e-12)
        TurboQuantKVCache(head_dim=128, qjl_correction=True, qjl_n_proj=m)  # accepted
    for bad in (0, 257, -3, 2.5):
        with pytest.raises(ValueError):
            TurboQuantKVCache(head_dim=128, qjl_correction=True, qjl_n_proj=bad)
