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
"""

import numpy as np
import pytest

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


def _prefill(kw, T, tq, G, seed, B=1):
    k, v = _kv(B, kw["num_kv_heads"], T, kw["head_dim"], seed)
    c, o = build(kw, k, v)
    q = np.random.RandomState(seed + 1).randn(B, kw["num_kv_heads"] * G, tq, kw["head_dim"]).astype(np.float16)
    out = c.attend(to_dev(q)).cpu().numpy()
    assert out.shape == q.shape
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv, causal_offset=T - tq)
    e, cs = rel_err(out, ref), min_cos(out, ref)
    print(f"T_kv={T} T_q={tq} {kw.get('key_bits')}/{kw.get('value_bits')} G={G}: rel {e:.3e} min cos {cs:.7f} "
          f"(compressed {c._compressed_len})")
    assert e < REL_TOL and cs >= COS_TOL
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
