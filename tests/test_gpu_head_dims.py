"""head_dims beyond the shipped tables (the reference builds a codebook for any
d at runtime, codebook.py:146-174, and its cache takes any d its packers
accept, packing.py:20, 71, 143): multiples of 16 in [16, 256] on the general
compress / dequantize / attention kernels, which run at the head_dim rounded
up to 32 columns with zeros in the padded columns (none stored or read).

Codebooks of these sizes come from the runtime Lloyd-Max (equal to the
oracle's restatement, tests/test_oracle.py). Against the oracle: codes
bit-exact outside the float32 band and norms bit-exact (code_parity);
dequantize at 1e-5; the QJL sketch's signs outside its band and gamma at
1e-5; decode and prefill attention over the stored codes against float64 at
1e-3 / cosine 0.9999. Rows of 30 bytes (80 dims at 3 bits) and other rows
that are not whole dwords are written and read byte by byte.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import code_parity, gpu_compress, min_cos, rel_err, to_dev
from test_gpu_attention import build, dense_from_gpu_codes

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
COS_TOL = 0.9999


def _kv(B, H, T, D, seed):
    rng = np.random.RandomState(seed)
    s = np.exp(rng.randn(D) * 0.5)
    return (rng.randn(B, H, T, D) * s).astype(np.float16), rng.randn(B, H, T, D).astype(np.float16)


CASES = [(80, 2), (80, 3), (80, 4), (48, 3), (112, 4), (16, 2), (32, 3), (160, 3), (192, 2), (224, 4),
         (160, 3.5), (192, 2.5), (224, 3.5)]


@pytest.mark.parametrize("d,bits", CASES, ids=[f"d{d}_b{b}" for d, b in CASES])
def test_compress_dequantize_parity(d, bits):
    from turboquant_amd import _codec
    x = _kv(1, 2, 203, d, seed=d + int(bits * 10))[0]
    gpu = gpu_compress(x, bits)
    _, outside, _, _, norms_eq, _ = code_parity(x, bits, gpu=gpu)
    assert norms_eq and outside == 0
    xt = to_dev(x)
    codec = _codec.get_codec(d, bits, 42, 0, xt.device)
    st = _codec.PackedStore(codec, 1, 2, qjl=False)
    st.reserve(203, 0)
    _codec.compress_into(codec, xt, 0, 203, st, 0)
    out = torch.empty(1, 2, 203, d, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 203, out, 0, apply_qjl=False)
    ref = O.dequantize(gpu[0], gpu[1], gpu[2], O.rotation_matrix(d), bits, d)
    assert rel_err(out.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("d,m", [(80, 64), (48, 96), (160, 128)])
def test_qjl_sketch(d, m):
    """The sketch at head_dims that are not multiples of 32 (the residual's
    padded columns are zero) and with more projections than one tile pass."""
    from turboquant_amd import _codec
    x = _kv(1, 2, 130, d, seed=d + m)[0]
    ch, cl, n, signs, gamma = gpu_compress(x, 3, qjl_m=m)
    R, S = O.rotation_matrix(d), O.projection_matrix(d, m)
    deq = O.dequantize(ch, cl, n, R, 3, d)
    r = x.astype(np.float64) - deq
    s_ref, g_ref, proj = O.qjl_sketch(r.reshape(-1, d), S)
    s_got = np.unpackbits(signs.reshape(-1, m // 8), axis=-1, bitorder="little").astype(bool)
    band = 1e-5 * np.abs(r.reshape(-1, d)) @ np.abs(S).T.astype(np.float64)
    assert not np.any((s_got != s_ref) & (np.abs(proj) > band))
    assert np.allclose(gamma.reshape(-1), g_ref, rtol=1e-5, atol=1e-6)
    xt = to_dev(x)
    codec = _codec.get_codec(d, 3, 42, m, xt.device)
    st = _codec.PackedStore(codec, 1, 2, qjl=True)
    st.reserve(130, 0)
    _codec.compress_into(codec, xt, 0, 130, st, 0)
    out = torch.empty(1, 2, 130, d, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 130, out, 0, apply_qjl=True)
    corr = O.qjl_correction(s_got, gamma.reshape(-1), S, d).reshape(deq.shape)
    assert rel_err(out.cpu().numpy(), deq + corr) < 1e-5


ATT = [(80, 4, 2, 4), (80, 3, 3, 1), (48, 2, 2, 3), (112, 4, 4, 2), (160, 3.5, 2, 4), (192, 2.5, 2.5, 8),
       (32, 4, 2, 2)]


@pytest.mark.parametrize("d,kb,vb,G", ATT, ids=[f"d{d}_K{k}V{v}_G{g}" for d, k, v, g in ATT])
def test_attention_decode_and_prefill(d, kb, vb, G):
    """Decode (one query token) and a causal prefill chunk (12 query tokens)
    on the general kernels, against float64 over the stored codes."""
    k, v = _kv(1, 2, 700, d, seed=d * 3 + G)
    kw = dict(head_dim=d, num_kv_heads=2, key_bits=kb, value_bits=vb, residual_window=32, fp16_sink_size=8)
    c, o = build(kw, k, v)
    assert c._compressed_len > 0
    kk, vv = dense_from_gpu_codes(c, o)
    for tq in (1, 12):
        q = np.random.RandomState(d + tq).randn(1, 2 * G, tq, d).astype(np.float16)
        out = c.attend(to_dev(q)).cpu().numpy()
        ref = O.attention(q, kk, vv, causal_offset=700 - tq)
        e, cs = rel_err(out, ref), min_cos(out, ref)
        print(f"d{d} K{kb}/V{vb} G={G} T_q={tq}: rel {e:.3e} min cos {cs:.7f}")
        assert np.isfinite(out).all() and e < REL_TOL and cs >= COS_TOL


def test_attention_qjl_d80():
    k, v = _kv(1, 2, 600, 80, seed=81)
    kw = dict(head_dim=80, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, fp16_sink_size=8,
              qjl_correction=True, qjl_n_proj=64)
    c, o = build(kw, k, v)
    q = np.random.RandomState(82).randn(1, 8, 1, 80).astype(np.float16)
    out = c.attend(to_dev(q)).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv)
    assert rel_err(out, ref) < REL_TOL and min_cos(out, ref) >= COS_TOL
