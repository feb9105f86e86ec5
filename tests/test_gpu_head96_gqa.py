"""head_dim 96 (the reference ships codebook_d96_b{1..4}.npz; its fused
attention tests cover Phi-3.5-mini's 96, tests/test_fused_attention.py:200-202)
and query-head ratios outside 1 / 2 / 4 / 8 (kv head h // (Hq / Hkv) for any
integer ratio, docs/FULL_FUSED_ATTENTION_RESULTS.md:51) on the GPU against
the oracle.

head_dim 96 at 2 / 3 / 4 bits and the fractional 2.5 / 3.5 (the rotated
vector split at 48: 16-code halves of a 32-code segment take different
widths, and 18-byte rows are written byte by byte): codes bit-exact outside
the float32 band and norms bit-exact (code_parity), dequantize at 1e-5, and
decode attention over the stored codes at 1e-3 / cos 0.9999. Ratios 3, 5, 6,
7, 11, 12 and 16 (launch groups of up to 8 heads per kv head) through the
general kernel, with and without the QJL sketch, on head_dim 128 and 96.
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


def _kv(B, H, T, D, seed, kscale=0.5):
    rng = np.random.RandomState(seed)
    s = np.exp(rng.randn(D) * kscale)
    k = (rng.randn(B, H, T, D) * s).astype(np.float16)
    v = rng.randn(B, H, T, D).astype(np.float16)
    return k, v


@pytest.mark.parametrize("bits", [2, 3, 4, 2.5, 3.5])
def test_d96_compress_dequantize_parity(bits):
    from turboquant_amd import _codec
    x = _kv(1, 3, 301, 96, seed=int(bits * 10))[0]
    gpu = gpu_compress(x, bits)
    _, outside, _, _, norms_eq, _ = code_parity(x, bits, gpu=gpu)
    assert norms_eq and outside == 0
    # dequantize the stored codes
    xt = to_dev(x)
    codec = _codec.get_codec(96, bits, 42, 0, xt.device)
    st = _codec.PackedStore(codec, 1, 3, qjl=False)
    st.reserve(301, 0)
    _codec.compress_into(codec, xt, 0, 301, st, 0)
    out = torch.empty(1, 3, 301, 96, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 301, out, 0, apply_qjl=False)
    ch, cl, nrm = gpu[0], gpu[1], gpu[2]
    ref = O.dequantize(ch, cl, nrm, O.rotation_matrix(96), bits, 96)
    assert rel_err(out.cpu().numpy(), ref) < 1e-5
    assert min_cos(out.cpu().numpy(), x.astype(np.float64)) > (0.95 if bits >= 3 else 0.85)


def test_d96_qjl_sketch():
    """The QJL sketch on head_dim 96 (m = 128 projections: a partial chunk of
    the projection matrix in the dequantize kernel)."""
    from turboquant_amd import _codec
    x = _kv(1, 2, 130, 96, seed=7)[0]
    ch, cl, n, signs, gamma = gpu_compress(x, 3, qjl_m=128)
    R, S = O.rotation_matrix(96), O.projection_matrix(96, 128)
    deq = O.dequantize(ch, cl, n, R, 3, 96)
    r = x.astype(np.float64) - deq
    s_ref, g_ref, proj = O.qjl_sketch(r.reshape(-1, 96), S)
    s_got = np.unpackbits(signs.reshape(-1, 16), axis=-1, bitorder="little").astype(bool)
    band = 1e-5 * np.abs(r.reshape(-1, 96)) @ np.abs(S).T.astype(np.float64)
    assert not np.any((s_got != s_ref) & (np.abs(proj) > band))
    assert np.allclose(gamma.reshape(-1), g_ref, rtol=1e-5, atol=1e-6)
    xt = to_dev(x)
    codec = _codec.get_codec(96, 3, 42, 128, xt.device)
    st = _codec.PackedStore(codec, 1, 2, qjl=True)
    st.reserve(130, 0)
    _codec.compress_into(codec, xt, 0, 130, st, 0)
    out = torch.empty(1, 2, 130, 96, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 130, out, 0, apply_qjl=True)
    corr = O.qjl_correction(s_got, gamma.reshape(-1), S, 96).reshape(deq.shape)
    assert rel_err(out.cpu().numpy(), deq + corr) < 1e-5


def _check(kw, k, v, G, seed, label):
    c, o = build(kw, k, v)
    B, H = k.shape[:2]
    q = np.random.RandomState(seed).randn(B, H * G, 1, kw["head_dim"]).astype(np.float16)
    out = c.attend(to_dev(q)).cpu().numpy()
    kk, vv = dense_from_gpu_codes(c, o)
    ref = O.attention(q, kk, vv)
    e, cs = rel_err(out, ref), min_cos(out, ref)
    print(f"{label}: rel {e:.3e} min cos {cs:.7f}")
    assert e < REL_TOL and cs >= COS_TOL
    return c, q, out


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 2), (3.5, 2.5), (4, 4), (2.5, 2), (2.5, 3.5)])
def test_d96_attention(kb, vb):
    """head_dim 96 on the general kernels; K2.5 keys have an 18-byte 3-bit hi
    segment, so their 2-bit lo segment is staged at the next dword column."""
    k, v = _kv(2, 2, 900, 96, seed=int(kb * 7 + vb))
    kw = dict(head_dim=96, num_kv_heads=2, key_bits=kb, value_bits=vb, residual_window=64, fp16_sink_size=16)
    _check(kw, k, v, 4, 3, f"d96 K{kb}/V{vb}")


@pytest.mark.parametrize("G", [3, 5, 6, 7, 11, 12, 16])
def test_gqa_ratios_d128(G):
    k, v = _kv(2, 2, 700, 128, seed=50 + G)
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=64, fp16_sink_size=16)
    c, q, out = _check(kw, k, v, G, 60 + G, f"d128 G={G}")
    # head h reads kv head h // G: each head alone equals its slice of the batched call
    h = G + 1  # a head of kv head 1
    one = c.attend(to_dev(np.ascontiguousarray(q[:, :: G])), general_kernel=True).cpu().numpy()
    assert rel_err(out[:, ::G], one) < 1e-6
    assert np.isfinite(out[:, h]).all()


@pytest.mark.parametrize("G,d", [(3, 128), (7, 96)])
def test_gqa_ratios_qjl(G, d):
    k, v = _kv(1, 2, 600, d, seed=70 + G)
    kw = dict(head_dim=d, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=32, fp16_sink_size=8,
              qjl_correction=True, qjl_n_proj=64)
    _check(kw, k, v, G, 80 + G, f"qjl d{d} G={G}")


def test_gqa_ratio_uncompressed_only():
    """Ratio 3 before anything is compressed: the general kernel over the fp16
    sink and ring (the dense decode kernel serves ratios 1 / 2 / 4 / 8)."""
    k, v = _kv(1, 2, 100, 128, seed=90)
    kw = dict(head_dim=128, num_kv_heads=2, key_bits=4, value_bits=2, residual_window=256, fp16_sink_size=16)
    c, _, _ = _check(kw, k, v, 3, 91, "d128 G=3 fp16 only")
    assert c._compressed_len == 0
