"""Tensor-level quantizers (quantizer.py:33-195) on the GPU against the oracle.

TurboQuantMSE.quantize: codes bit-exact with O.compress outside the float32
boundary band (code_parity, which records and asserts the counts), norms
bit-exact; dequantize against O.dequantize at 1e-5. TurboQuantProd: the
(bits - 1)-bit stage the same way, the QJL signs against O.qjl_sketch of the
residual x - O.dequantize(stored codes) (equal wherever the projection is
outside float32 error of 0), gamma at 1e-5, and the corrected output against
O.dequantize + O.qjl_correction at 1e-5. Leading batch shapes, float32 /
fp16 / bf16 inputs, and the reference's edge cases
(tests/test_edge_cases.py:131-202): large and tiny norms, identical vectors,
batch against single, TurboQuantProd at 2 bits, zero-token and one-token
cache updates.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import code_parity, rel_err, to_dev

pytestmark = pytest.mark.gpu

R128 = None


def _R():
    global R128
    if R128 is None:
        R128 = O.rotation_matrix(128)
    return R128


def _mse_parity(x_np: np.ndarray, bits: int, dtype=torch.float32):
    """Quantize x (any leading shape, last dim 128) with TurboQuantMSE; check
    codes / norms against the oracle and dequantize against O.dequantize."""
    from turboquant_amd import TurboQuantMSE
    tq = TurboQuantMSE(128, bits=bits)
    xt = torch.from_numpy(np.ascontiguousarray(x_np)).to("cuda", dtype)
    x_in = xt.cpu().float().numpy() if dtype == torch.bfloat16 else xt.cpu().numpy()
    qt = tq.quantize(xt)
    lead = x_np.shape[:-1]
    assert qt.packed_indices.shape == (*lead, 128 * bits // 8) and qt.norms.shape == lead
    n = int(np.prod(lead, dtype=np.int64))
    ch = qt.packed_indices.reshape(n, -1).cpu().numpy()
    nrm = qt.norms.reshape(n).cpu().numpy()
    mism, outside, _, _, norms_eq, _ = code_parity(x_in.reshape(n, 128), bits, gpu=(ch, None, nrm, None, None))
    assert norms_eq and outside == 0
    got = tq.dequantize(qt)
    assert got.shape == (*lead, 128) and got.dtype == torch.float32
    ref = O.dequantize(ch, None, nrm, _R(), bits, 128).reshape(*lead, 128)
    assert rel_err(got.cpu().numpy(), ref) < 1e-5
    return qt, got


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("lead", [(7,), (3, 5), (2, 3, 4)])
def test_mse_quantize_dequantize_parity(bits, lead):
    x = np.random.RandomState(bits * 10 + len(lead)).randn(*lead, 128).astype(np.float32)
    _mse_parity(x, bits)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mse_half_inputs(dtype):
    x = (np.random.RandomState(5).randn(64, 128) * 3).astype(np.float32)
    _mse_parity(x, 4, dtype)


def test_mse_large_and_tiny_norms():
    """Norms of ~1e4 and ~1e-7 (reference: x * 1000 and x * 1e-8): the same
    codes as the oracle, finite outputs, norms preserved by the round trip."""
    rng = np.random.RandomState(6)
    big = (rng.randn(10, 128) * 1000).astype(np.float32)
    _, xh = _mse_parity(big, 4)
    ratio = np.linalg.norm(xh.cpu().numpy(), axis=-1) / np.linalg.norm(big, axis=-1)
    assert 0.9 < np.median(ratio) < 1.1
    tiny = (rng.randn(10, 128) * 1e-8).astype(np.float32)
    _, xh = _mse_parity(tiny, 4)
    assert torch.isfinite(xh).all()
    zero = np.zeros((3, 128), np.float32)  # the norm floor 1e-10: codes of y = 0, output 0
    _, xh = _mse_parity(zero, 4)
    assert torch.equal(xh, torch.zeros_like(xh))


def test_mse_identical_and_batch_vs_single():
    from turboquant_amd import TurboQuantMSE
    tq = TurboQuantMSE(128, bits=4)
    x = torch.from_numpy(np.random.RandomState(42).randn(5, 128).astype(np.float32)).cuda()
    a, b = tq.quantize(x[0]), tq.quantize(x[0])
    assert torch.equal(a.packed_indices, b.packed_indices) and torch.equal(a.norms, b.norms)
    assert a.packed_indices.shape == (64,) and a.norms.shape == ()
    qb = tq.quantize(x)
    xb = tq.dequantize(qb)
    for i in range(5):
        qs = tq.quantize(x[i])
        assert torch.equal(qs.packed_indices, qb.packed_indices[i]) and torch.equal(qs.norms, qb.norms[i])
        assert torch.equal(tq.dequantize(qs), xb[i])


@pytest.mark.parametrize("bits,m,seed", [(4, 128, 12345), (3, 64, 12345), (2, 128, 12345), (4, 256, 12345),
                                         (4, 48, 12345), (3, 100, 12345), (4, 128, 7), (2, 17, 2024)])
def test_prod_parity(bits, m, seed):
    """Any qjl_dim in [1, 256] and any qjl_seed (quantizer.py:122-139)."""
    from turboquant_amd import TurboQuantProd
    x = np.random.RandomState(bits + m).randn(6, 40, 128).astype(np.float32)
    tq = TurboQuantProd(128, bits=bits, qjl_dim=m, qjl_seed=seed)
    qt = tq.quantize(to_dev(x))
    assert qt.qjl_signs.shape == (6, 40, m) and qt.qjl_norms.shape == (6, 40)
    n = 240
    ch = qt.packed_indices.reshape(n, -1).cpu().numpy()
    nrm = qt.norms.reshape(n).cpu().numpy()
    _, outside, _, _, norms_eq, _ = code_parity(x.reshape(n, 128), bits - 1, gpu=(ch, None, nrm, None, None))
    assert norms_eq and outside == 0
    S = O.projection_matrix(128, m, seed)
    deq = O.dequantize(ch, None, nrm, _R(), bits - 1, 128)
    r = x.reshape(n, 128).astype(np.float64) - deq
    s_ref, g_ref, proj = O.qjl_sketch(r, S)
    s_got = qt.qjl_signs.reshape(n, m).cpu().numpy()
    band = 1e-5 * np.abs(r) @ np.abs(S).T.astype(np.float64)
    assert not np.any((s_got != s_ref) & (np.abs(proj) > band))
    g_got = qt.qjl_norms.reshape(n).cpu().numpy()
    assert np.allclose(g_got, g_ref, rtol=1e-5, atol=1e-7)
    got = tq.dequantize(qt).reshape(n, 128).cpu().numpy()
    ref = deq + O.qjl_correction(s_got, g_got, S, 128)
    assert rel_err(got, ref) < 1e-5
    assert np.isfinite(got).all()
    # without the sketch: the (bits - 1)-bit stage alone
    from turboquant_amd.quantizer import QuantizedTensor
    mse_only = tq.dequantize(QuantizedTensor(qt.packed_indices, qt.norms, bits, 128))
    assert rel_err(mse_only.reshape(n, 128).cpu().numpy(), deq) < 1e-5


def test_cache_zero_and_one_token_updates():
    """update_and_fetch with zero tokens returns an empty view and changes
    nothing; a single token comes back exactly (reference
    test_edge_cases.py:185-202)."""
    from turboquant_amd import TurboQuantKVCache
    c = TurboQuantKVCache(head_dim=128, key_bits=4, value_bits=2)
    k0 = torch.randn(1, 2, 0, 128, device="cuda")
    ko, vo = c.update_and_fetch(k0, k0.clone())
    assert ko.shape[2] == 0 and vo.shape[2] == 0 and c.offset == 0
    c1 = TurboQuantKVCache(head_dim=128, key_bits=4, value_bits=2, residual_window=128)
    k1 = torch.randn(1, 2, 1, 128, device="cuda")
    v1 = torch.randn(1, 2, 1, 128, device="cuda")
    ko, vo = c1.update_and_fetch(k1, v1)
    assert ko.shape == (1, 2, 1, 128) and torch.equal(ko.float(), k1) and torch.equal(vo.float(), v1)
    ko, vo = c1.update_and_fetch(k0, k0.clone())  # zero tokens after one: the same single token
    assert ko.shape == (1, 2, 1, 128) and c1.offset == 1 and torch.equal(ko.float(), k1)
    # a compressed cache: zero-token update after drains leaves the dense view unchanged
    c2 = TurboQuantKVCache(head_dim=128, key_bits=4, value_bits=2, residual_window=16)
    k = torch.randn(1, 2, 100, 128, device="cuda").half()
    kd, vd = c2.update_and_fetch(k, k.clone())
    kd, vd = kd.clone(), vd.clone()
    assert c2._compressed_len > 0
    ke, ve = c2.update_and_fetch(k[:, :, :0], k[:, :, :0])
    assert torch.equal(ke, kd) and torch.equal(ve, vd) and c2.offset == 100
