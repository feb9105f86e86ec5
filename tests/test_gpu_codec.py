"""GPU parity of the compress / dequantize / packing kernels against the oracle.

Bar: norms bit-exact; codes bit-exact except coordinates whose exact value lies
inside the float32 dot-product band around a boundary (oracle module docstring);
the count of such mismatches, and how many are within 1 ulp, is printed.
"""

import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import code_parity, gpu_compress, min_cos, rel_err, to_dev, unpack_codes

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _x(shape, seed, dtype=np.float16, scale=None):
    rng = np.random.RandomState(seed)
    x = rng.randn(*shape)
    if scale is not None:
        x = x * np.exp(rng.randn(shape[-1]) * scale)
    return x.astype(dtype)


@pytest.mark.parametrize("bits", [4, 2, 3, 3.5, 2.5, 1])
def test_compress_parity_config1_shape(bits):
    x = _x((1, 8, 1024, 128), seed=0)
    mism, outside, ulp1, total, norms_eq, _ = code_parity(x, bits)
    print(f"bits={bits}: mismatches {mism}/{total} (outside band {outside}, within 1 ulp {ulp1})")
    assert norms_eq
    assert outside == 0


@pytest.mark.parametrize("dtype", [np.float32, "bf16"])
def test_compress_parity_input_dtypes(dtype):
    if dtype == "bf16":
        x32 = _x((1, 4, 256, 128), seed=3, dtype=np.float32)
        xt = torch.from_numpy(x32).to(torch.bfloat16)
        x = xt.float().numpy()  # exact bf16 values for the oracle
        from turboquant_amd import _codec
        xd = xt.cuda()
        codec = _codec.get_codec(128, 4, 42, 0, xd.device)
        st = _codec.PackedStore(codec, 1, 4, qjl=False)
        st.reserve(256, 0)
        _codec.compress_into(codec, xd, 0, 256, st, 0)
        gpu = (st.codes_hi[:, :, :256].cpu().numpy(), None, st.norms[:, :, :256].cpu().numpy(), None, None)
        mism, outside, _, _, norms_eq, _ = code_parity(x, 4, gpu=gpu)
    else:
        x = _x((1, 4, 256, 128), seed=3, dtype=dtype, scale=0.5)
        mism, outside, _, _, norms_eq, _ = code_parity(x, 4)
    assert norms_eq and outside == 0


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("bits", [4, 3, 2, 3.5])
def test_compress_parity_head_dims(d, bits):
    x = _x((1, 2, 300, d), seed=d + int(bits * 10))
    mism, outside, _, _, norms_eq, _ = code_parity(x, bits)
    assert norms_eq and outside == 0


def test_compress_golden_config1():
    """Oracle and GPU both reproduce the committed config-1 digests/slice."""
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        gold = json.load(f)["config1"]
    rng = np.random.RandomState(0)
    k = rng.randn(1, 8, 1024, 128).astype(np.float16)
    v = rng.randn(1, 8, 1024, 128).astype(np.float16)
    # config 1 drains tokens [128, 896) (sink 128, window 128)
    kd, vd = k[:, :, 128:896], v[:, :, 128:896]
    kh, _, kn, _, _ = gpu_compress(kd, 4)
    vh, _, vn, _, _ = gpu_compress(vd, 2)
    sl = np.load(os.path.join(GOLDEN, "config1_slice.npz"))
    assert np.array_equal(kn[:, :2, :32].view(np.uint32), sl["k_norms"].view(np.uint32))
    assert np.array_equal(vn[:, :2, :32].view(np.uint32), sl["v_norms"].view(np.uint32))
    for got, want, near, bits in ((kh, sl["k_codes"], sl["k_near"], 4), (vh, sl["v_codes"], sl["v_near"], 2)):
        gi = O.unpack_bits(got[:, :2, :32], bits, 128)
        wi = O.unpack_bits(want, bits, 128)
        assert not np.any((gi != wi) & ~near)
    import hashlib
    assert hashlib.sha256(np.ascontiguousarray(kn).tobytes()).hexdigest() == gold["k_norms"]
    assert hashlib.sha256(np.ascontiguousarray(vn).tobytes()).hexdigest() == gold["v_norms"]


def test_zero_vector():
    x = np.zeros((1, 1, 4, 128), np.float16)
    ch, _, n, _, _ = gpu_compress(x, 4)
    assert np.all(n == 0)
    assert np.all(O.unpack_bits(ch, 4, 128) == 7)  # y = 0 < middle boundary +2.3e-17


@pytest.mark.parametrize("bits", [4, 2, 3.5])
def test_dequantize_parity(bits):
    from turboquant_amd import _codec
    x = _x((1, 4, 200, 128), seed=11)
    xt = to_dev(x)
    codec = _codec.get_codec(128, bits, 42, 0, xt.device)
    st = _codec.PackedStore(codec, 1, 4, qjl=False)
    st.reserve(200, 0)
    _codec.compress_into(codec, xt, 0, 200, st, 0)
    out = torch.empty(1, 4, 200, 128, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 200, out, 0, apply_qjl=False)
    ch = st.codes_hi[:, :, :200].cpu().numpy()
    cl = None if st.codes_lo is None else st.codes_lo[:, :, :200].cpu().numpy()
    ref = O.dequantize(ch, cl, st.norms[:, :, :200].cpu().numpy(), O.rotation_matrix(128), bits, 128)
    got = out.cpu().numpy()
    assert rel_err(got, ref) < 1e-5
    assert min_cos(got, x.astype(np.float64)) > (0.95 if bits >= 3 else 0.8)


def test_qjl_sketch_parity():
    from turboquant_amd import _codec
    x = _x((1, 2, 128, 128), seed=5)
    ch, _, n, signs, gamma = gpu_compress(x, 4, qjl_m=128)
    R = O.rotation_matrix(128)
    S = O.projection_matrix(128, 128)
    ref = O.compress(x, R, 4)
    deq = O.dequantize(ch, None, n, R, 4, 128)
    r = x.astype(np.float64) - deq
    s_ref, g_ref, proj = O.qjl_sketch(r.reshape(-1, 128), S)
    s_got = np.unpackbits(signs.reshape(-1, 16), axis=-1, bitorder="little").astype(bool)
    # signs may differ only where the projection is within float32 error of 0
    band = 1e-5 * np.abs(r.reshape(-1, 128)) @ np.abs(S).T.astype(np.float64)
    assert not np.any((s_got != s_ref) & (np.abs(proj) > band))
    assert np.allclose(gamma.reshape(-1), g_ref, rtol=1e-5, atol=1e-6)
    # dequantize with correction
    xt = to_dev(x)
    codec = _codec.get_codec(128, 4, 42, 128, xt.device)
    st = _codec.PackedStore(codec, 1, 2, qjl=True)
    st.reserve(128, 0)
    _codec.compress_into(codec, xt, 0, 128, st, 0)
    out = torch.empty(1, 2, 128, 128, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, 128, out, 0, apply_qjl=True)
    corr = O.qjl_correction(s_got, gamma.reshape(-1), S, 128).reshape(deq.shape)
    assert rel_err(out.cpu().numpy(), deq + corr) < 1e-5
    assert ref.norms.shape == n.shape


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_unpack_kernels(bits):
    from turboquant_amd.packing import pack_indices, unpack_indices
    rng = np.random.RandomState(bits)
    for d in (8, 48, 128):
        if (d * bits) % 8:
            continue
        idx = rng.randint(0, 1 << bits, size=(3, 5, d)).astype(np.uint8)
        p = pack_indices(to_dev(idx), bits).cpu().numpy()
        assert np.array_equal(p, O.pack_bits(idx, bits))
        u = unpack_indices(to_dev(p), bits, d).cpu().numpy()
        assert np.array_equal(u, idx)


def test_pack_errors():
    from turboquant_amd.packing import pack_indices
    with pytest.raises(ValueError):
        pack_indices(torch.zeros(1, 8, dtype=torch.uint8, device="cuda"), 5)


def test_quantize_scalar_known_answers():
    from turboquant_amd.codebook import get_codebook, quantize_scalar
    c, b = get_codebook(128, 4)
    y = torch.tensor([10.0, -10.0, 0.0, float("nan")], device="cuda")
    assert quantize_scalar(y, c, b).cpu().tolist() == [15, 0, 7, 0]
    y = b[7:8] + 1e-7
    assert quantize_scalar(y, c, b).item() == 8


def test_mse_quantizer_roundtrip():
    from turboquant_amd import TurboQuantMSE
    x = torch.randn(500, 128, device="cuda")
    q = TurboQuantMSE(128, bits=4)
    qt = q.quantize(x)
    assert qt.packed_indices.shape == (500, 64) and qt.norms.shape == (500,)
    xh = q.dequantize(qt)
    mse = ((xh - x) ** 2).sum(-1) / (x ** 2).sum(-1)
    assert float(mse.median()) < 0.015   # reference test_phase1.py:321-337


def test_prod_quantizer():
    from turboquant_amd import TurboQuantProd
    x = torch.randn(256, 128, device="cuda")
    q = TurboQuantProd(128, bits=4)
    qt = q.quantize(x)
    assert qt.qjl_signs.shape == (256, 128) and qt.qjl_norms.shape == (256,)
    xh = q.dequantize(qt)
    assert xh.shape == x.shape and torch.isfinite(xh).all()
