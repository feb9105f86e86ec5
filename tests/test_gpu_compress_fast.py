"""GPU parity of the MFMA compress kernel (fp16, head_dim 128, no QJL) that
tq_compress selects, against the oracle and against the general kernel.

Bar (as tests/test_gpu_codec.py): norms bit-exact; codes bit-exact outside the
float32 dot-product band of the oracle's module docstring. Covers partial
tiles, ragged per-batch spans through the C ABI, strided sources and offset
destinations, extreme magnitudes, NaN inputs, every width, and the
configs[2] prefill size through size-independent properties.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import code_parity, gpu_compress, min_cos, to_dev, unpack_codes

pytestmark = pytest.mark.gpu


def _x(shape, seed, scale=None, vec_scale=None):
    rng = np.random.RandomState(seed)
    x = rng.randn(*shape)
    if scale is not None:
        x = x * np.exp(rng.randn(shape[-1]) * scale)
    if vec_scale is not None:
        x = x * np.exp(rng.randn(*shape[:-1], 1) * vec_scale)
    return np.clip(x, -6e4, 6e4).astype(np.float16)


@pytest.mark.parametrize("T", [1, 17, 63, 64, 65, 200, 1000])
def test_partial_tiles(T):
    x = _x((1, 3, T, 128), seed=T, scale=0.5)
    mism, outside, ulp1, total, norms_eq, _ = code_parity(x, 4)
    print(f"T={T}: mismatches {mism}/{total} (outside band {outside}, within 1 ulp {ulp1})")
    assert norms_eq and outside == 0


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 1.5, 2.5, 3.5])
def test_every_width_mixed_scales(bits):
    x = _x((2, 4, 130, 128), seed=int(bits * 10), scale=0.5, vec_scale=2.5)
    mism, outside, ulp1, total, norms_eq, _ = code_parity(x, bits)
    print(f"bits={bits}: mismatches {mism}/{total} (outside band {outside}, within 1 ulp {ulp1})")
    assert norms_eq and outside == 0


def test_extreme_magnitudes():
    rng = np.random.RandomState(3)
    x = rng.randn(1, 2, 96, 128)
    x[0, 0, :32] *= 6e4 / np.abs(x[0, 0, :32]).max(axis=-1, keepdims=True)  # up to fp16 max
    x[0, 0, 32:64] *= 1e-6                                                # fp16 subnormals
    x[0, 1, :16] = 0.0
    x[0, 1, 16:32, 1:] = 0.0                                              # one-hot vectors
    x[0, 1, 32:48] = np.where(rng.rand(16, 128) < 0.9, 0.0, x[0, 1, 32:48])  # sparse
    x = x.astype(np.float16)
    for bits in (4, 3, 2):
        mism, outside, _, _, norms_eq, _ = code_parity(x, bits)
        assert norms_eq and outside == 0, bits


def test_nan_vector_codes_zero():
    x = _x((1, 1, 8, 128), seed=1)
    x[0, 0, 3, 5] = np.nan
    ch, _, n, _, _ = gpu_compress(x, 4)
    assert np.isnan(n[0, 0, 3])
    assert np.all(O.unpack_bits(ch[0, 0, 3], 4, 128) == 0)  # NaN -> 0 (codebook.py:220-223)
    ref = O.compress(np.delete(x, 3, axis=2), O.rotation_matrix(128), 4)
    got = np.delete(O.unpack_bits(ch, 4, 128), 3, axis=2)
    assert not np.any((got != ref.idx) & ~ref.near)


@pytest.mark.parametrize("bits", [4, 3, 2, 3.5])
def test_axis_vectors_and_infinities(bits):
    """Vectors along rotated axes (x = +-s R_j, so y_j = +-1: the outermost
    quantizer cells) and vectors holding an infinity (norm inf, codes 0)."""
    R = O.rotation_matrix(128)
    rows = [0, 1, 37, 64, 100, 127]
    x = np.concatenate([np.stack([R[j] * sg * sc for j in rows]) for sg in (1.0, -1.0) for sc in (1.0, 300.0)])
    x = x.astype(np.float16)[None, None]
    mism, outside, ulp1, total, norms_eq, _ = code_parity(x, bits)
    print(f"bits={bits}: axis vectors, mismatches {mism}/{total} (outside band {outside})")
    assert norms_eq and outside == 0
    y = _x((1, 1, 8, 128), seed=11)
    y[0, 0, 2, 7] = np.inf
    y[0, 0, 5, 0] = -np.inf
    ch, cl, n, _, _ = gpu_compress(y, bits)
    assert np.isinf(n[0, 0, 2]) and np.isinf(n[0, 0, 5])
    for t in (2, 5):
        assert not ch[0, 0, t].any() and (cl is None or not cl[0, 0, t].any())


def test_fast_and_general_kernels_agree():
    """Both kernels against the oracle on the same input, and with each other
    outside the band."""
    x = _x((1, 8, 512, 128), seed=9, scale=0.5)
    fast = gpu_compress(x, 3.5)
    gen = gpu_compress(x, 3.5, general=True)
    r_fast = code_parity(x, 3.5, gpu=fast)
    r_gen = code_parity(x, 3.5, gpu=gen, ref=r_fast[5])
    assert r_fast[4] and r_gen[4] and r_fast[1] == 0 and r_gen[1] == 0
    assert np.array_equal(fast[2].view(np.uint32), gen[2].view(np.uint32))
    i_f = unpack_codes(fast[0], fast[1], 3.5, 128)
    i_g = unpack_codes(gen[0], gen[1], 3.5, 128)
    assert not np.any((i_f != i_g) & ~r_fast[5].near)


def _compress_span(codec, x, heads, n_tok, n_tok_b, src0_b, dst0_b, store):
    from turboquant_amd import _lib
    lib = _lib.load()
    keep = [torch.tensor(a, dtype=torch.int32, device="cuda") if a is not None else None
            for a in (n_tok_b, src0_b, dst0_b)]
    span = _lib.Span(rows=x.shape[0] * x.shape[1], heads=heads, n_tok=n_tok, reserved=0,
                     n_tok_b=_lib.ptr(keep[0]), src_tok0_b=_lib.ptr(keep[1]), dst_tok0_b=_lib.ptr(keep[2]))
    st = store.struct(0)
    _lib.check(lib.tq_compress(codec.ref(), x.data_ptr(), _lib.TQ_F16, x.stride(1), ctypes.byref(span),
                               ctypes.byref(st), _lib.stream_ptr(x.device)), "tq_compress")
    torch.cuda.synchronize()


@pytest.mark.parametrize("bits", [4, 2.5])
def test_ragged_span_offsets(bits):
    """Per-batch token counts and source / destination offsets (C ABI)."""
    from turboquant_amd import _codec
    B, H, T, D = 3, 2, 300, 128
    x = _x((B, H, T, D), seed=21, scale=0.5)
    xt = to_dev(x)
    n_b, s_b, d_b = [70, 0, 129], [5, 0, 100], [0, 3, 64]
    codec = _codec.get_codec(D, bits, 42, 0, xt.device)
    st = _codec.PackedStore(codec, B, H, qjl=False)
    st.reserve(512, 0)
    for t in (st.codes_hi, st.codes_lo, st.norms):
        if t is not None:
            t.fill_(0xAB if t.dtype == torch.uint8 else 7.0)
    _compress_span(codec, xt, H, max(n_b), n_b, s_b, d_b, st)
    R = O.rotation_matrix(D)
    for b in range(B):
        n, s0, d0 = n_b[b], s_b[b], d_b[b]
        hi = st.codes_hi[b].cpu().numpy()
        lo = None if st.codes_lo is None else st.codes_lo[b].cpu().numpy()
        nr = st.norms[b].cpu().numpy()
        # untouched outside [d0, d0 + n)
        assert np.all(hi[:, :d0] == 0xAB) and np.all(hi[:, d0 + n:] == 0xAB)
        assert np.all(nr[:, :d0] == 7.0) and np.all(nr[:, d0 + n:] == 7.0)
        if n == 0:
            continue
        gpu = (hi[None, :, d0:d0 + n], None if lo is None else lo[None, :, d0:d0 + n], nr[None, :, d0:d0 + n],
               None, None)
        mism, outside, _, _, norms_eq, _ = code_parity(x[b:b + 1, :, s0:s0 + n], bits, gpu=gpu)
        assert norms_eq and outside == 0


@pytest.mark.parametrize("bits", [3, 2, 3.5])
def test_prefill_config2_size_properties(bits):
    """configs[2] shape (8 heads x 126,976 compressed tokens, fp16, keys with
    per-channel LogNormal(0, 0.5) scale): a seeded sample of rows against the
    oracle, every vector's norm against a float64 norm, and the dequantized
    reconstruction quality of every vector."""
    from turboquant_amd import _codec
    H, T, D = 8, 126976, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    scale = torch.exp(torch.randn(D, generator=g, device="cuda") * 0.5)
    x = (torch.randn(1, H, T, D, generator=g, device="cuda") * scale).half()
    codec = _codec.get_codec(D, bits, 42, 0, x.device)
    st = _codec.PackedStore(codec, 1, H, qjl=False)
    st.reserve(T, 0)
    _codec.compress_into(codec, x, 0, T, st, 0)
    torch.cuda.synchronize()
    # norms of every vector vs float64 (the exact norm rounds to the same float32
    # except within ~2^-29 of a rounding tie)
    n64 = torch.linalg.vector_norm(x.double(), dim=-1).float()
    assert torch.equal(st.norms[:, :, :T], n64)
    # 512 sampled tokens x 8 heads for exact code parity
    rng = np.random.RandomState(int(bits * 10) + 1)
    ts = np.sort(rng.choice(T, 512, replace=False))
    xs = x[:, :, ts].cpu().numpy()
    gpu = (st.codes_hi[:, :, ts].cpu().numpy(),
           None if st.codes_lo is None else st.codes_lo[:, :, ts].cpu().numpy(),
           st.norms[:, :, ts].cpu().numpy(), None, None)
    mism, outside, ulp1, total, norms_eq, _ = code_parity(xs, bits, gpu=gpu)
    print(f"bits={bits}: sample mismatches {mism}/{total} (outside band {outside}, within 1 ulp {ulp1})")
    assert norms_eq and outside == 0
    # reconstruction of every vector (GPU dequantize), reference bounds of
    # test_phase2.py:583-639 (median cos > 0.99 for 4-bit, > 0.85 for 2-bit)
    out = torch.empty(1, H, T, D, dtype=torch.float32, device="cuda")
    _codec.dequantize_into(codec, st, 0, T, out, 0, apply_qjl=False)
    cos = torch.nn.functional.cosine_similarity(out, x.float(), dim=-1)
    med = float(cos.median())
    print(f"bits={bits}: median cos {med:.5f}, min {float(cos.min()):.5f}")
    assert med > {2: 0.9, 3: 0.97, 3.5: 0.98}[bits]
