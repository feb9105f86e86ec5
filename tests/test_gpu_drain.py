"""The one-vector drain kernel of tq_compress (spans of at most 8 tokens per
row, head_dim 128, with the QJL sketch: the one-token ragged drains of a
decode step, cache.py:529-533 with qjl_correction) against the tiled general
compress kernel (TQ_CODEC_GENERAL_COMPRESS): both compute the same float32 /
float64 operations in the same order, so codes, norms, residual norms and
sign words must be bit-identical. The general kernel itself is checked
against the oracle in test_gpu_codec.py / test_gpu_ragged.py.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
D = 128


def drain(codec, ring, n_b, src_b, dst_b, heads, general):
    from turboquant_amd import _codec, _lib
    B = ring.shape[0]
    store = _codec.PackedStore(codec, B, heads, qjl=True)
    store.reserve(64, 0)
    for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
        t = getattr(store, name)
        if t is not None:
            t.zero_()
    i32 = lambda a: torch.tensor(np.asarray(a, np.int32), device=DEV)
    nb, sb, db = i32(n_b), i32(src_b), i32(dst_b)
    span = _lib.Span(rows=B * heads, heads=heads, n_tok=int(max(n_b)), reserved=0, n_tok_b=nb.data_ptr(),
                     src_tok0_b=sb.data_ptr(), dst_tok0_b=db.data_ptr())
    lib = _lib.load()
    st = store.struct(0)
    _lib.check(lib.tq_compress(codec.ref(general), ring.data_ptr(), _lib.dtype_code(ring.dtype), ring.shape[2] * D,
                               ctypes.byref(span), ctypes.byref(st), _lib.stream_ptr(DEV)), "tq_compress")
    torch.cuda.synchronize()
    return {n: getattr(store, n).cpu().numpy() for n in ("codes_hi", "codes_lo", "norms", "signs", "gamma")
            if getattr(store, n) is not None}


@pytest.mark.parametrize("bits,qjl_m,dtype,n_b", [
    (4, 128, torch.float16, [1, 1, 1, 1, 1]),           # the configs[4] drain: one token per sequence
    (4, 64, torch.float32, [1, 0, 1, 0, 1]),            # sequences without a drain this step
    (3, 128, torch.float16, [3, 8, 1, 0, 5]),           # up to 8 tokens per row
    (3.5, 96, torch.bfloat16, [2, 2, 7, 1, 4]),         # fractional width (hi / lo codes), m = 96
])
def test_drain_kernel_matches_general(bits, qjl_m, dtype, n_b):
    from turboquant_amd import _codec
    B, H, cap = len(n_b), 3, 40
    g = torch.Generator(device=DEV).manual_seed(17)
    ring = (torch.randn(B, H, cap, D, generator=g, device=DEV) * 2.5).to(dtype)
    codec = _codec.get_codec(D, bits, 42, qjl_m, DEV)
    rng = np.random.RandomState(3)
    src_b = rng.randint(0, cap - 8, size=B)
    dst_b = rng.randint(0, 50, size=B)
    a = drain(codec, ring, n_b, src_b, dst_b, H, general=False)
    b = drain(codec, ring, n_b, src_b, dst_b, H, general=True)
    for name in a:
        assert np.array_equal(a[name], b[name]), f"{name} differs between the drain and general kernels"
    # something was written where a drain happened, nothing elsewhere
    norms = a["norms"]
    for s, n in enumerate(n_b):
        assert (norms[s, :, dst_b[s]:dst_b[s] + n] > 0).all()
        assert (norms[s, :, :dst_b[s]] == 0).all() and (norms[s, :, dst_b[s] + n:] == 0).all()
