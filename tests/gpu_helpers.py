"""Helpers shared by the GPU parity tests: run the HIP path through the C ABI
and compare with the numpy oracle (test infrastructure)."""

from __future__ import annotations

import os

import numpy as np
import torch

import oracle as O


def to_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_compress(x: np.ndarray, bits: float, qjl_m: int = 0, seed: int = 42, general: bool = False):
    """Compress (B, H, T, D) on the GPU; returns numpy (codes_hi, codes_lo, norms, signs, gamma).
    ``general`` routes the call through the general compress kernel."""
    from turboquant_amd import _codec

    xt = to_dev(x)
    B, H, T, D = xt.shape
    codec = _codec.get_codec(D, bits, seed, qjl_m, xt.device)
    st = _codec.PackedStore(codec, B, H, qjl=qjl_m > 0)
    st.reserve(max(T, 1), 0)
    _codec.compress_into(codec, xt, 0, T, st, 0, general=general)
    torch.cuda.synchronize()

    def np_(t):
        return None if t is None else t[:, :, :T].cpu().numpy()

    return np_(st.codes_hi), np_(st.codes_lo), np_(st.norms), np_(st.signs), np_(st.gamma)


def unpack_codes(codes_hi, codes_lo, bits: float, d: int) -> np.ndarray:
    bh, bl, split = O.split_bits(bits, d)
    lead = codes_hi.shape[:-1]
    idx = np.empty((*lead, d), dtype=np.uint8)
    idx[..., :split] = O.unpack_bits(codes_hi, bh, split)
    if split < d:
        idx[..., split:] = O.unpack_bits(codes_lo, bl, d - split)
    return idx


# Every code_parity call of the session: (test, bits, coordinates compared,
# mismatches, mismatches inside the float32 band, of those within 1 ulp of a
# boundary, mismatches outside the band), printed by conftest's terminal
# summary (also under -q).
PARITY_LOG: list[tuple] = []


def code_parity(x: np.ndarray, bits: float, gpu=None, ref=None):
    """Compare GPU codes/norms with the oracle (``ref``: a precomputed
    ``O.compress`` result of the same input). Records the counts in
    PARITY_LOG and asserts that every mismatch lies inside the band.

    Returns (n_mismatch, n_outside_band, n_within_1ulp, total, norms_equal, ref)."""
    D = x.shape[-1]
    R = O.rotation_matrix(D)
    if ref is None:
        ref = O.compress(x, R, bits)
    ch, cl, nrm, _, _ = gpu if gpu is not None else gpu_compress(x, bits)
    idx = unpack_codes(ch, cl, bits, D)
    mism = idx != ref.idx
    outside = mism & ~ref.near
    # strict class: exact coordinate within one float32 ulp of a boundary
    bh, bl, split = O.split_bits(bits, D)
    _, b_hi = O.codebook(D, bh)
    _, b_lo = O.codebook(D, bl)
    y = ref.y64
    ulp1 = np.zeros_like(mism)
    for sl, b in ((slice(0, split), b_hi), (slice(split, D), b_lo)):
        yy = y[..., sl]
        bb = b.astype(np.float64)
        dist = np.min(np.abs(yy[..., None] - bb), axis=-1)
        ulp = np.spacing(np.abs(yy).astype(np.float32)).astype(np.float64)
        ulp1[..., sl] = dist <= ulp
    norms_equal = np.array_equal(nrm.view(np.uint32), ref.norms.view(np.uint32))
    n_m, n_out, n_ulp = int(mism.sum()), int(outside.sum()), int((mism & ulp1).sum())
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    PARITY_LOG.append((test, bits, int(mism.size), n_m, n_m - n_out, n_ulp, n_out))
    assert n_out == 0, f"{n_out} code mismatches outside the float32 boundary band ({n_m} in all)"
    return n_m, n_out, n_ulp, int(mism.size), norms_equal, ref


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def min_cos(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64).reshape(-1, a.shape[-1])
    b = np.asarray(b, np.float64).reshape(-1, b.shape[-1])
    num = (a * b).sum(-1)
    den = np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1)
    ok = den > 0
    return float(np.min(num[ok] / den[ok])) if ok.any() else 1.0
