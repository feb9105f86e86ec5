"""numpy restatement of mlx-turboquant's compress / dequantize / attention path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the product package never
imports this module.

Numeric contract (what "bit-exact" is measured against):

* norms: ``n = f32(sqrt(S))`` where ``S`` is the float64 sum of squares in a
  fixed order: dims in blocks of 32, each block summed sequentially from 0.0,
  block sums combined pairwise level by level in index order ((B0+B1)+(B2+B3)
  for d = 128; an odd block at a level carries up unchanged). Squares of
  fp16/fp32 inputs are exact in float64. This restates ``mx.linalg.norm`` of
  the float32 cast (cache.py:235-236) with an order every kernel can follow;
  any float64 order gives the correctly rounded float32 norm except within
  ~2^-29 of a float32 rounding tie (``test_norms_correctly_rounded``).
* normalised input: ``x_n = f32(x) / max(n, f32(1e-10))`` with IEEE float32
  division (cache.py:237-238).
* rotated coordinate: ``y = x_n @ R.T`` (rotation.py:65) evaluated in float64
  from the float32 operands; the code of coordinate j is
  ``#{k : f32(y_j) > b_k}`` (codebook.py:220-223).
* a coordinate is "near-boundary" when ``|y_j - b_k| <= gamma * sum_i |x_n,i R_ji|``
  for some boundary ``b_k``, with ``gamma = m u / (1 - m u)``, ``u = 2**-24``,
  ``m = d + 2``: the standard worst-case bound of a float32 dot product of
  length d plus the rounding of the normalisation. Inside that band the
  reference's own float32 GEMM does not determine the code, so a
  mismatch there is reported, not failed. Outside it codes must be identical.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_REPO = os.path.dirname(_HERE)
CODEBOOK_DIR = os.path.join(_REPO, "mlx-turboquant_amd", "turboquant_amd", "codebooks")

ROTATION_SEED = 42      # rotation.py:14, cache.py:35, patch.py:144
QJL_SEED = 12345        # qjl.py:20
NORM_EPS = np.float32(1e-10)  # cache.py:237

__all__ = [
    "CODEBOOK_DIR", "rotation_matrix", "projection_matrix", "codebook", "lloyd_max_table",
    "quantize_scalar", "dequantize_scalar", "pack_bits", "unpack_bits",
    "sumsq_f64", "vector_norms", "normalize", "rotate_f64", "split_bits", "compress",
    "CompressResult", "dequantize", "boundary_margin", "near_boundary_mask",
    "qjl_sketch", "qjl_correction", "attention", "detect_outlier_layers",
    "CacheOracle", "compress_f32", "reference_decode_step_f32",
]


# --------------------------------------------------------------------------
# a1: rotation
# --------------------------------------------------------------------------
def rotation_matrix(d: int, seed: int = ROTATION_SEED) -> np.ndarray:
    """Seeded orthogonal matrix (rotation.py:17-36).

    ``G = RandomState(seed).randn(d, d)`` cast to float32; numpy's QR promotes
    float32 to float64 internally and casts Q back to float32; columns are
    multiplied by sign(diag(R)) with zero signs replaced by +1.
    """
    rng = np.random.RandomState(seed)
    g = rng.randn(d, d).astype(np.float32)
    q, r = np.linalg.qr(g)
    signs = np.sign(np.diag(r))
    signs[signs == 0] = 1
    return (q * signs[np.newaxis, :]).astype(np.float32)


def projection_matrix(d: int, m: int, seed: int = QJL_SEED) -> np.ndarray:
    """QJL Gaussian projection S of shape (m, d), float32 (qjl.py:23-36)."""
    rng = np.random.RandomState(seed)
    return rng.randn(m, d).astype(np.float32)


# --------------------------------------------------------------------------
# a3-a5: codebook, scalar quantizer
# --------------------------------------------------------------------------
_LM_CACHE: dict = {}


def lloyd_max_table(d: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Lloyd-Max quantizer of one coordinate of a rotated unit vector, as the
    reference computes the tables it does not ship (codebook.py:55-116): a
    10,000-point grid over +-6/sqrt(d); the density N(0, 1/d) for d >= 32,
    else Beta((d-1)/2, (d-1)/2) on [-1, 1] (codebook.py:35-52), normalised on
    the grid; centroids initialised at the quantiles (i + 1/2)/L of the grid
    CDF; each step sets the boundaries to the centroid midpoints and every
    centroid to the grid mean of its cell (cells [b_i, b_i+1), the last one
    closed; an empty cell keeps its centroid); the loop stops, keeping the
    centroids from before the step, once a step moves none by 1e-12, or after
    500 steps. float32 (centroids, boundaries)."""
    key = (d, bits)
    if key in _LM_CACHE:
        return _LM_CACHE[key]
    L = 1 << bits
    sig = 1.0 / math.sqrt(d)
    a, b = -6.0 * sig, 6.0 * sig
    grid = np.linspace(a, b, 10000)
    step = grid[1] - grid[0]
    if d >= 32:  # the same float64 operations as the reference's gaussian_pdf (codebook.py:46-49)
        var = 1.0 / d
        dens = np.exp(-0.5 * grid * grid / var) / math.sqrt(2.0 * math.pi * var)
    else:
        from scipy.special import gammaln
        al = 0.5 * (d - 1)
        lc = gammaln(2 * al) - 2 * gammaln(al) - (2 * al - 1) * math.log(2.0)
        dens = np.exp(lc + (al - 1) * np.log(np.maximum(1.0 - grid * grid, 1e-300)))
    dens = dens / (dens.sum() * step)
    cum = np.cumsum(dens) * step
    cum = cum / cum[-1]
    cen = np.interp(np.linspace(0.5 / L, 1 - 0.5 / L, L), cum, grid)
    for _ in range(500):
        edges = np.concatenate(([a], (cen[:-1] + cen[1:]) / 2.0, [b]))
        upd = cen.copy()
        for i in range(L):
            inside = (grid >= edges[i]) & ((grid <= edges[i + 1]) if i == L - 1 else (grid < edges[i + 1]))
            wt = dens[inside]
            if wt.sum() > 0:
                upd[i] = (grid[inside] * wt).sum() / wt.sum()
        if np.abs(upd - cen).max() < 1e-12:
            break
        cen = upd
    out = (cen.astype(np.float32), ((cen[:-1] + cen[1:]) / 2.0).astype(np.float32))
    _LM_CACHE[key] = out
    return out


def codebook(d: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Shipped Lloyd-Max table (codebook.py:146-174): (centroids, boundaries)
    f32; sizes the reference does not ship are computed as it computes them
    (``lloyd_max_table``)."""
    path = os.path.join(CODEBOOK_DIR, f"codebook_d{d}_b{bits}.npz")
    if not os.path.exists(path):
        return lloyd_max_table(d, bits)
    with np.load(path, allow_pickle=False) as z:
        return z["centroids"].astype(np.float32), z["boundaries"].astype(np.float32)


def quantize_scalar(y: np.ndarray, boundaries: np.ndarray) -> np.ndarray:
    """``idx = #{k : y > b_k}`` as uint8 (codebook.py:203-225). NaN -> 0."""
    y = np.asarray(y, dtype=np.float32)
    b = np.asarray(boundaries, dtype=np.float32)
    return (y[..., None] > b).sum(axis=-1).astype(np.uint8)


def dequantize_scalar(idx: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """``centroids[idx]`` (codebook.py:228-238)."""
    return np.asarray(centroids)[np.asarray(idx).astype(np.int64)]


# --------------------------------------------------------------------------
# a6-a7: packing (LSB-first bitstream per row)
# --------------------------------------------------------------------------
def pack_bits(idx: np.ndarray, bits: int) -> np.ndarray:
    """Pack codes into a little-endian LSB-first bitstream per row.

    Code j of a row occupies bits [bits*j, bits*j + bits) of the row's byte
    string. This is the layout of pack_1bit/2bit/3bit/4bit
    (packing.py:9-32, 60-97, 132-152, 176-194); ``ValueError`` for other
    widths (packing.py:211-222) and ``AssertionError`` when the row does not
    fill whole bytes (packing.py:20, 71, 143, 180).
    """
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"Unsupported bit-width: {bits}. Use 1, 2, 3, or 4.")
    idx = np.asarray(idx, dtype=np.uint8)
    d = idx.shape[-1]
    assert (d * bits) % 8 == 0, f"Last dimension {d} cannot be packed at {bits} bits"
    flat = idx.reshape(-1, d)
    shifts = np.arange(bits, dtype=np.uint8)
    bitplane = ((flat[:, :, None] >> shifts) & 1).reshape(flat.shape[0], d * bits)
    packed = np.packbits(bitplane.reshape(flat.shape[0], -1, 8), axis=-1, bitorder="little")
    return packed.reshape(*idx.shape[:-1], d * bits // 8)


def unpack_bits(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    """Inverse of :func:`pack_bits` (packing.py:35-57, 100-129, 155-173, 225-236)."""
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"Unsupported bit-width: {bits}. Use 1, 2, 3, or 4.")
    packed = np.asarray(packed, dtype=np.uint8)
    nbytes = packed.shape[-1]
    assert nbytes * 8 == d * bits
    flat = packed.reshape(-1, nbytes)
    bitplane = np.unpackbits(flat, axis=-1, bitorder="little").reshape(flat.shape[0], d, bits)
    weights = (1 << np.arange(bits)).astype(np.uint8)
    idx = (bitplane * weights).sum(axis=-1).astype(np.uint8)
    return idx.reshape(*packed.shape[:-1], d)


# --------------------------------------------------------------------------
# a8: norm / normalise / rotate
# --------------------------------------------------------------------------
def sumsq_f64(x: np.ndarray) -> np.ndarray:
    """float64 sum of squares over the last axis in the norm order of the
    module docstring: 32-dim blocks summed sequentially from 0.0, block sums
    combined pairwise level by level (an odd block carries up)."""
    x = np.asarray(x)
    d = x.shape[-1]
    xf = x.reshape(-1, d).astype(np.float64)
    blocks = []
    for b0 in range(0, d, 32):
        acc = np.zeros(xf.shape[0], dtype=np.float64)
        for j in range(b0, min(b0 + 32, d)):
            acc = acc + xf[:, j] * xf[:, j]
        blocks.append(acc)
    while len(blocks) > 1:
        nxt = [blocks[i] + blocks[i + 1] for i in range(0, len(blocks) - 1, 2)]
        if len(blocks) % 2:
            nxt.append(blocks[-1])
        blocks = nxt
    return blocks[0].reshape(x.shape[:-1])


def vector_norms(x: np.ndarray) -> np.ndarray:
    """L2 norm over the last axis (cache.py:235-236), float32 result.

    ``sqrt(sumsq_f64(x))`` in float64 rounded to float32 (equal to the
    correctly rounded float32 square root of the float64 sum, since
    53 >= 2*24 + 2).
    """
    return np.sqrt(sumsq_f64(x)).astype(np.float32)


def normalize(x: np.ndarray, norms: np.ndarray) -> np.ndarray:
    """``f32(x) / max(n, 1e-10)`` in float32 (cache.py:237-238)."""
    safe = np.maximum(np.asarray(norms, dtype=np.float32), NORM_EPS)
    return (np.asarray(x).astype(np.float32) / safe[..., None]).astype(np.float32)


def rotate_f64(x: np.ndarray, rotation: np.ndarray) -> np.ndarray:
    """``x @ R.T`` (rotation.py:55-65) evaluated in float64."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(rotation, dtype=np.float64).T


def split_bits(bits: float, d: int) -> tuple[int, int, int]:
    """(bits_hi, bits_lo, split) for integer or fractional widths.

    Integer widths use one codebook over all d dims. A fractional width
    quantises rotated dims [0, d/2) at ceil(bits) and [d/2, d) at floor(bits)
    (cache.py:63-84, 253-274). ``split`` is the number of dims at bits_hi.
    """
    if bits != int(bits):
        return int(bits) + 1, int(bits), d // 2
    return int(bits), int(bits), d


def boundary_margin(y64: np.ndarray, xn: np.ndarray, rotation: np.ndarray,
                    boundaries: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Distance of each exact coordinate to its nearest boundary, and the band.

    Returns ``(dist, band)`` both shaped like ``y64``: ``dist = min_k |y - b_k|``
    and ``band = gamma_{d+2} * sum_i |x_n,i * R_ji|`` (see module docstring).
    """
    d = y64.shape[-1]
    u = 2.0 ** -24
    m = d + 2
    gamma = m * u / (1.0 - m * u)
    absdot = np.abs(np.asarray(xn, np.float64)) @ np.abs(np.asarray(rotation, np.float64)).T
    b = np.asarray(boundaries, np.float64)
    dist = np.min(np.abs(y64[..., None] - b), axis=-1)
    return dist, gamma * absdot


def near_boundary_mask(y64, xn, rotation, boundaries) -> np.ndarray:
    dist, band = boundary_margin(y64, xn, rotation, boundaries)
    return dist <= band


@dataclass
class CompressResult:
    codes_hi: np.ndarray          # (..., split*bits_hi/8) uint8
    codes_lo: np.ndarray | None   # (..., (d-split)*bits_lo/8) uint8 or None
    norms: np.ndarray             # (...) float32
    idx: np.ndarray               # (..., d) uint8 unpacked codes
    y64: np.ndarray               # (..., d) float64 exact rotated coordinates
    near: np.ndarray              # (..., d) bool: coordinate inside the f32 band
    xn: np.ndarray = field(repr=False, default=None)


def compress(x: np.ndarray, rotation: np.ndarray, bits: float) -> CompressResult:
    """norm -> normalise -> rotate -> quantize -> pack (cache.py:232-274).

    ``x``: (..., d) fp16 or fp32. Integer ``bits`` in {1,2,3,4}; fractional
    widths split the rotated vector (cache.py:253-274).
    """
    x = np.asarray(x)
    d = x.shape[-1]
    lead = x.shape[:-1]
    bits_hi, bits_lo, split = split_bits(bits, d)
    norms = vector_norms(x)
    xn = normalize(x, norms)
    y64 = rotate_f64(xn.reshape(-1, d), rotation)
    y32 = y64.astype(np.float32)
    _, b_hi = codebook(d, bits_hi)
    idx = np.empty(y32.shape, dtype=np.uint8)
    idx[:, :split] = quantize_scalar(y32[:, :split], b_hi)
    near = np.empty(y32.shape, dtype=bool)
    near[:, :split] = near_boundary_mask(y64, xn.reshape(-1, d), rotation, b_hi)[:, :split]
    codes_lo = None
    if split < d:
        _, b_lo = codebook(d, bits_lo)
        idx[:, split:] = quantize_scalar(y32[:, split:], b_lo)
        near[:, split:] = near_boundary_mask(y64, xn.reshape(-1, d), rotation, b_lo)[:, split:]
        codes_lo = pack_bits(idx[:, split:], bits_lo).reshape(*lead, -1)
    codes_hi = pack_bits(idx[:, :split], bits_hi).reshape(*lead, -1)
    return CompressResult(codes_hi=codes_hi, codes_lo=codes_lo, norms=norms,
                          idx=idx.reshape(*lead, d), y64=y64.reshape(*lead, d),
                          near=near.reshape(*lead, d), xn=xn)


# --------------------------------------------------------------------------
# a11-a12: dequantize
# --------------------------------------------------------------------------
def dequantize(codes_hi: np.ndarray, codes_lo: np.ndarray | None, norms: np.ndarray,
               rotation: np.ndarray, bits: float, d: int) -> np.ndarray:
    """``x_hat = n * (c[idx] @ R)`` in float64 (cache.py:276-300, 336-343)."""
    bits_hi, bits_lo, split = split_bits(bits, d)
    lead = np.asarray(norms).shape
    c_hi, _ = codebook(d, bits_hi)
    y = np.empty((int(np.prod(lead, dtype=np.int64)), d), dtype=np.float64)
    y[:, :split] = dequantize_scalar(unpack_bits(np.asarray(codes_hi).reshape(-1, codes_hi.shape[-1]),
                                                 bits_hi, split), c_hi)
    if split < d:
        c_lo, _ = codebook(d, bits_lo)
        y[:, split:] = dequantize_scalar(unpack_bits(np.asarray(codes_lo).reshape(-1, codes_lo.shape[-1]),
                                                     bits_lo, d - split), c_lo)
    x = (y @ np.asarray(rotation, np.float64)) * np.asarray(norms, np.float64).reshape(-1, 1)
    return x.reshape(*lead, d)


# --------------------------------------------------------------------------
# a13: QJL sign sketch
# --------------------------------------------------------------------------
def qjl_sketch(residual: np.ndarray, projection: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``(signs, gamma, proj)``: ``signs = (r @ S.T >= 0)``, ``gamma = ||r||``
    (qjl.py:47-67). Evaluated in float64; ``proj`` returned for margin checks."""
    r = np.asarray(residual, np.float64)
    proj = r @ np.asarray(projection, np.float64).T
    gamma = np.sqrt(np.sum(r * r, axis=-1))
    return proj >= 0, gamma, proj


def qjl_correction(signs: np.ndarray, gamma: np.ndarray, projection: np.ndarray, d: int) -> np.ndarray:
    """``(sqrt(pi/2)/d) * gamma * (z @ S)`` with z = +-1 (qjl.py:70-94; d = head_dim)."""
    z = np.where(signs, 1.0, -1.0)
    return (math.sqrt(math.pi / 2) / d) * np.asarray(gamma, np.float64)[..., None] * (
        z @ np.asarray(projection, np.float64))


# --------------------------------------------------------------------------
# a19-a20: attention
# --------------------------------------------------------------------------
def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
              causal_offset: int | None = None) -> np.ndarray:
    """float64 softmax attention with grouped heads.

    q: (B, Hq, Tq, D); k, v: (B, Hkv, T, D). Query head h reads kv head
    ``h // (Hq // Hkv)`` and scores are scaled by ``D**-0.5`` by default
    (docs/attention_source_dump.txt:30-31, 49). With ``causal_offset`` the
    query at row i sees keys [0, causal_offset + i].
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, Tq, D = q.shape
    Hkv = k.shape[1]
    rep = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    kk = np.repeat(k, rep, axis=1)
    vv = np.repeat(v, rep, axis=1)
    s = np.einsum("bhqd,bhtd->bhqt", q, kk) * scale
    if causal_offset is not None:
        T = k.shape[2]
        qi = np.arange(Tq)[:, None] + causal_offset
        ti = np.arange(T)[None, :]
        s = np.where(ti <= qi, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqt,bhtd->bhqd", p, vv)


# --------------------------------------------------------------------------
# a22: outlier-layer rule
# --------------------------------------------------------------------------
def detect_outlier_layers(max_norms, threshold: float = 3.0) -> list[int]:
    """Layers whose max key norm exceeds threshold x median of the positive
    maxima; empty when no maximum is positive (patch.py:119-133)."""
    m = np.asarray(max_norms, dtype=np.float64)
    pos = m[m > 0]
    if pos.size == 0:
        return []
    med = float(np.median(pos))
    return [i for i, n in enumerate(m) if n > threshold * med]


# --------------------------------------------------------------------------
# a14-a18: cache state machine
# --------------------------------------------------------------------------
class CacheOracle:
    """State machine of ``TurboQuantKVCache`` (cache.py:28-116, 429-706).

    Holds float64 dequantised tensors in place of the reference's float32
    decompressed cache, and also keeps the QJL sign sketch / residual norm of
    every compressed vector so that fused attention can be checked against
    the corrected dense cache.
    """

    def __init__(self, head_dim=128, num_kv_heads=1, key_bits=4, value_bits=2,
                 residual_window=128, rotation_seed=ROTATION_SEED, fp16_sink_size=0,
                 chunk_size=0, qjl_correction=False, qjl_n_proj=32):
        self.d = head_dim
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.window = residual_window
        self.sink_size = fp16_sink_size
        self.chunk = chunk_size
        self.qjl = qjl_correction
        self.R = rotation_matrix(head_dim, rotation_seed)
        self.S = projection_matrix(head_dim, qjl_n_proj) if qjl_correction else None
        self.offset = 0
        self.sink_k = self.sink_v = None
        self.sink_len = 0
        self.buf_k = self.buf_v = None   # fp16 residual window (B,H,n,D)
        self.comp = {"k": [], "v": []}   # list of CompressResult per drain
        self.deq = {"k": [], "v": []}    # float64 dequantised (+QJL) chunks
        self.sketch = {"k": [], "v": []} # (signs, gamma) per drain when QJL on
        self.compressed_len = 0
        self.drains: list[int] = []

    @property
    def fp16_len(self) -> int:
        return 0 if self.buf_k is None else self.buf_k.shape[2]

    def _route_sink(self, k, v):
        # cache.py:577-618
        if self.sink_size <= 0 or self.offset >= self.sink_size:
            return k, v
        T = k.shape[2]
        n = min(self.sink_size - self.offset, T)
        if n <= 0:
            return k, v
        if self.sink_k is None:
            B, H, _, D = k.shape
            self.sink_k = np.zeros((B, H, self.sink_size, D), dtype=k.dtype)
            self.sink_v = np.zeros((B, H, self.sink_size, D), dtype=v.dtype)
        self.sink_k[:, :, self.offset:self.offset + n] = k[:, :, :n]
        self.sink_v[:, :, self.offset:self.offset + n] = v[:, :, :n]
        self.sink_len = self.offset + n
        return k[:, :, n:], v[:, :, n:]

    def _compress_side(self, x, bits):
        res = compress(x, self.R, bits)
        deq = dequantize(res.codes_hi, res.codes_lo, res.norms, self.R, bits, self.d)
        sk = None
        if self.qjl:
            # cache.py:396-427: residual against the MSE reconstruction
            r = np.asarray(x, np.float64) - deq
            signs, gamma, _ = qjl_sketch(r.reshape(-1, self.d), self.S)
            deq = deq + qjl_correction(signs, gamma, self.S, self.d).reshape(deq.shape)
            sk = (signs.reshape(*deq.shape[:-1], -1), gamma.reshape(deq.shape[:-1]))
        return res, deq, sk

    def _drain(self, n):
        # cache.py:535-575
        old_k, old_v = self.buf_k[:, :, :n], self.buf_v[:, :, :n]
        self.buf_k, self.buf_v = self.buf_k[:, :, n:], self.buf_v[:, :, n:]
        for side, x, bits in (("k", old_k, self.key_bits), ("v", old_v, self.value_bits)):
            res, deq, sk = self._compress_side(x, bits)
            self.comp[side].append(res)
            self.deq[side].append(deq)
            self.sketch[side].append(sk)
        self.compressed_len += n
        self.drains.append(n)

    def _compress_old(self):
        # cache.py:497-533
        if self.buf_k is None:
            return
        if self.chunk <= 0:
            if self.fp16_len <= 2 * self.window:
                return
            self._drain(self.fp16_len - self.window)
            return
        while self.fp16_len >= self.window + self.chunk:
            self._drain(self.chunk)

    def update(self, k, v):
        """Append (B,H,T,D) fp16 keys/values (cache.py:620-672)."""
        T = k.shape[2]
        rk, rv = self._route_sink(k, v)
        if rk.shape[2] > 0:
            if self.buf_k is None:
                self.buf_k, self.buf_v = rk.copy(), rv.copy()
            else:
                self.buf_k = np.concatenate([self.buf_k, rk], axis=2)
                self.buf_v = np.concatenate([self.buf_v, rv], axis=2)
        self.offset += T
        self._compress_old()

    def dense(self) -> tuple[np.ndarray, np.ndarray]:
        """``[sink | decompressed | residual]`` in float64 (cache.py:682-706)."""
        ks, vs = [], []
        if self.sink_len > 0:
            ks.append(self.sink_k[:, :, :self.sink_len].astype(np.float64))
            vs.append(self.sink_v[:, :, :self.sink_len].astype(np.float64))
        if self.compressed_len > 0:
            ks.append(np.concatenate(self.deq["k"], axis=2))
            vs.append(np.concatenate(self.deq["v"], axis=2))
        if self.fp16_len > 0:
            ks.append(self.buf_k.astype(np.float64))
            vs.append(self.buf_v.astype(np.float64))
        return np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)

    def packed(self, side: str):
        """Concatenated (codes_hi, codes_lo, norms) of all drains for a side."""
        rs = self.comp[side]
        hi = np.concatenate([r.codes_hi for r in rs], axis=2)
        lo = None if rs[0].codes_lo is None else np.concatenate([r.codes_lo for r in rs], axis=2)
        n = np.concatenate([r.norms for r in rs], axis=2)
        return hi, lo, n

    def attend(self, q: np.ndarray, scale: float | None = None) -> np.ndarray:
        k, v = self.dense()
        return attention(q, k, v, scale)


# --------------------------------------------------------------------------
# float32 restatements of the reference's per-step CPU work, used only as the
# timed CPU baseline of bench.py (not as a parity checker)
# --------------------------------------------------------------------------
def compress_f32(x: np.ndarray, rotation: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """The reference's compress arithmetic in float32 numpy/OpenBLAS:
    norm, normalise, ``x_n @ R.T``, boundary count, pack (cache.py:232-251)."""
    d = x.shape[-1]
    xf = np.asarray(x, np.float32).reshape(-1, d)
    n = np.sqrt(np.einsum("ij,ij->i", xf, xf)).astype(np.float32)
    y = (xf / np.maximum(n, NORM_EPS)[:, None]) @ np.asarray(rotation, np.float32).T
    _, b = codebook(d, bits)
    idx = np.searchsorted(b, y, side="left").astype(np.uint8)  # == #{k: y > b_k}
    return pack_bits(idx, bits), n


def reference_decode_step_f32(sink_k, sink_v, deq_k, deq_v, res_k, res_v, q, scale=None):
    """One decode step of the reference for one layer: concatenate
    [sink | decompressed | residual] (cache.py:682-706) and run grouped
    scaled-dot-product attention over the float32 result (mlx-lm SDPA)."""
    k = np.concatenate([sink_k.astype(np.float32), deq_k, res_k.astype(np.float32)], axis=2)
    v = np.concatenate([sink_v.astype(np.float32), deq_v, res_v.astype(np.float32)], axis=2)
    B, Hq, _, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    qq = (q.astype(np.float32) * np.float32(scale)).reshape(B, Hkv, g, D)
    s = np.matmul(qq, k.transpose(0, 1, 3, 2))          # (B, Hkv, g, T)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v).reshape(B, Hq, 1, D)
