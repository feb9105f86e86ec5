"""The C-ABI library loads and exports every entry point include/*.h declares
(CPU only: no kernel is launched)."""

import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(tq_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("tq_compress", "tq_dequantize", "tq_decode_attention", "tq_last_error",
                 "tq_pack_codes", "tq_unpack_codes", "tq_quantize_scalar", "tq_decode_workspace_bytes"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from turboquant_amd import _lib
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} not bound in _lib.SIGNATURES"
    assert lib.tq_abi_version() == 3


def test_struct_layouts_match_header():
    """Compile a tiny C program printing sizeof/offsetof and compare with ctypes."""
    import shutil
    import subprocess
    import tempfile
    from turboquant_amd import _lib
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    fields = {"tq_codec": _lib.Codec, "tq_store": _lib.Store, "tq_span": _lib.Span, "tq_attn_desc": _lib.AttnDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "tq_abi.h"', "int main(void){"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "l.c")
        open(src, "w").write("\n".join(lines))
        exe = os.path.join(d, "l")
        subprocess.run([cc, "-I", os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(line.rsplit(" ", 1) for line in out if line)
    for cname, cls in fields.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, f"{cname}.{f}"


def test_host_side_validation_errors():
    """Argument checks return error codes before any device work."""
    from turboquant_amd import _lib
    lib = _lib.load()
    assert lib.tq_pack_codes(None, 1, 128, 5, None, None) == _lib.TQ_ERR_UNSUPPORTED
    assert b"Unsupported bit-width" in lib.tq_last_error()
    assert lib.tq_unpack_codes(None, 1, 5, 3, None, None) == _lib.TQ_ERR_INVALID
    codec = _lib.Codec(d=72, bits_hi=4, bits_lo=4, split=72)  # head_dims are multiples of 16 in [16, 256]
    assert lib.tq_compress(ctypes.byref(codec), None, 0, 0, None, None, None) == _lib.TQ_ERR_UNSUPPORTED
    assert b"head_dim 72" in lib.tq_last_error()
    codec = _lib.Codec(d=272, bits_hi=4, bits_lo=4, split=272)
    assert lib.tq_compress(ctypes.byref(codec), None, 0, 0, None, None, None) == _lib.TQ_ERR_UNSUPPORTED
    codec = _lib.Codec(d=80, bits_hi=4, bits_lo=4, split=80)  # a valid shape: the NULL rotation is refused
    assert lib.tq_compress(ctypes.byref(codec), None, 0, 0, None, None, None) == _lib.TQ_ERR_INVALID
    codec = _lib.Codec(d=96, bits_hi=4, bits_lo=3, split=40)  # halves of 16 codes at most
    assert lib.tq_compress(ctypes.byref(codec), None, 0, 0, None, None, None) == _lib.TQ_ERR_UNSUPPORTED
    codec = _lib.Codec(d=96, bits_hi=4, bits_lo=3, split=48)  # a valid shape: the NULL rotation is refused
    assert lib.tq_compress(ctypes.byref(codec), None, 0, 0, None, None, None) == _lib.TQ_ERR_INVALID
    assert lib.tq_pack_codes(None, 0, 128, 4, None, None) == _lib.TQ_OK  # empty is a no-op
    # dense decode attention: head_dim, compressed tokens, K/V dtype, group size
    d = _lib.AttnDesc(batch=1, hq=8, hkv=2, max_sink=4, q_dtype=_lib.TQ_F16, kv_dtype=_lib.TQ_F16,
                      q=16, out=16, sink_k=16, sink_v=16, sink_head_stride=512)
    assert lib.tq_dense_decode_attention(ctypes.byref(d), 64, None, 0, None) == _lib.TQ_ERR_UNSUPPORTED
    assert b"head_dim 64" in lib.tq_last_error()
    d.max_comp = 5
    assert lib.tq_dense_decode_attention(ctypes.byref(d), 128, None, 0, None) == _lib.TQ_ERR_INVALID
    d.max_comp, d.kv_dtype = 0, _lib.TQ_F32
    assert lib.tq_dense_decode_attention(ctypes.byref(d), 128, None, 0, None) == _lib.TQ_ERR_UNSUPPORTED
    d.kv_dtype, d.hq = _lib.TQ_F16, 6
    assert lib.tq_dense_decode_attention(ctypes.byref(d), 128, None, 0, None) == _lib.TQ_ERR_UNSUPPORTED
    d.hq, d.sink_k = 8, 18  # rows not 16-byte aligned
    assert lib.tq_dense_decode_attention(ctypes.byref(d), 128, None, 0, None) == _lib.TQ_ERR_UNSUPPORTED
    # ring append: dtype, NULL pointers, shapes, alignment (fake non-NULL addresses: nothing is launched)
    ra = lib.tq_ring_append
    assert ra(16, 16, _lib.TQ_F32, 16, 16, 1024, 8, 1, 1, 128, 16, None) == _lib.TQ_ERR_UNSUPPORTED
    assert ra(None, 16, _lib.TQ_F16, 16, 16, 1024, 8, 1, 1, 128, 16, None) == _lib.TQ_ERR_INVALID
    assert ra(16, 16, _lib.TQ_F16, 16, 16, 1024, 8, 1, 1, 100, 16, None) == _lib.TQ_ERR_INVALID  # d % 8
    assert ra(16, 16, _lib.TQ_F16, 16, 16, 512, 8, 1, 1, 128, 16, None) == _lib.TQ_ERR_INVALID  # stride < cap * d
    assert b"bad shape" in lib.tq_last_error()
    assert ra(16, 24, _lib.TQ_F16, 16, 16, 1024, 8, 1, 1, 128, 16, None) == _lib.TQ_ERR_INVALID  # alignment
    assert ra(16, 16, _lib.TQ_BF16, 16, 16, 1024, 8, 0, 1, 128, 16, None) == _lib.TQ_OK  # empty batch: no-op
    # ragged step (fake 16-byte aligned addresses: every case fails its checks before a launch)
    f = 4096
    sk = _lib.Codec(d=128, bits_hi=4, bits_lo=4, split=128, rotation=f, centroids_hi=f, boundaries_hi=f,
                    qjl_proj=f, qjl_m=128)
    nsk = _lib.Codec(d=128, bits_hi=2, bits_lo=2, split=128, rotation=f, centroids_hi=f, boundaries_hi=f)
    st = _lib.Store(codes_hi=f, norms=f, signs=f, gamma=f)
    ints = (ctypes.c_int32 * 8)(5, 6, 1, 1, 5, 2, 0, 0)  # batch 2: slots 5 / 6, both drain ring slots 5 / 2
    rs = lambda kc, vc, dt=_lib.TQ_F16, n=8, i=ints: lib.tq_ragged_step(
        ctypes.byref(kc), ctypes.byref(vc), f, f, dt, f, f, 129 * 128, 129, ctypes.byref(st), ctypes.byref(st), 2, 8,
        i, n, f, None)
    d96 = _lib.Codec(d=96, bits_hi=4, bits_lo=4, split=96, rotation=f, centroids_hi=f, boundaries_hi=f)
    assert rs(sk, d96) == _lib.TQ_ERR_UNSUPPORTED  # head_dim 96: tq_ring_append + tq_compress
    assert b"no one-launch step" in lib.tq_last_error()
    assert rs(sk, nsk) == _lib.TQ_ERR_INVALID  # a side without a sketch is served: the ints are checked next
    assert b"sequence 0 drains ring slot 5" in lib.tq_last_error()
    assert rs(sk, sk, dt=_lib.TQ_F32) == _lib.TQ_ERR_UNSUPPORTED
    assert rs(sk, sk, n=7) == _lib.TQ_ERR_INVALID  # fewer than 4 * batch ints
    assert rs(sk, sk) == _lib.TQ_ERR_INVALID  # sequence 0 drains the slot it appends to
    assert b"sequence 0 drains ring slot 5" in lib.tq_last_error()
    bad = (ctypes.c_int32 * 8)(4, 6, 2, 1, 5, 2, 0, 0)  # drain count 2
    assert rs(sk, sk, i=bad) == _lib.TQ_ERR_INVALID


def test_value_table_is_an_exact_fp16_copy_of_the_2bit_codebook():
    """tq_codec_prepare (host only): centroid i == value_scale *
    fp16(value_table[i]) for the shipped d=128 2-bit codebook to within 2e-7,
    the bar of the K4/V2 decode route; other sizes are refused (error inf)."""
    import numpy as np
    from turboquant_amd import _lib
    from turboquant_amd.codebook import codebook_arrays
    lib = _lib.load()
    cen, _ = codebook_arrays(128, 2)
    cen = np.ascontiguousarray(cen, np.float32)
    c = _lib.Codec()
    assert lib.tq_codec_prepare(ctypes.byref(c), cen.ctypes.data, 4) == _lib.TQ_OK
    assert c.n_host_centroids == 4 and np.array_equal(np.array(list(c.host_centroids))[:4], cen)
    tab = np.array(list(c.value_table), np.uint16).view(np.float16).astype(np.float64)
    got = float(np.float32(c.value_scale)) * tab
    rel = np.abs(got - cen) / np.abs(cen)
    assert rel.max() <= 2e-7 and c.value_table_err <= 2e-7, rel
    assert np.isclose(rel.max(), c.value_table_err, rtol=1e-3, atol=1e-12)
    # the table entries are fp16 numbers in the normal range, antisymmetric like the codebook
    assert np.all(np.abs(tab) >= 2.0 ** -14) and np.array_equal(tab[::-1], -tab)
    c16 = np.linspace(-1, 1, 16, dtype=np.float32)
    assert lib.tq_codec_prepare(ctypes.byref(c), c16.ctypes.data, 16) == _lib.TQ_OK
    assert c.value_table_err == float("inf")
