"""ctypes binding of ``libtq_hip.so`` (the C ABI declared in include/tq_abi.h).

The library is the only compute path of this package: there is no CPU or
PyTorch fallback. Loading fails loudly when the shared object is missing, and
every call raises when the library reports an error (ValueError for invalid or
unsupported arguments, as the reference does in packing.py:222 and
kernels.py:349; RuntimeError for launch failures).
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtq_hip.so")

TQ_OK = 0
TQ_ERR_INVALID = -1
TQ_ERR_UNSUPPORTED = -2
TQ_ERR_LAUNCH = -3
TQ_ERR_WORKSPACE = -4

TQ_F16, TQ_BF16, TQ_F32 = 0, 1, 2
_DTYPE = {torch.float16: TQ_F16, torch.bfloat16: TQ_BF16, torch.float32: TQ_F32}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class Codec(ctypes.Structure):
    _fields_ = [("d", _i32), ("bits_hi", _i32), ("bits_lo", _i32), ("split", _i32),
                ("rotation", _p), ("centroids_hi", _p), ("boundaries_hi", _p),
                ("centroids_lo", _p), ("boundaries_lo", _p), ("qjl_proj", _p),
                ("qjl_m", _i32), ("flags", _i32), ("rotation_parts", _p),
                ("host_centroids", ctypes.c_float * 16), ("n_host_centroids", _i32),
                ("value_table", ctypes.c_uint16 * 4), ("value_scale", ctypes.c_float),
                ("value_table_err", ctypes.c_float), ("decode_table", _p)]

TQ_CODEC_GENERAL_COMPRESS = 1


class Store(ctypes.Structure):
    _fields_ = [("codes_hi", _p), ("hi_head_stride", _i64),
                ("codes_lo", _p), ("lo_head_stride", _i64),
                ("norms", _p), ("norm_head_stride", _i64),
                ("signs", _p), ("sign_head_stride", _i64),
                ("gamma", _p), ("gamma_head_stride", _i64)]


class Span(ctypes.Structure):
    _fields_ = [("rows", _i32), ("heads", _i32), ("n_tok", _i32), ("reserved", _i32),
                ("n_tok_b", _p), ("src_tok0_b", _p), ("dst_tok0_b", _p)]


class AttnDesc(ctypes.Structure):
    _fields_ = [("batch", _i32), ("hq", _i32), ("hkv", _i32), ("qjl", _i32),
                ("scale", ctypes.c_float),
                ("max_comp", _i32), ("max_sink", _i32), ("max_res", _i32),
                ("q_dtype", _i32), ("kv_dtype", _i32),
                ("q", _p), ("out", _p),
                ("kstore", Store), ("vstore", Store),
                ("comp_len", _p),
                ("sink_k", _p), ("sink_v", _p), ("sink_head_stride", _i64), ("sink_len", _p),
                ("res_k", _p), ("res_v", _p), ("res_head_stride", _i64),
                ("res_cap", _i32), ("res_start0", _i32),
                ("res_start", _p), ("res_len", _p), ("flags", _i32), ("n_q", _i32)]

TQ_ATTN_GENERAL = 1


_PC = ctypes.POINTER(Codec)
_PS = ctypes.POINTER(Store)
_PSp = ctypes.POINTER(Span)
_PA = ctypes.POINTER(AttnDesc)

# name -> (restype, argtypes); the set of entry points of include/tq_abi.h
SIGNATURES = {
    "tq_abi_version": (_i32, []),
    "tq_last_error": (ctypes.c_char_p, []),
    "tq_device_supported": (_i32, []),
    "tq_compress": (_i32, [_PC, _p, _i32, _i64, _PSp, _PS, _p]),
    "tq_ring_append": (_i32, [_p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p]),
    "tq_ragged_step": (_i32, [_PC, _PC, _p, _p, _i32, _p, _p, _i64, _i32, _PS, _PS, _i32, _i32, _p, _i32, _p, _p]),
    "tq_codec_prepare": (_i32, [_PC, _p, _i32]),
    "tq_codec_decode_table": (_i32, [_PC, _p]),
    "tq_dequantize": (_i32, [_PC, _PS, _PSp, _p, _i64, _i32, _p]),
    "tq_pack_codes": (_i32, [_p, _i64, _i32, _i32, _p, _p]),
    "tq_unpack_codes": (_i32, [_p, _i64, _i32, _i32, _p, _p]),
    "tq_quantize_scalar": (_i32, [_p, _i64, _p, _i32, _p, _p]),
    "tq_decode_workspace_bytes": (ctypes.c_size_t, [_PC, _PA]),
    "tq_attention_workspace_bytes": (ctypes.c_size_t, [_PC, _PC, _PA]),
    "tq_decode_attention": (_i32, [_PC, _PC, _PA, _p, ctypes.c_size_t, _p]),
    "tq_decode_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "tq_decode_attention_noalloc": (_i32, [_PC, _PC, _PA, _p]),
    "tq_dense_decode_workspace_bytes": (ctypes.c_size_t, [_PA, _i32]),
    "tq_dense_decode_attention": (_i32, [_PA, _i32, _p, ctypes.c_size_t, _p]),
}

_lib = None


class TurboQuantLibraryError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load ``libtq_hip.so`` (once). Raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise TurboQuantLibraryError(
            f"turboquant_amd: HIP library not built ({LIB_PATH} missing); "
            "run `make -C mlx-turboquant_amd/csrc` or __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.tq_abi_version() != 3:
        raise TurboQuantLibraryError("turboquant_amd: ABI version mismatch")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == TQ_OK:
        return
    msg = (load().tq_last_error() or b"").decode(errors="replace")
    if rc in (TQ_ERR_INVALID, TQ_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError("turboquant_amd runs on the GPU only; got a CPU tensor")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device | None = None) -> int:
    """The hipStream_t of torch's current stream on ``device`` (the raw
    handle through torch's direct query where it has one: a decode step's
    host path calls this per launch)."""
    if _raw_stream is not None:
        idx = device.index if device is not None and device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE[dt]
    except KeyError:
        raise ValueError(f"unsupported floating dtype {dt}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
