"""ctypes binding of the sunshape_amd C ABI (include/sunshape_amd.h).

torch is imported before the library is loaded so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
mapped: one HIP runtime per process, so torch's streams and device pointers
are valid in the library.

There is no CPU fallback anywhere in this package: if the library is missing,
every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libsunshape_amd.so")

SSQ_OK = 0
SSQ_ERR_INVALID = 1
SSQ_ERR_HIP = 2
SSQ_ERR_ABI = 3
SSQ_ERR_UNSUPPORTED = 4

SSQ_F32, SSQ_BF16, SSQ_F16 = 0, 1, 2
SSQ_CONTIGUOUS, SSQ_PAGED = 0, 1

DTYPE_CODE = {torch.float32: SSQ_F32, torch.bfloat16: SSQ_BF16, torch.float16: SSQ_F16}

ABI_VERSION = 5  # SSQ_ABI_VERSION in include/sunshape_amd.h
NOALLOC_SCRATCH_BYTES = 32 << 20  # SSQ_NOALLOC_SCRATCH_BYTES

# every function include/sunshape_amd.h declares
EXPORTED_SYMBOLS = (
    "ssq_decode_workspace_size",
    "ssq_decode",
    "ssq_decode_noalloc",
    "ssq_attention_scores",
    "ssq_lut_build",
    "ssq_encode",
    "ssq_encode_grid_bytes",
    "ssq_encode_grid_build",
    "ssq_dequantize",
    "ssq_transform_rows",
    "ssq_pack_codes",
    "ssq_unpack_codes",
    "ssq_last_error",
    "ssq_abi_version",
)

from ._abi import DecodeArgs, EncodeArgs  # noqa: E402  (the structs, torch-free)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float


_lib = None
_ops = None
_lock = threading.Lock()
TORCH_OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libsunshape_torch_ops.so")


def _declare(lib: ctypes.CDLL) -> None:
    P = ctypes.POINTER
    lib.ssq_decode_workspace_size.argtypes = [P(DecodeArgs)]
    lib.ssq_decode_workspace_size.restype = ctypes.c_size_t
    lib.ssq_decode.argtypes = [P(DecodeArgs), _vp, ctypes.c_size_t, _vp]
    lib.ssq_decode.restype = ctypes.c_int
    lib.ssq_decode_noalloc.argtypes = [P(DecodeArgs), _vp]
    lib.ssq_decode_noalloc.restype = ctypes.c_int
    lib.ssq_attention_scores.argtypes = [P(DecodeArgs), _vp]
    lib.ssq_attention_scores.restype = ctypes.c_int
    lib.ssq_lut_build.argtypes = [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _vp, _vp]
    lib.ssq_lut_build.restype = ctypes.c_int
    lib.ssq_encode.argtypes = [P(EncodeArgs), _vp]
    lib.ssq_encode.restype = ctypes.c_int
    lib.ssq_encode_grid_bytes.argtypes = [P(EncodeArgs)]
    lib.ssq_encode_grid_bytes.restype = ctypes.c_uint64
    lib.ssq_encode_grid_build.argtypes = [P(EncodeArgs), _vp, ctypes.c_uint64, _vp]
    lib.ssq_encode_grid_build.restype = ctypes.c_int
    lib.ssq_dequantize.argtypes = [_vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _i64,
                                   _vp, _i64, _vp]
    lib.ssq_dequantize.restype = ctypes.c_int
    lib.ssq_transform_rows.argtypes = [_vp, _i32, _i64, _i64, _i32, _i32, _f32, _vp, _i32, _vp, _i64, _vp]
    lib.ssq_transform_rows.restype = ctypes.c_int
    lib.ssq_pack_codes.argtypes = [_vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]
    lib.ssq_pack_codes.restype = ctypes.c_int
    lib.ssq_unpack_codes.argtypes = [_vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]
    lib.ssq_unpack_codes.restype = ctypes.c_int
    lib.ssq_last_error.argtypes = []
    lib.ssq_last_error.restype = ctypes.c_char_p
    lib.ssq_abi_version.argtypes = []
    lib.ssq_abi_version.restype = ctypes.c_int


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"sunshape_amd HIP library is not built ({LIB_PATH}); run `python -m sunshape_amd.build`"
                )
            handle = ctypes.CDLL(LIB_PATH)
            _declare(handle)
            if handle.ssq_abi_version() != ABI_VERSION:
                raise RuntimeError("sunshape_amd library ABI version mismatch")
            _lib = handle
    return _lib


def torch_ops():
    """torch.ops.sunshape (operators of libsunshape_torch_ops.so, over the same library); raises if
    it was not built."""
    global _ops
    if _ops is not None:
        return _ops
    lib()
    with _lock:
        if _ops is None:
            if not os.path.exists(TORCH_OPS_PATH):
                raise RuntimeError(
                    f"sunshape_amd torch operators are not built ({TORCH_OPS_PATH}); run `python -m sunshape_amd.build`"
                )
            torch.ops.load_library(TORCH_OPS_PATH)
            _ops = torch.ops.sunshape
    return _ops


_STATUS_RE = None


def kernel_error(e: RuntimeError) -> RuntimeError:
    """A torch operator's RuntimeError as SunShapeKernelError when the library returned a status."""
    global _STATUS_RE
    if _STATUS_RE is None:
        import re

        _STATUS_RE = re.compile(r"sunshape_amd status (\d+): ([^\n]*)")
    m = _STATUS_RE.search(str(e))
    if m is None:
        return e
    return SunShapeKernelError(int(m.group(1)), m.group(2))


def signed64(w: int) -> int:
    """An unsigned 64-bit mask word as the signed int64 the operators' int arguments carry."""
    return w - (1 << 64) if w >= (1 << 63) else w


def mask_words_signed(mask) -> tuple[int, int]:
    """heavy_mask_words as two signed int64 (the operators' int arguments), cached per mask tuple."""
    key = None if mask is None else tuple(bool(x) for x in (mask.tolist() if hasattr(mask, "tolist") else mask))
    hit = _WORDS.get(key)
    if hit is None:
        w0, w1 = heavy_mask_words(key)
        hit = (signed64(w0), signed64(w1))
        _WORDS[key] = hit
    return hit


_WORDS: dict = {}


class SunShapeKernelError(RuntimeError):
    """A sunshape_amd entry point returned an error status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def check(status: int) -> None:
    if status != SSQ_OK:
        msg = lib().ssq_last_error().decode("utf-8", "replace")
        raise SunShapeKernelError(status, msg)


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from None


def heavy_mask_words(mask) -> tuple[int, int]:
    """bool [nb] (tensor or sequence) -> two uint64 bit words."""
    if mask is None:
        return 0, 0
    bits = [bool(x) for x in (mask.tolist() if hasattr(mask, "tolist") else mask)]
    if len(bits) > 128:
        raise RuntimeError("at most 128 blocks are supported")
    w0 = sum(1 << i for i, x in enumerate(bits[:64]) if x)
    w1 = sum(1 << i for i, x in enumerate(bits[64:]) if x)
    return w0, w1
