"""ctypes binding of libafterimage_decode.so (declared in include/afterimage_decode.h).

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already holds (both name it libamdhip64.so.7). The
library is never built implicitly here: a missing library raises, it does not
fall back to anything.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the library; see module doc)

LIB_PATH = Path(__file__).resolve().parent / "libafterimage_decode.so"
ABI_VERSION = 11
MAX_TENSORS = 32

AIMG_OK = 0
AIMG_ERR_INVALID_ARGUMENT = 1
AIMG_ERR_BAD_TABLE = 2
AIMG_ERR_HIP = 3
AIMG_ERR_UNSUPPORTED = 4


class NativeError(RuntimeError):
    """A non-OK status from the native library."""

    def __init__(self, code: int, message: str):
        super().__init__("afterimage_decode error %d: %s" % (code, message))
        self.code = code
        self.message = message


class AimgTensor(ctypes.Structure):
    """Mirror of ``aimg_tensor``."""

    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("chunk_offsets", ctypes.c_void_p),
        ("chunk_nbytes", ctypes.c_void_p),
        ("sign_mantissa", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("table", ctypes.c_void_p),
        ("index", ctypes.c_void_p),
        ("index_nbytes", ctypes.c_int64),
        ("packed_nbytes", ctypes.c_int64),
        ("n_symbols", ctypes.c_int64),
        ("chunk_size", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32),
    ]


_lib = None
_lock = threading.Lock()

# (name, restype, argtypes) for every entry point declared in the header.
_SIGNATURES = [
    ("aimg_abi_version", ctypes.c_int, []),
    ("aimg_last_error", ctypes.c_char_p, []),
    ("aimg_table_nbytes", ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]),
    ("aimg_build_table", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]),
    ("aimg_index_nbytes", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    ("aimg_build_index", ctypes.c_int,
     [ctypes.POINTER(AimgTensor), ctypes.c_int, ctypes.c_void_p]),
    ("aimg_decode_bf16", ctypes.c_int,
     [ctypes.POINTER(AimgTensor), ctypes.c_int, ctypes.c_void_p]),
    ("aimg_decode_u8", ctypes.c_int,
     [ctypes.POINTER(AimgTensor), ctypes.c_int, ctypes.c_void_p]),
    ("aimg_decode_gemv_bf16", ctypes.c_int,
     [ctypes.POINTER(AimgTensor), ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
      ctypes.c_void_p, ctypes.c_void_p]),
    ("aimg_decode_gemm_bf16", ctypes.c_int,
     [ctypes.POINTER(AimgTensor), ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
      ctypes.c_void_p, ctypes.c_void_p]),
    ("aimg_recombine_bf16", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]),
    ("aimg_cpu_decode_bf16", ctypes.c_int, [ctypes.POINTER(AimgTensor), ctypes.c_int, ctypes.c_int]),
    ("aimg_cpu_decode_u8", ctypes.c_int, [ctypes.POINTER(AimgTensor), ctypes.c_int, ctypes.c_int]),
    ("aimg_cpu_recombine_bf16", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    ("aimg_pack_chunked", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
      ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64)]),
]

EXPORTED_SYMBOLS = tuple(name for name, _, _ in _SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    "%s is not built; run `python -m afterimage_amd.build` "
                    "(this decoder has no non-native path)" % LIB_PATH)
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, restype, argtypes in _SIGNATURES:
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            got = handle.aimg_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError("libafterimage_decode ABI %d, expected %d (rebuild it)"
                                   % (got, ABI_VERSION))
            _lib = handle
    return _lib


def check(status: int) -> None:
    """Raise NativeError for a non-OK status, with the library's message."""
    if status != AIMG_OK:
        msg = lib().aimg_last_error()
        raise NativeError(status, msg.decode() if msg else "")
