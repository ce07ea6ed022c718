"""CPU oracle for the BF16 decode path -- TEST INFRASTRUCTURE, not product code.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this package: as the reference that the GPU decoder's outputs are
compared with, or as the timed CPU baseline. ``afterimage_amd`` never imports
it.

The arithmetic is C (aimg_oracle.c, built by ``make -C oracle``); this module
loads it with ctypes. What each function restates:

* ``decode_chunks``: the engine's CPU decode, decode_chunks_numba/_decode_numba
  (afterimage/runtime/cpu_decode.py:67-113) -- a 32-bit MSB-aligned reader,
  byte refills bounded by the chunk end, flat-LUT lookup; OpenMP over chunks.
  Pinned against the reference's own decoded outputs in
  tests/golden/codec_vectors.npz (including whole-chunk decodes of a sliced
  stream whose last chunk is partial).
* ``decode_chunked_reference``: decode_chunked_cpu_reference
  (afterimage/runtime/huffman_chunked.py:256-267), i.e. the above truncated
  to ``n_symbols``.
* ``recombine`` / ``decompress_layer_reference``: _recombine and
  decompress_layer_cpu_reference (afterimage/runtime/compressed_store.py:94-114,
  :243-251). Pinned by the reference's known-answer int16 patterns and
  special values.
* ``decode_bitwise``: the bit-by-bit decoder (afterimage/runtime/huffman.py:195-217),
  an independent check on LUT decoding. Pinned by the reference's
  single-stream decodes in the golden file.
* ``pack_bitwise``: chunk packing bit by bit (huffman_chunked.py:41-78).
  Pinned by the reference's packed bytes in the golden file.
"""
from __future__ import annotations

import ctypes
import subprocess
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        h.oracle_decode_chunks.restype = i32
        h.oracle_decode_chunks.argtypes = [vp, i64, vp, vp, i64, i64, vp, vp, i32, i64, vp, i32]
        h.oracle_recombine.restype = None
        h.oracle_recombine.argtypes = [vp, vp, vp, i64, i32]
        h.oracle_decode_bitwise.restype = i64
        h.oracle_decode_bitwise.argtypes = [vp, i64, vp, vp, vp, i32, i32, i64, vp]
        h.oracle_pack_bitwise.restype = i64
        h.oracle_pack_bitwise.argtypes = [vp, i64, vp, vp, i64, vp, i64, vp]
        h.oracle_max_threads.restype = i32
        h.oracle_max_threads.argtypes = []
        _lib = h
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def decode_chunks(enc, chunk_lo: int = 0, chunk_hi: int | None = None,
                  n_threads: int = 1) -> np.ndarray:
    """uint8[(chunk_hi - chunk_lo) * chunk_size]: whole chunks, padding included."""
    chunk_hi = enc.n_chunks if chunk_hi is None else chunk_hi
    packed = _c(enc.packed, np.uint8)
    offs = _c(enc.chunk_offsets, np.int32)
    nbytes = _c(enc.chunk_nbytes, np.int32)
    sym = _c(enc.sym_lut, np.int32)
    ln = _c(enc.len_lut, np.int8)
    out = np.zeros(max(0, chunk_hi - chunk_lo) * enc.chunk_size, dtype=np.uint8)
    if out.size == 0:
        return out
    rc = lib().oracle_decode_chunks(packed.ctypes.data, packed.size, offs.ctypes.data,
                                    nbytes.ctypes.data, chunk_lo, chunk_hi, sym.ctypes.data,
                                    ln.ctypes.data, int(enc.max_bits), int(enc.chunk_size),
                                    out.ctypes.data, int(n_threads))
    if rc != 0:
        raise ValueError("oracle_decode_chunks rejected its arguments")
    return out


def decode_chunked_reference(enc) -> np.ndarray:
    """uint8[n_symbols]."""
    return decode_chunks(enc)[: enc.n_symbols]


def recombine(exponent: np.ndarray, sign_mantissa: np.ndarray, n_threads: int = 1) -> np.ndarray:
    """uint16 bf16 bit patterns."""
    e = _c(exponent, np.uint8)
    sm = _c(sign_mantissa, np.uint8)
    if e.size != sm.size:
        raise ValueError("exponent and sign_mantissa lengths differ")
    out = np.zeros(e.size, dtype=np.uint16)
    lib().oracle_recombine(e.ctypes.data, sm.ctypes.data, out.ctypes.data, e.size, int(n_threads))
    return out


def decompress_layer_reference(layer):
    """bf16 torch tensor of ``layer.shape`` rebuilt on the CPU."""
    import torch

    exps = decode_chunked_reference(layer.encoded)
    sm = np.asarray(layer.sign_mantissa.reshape(-1).cpu().numpy() if hasattr(
        layer.sign_mantissa, "numpy") else layer.sign_mantissa, dtype=np.uint8)
    bits = recombine(exps, sm)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).reshape(layer.shape)


def decode_bitwise(packed: np.ndarray, symbols, lengths, codes, n_symbols: int) -> np.ndarray:
    """int32[n_symbols]; raises ValueError on a stream with no matching code."""
    p = _c(packed, np.uint8)
    sym = _c(symbols, np.int32)
    ln = _c(lengths, np.int32)
    cd = _c(codes, np.uint32)
    out = np.zeros(n_symbols, dtype=np.int32)
    mb = int(ln.max()) if ln.size else 0
    bad = lib().oracle_decode_bitwise(p.ctypes.data, p.size, sym.ctypes.data, ln.ctypes.data,
                                      cd.ctypes.data, int(sym.size), mb, int(n_symbols),
                                      out.ctypes.data)
    if bad:
        raise ValueError("no matching code found -- corrupt stream or bad table "
                         "(symbol %d)" % (bad - 1))
    return out


def pack_bitwise(symbols: np.ndarray, code_of: np.ndarray, len_of: np.ndarray,
                 chunk_size: int) -> tuple[np.ndarray, np.ndarray]:
    """(packed bytes without slack, chunk_nbytes int32)."""
    s = _c(symbols, np.uint8)
    n = s.size
    n_chunks = (n + chunk_size - 1) // chunk_size
    cap = (n * 16 + 7) // 8 + n_chunks + 8
    out = np.zeros(cap, dtype=np.uint8)
    nb = np.zeros(n_chunks, dtype=np.int32)
    total = lib().oracle_pack_bitwise(s.ctypes.data, n, _c(code_of, np.uint32).ctypes.data,
                                      _c(len_of, np.uint8).ctypes.data, chunk_size,
                                      out.ctypes.data, cap, nb.ctypes.data)
    if total < 0:
        raise ValueError("oracle_pack_bitwise failed")
    return out[:total].copy(), nb


def max_threads() -> int:
    return int(lib().oracle_max_threads())


def time_cpu_decode(enc, sign_mantissa: np.ndarray, n_threads: int, min_seconds: float = 10.0,
                    max_reps: int = 50) -> dict:
    """Time the reference CPU path (chunk decode + recombine) on ``enc``.

    Repeats until ``min_seconds`` of work or ``max_reps``; returns per-rep
    medians. Used as the reported CPU baseline, never as a target.
    """
    sm = _c(sign_mantissa, np.uint8)
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps:
        t0 = time.perf_counter()
        exps = decode_chunks(enc, n_threads=n_threads)[: enc.n_symbols]
        recombine(exps, sm, n_threads=n_threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= min_seconds and len(times) >= 3:
            break
    times.sort()
    return {"median_s": times[len(times) // 2], "reps": len(times),
            "n_symbols": int(enc.n_symbols), "threads": int(n_threads)}
