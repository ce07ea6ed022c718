"""Chunked canonical-Huffman encoding of exponent bytes.

Same container and byte layout as the reference
(afterimage/runtime/huffman_chunked.py:134-207): one shared code per tensor;
the symbol stream is cut into chunks of ``chunk_size`` symbols, each packed
MSB-first into its own byte-aligned bitstream; ``chunk_offsets`` are the
prefix sums of ``chunk_nbytes``; eight zero bytes follow the last chunk.

Chunks are what the GPU decoder parallelises over, and every chunk boundary is
a known codeword boundary, which is also where the decoder's speculative
segment parse starts from.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from .. import _native
from .huffman import build_decode_lut, build_lengths, canonical_codes, code_arrays

SLACK_BYTES = 8


@dataclasses.dataclass
class ChunkedEncoded:
    """Entropy-coded exponent stream (huffman_chunked.py:134-148)."""

    packed: np.ndarray          # uint8: chunk bitstreams back to back + 8 zero bytes
    chunk_offsets: np.ndarray   # int32: byte offset of each chunk in packed
    chunk_nbytes: np.ndarray    # int32: byte length of each chunk
    sym_lut: np.ndarray         # int32[2**max_bits]
    len_lut: np.ndarray         # int8[2**max_bits]
    max_bits: int               # actual LUT width (longest code length)
    chunk_size: int             # symbols per chunk
    n_symbols: int
    shape: tuple[int, ...]

    @property
    def n_chunks(self) -> int:
        return len(self.chunk_offsets)


def _as_symbols(exponents) -> np.ndarray:
    if hasattr(exponents, "detach"):
        flat = exponents.detach().flatten().cpu().numpy()
    else:
        flat = np.asarray(exponents).reshape(-1)
    if flat.dtype == np.uint8:
        return np.ascontiguousarray(flat)
    if flat.size and (int(flat.min()) < 0 or int(flat.max()) > 255):
        raise ValueError("exponent symbols must lie in 0..255")
    return flat.astype(np.uint8)


def pack_chunks(flat: np.ndarray, codes: dict[int, int], lengths: dict[int, int],
                chunk_size: int, max_bits: int) -> tuple[np.ndarray, np.ndarray]:
    """(packed body without slack, chunk_nbytes) via the native packer."""
    n = int(flat.shape[0])
    n_chunks = (n + chunk_size - 1) // chunk_size
    code_of, len_of = code_arrays(codes, lengths)
    cap = (n * max(max_bits, 1) + 7) // 8 + n_chunks + 8
    out = np.zeros(cap, dtype=np.uint8)
    nbytes = np.zeros(n_chunks, dtype=np.int32)
    total = ctypes.c_int64(0)
    lib = _native.lib()
    _native.check(lib.aimg_pack_chunked(
        flat.ctypes.data, n, code_of.ctypes.data, len_of.ctypes.data, int(chunk_size),
        out.ctypes.data, cap, nbytes.ctypes.data, ctypes.byref(total)))
    return out[: total.value].copy(), nbytes


def symbol_counts(exponents) -> np.ndarray:
    """Histogram of a symbol tensor/array over 0..255 (int64[256])."""
    return np.bincount(_as_symbols(exponents), minlength=256).astype(np.int64)


def lengths_from_counts(counts: np.ndarray, max_bits: int = 16) -> dict[int, int]:
    """Code lengths for a histogram, as encode_chunked builds them."""
    freqs = {int(s): int(c) for s, c in enumerate(counts) if c > 0}
    return build_lengths(freqs, max_bits=max_bits)


def encode_chunked(exponents, chunk_size: int = 512, max_bits: int = 16, *,
                   lengths: dict[int, int] | None = None) -> ChunkedEncoded:
    """Chunked encode of a symbol tensor/array (huffman_chunked.py:151-207).

    ``lengths`` (keyword-only, not in the reference) encodes with a given
    codebook instead of one built from this array's histogram, so several
    tensors can share one codebook and one decode table; every symbol that
    occurs must have a length."""
    if chunk_size < 1:
        raise ValueError("chunk_size must be >= 1, got %d" % chunk_size)
    shape = tuple(exponents.shape)
    flat = _as_symbols(exponents)
    n = int(flat.shape[0])
    if lengths is None:
        lengths = lengths_from_counts(np.bincount(flat, minlength=256), max_bits)
    else:
        present = np.flatnonzero(np.bincount(flat, minlength=256))
        missing = [int(s) for s in present if int(s) not in lengths]
        if missing:
            raise ValueError("symbols %s occur but have no code" % missing[:8])
    table, codes = canonical_codes(lengths)
    sym_lut, len_lut = build_decode_lut(table, codes)
    # The LUT is indexed at the code's real width, which can be below the cap.
    width = table.max_bits
    n_chunks = (n + chunk_size - 1) // chunk_size
    body, chunk_nbytes = pack_chunks(flat, codes, lengths, chunk_size, width)
    chunk_offsets = np.zeros(n_chunks, dtype=np.int32)
    if n_chunks:
        chunk_offsets[1:] = np.cumsum(chunk_nbytes, dtype=np.int64)[:-1]
    packed = np.concatenate([body, np.zeros(SLACK_BYTES, dtype=np.uint8)])
    return ChunkedEncoded(packed=packed, chunk_offsets=chunk_offsets, chunk_nbytes=chunk_nbytes,
                          sym_lut=sym_lut, len_lut=len_lut, max_bits=width,
                          chunk_size=chunk_size, n_symbols=n, shape=shape)
