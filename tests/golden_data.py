"""Loader for tests/golden/codec_vectors.npz (data written by tests/golden/make_golden.py)."""
from __future__ import annotations

import functools
from pathlib import Path

import numpy as np

from afterimage_amd.runtime.huffman_chunked import ChunkedEncoded

PATH = Path(__file__).resolve().parent / "golden" / "codec_vectors.npz"
GOLDEN = np.load(PATH, allow_pickle=False)


def case_names() -> list[str]:
    return [str(x) for x in GOLDEN["case_names"]]


@functools.lru_cache(maxsize=None)
def case(name: str) -> dict:
    p = "case/%s/" % name
    chunk_size, max_bits, actual, n = (int(x) for x in GOLDEN[p + "params"])
    enc = ChunkedEncoded(
        packed=GOLDEN[p + "packed"], chunk_offsets=GOLDEN[p + "chunk_offsets"],
        chunk_nbytes=GOLDEN[p + "chunk_nbytes"], sym_lut=GOLDEN[p + "sym_lut"],
        len_lut=GOLDEN[p + "len_lut"], max_bits=actual, chunk_size=chunk_size,
        n_symbols=n, shape=(n,))
    tail = None
    if p + "slice_tail" in GOLDEN:
        tail = tuple(int(x) for x in GOLDEN[p + "slice_tail"])
    return {
        "symbols": GOLDEN[p + "symbols"], "chunk_size": chunk_size, "max_bits": max_bits,
        "actual_max_bits": actual, "n_symbols": n, "lengths": GOLDEN[p + "lengths"],
        "packed": GOLDEN[p + "packed"], "chunk_offsets": GOLDEN[p + "chunk_offsets"],
        "chunk_nbytes": GOLDEN[p + "chunk_nbytes"], "sym_lut": GOLDEN[p + "sym_lut"],
        "len_lut": GOLDEN[p + "len_lut"], "encoded": enc, "slice_tail": tail,
        "slice_tail_decoded": GOLDEN[p + "slice_tail_decoded"] if tail else None,
    }
