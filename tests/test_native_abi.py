"""The C ABI library on the CPU: it loads, exports what include/afterimage_decode.h
declares, and its host functions (table builder, packer) are right. No kernel
is launched here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from afterimage_amd import _native
from afterimage_amd.runtime.device import build_table_blob
from afterimage_amd.runtime.huffman import build_lengths, canonical_codes, code_arrays
from afterimage_amd.runtime.huffman_chunked import ChunkedEncoded, encode_chunked, pack_chunks
from tests.distributions import many_escape_windows
from tests.golden_data import case, case_names

HEADER = Path(__file__).resolve().parent.parent / "include" / "afterimage_decode.h"
WIN_BITS = 12


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aimg_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _native.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.EXPORTED_SYMBOLS)


def test_abi_version_and_error_channel():
    lib = _native.lib()
    assert lib.aimg_abi_version() == _native.ABI_VERSION
    n = ctypes.c_size_t()
    assert lib.aimg_table_nbytes(17, ctypes.byref(n)) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"max_bits" in lib.aimg_last_error()
    assert lib.aimg_table_nbytes(16, ctypes.byref(n)) == _native.AIMG_OK
    assert n.value == 64 + 4 * 4096 + 4096 + 256 + 2 * 16 * 256


def test_decode_entry_points_validate_before_launching():
    lib = _native.lib()
    arr = (_native.AimgTensor * 1)()
    arr[0].chunk_size = 0
    assert lib.aimg_decode_bf16(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"chunk_size" in lib.aimg_last_error()
    arr[0].chunk_size = 16
    arr[0].n_chunks = 1
    arr[0].n_symbols = 17
    assert lib.aimg_decode_u8(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert lib.aimg_decode_u8(arr, 33, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    arr[0].n_symbols = 16  # null device pointers
    assert lib.aimg_decode_bf16(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"null" in lib.aimg_last_error()
    # Nothing to decode is not an error and launches nothing.
    arr[0].n_symbols = 0
    assert lib.aimg_decode_bf16(arr, 1, None) == _native.AIMG_OK
    assert lib.aimg_decode_bf16(arr, 0, None) == _native.AIMG_OK


def test_gemv_entry_point_validates_before_launching():
    lib = _native.lib()
    arr = (_native.AimgTensor * 1)()
    arr[0].chunk_size = 16
    arr[0].n_chunks = 1
    arr[0].n_symbols = 16
    x = ctypes.c_void_p(16)
    y = ctypes.c_void_p(16)
    assert lib.aimg_decode_gemv_bf16(None, 4, 4, x, 1, y, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert lib.aimg_decode_gemv_bf16(arr, 4, 5, x, 1, y, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"rows * cols" in lib.aimg_last_error()
    assert lib.aimg_decode_gemv_bf16(arr, 4, 4, x, 5, y, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"batch" in lib.aimg_last_error()
    assert lib.aimg_decode_gemv_bf16(arr, 4, 4, None, 1, y, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    # A tensor without device pointers fails in the shared checks.
    assert lib.aimg_decode_gemv_bf16(arr, 4, 4, x, 1, y, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"null" in lib.aimg_last_error()
    arr[0].n_symbols = 1 << 31
    arr[0].n_chunks = 1 << 27
    assert lib.aimg_decode_bf16(arr, 1, None) == _native.AIMG_ERR_UNSUPPORTED


def test_table_builder_rejects_a_symbol_with_two_code_lengths():
    # A valid prefix code, but symbol 5 has codes "0" and "10".
    sym = np.array([5, 5, 5, 6], np.int32)
    ln = np.array([1, 1, 2, 2], np.int8)
    with pytest.raises(_native.NativeError, match="two lengths"):
        build_table_blob(sym, ln, 2)


def test_table_builder_rejects_wide_symbols():
    sym = np.array([0, 300], np.int32)
    ln = np.array([1, 1], np.int8)
    with pytest.raises(_native.NativeError, match="fit in a byte"):
        build_table_blob(sym, ln, 1)


def test_table_builder_rejects_non_prefix_lut():
    sym = np.array([1, 1, 2, 2], np.int32)
    ln = np.array([1, 2, 2, 2], np.int8)  # entry 1 claims length 2 inside a length-1 span
    with pytest.raises(_native.NativeError, match="prefix"):
        build_table_blob(sym, ln, 2)


def _window_expectation(lengths, w, max_syms=4):
    """Codewords read one after another from the 12-bit window w, found by
    matching each canonical code against the window's bits; kept while they
    lie wholly inside the window (at most max_syms)."""
    _, codes = canonical_codes(lengths)
    bits = format(w, "012b")
    out, pos = [], 0
    while len(out) < max_syms:
        hit = [s for s, c in codes.items()
               if pos + lengths[s] <= WIN_BITS
               and bits[pos: pos + lengths[s]] == format(c, "0%db" % lengths[s])]
        assert len(hit) <= 1  # prefix property
        if not hit:
            break
        out.append(hit[0])
        pos += lengths[hit[0]]
    return out


def test_window_expectation_agrees_with_oracle_reader():
    """The code-matching expectation and the oracle's LUT reader agree on
    windows made of whole codewords."""
    c = case("bf16_outliers_64k")
    enc = c["encoded"]
    lengths = {s: int(ln) for s, ln in enumerate(c["lengths"]) if ln > 0}
    for w in range(0, 4096, 37):
        want = _window_expectation(lengths, w, max_syms=6)
        body = np.array([(w >> 4) & 0xFF, (w & 0xF) << 4], np.uint8)
        one = ChunkedEncoded(packed=body, chunk_offsets=np.array([0], np.int32),
                             chunk_nbytes=np.array([2], np.int32), sym_lut=enc.sym_lut,
                             len_lut=enc.len_lut, max_bits=enc.max_bits, chunk_size=8,
                             n_symbols=8, shape=(8,))
        assert list(oracle.decode_chunks(one)[: len(want)]) == want


def _first_codeword(lengths, bits16):
    """(symbol, length) of the canonical codeword that the 16-bit string
    bits16 starts with, or None."""
    _, codes = canonical_codes(lengths)
    for s, c in codes.items():
        ln = lengths[s]
        if ln <= 16 and bits16 >> (16 - ln) == c:
            return s, ln
    return None


@pytest.mark.parametrize("name", ["bf16_outliers_64k", "dirichlet_6", "skewed_2sym",
                                  "single_symbol", "fibonacci40_mb6", "uniform256",
                                  "scales_3p0"])
def test_window_table_matches_canonical_code(name):
    c = case(name)
    enc = c["encoded"]
    lengths = {s: int(ln) for s, ln in enumerate(c["lengths"]) if ln > 0}
    blob = build_table_blob(enc.sym_lut, enc.len_lut, enc.max_bits)
    hdr = blob[:64].view(np.uint32)
    assert hdr[0] == 0x474D4941 and hdr[2] == enc.max_bits
    assert hdr[3] == min(lengths.values())
    assert hdr[4] == enc.sym_lut[0]
    n_blocks = int(hdr[6])
    wsyms = blob[64: 64 + 4 * 4096].view(np.uint32)
    wmeta = blob[64 + 4 * 4096: 64 + 5 * 4096]
    len_of = blob[64 + 5 * 4096: 64 + 5 * 4096 + 256]
    esc = blob[64 + 5 * 4096 + 256:].view(np.uint16)
    for sym in range(256):
        assert int(len_of[sym]) == lengths.get(sym, 0)
    long_prefixes = {codes_prefix for codes_prefix in range(4096)
                     if (fc := _first_codeword(lengths, codes_prefix << 4)) is not None
                     and fc[1] > WIN_BITS}
    assert n_blocks == len(long_prefixes)
    rng = np.random.default_rng(0)
    windows = set(rng.integers(0, 4096, 400).tolist()) | {0, 4095} | long_prefixes
    for w in sorted(windows):
        want = _window_expectation(lengths, w)
        ent = int(wsyms[w])
        total = int(wmeta[w]) & 31
        count = int(wmeta[w]) >> 5 if total else 0
        if not want:
            # Escape window: its block gives the first codeword for every
            # value of the next four bits.
            assert total == 0 and count == 0
            blk = ent & 0xFFFF
            if w not in long_prefixes:
                assert blk == 0xFFFF
                continue
            assert blk < n_blocks
            for e4 in range(16):
                got = int(esc[blk * 16 + e4])
                fc = _first_codeword(lengths, (w << 4) | e4)
                if fc is None:
                    assert got >> 8 == 0
                else:
                    assert (got & 0xFF, got >> 8) == fc
            continue
        got = [(ent >> (8 * j)) & 0xFF for j in range(len(want))]
        assert got == want
        assert ent >> (8 * len(want)) == 0
        assert count == len(want) and total == sum(lengths[s] for s in want)


@pytest.mark.parametrize("name", case_names())
def test_native_packer_matches_reference(name):
    c = case(name)
    counts = np.bincount(c["symbols"], minlength=256)
    freqs = {int(s): int(k) for s, k in enumerate(counts) if k > 0}
    lengths = build_lengths(freqs, max_bits=c["max_bits"])
    _, codes = canonical_codes(lengths)
    body, nbytes = pack_chunks(c["symbols"], codes, lengths, c["chunk_size"],
                               c["actual_max_bits"])
    assert np.array_equal(nbytes, c["chunk_nbytes"])
    assert np.array_equal(body, c["packed"][: body.size])


def test_native_packer_rejects_symbol_without_code():
    codes, lengths = {0: 0, 1: 1}, {0: 1, 1: 1}
    with pytest.raises(_native.NativeError, match="no code"):
        pack_chunks(np.array([0, 1, 5], np.uint8), codes, lengths, 4, 1)
    with pytest.raises(ValueError):
        code_arrays({300: 0}, {300: 1})


def test_escape_blocks_can_exceed_the_lds_share():
    """The premise of the GPU test of escape blocks held in global memory."""
    data = many_escape_windows(7, 400_000)
    enc = encode_chunked(torch.from_numpy(data), chunk_size=4096, max_bits=16)
    blob = build_table_blob(enc.sym_lut, enc.len_lut, enc.max_bits)
    hdr = np.frombuffer(blob[:64].tobytes(), dtype=np.uint32)
    assert hdr[6] > 64  # n_esc_blocks
    assert int(enc.len_lut.max()) > 12



def _bf16_table():
    W = (torch.randn(64, 512, generator=torch.Generator().manual_seed(3)) * 0.02).to(torch.bfloat16)
    bits = W.view(torch.int16).to(torch.int32) & 0xFFFF
    enc = encode_chunked(((bits >> 7) & 0xFF).reshape(-1), chunk_size=1024)
    return enc, build_table_blob(enc.sym_lut, enc.len_lut, enc.max_bits)


def test_table_blob_records_a_checksum_of_its_tables():
    _, blob = _bf16_table()
    h = 2166136261
    for b in blob[64:].tobytes():
        h = ((h ^ b) * 16777619) & 0xFFFFFFFF
    assert int(blob[28:32].view(np.uint32)[0]) == h


def test_index_size_is_four_bytes_per_segment_plus_chunk_tables():
    lib = _native.lib()
    enc, blob = _bf16_table()
    min_len = int(blob[12:16].view(np.uint32)[0])
    seg = min(84 * min_len, 168) & ~7
    n = ctypes.c_size_t()
    packed, chunks = 1_000_003, 77
    assert lib.aimg_index_nbytes(blob.ctypes.data, packed, chunks, ctypes.byref(n)) == 0
    # 64-byte header, first segment (chunks + 1) and real end (chunks) of
    # each chunk, 4 bytes per segment of the packed bytes (one partial
    # segment per chunk), and 16 bytes for every 512th segment (where a
    # segment run may start: chunk, element, byte, chunk's first segment)
    # and one more for the end.
    cap = -(-8 * packed // seg) + chunks
    entries_at = (64 + 4 * (chunks + 1) + 4 * chunks + 15) & ~15
    rounds_at = (entries_at + 4 * cap + 15) & ~15
    assert n.value == rounds_at + 16 * (cap // 512 + 2)
    assert n.value < 4.05 * cap + 12 * chunks + 128
    bad = blob.copy()
    bad[0] ^= 1
    assert lib.aimg_index_nbytes(bad.ctypes.data, packed, chunks, ctypes.byref(n)) == \
        _native.AIMG_ERR_BAD_TABLE
    assert lib.aimg_index_nbytes(blob.ctypes.data, -1, chunks, ctypes.byref(n)) == \
        _native.AIMG_ERR_INVALID_ARGUMENT
    assert lib.aimg_index_nbytes(None, packed, chunks, ctypes.byref(n)) == \
        _native.AIMG_ERR_INVALID_ARGUMENT


def test_build_index_validates_before_launching():
    lib = _native.lib()
    arr = (_native.AimgTensor * 1)()
    arr[0].chunk_size = 16
    arr[0].n_chunks = 4
    arr[0].n_symbols = 64
    # No index: nothing to build, nothing launched.
    assert lib.aimg_build_index(arr, 1, None) == _native.AIMG_OK
    assert lib.aimg_build_index(arr, 33, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    arr[0].index = 4096
    arr[0].index_nbytes = 32  # below the 64-byte header
    assert lib.aimg_build_index(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"index_nbytes" in lib.aimg_last_error()
    arr[0].index = 4100
    arr[0].index_nbytes = 4096
    assert lib.aimg_build_index(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"aligned" in lib.aimg_last_error()
    arr[0].index = 4096  # the shared checks: null device pointers
    assert lib.aimg_build_index(arr, 1, None) == _native.AIMG_ERR_INVALID_ARGUMENT
    assert b"null" in lib.aimg_last_error()
