"""Encoder and oracle against the reference's own outputs (tests/golden/codec_vectors.npz,
written by tests/golden/make_golden.py from the reference codec)."""
import numpy as np
import pytest
import torch

import oracle
from afterimage_amd.runtime.compressed_store import _slice_encoded, compress_layer
from afterimage_amd.runtime.huffman import (
    build_decode_lut,
    build_lengths,
    canonical_codes,
    code_arrays,
)
from afterimage_amd.runtime.huffman_chunked import encode_chunked
from tests.golden_data import GOLDEN, case, case_names


@pytest.mark.parametrize("name", case_names())
def test_encoder_matches_reference_bytes(name):
    c = case(name)
    enc = encode_chunked(c["symbols"], chunk_size=c["chunk_size"], max_bits=c["max_bits"])
    assert enc.max_bits == c["actual_max_bits"]
    assert enc.n_symbols == c["n_symbols"]
    assert np.array_equal(enc.sym_lut, c["sym_lut"])
    assert np.array_equal(enc.len_lut, c["len_lut"])
    assert np.array_equal(enc.chunk_nbytes, c["chunk_nbytes"])
    assert np.array_equal(enc.chunk_offsets, c["chunk_offsets"])
    assert np.array_equal(enc.packed, c["packed"])


@pytest.mark.parametrize("name", case_names())
def test_code_lengths_match_reference(name):
    c = case(name)
    counts = np.bincount(c["symbols"], minlength=256)
    freqs = {int(s): int(k) for s, k in enumerate(counts) if k > 0}
    lengths = build_lengths(freqs, max_bits=c["max_bits"])
    got = np.zeros(256, dtype=np.int8)
    for s, ln in lengths.items():
        got[s] = ln
    assert np.array_equal(got, c["lengths"])


@pytest.mark.parametrize("mb", [6, 8, 16])
def test_package_merge_lengths_on_fibonacci_weights(mb):
    fib = [1, 1]
    while len(fib) < 40:
        fib.append(fib[-1] + fib[-2])
    lengths = build_lengths({s: f for s, f in enumerate(fib)}, max_bits=mb)
    got = np.array([lengths[s] for s in range(40)], dtype=np.int8)
    assert np.array_equal(got, GOLDEN["fib_lengths/mb%d" % mb])
    assert got.max() <= mb
    # A length-limited code must still satisfy Kraft's inequality with equality.
    assert sum(2.0 ** -int(x) for x in got) == pytest.approx(1.0)


@pytest.mark.parametrize("name", case_names())
def test_oracle_decodes_reference_stream(name):
    c = case(name)
    enc = c["encoded"]
    assert np.array_equal(oracle.decode_chunked_reference(enc), c["symbols"])


@pytest.mark.parametrize("name", [n for n in case_names() if case(n)["slice_tail"] is not None])
def test_oracle_whole_chunk_decode_of_partial_slice_matches_reference(name):
    """Positions past the real symbols of a partial last chunk: the reference
    decodes them from zero bits; the oracle must produce the same bytes."""
    c = case(name)
    c0, c1 = c["slice_tail"]
    sub = _slice_encoded(c["encoded"], c0, c1)
    assert np.array_equal(oracle.decode_chunks(sub), c["slice_tail_decoded"])


def test_oracle_threads_agree():
    c = case("bf16_outliers_64k")
    one = oracle.decode_chunks(c["encoded"], n_threads=1)
    many = oracle.decode_chunks(c["encoded"], n_threads=4)
    assert np.array_equal(one, many)


def test_bitwise_decoder_matches_reference_single_stream():
    sym = GOLDEN["stream/symbols"]
    counts = np.bincount(sym, minlength=256)
    freqs = {int(s): int(k) for s, k in enumerate(counts) if k > 0}
    lengths = build_lengths(freqs)
    table, codes = canonical_codes(lengths)
    code_of, len_of = code_arrays(codes, lengths)
    # The whole stream as one chunk is the single-stream packing of huffman.py.
    packed, nbytes = oracle.pack_bitwise(sym, code_of, len_of, chunk_size=len(sym))
    assert np.array_equal(packed, GOLDEN["stream/packed"])
    dec = oracle.decode_bitwise(packed, table.symbols, table.lengths,
                                [codes[s] for s in table.symbols], len(sym))
    assert np.array_equal(dec, GOLDEN["stream/decode_reference"])
    assert np.array_equal(dec, GOLDEN["stream/decode_lut_cpu"])
    assert np.array_equal(dec, sym)


@pytest.mark.parametrize("name", case_names())
def test_bitwise_packer_matches_reference(name):
    c = case(name)
    counts = np.bincount(c["symbols"], minlength=256)
    freqs = {int(s): int(k) for s, k in enumerate(counts) if k > 0}
    lengths = build_lengths(freqs, max_bits=c["max_bits"])
    _, codes = canonical_codes(lengths)
    code_of, len_of = code_arrays(codes, lengths)
    body, nbytes = oracle.pack_bitwise(c["symbols"], code_of, len_of, c["chunk_size"])
    assert np.array_equal(nbytes, c["chunk_nbytes"])
    assert np.array_equal(body, c["packed"][: body.size])
    assert np.all(c["packed"][body.size:] == 0) and c["packed"].size - body.size == 8


def test_bitwise_decoder_detects_corrupt_stream():
    # Code {0: '0', 1: '10'}: the bits '11' match no codeword.
    with pytest.raises(ValueError, match="no matching code"):
        oracle.decode_bitwise(np.array([0xC0], np.uint8), [0, 1], [1, 2], [0, 2], 1)


@pytest.mark.parametrize("name", ["kat_int16", "special_values", "randn_128x512"])
def test_bf16_known_answers(name):
    p = "bf16/%s/" % name
    bits = GOLDEN[p + "bits"]
    shape = tuple(int(x) for x in GOLDEN[p + "shape"])
    w = torch.from_numpy(bits.copy()).view(torch.bfloat16).reshape(shape)
    layer = compress_layer(w, chunk_size=int(GOLDEN[p + "chunk_size"][0]))
    assert np.array_equal(layer.sign_mantissa.numpy(), GOLDEN[p + "sign_mantissa"])
    assert np.array_equal(layer.encoded.packed, GOLDEN[p + "packed"])
    recon = oracle.decompress_layer_reference(layer)
    assert np.array_equal(recon.view(torch.int16).numpy().reshape(-1), GOLDEN[p + "decoded_bits"])
    assert np.array_equal(GOLDEN[p + "decoded_bits"], bits)


def test_recombine_closed_form_on_every_byte_pair():
    e = np.repeat(np.arange(256, dtype=np.uint8), 256)
    sm = np.tile(np.arange(256, dtype=np.uint8), 256)
    got = oracle.recombine(e, sm)
    want = ((sm.astype(np.uint32) >> 7) << 15) | (e.astype(np.uint32) << 7) | (sm & 0x7F)
    assert np.array_equal(got, want.astype(np.uint16))
    # Every bf16 bit pattern appears exactly once.
    assert np.unique(got).size == 65536


def test_planted_sign_error_in_oracle_recombine_is_caught():
    """A recombine that drops the sign bit must fail the known-answer vector."""
    p = "bf16/kat_int16/"
    sm = GOLDEN[p + "sign_mantissa"]
    exps = ((GOLDEN[p + "bits"].view(np.uint16) >> 7) & 0xFF).astype(np.uint8)
    wrong = oracle.recombine(exps, sm & 0x7F)
    assert not np.array_equal(wrong.view(np.int16), GOLDEN[p + "decoded_bits"])
    right = oracle.recombine(exps, sm)
    assert np.array_equal(right.view(np.int16), GOLDEN[p + "decoded_bits"])


def test_decode_lut_structure():
    """Every window's LUT entry is the codeword it starts with."""
    c = case("dirichlet_3")
    enc = c["encoded"]
    lengths = {s: int(ln) for s, ln in enumerate(c["lengths"]) if ln > 0}
    table, codes = canonical_codes(lengths)
    sym_lut, len_lut = build_decode_lut(table, codes)
    mb = table.max_bits
    for s, code in codes.items():
        ln = lengths[s]
        lo = code << (mb - ln)
        assert np.all(sym_lut[lo: lo + (1 << (mb - ln))] == s)
        assert np.all(len_lut[lo: lo + (1 << (mb - ln))] == ln)
    assert np.array_equal(sym_lut, enc.sym_lut)
