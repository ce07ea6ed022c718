"""GPU exponent decode (decode_gpu_v2) against the oracle and the reference's outputs.

Mirrors the reference's tests/test_gpu_decode.py and tests/test_gpu_decode_v2.py
cases, run through this package's gfx950 kernel.
"""
import numpy as np
import pytest
import torch

import oracle
from afterimage_amd.runtime.compressed_store import _slice_encoded
from afterimage_amd.runtime.gpu_decode_v2 import decode_gpu_v2
from afterimage_amd.runtime.huffman_chunked import encode_chunked
from tests.distributions import many_escape_windows
from tests.golden_data import case, case_names

pytestmark = pytest.mark.gpu


def _check(exponents, chunk_size, block_chunks=32, max_bits=16):
    exps = exponents.numpy() if hasattr(exponents, "numpy") else np.asarray(exponents)
    enc = encode_chunked(exponents, chunk_size=chunk_size, max_bits=max_bits)
    cpu = oracle.decode_chunked_reference(enc)
    assert np.array_equal(cpu, exps), "oracle itself is wrong"
    gpu = decode_gpu_v2(enc, block_chunks=block_chunks).cpu().numpy()
    assert gpu.shape == exps.shape
    assert np.array_equal(gpu, exps), (
        "GPU decode mismatch: %d / %d symbols wrong" % (int((gpu != exps).sum()), exps.size))


def test_small_skewed_distribution():
    torch.manual_seed(0)
    _check(torch.randint(100, 140, (2000,)), chunk_size=64)


def test_full_256_symbol_alphabet_uniform():
    torch.manual_seed(1)
    _check(torch.randint(0, 256, (8000,)), chunk_size=256)


def test_real_bf16_exponent_distribution():
    torch.manual_seed(2)
    W = (torch.randn(512, 4096) * 0.02).to(torch.bfloat16)
    bits = W.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    _check(((bits >> 7) & 0xFF).flatten(), chunk_size=512)


def test_various_chunk_sizes():
    torch.manual_seed(3)
    exps = torch.randint(50, 90, (10000,))
    for cs in [32, 128, 512, 1024]:
        _check(exps, chunk_size=cs)


def test_chunk_size_not_dividing_data_evenly():
    torch.manual_seed(4)
    _check(torch.randint(0, 200, (7777,)), chunk_size=333)


def test_single_symbol_degenerate_case():
    _check(torch.full((5000,), 42, dtype=torch.int64), chunk_size=256)


def test_two_symbol_extreme_skew():
    data = np.random.default_rng(5).choice([10, 200], size=6000, p=[0.99, 0.01])
    _check(torch.from_numpy(data), chunk_size=256)


@pytest.mark.parametrize("seed", range(10))
def test_many_random_distributions(seed):
    rng = np.random.default_rng(seed)
    k = rng.integers(2, 200)
    probs = rng.dirichlet(np.ones(k) * rng.uniform(0.1, 3.0))
    data = rng.choice(k, size=rng.integers(2000, 8000), p=probs)
    _check(torch.from_numpy(data.astype(np.int64)), chunk_size=int(rng.choice([64, 128, 256, 512])))


@pytest.mark.parametrize("block_chunks", [1, 4, 32, 128, 256])
def test_block_chunks_values_are_accepted(block_chunks):
    torch.manual_seed(0)
    _check(torch.randint(100, 140, (20000,)), chunk_size=64, block_chunks=block_chunks)


def test_n_chunks_not_multiple_of_block_chunks():
    torch.manual_seed(1)
    _check(torch.randint(0, 256, (7777,)), chunk_size=100, block_chunks=32)


@pytest.mark.parametrize("chunk_size", [256, 4096, 65536])
def test_escape_blocks_beyond_the_lds_share(chunk_size):
    """Tables with more than 64 escape blocks read the rest from global memory."""
    _check(torch.from_numpy(many_escape_windows(7, 400_000)), chunk_size=chunk_size)


@pytest.mark.parametrize("max_bits", [8, 12, 16])
@pytest.mark.parametrize("chunk_size", [32, 128, 1024])
def test_length_limited_codes(chunk_size, max_bits):
    torch.manual_seed(chunk_size + max_bits)
    w = (torch.randn(80_000) * 0.02).to(torch.bfloat16)
    bits = w.view(torch.int16).to(torch.int32) & 0xFFFF
    _check((bits >> 7) & 0xFF, chunk_size=chunk_size, max_bits=max_bits)


@pytest.mark.parametrize("name", case_names())
def test_golden_streams(name):
    c = case(name)
    gpu = decode_gpu_v2(c["encoded"]).cpu().numpy()
    assert np.array_equal(gpu, c["symbols"])


@pytest.mark.parametrize("name", [n for n in case_names() if case(n)["slice_tail"] is not None])
def test_golden_whole_chunk_decode_of_partial_slice(name):
    """n_symbols of a chunk-range slice counts whole chunks; the positions past
    the real symbols must read like the reference's bounded reader."""
    c = case(name)
    c0, c1 = c["slice_tail"]
    sub = _slice_encoded(c["encoded"], c0, c1)
    gpu = decode_gpu_v2(sub).cpu().numpy()
    assert np.array_equal(gpu, c["slice_tail_decoded"])


def test_rejects_invalid_block_width_before_touching_enc():
    for value in (0, -1, 3):
        with pytest.raises(ValueError, match="power of 2"):
            decode_gpu_v2(None, block_chunks=value)


def test_exponent_decode_at_64k_chunks_with_outliers():
    """4 chunks of 65536 symbols drawn like the 5120x17408 layer."""
    c = case("bf16_outliers_64k")
    gpu = decode_gpu_v2(c["encoded"]).cpu().numpy()
    assert np.array_equal(gpu, c["symbols"])


def test_repeat_runs_are_identical_across_streams():
    c = case("bf16_n002")
    enc = c["encoded"]
    base = decode_gpu_v2(enc)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        again = [decode_gpu_v2(enc, synchronize=False) for _ in range(3)]
    s.synchronize()
    for a in again:
        assert torch.equal(a, base)


@pytest.mark.parametrize("chunk_size", [16, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536])
def test_every_subgroup_width(chunk_size):
    """Chunk sizes that select each threads-per-chunk width (16..1024)."""
    w = (torch.randn(3 * chunk_size + 77, generator=torch.Generator().manual_seed(chunk_size))
         * 0.02).to(torch.bfloat16)
    bits = w.view(torch.int16).to(torch.int32) & 0xFFFF
    _check((bits >> 7) & 0xFF, chunk_size=chunk_size)


def test_round_with_more_symbols_than_the_staging_area():
    """1-bit codes in 70000-symbol chunks: one round carries more symbols
    than a sub-group can stage, so the decode runs in several windows."""
    rng = np.random.default_rng(0)
    data = rng.choice([5, 9], size=140013, p=[0.7, 0.3])
    _check(torch.from_numpy(data), chunk_size=70000)


def test_chunks_that_need_several_rounds():
    """8-bit codes in 65536-symbol chunks: 512 Kbit per chunk, several rounds."""
    rng = np.random.default_rng(1)
    _check(torch.from_numpy(rng.integers(0, 256, size=65536 + 5000)), chunk_size=65536)
    c = case("uniform256")
    gpu = decode_gpu_v2(c["encoded"]).cpu().numpy()
    assert np.array_equal(gpu, c["symbols"])


def test_whole_chunk_decode_with_padding_across_rounds():
    rng = np.random.default_rng(2)
    data = rng.integers(0, 256, size=65536 + 5000)
    enc = encode_chunked(torch.from_numpy(data), chunk_size=65536)
    sub = _slice_encoded(enc, 0, enc.n_chunks)
    gpu = decode_gpu_v2(sub).cpu().numpy()
    assert np.array_equal(gpu, oracle.decode_chunks(sub))


def test_segment_guesses_all_wrong():
    # Eight equiprobable symbols get 3-bit codes. Segment starts are multiples
    # of 168 bits and the 32-bit lead-in before each lands one bit past a
    # codeword boundary, which fixed-length codes never leave: every thread but
    # the first of each round is wrong on its first pass, and the output rests
    # on the re-decode from the predecessor's end (up to one pass per thread).
    rng = np.random.default_rng(8)
    _check(rng.integers(0, 8, 20000), chunk_size=4096)
    _check(rng.integers(0, 8, 70000), chunk_size=65536)
