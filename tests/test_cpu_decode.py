"""The product's CPU decode path (aimg_cpu_decode_bf16 / _u8 and the
device="cpu" branch of the reference API), checked against the reference's own
decoded vectors (tests/golden/codec_vectors.npz) and the oracle.

Mirrors the reference's tests/test_cpu_decode.py (numba decoder vs the
reference reader) and the CPU cases of tests/test_compressed_store.py.
"""
import numpy as np
import pytest
import torch

import oracle
from afterimage_amd import _native, workloads
from afterimage_amd.runtime import compressed_store as cs
from afterimage_amd.runtime import device as devmod
from afterimage_amd.runtime import gpu_decode_v2 as gd
from afterimage_amd.runtime.compressed_store import (
    _slice_encoded,
    compress_layer,
    decompress_layer_cpu_reference,
    decompress_layer_gpu,
    decompress_rows_gpu,
    recombine_exponent_and_sign_mantissa,
)
from tests.golden_data import GOLDEN, case, case_names
from tests.store_views import store_views


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def _decode_u8(enc, n_out, threads):
    out = torch.empty(n_out, dtype=torch.uint8)
    devmod.cpu_decode([(enc, None, out, n_out)], n_threads=threads, exponents_only=True)
    return out.numpy()


@pytest.mark.parametrize("name", case_names())
@pytest.mark.parametrize("threads", [1, 3])
def test_cpu_decoder_matches_reference_symbols(name, threads):
    c = case(name)
    enc = c["encoded"]
    assert np.array_equal(_decode_u8(enc, enc.n_symbols, threads), c["symbols"])


@pytest.mark.parametrize("name", [n for n in case_names() if case(n)["slice_tail"] is not None])
def test_cpu_whole_chunk_decode_of_partial_slice_matches_reference(name):
    """Past a partial last chunk's coded symbols the reference decodes zero bits."""
    c = case(name)
    c0, c1 = c["slice_tail"]
    sub = _slice_encoded(c["encoded"], c0, c1)
    got = _decode_u8(sub, sub.n_chunks * sub.chunk_size, 2)
    assert np.array_equal(got, c["slice_tail_decoded"])


@pytest.mark.parametrize("name", ["kat_int16", "special_values", "randn_128x512"])
def test_cpu_bf16_known_answers(name):
    p = "bf16/%s/" % name
    bits = GOLDEN[p + "bits"]
    shape = tuple(int(x) for x in GOLDEN[p + "shape"])
    w = torch.from_numpy(bits.copy()).view(torch.bfloat16).reshape(shape)
    layer = compress_layer(w, chunk_size=int(GOLDEN[p + "chunk_size"][0]))
    for out in (decompress_layer_gpu(layer, device="cpu"), decompress_layer_cpu_reference(layer)):
        assert out.dtype == torch.bfloat16 and out.device.type == "cpu"
        assert tuple(out.shape) == shape
        assert np.array_equal(out.view(torch.int16).numpy().reshape(-1), GOLDEN[p + "decoded_bits"])


def test_cpu_layer_1024x3072_against_oracle_and_original():
    W, layer = workloads.small_layer()
    out = decompress_layer_gpu(layer, device=torch.device("cpu"))
    assert torch.equal(_bits(out), _bits(W))
    assert torch.equal(_bits(out), _bits(oracle.decompress_layer_reference(layer)))


@pytest.mark.parametrize("chunk_size", [16, 1000, 4096, 70000])
def test_cpu_decode_thread_counts_agree(chunk_size):
    g = torch.Generator().manual_seed(chunk_size)
    W = (torch.randn(300, 700, generator=g) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=chunk_size)
    outs = []
    for threads in (1, 2, 7):
        out = torch.empty(W.numel(), dtype=torch.bfloat16)
        devmod.cpu_decode([(layer.encoded, layer.sign_mantissa, out, W.numel())], n_threads=threads)
        outs.append(out)
    for out in outs:
        assert torch.equal(_bits(out), _bits(W.reshape(-1)))


def test_cpu_rows_match_full_decode():
    W, layer = workloads.small_layer(seed=4, rows=96, cols=640, chunk_size=1000)
    for r0, r1 in [(0, 96), (5, 6), (17, 60), (95, 200), (50, 50)]:
        rows = decompress_rows_gpu(layer, r0, r1, device="cpu")
        want = W[max(0, r0):min(96, r1)]
        assert rows.shape == want.shape
        assert torch.equal(_bits(rows), _bits(want))


def test_cpu_sliced_call_matches_whole():
    W, layer = workloads.small_layer(seed=6, rows=64, cols=1000, chunk_size=512)
    a = decompress_layer_gpu(layer, device="cpu", max_slice_elems=1 << 25)
    b = decompress_layer_gpu(layer, device="cpu", max_slice_elems=1500, reuse_decode_tables=True)
    assert torch.equal(_bits(a), _bits(W)) and torch.equal(_bits(b), _bits(W))


def test_cpu_empty_layer():
    layer = compress_layer(torch.zeros(0, 8, dtype=torch.bfloat16))
    out = decompress_layer_gpu(layer, device="cpu")
    assert out.shape == (0, 8)


def test_recombine_public_entry_on_every_byte_pair():
    e = np.repeat(np.arange(256, dtype=np.uint8), 256)
    sm = np.tile(np.arange(256, dtype=np.uint8), 256)
    got = recombine_exponent_and_sign_mantissa(e, sm, (256, 256), "cpu")
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == (256, 256)
    bits = got.view(torch.int16).numpy().reshape(-1).view(np.uint16)
    assert np.array_equal(bits, oracle.recombine(e, sm))
    assert np.unique(bits).size == 65536


def test_recombine_public_entry_on_known_answers():
    p = "bf16/kat_int16/"
    sm = GOLDEN[p + "sign_mantissa"]
    exps = ((GOLDEN[p + "bits"].view(np.uint16) >> 7) & 0xFF).astype(np.uint8)
    # The reference passes int32 exponents (decompress_layer_cpu_reference).
    got = recombine_exponent_and_sign_mantissa(torch.from_numpy(exps).to(torch.int32),
                                               torch.from_numpy(sm), (exps.size,), "cpu")
    assert np.array_equal(got.view(torch.int16).numpy(), GOLDEN[p + "decoded_bits"])


def test_recombine_rejects_mismatched_lengths():
    with pytest.raises(ValueError, match="elements"):
        recombine_exponent_and_sign_mantissa(np.zeros(4, np.uint8), np.zeros(5, np.uint8), (4,), "cpu")


@pytest.mark.filterwarnings("ignore::UserWarning")
@pytest.mark.parametrize("misalign", [1, 3])
def test_cpu_decode_from_unaligned_non_owning_views(misalign):
    W, layer = workloads.small_layer(seed=9, rows=128, cols=768, chunk_size=4096)
    view_layer, views = store_views(layer, misalign)
    assert all(not v.flags.owndata for v in views)
    assert not views[2].flags.aligned  # int32 chunk offsets at an odd address
    out = decompress_layer_gpu(view_layer, device="cpu")
    assert torch.equal(_bits(out), _bits(W))


def test_prepare_decode_tables_unpacks_like_the_reference():
    c = case("bf16_outliers_64k")
    enc = c["encoded"]
    tables = gd.prepare_decode_tables(enc, "cpu")
    sym, ln = tables
    assert sym.dtype == torch.int32 and ln.dtype == torch.int32
    assert np.array_equal(sym.numpy(), enc.sym_lut) and np.array_equal(ln.numpy(), enc.len_lut)
    assert len(tables) == 2 and tables[0] is sym


def test_table_cache_hits_by_identity_then_by_content():
    c = case("dirichlet_4")
    enc = c["encoded"]
    devmod.TABLES.clear()
    h0, b0 = devmod.TABLES.hashes, devmod.TABLES.builds
    t1 = devmod.TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, "cpu")
    t2 = devmod.TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, "cpu")
    assert t1 is t2
    assert devmod.TABLES.hashes == h0 + 1 and devmod.TABLES.builds == b0 + 1
    # Equal content in new arrays: hashed, not rebuilt.
    t3 = devmod.TABLES.get(enc.sym_lut.copy(), enc.len_lut.copy(), enc.max_bits, "cpu")
    assert t3 is t1 and devmod.TABLES.hashes == h0 + 2 and devmod.TABLES.builds == b0 + 1
    # Another codebook never shares the table.
    other = case("dirichlet_5")["encoded"]
    t4 = devmod.TABLES.get(other.sym_lut, other.len_lut, other.max_bits, "cpu")
    assert t4.key != t1.key


def test_decode_tables_compare_and_hash_by_codebook():
    # DecodeTables unpacks like a 2-tuple but must not compare or hash as the
    # empty tuple it is built from: different codebooks differ.
    a = case("dirichlet_4")["encoded"]
    b = case("dirichlet_5")["encoded"]
    ta = devmod._TableCache().get(a.sym_lut, a.len_lut, a.max_bits, "cpu")
    ta2 = devmod._TableCache().get(a.sym_lut.copy(), a.len_lut.copy(), a.max_bits, "cpu")
    tb = devmod._TableCache().get(b.sym_lut, b.len_lut, b.max_bits, "cpu")
    assert ta is not ta2 and ta == ta2 and hash(ta) == hash(ta2)
    assert ta != tb and not (ta == tb)
    assert len({ta, ta2, tb}) == 2
    assert ta != () and () != ta


def test_table_cache_is_bounded_by_bytes():
    cache = devmod._TableCache(capacity_bytes=3 * 29000)
    names = ["dirichlet_%d" % k for k in range(6)]
    for n in names:
        enc = case(n)["encoded"]
        cache.get(enc.sym_lut, enc.len_lut, enc.max_bits, "cpu")
    assert len(cache._items) <= 3


def test_cpu_decoder_rejects_a_foreign_table_blob():
    c = case("uniform16")
    enc = c["encoded"]
    desc = (_native.AimgTensor * 1)()
    out = np.zeros(enc.n_symbols, np.uint8)
    junk = np.zeros(64 * 1024, np.uint8)
    packed = np.ascontiguousarray(enc.packed)
    offs = np.ascontiguousarray(enc.chunk_offsets, np.int32)
    nb = np.ascontiguousarray(enc.chunk_nbytes, np.int32)
    d = desc[0]
    d.packed, d.chunk_offsets, d.chunk_nbytes = packed.ctypes.data, offs.ctypes.data, nb.ctypes.data
    d.out, d.table = out.ctypes.data, junk.ctypes.data
    d.packed_nbytes, d.n_symbols = packed.size, enc.n_symbols
    d.chunk_size, d.n_chunks = enc.chunk_size, enc.n_chunks
    lib = _native.lib()
    assert lib.aimg_cpu_decode_u8(desc, 1, 1) == _native.AIMG_ERR_BAD_TABLE
    assert b"magic" in lib.aimg_last_error()
    d.n_symbols = enc.n_chunks * enc.chunk_size + 1
    assert lib.aimg_cpu_decode_u8(desc, 1, 1) == _native.AIMG_ERR_INVALID_ARGUMENT


def test_gpu_only_entry_points_name_the_cpu_route():
    enc = case("uniform16")["encoded"]
    with pytest.raises(RuntimeError, match="device='cpu'"):
        gd.decode_gpu_v2(enc, device="cpu")
