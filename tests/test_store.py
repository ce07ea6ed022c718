"""The compressed store on disk (runtime/store.py): the reference's weights.bin +
manifest.json layout, written and read here.

Mirrors the reference's tests/test_binstore.py (round trips, sequential
offsets, read_many extents and its non-owning unaligned views) and its
integrity checks (afterimage/runtime/binstore.py:222-247,
streaming_engine.py:843-870); tests/golden/store_vectors.npz pins the bytes
and blob references against the reference's own writer.
"""
import json
import zlib

import numpy as np
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import (
    compress_group,
    compress_layer,
    decompress_layer_gpu,
)
from afterimage_amd.runtime.store import (
    COMPRESSED_BLOBS,
    SCHEMA_VERSION,
    StoreError,
    StoreReader,
    StoreWriter,
    verify_store,
)
from afterimage_amd.runtime.stream_ring import HostBlock

GOLDEN = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "store_vectors.npz",
                 allow_pickle=False)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def test_writer_matches_the_reference_writer_byte_for_byte(tmp_path):
    rows, cols, chunk, max_bits, seed = (int(x) for x in GOLDEN["params"])
    w = workloads.bf16_normal((rows, cols), seed=seed, scale=0.02, outlier_frac=1e-3)
    assert np.array_equal(w.view(torch.int16).numpy().reshape(-1), GOLDEN["bits"])
    with StoreWriter(tmp_path, model_id="golden") as sw:
        sw.add_compressed("w", compress_layer(w, chunk_size=chunk, max_bits=max_bits))
    data = np.fromfile(tmp_path / "weights.bin", dtype=np.uint8)
    assert np.array_equal(data, GOLDEN["weights_bin"])
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    assert manifest["tensors"]["w"]["blobs"] == json.loads(str(GOLDEN["blobs_json"]))
    assert list(manifest["tensors"]["w"]["blobs"]) == list(COMPRESSED_BLOBS)


def _model(tmp_path, chunk_size=4096):
    """A small store: a block with shared per-role codebooks, a tensor
    compressed on its own, a raw norm vector and a raw small matrix."""
    blk = workloads.block_14b(scale=0.01, chunk_size=chunk_size)
    extra = workloads.bf16_normal((300, 400), seed=9, scale=0.02)
    small = workloads.bf16_normal((16, 16), seed=10, scale=0.02)
    with StoreWriter(tmp_path, model_id="tiny", chunk_size=chunk_size) as sw:
        for name, w, layer in blk:
            if layer.encoded.n_symbols > 65536 and w.dim() == 2:
                sw.add_compressed("layers.0." + name, layer)
            else:
                sw.add_tensor("layers.0." + name, w)
        sw.add_tensor("extra", extra)
        sw.add_tensor("small", small)
    want = {"layers.0." + n: w for n, w, _ in blk}
    want.update(extra=extra, small=small)
    return want


def test_round_trip_through_the_store(tmp_path):
    want = _model(tmp_path)
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    assert manifest["schema_version"] == SCHEMA_VERSION
    with StoreReader(tmp_path) as rd:
        assert set(rd.tensors) == set(want)
        for key, w in want.items():
            meta = rd.tensors[key]
            if meta["compressed"]:
                assert list(meta["blobs"]) == list(COMPRESSED_BLOBS)
                layer = rd.layer(key, verify=True)
                out = decompress_layer_gpu(layer, device="cpu")
                assert torch.equal(_bits(out), _bits(w)), key
                assert meta["n_symbols"] == w.numel() and meta["shape"] == list(w.shape)
            else:
                got = rd.raw(key, verify=True)
                assert got.dtype == w.dtype and torch.equal(_bits(got), _bits(w)), key
    # The storage rule of the reference: small or 1-D tensors stay raw.
    assert not manifest["tensors"]["small"]["compressed"]
    assert not manifest["tensors"]["layers.0.input_layernorm"]["compressed"]
    assert manifest["tensors"]["extra"]["compressed"]


def test_blobs_are_back_to_back_with_crc32(tmp_path):
    _model(tmp_path)
    data = (tmp_path / "weights.bin").read_bytes()
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    pos = 0
    for meta in manifest["tensors"].values():
        for ref in meta["blobs"].values():
            assert ref["offset"] == pos
            blob = data[pos: pos + ref["nbytes"]]
            assert zlib.crc32(blob) == ref["crc32"]
            pos += ref["nbytes"]
    assert pos == len(data)


def test_shared_codebooks_survive_the_store(tmp_path):
    ws = [workloads.bf16_normal((200, 700), seed=s, scale=0.02) for s in (1, 2)]
    layers = compress_group(ws, chunk_size=2048)
    with StoreWriter(tmp_path) as sw:
        for k, l in enumerate(layers):
            sw.add_compressed("t%d" % k, l)
    with StoreReader(tmp_path) as rd:
        a, b = rd.layer("t0"), rd.layer("t1")
        assert np.array_equal(a.encoded.sym_lut, b.encoded.sym_lut)
        for l, w in zip((a, b), ws):
            assert torch.equal(_bits(decompress_layer_gpu(l, device="cpu")), _bits(w))


def _blob_file(tmp_path, arrays):
    with StoreWriter(tmp_path) as sw:
        for k, a in enumerate(arrays):
            sw._entry("a%d" % k, {"orig_bytes": a.nbytes, "comp_bytes": a.nbytes,
                                  "shape": list(a.shape), "compressed": False,
                                  "dtype": str(a.dtype)}, {"raw": a})
    return [m["blobs"]["raw"] for m in json.loads((tmp_path / "manifest.json").read_text())
            ["tensors"].values()]


def test_offsets_are_sequential(tmp_path):
    refs = _blob_file(tmp_path, [np.zeros(100, np.uint8), np.zeros(50, np.uint8),
                                 np.zeros(200, np.uint8)])
    assert [r["offset"] for r in refs] == [0, 100, 150]
    assert (tmp_path / "weights.bin").stat().st_size == 350


def test_read_many_coalesces_and_keeps_the_callers_order(tmp_path):
    arrays = [np.arange(64, dtype=np.uint8), np.arange(20, dtype=np.float32).reshape(4, 5),
              np.arange(11, dtype=np.int32)]
    refs = _blob_file(tmp_path, arrays)
    with StoreReader(tmp_path) as rd:
        got, calls, nbytes = rd.read_many(refs, max_extent_bytes=4096)
        assert calls == 1 and nbytes == (tmp_path / "weights.bin").stat().st_size
        assert all(np.array_equal(a, b) for a, b in zip(got, arrays))
        got, calls, nbytes = rd.read_many([refs[2], refs[0], refs[1]], max_extent_bytes=150)
        assert calls == 2 and [g.dtype for g in got] == [np.int32, np.uint8, np.float32]
        with pytest.raises(ValueError):
            rd.read_many(refs, max_gap_bytes=-1)


def test_read_many_views_are_non_owning_and_may_be_unaligned(tmp_path):
    arrays = [np.arange(7, dtype=np.uint8), np.arange(5, dtype=np.uint32),
              np.arange(3, dtype=np.float32), np.arange(9, dtype=np.uint16).reshape(3, 3)]
    refs = _blob_file(tmp_path, arrays)
    with StoreReader(tmp_path) as rd:
        got, calls, _ = rd.read_many(refs, verify=True)
    assert calls == 1
    for a, g in zip(arrays, got):
        assert np.array_equal(a, g) and g.flags.writeable and not g.flags.owndata
    assert not got[1].flags.aligned


def test_a_flipped_byte_is_caught(tmp_path):
    _model(tmp_path)
    assert verify_store(tmp_path) == (True, [])
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    ref = manifest["tensors"]["extra"]["blobs"]["packed"]
    with open(tmp_path / "weights.bin", "r+b") as f:
        f.seek(ref["offset"] + ref["nbytes"] // 2)
        b = f.read(1)
        f.seek(-1, 1)
        f.write(bytes([b[0] ^ 0x10]))
    assert verify_store(tmp_path) == (False, ["extra"])
    with StoreReader(tmp_path) as rd:
        with pytest.raises(StoreError, match="checksum mismatch"):
            rd.layer("extra", verify=True)
        with pytest.raises(StoreError, match="checksum mismatch"):
            rd.host_block(["extra"], pin=False, verify=True)
        rd.layer("extra")  # unverified reads do not check


def test_truncated_and_foreign_stores_are_refused(tmp_path):
    _model(tmp_path)
    path = tmp_path / "weights.bin"
    with open(path, "r+b") as f:
        f.truncate(path.stat().st_size - 1)
    with pytest.raises(StoreError, match="truncated"):
        StoreReader(tmp_path)
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    manifest["schema_version"] = 1
    (tmp_path / "manifest.json").write_text(json.dumps(manifest))
    with pytest.raises(StoreError, match="schema_version"):
        StoreReader(tmp_path)


def test_host_block_read_from_the_store_equals_one_built_in_memory(tmp_path):
    blk = workloads.block_14b(scale=0.01, chunk_size=4096)
    keys = []
    with StoreWriter(tmp_path) as sw:
        for name, _, layer in blk:
            sw.add_compressed(name, layer)
            keys.append(name)
    with StoreReader(tmp_path) as rd:
        from_store = rd.host_block(keys, pin=False, verify=True)
    built = HostBlock([l for _, _, l in blk], pin=False)
    assert from_store.nbytes == built.nbytes
    a, b = from_store.buf.numpy(), built.buf.numpy()
    for t in built.layout:
        for at, n in (t.sign_mantissa, t.packed):
            assert np.array_equal(a[at: at + n], b[at: at + n])
        for at, n in (t.chunk_offsets, t.chunk_nbytes):
            assert np.array_equal(a[at: at + 4 * n], b[at: at + 4 * n])
    for x, y in zip(from_store.layout, built.layout):
        assert (x.chunk_size, x.n_symbols, x.shape, x.max_bits) == \
               (y.chunk_size, y.n_symbols, y.shape, y.max_bits)
        assert np.array_equal(x.sym_lut, y.sym_lut) and np.array_equal(x.len_lut, y.len_lut)


def _aligned_pread(data: bytes, alignment: int, calls: list):
    """A pread over `data` that enforces what O_DIRECT enforces: block-aligned
    file offset and length (a shorter read only at the end of the file)."""
    def pread(buf, at):
        assert at % alignment == 0 and buf.nbytes % alignment == 0
        calls.append((at, buf.nbytes))
        chunk = data[at: at + buf.nbytes]
        buf[: len(chunk)] = chunk
        return len(chunk)
    return pread


@pytest.mark.parametrize("offset,n", [(0, 1), (1, 4095), (4095, 2), (4096, 4096), (5000, 12000),
                                      (123, 30000), (40000 - 7, 7), (0, 40000)])
def test_direct_reads_are_aligned_and_exact(offset, n):
    import mmap
    from afterimage_amd.runtime.store import direct_readinto

    data = np.random.default_rng(offset + n).integers(0, 256, 40000, dtype=np.uint8).tobytes()
    bounce = mmap.mmap(-1, 3 * 4096)  # smaller than some reads: several bounces
    calls = []
    out = np.zeros(n, np.uint8)
    direct_readinto(_aligned_pread(data, 4096, calls), bounce, offset, memoryview(out))
    assert out.tobytes() == data[offset: offset + n]
    assert all(sz <= 3 * 4096 for _, sz in calls)
    with pytest.raises(StoreError):  # past the end of the file
        direct_readinto(_aligned_pread(data, 4096, []), bounce, 40000 - 3, memoryview(np.zeros(8, np.uint8)))
    bounce.close()


def test_direct_reader_reads_what_the_buffered_one_does(tmp_path):
    W = workloads.bf16_normal((300, 700), seed=3, scale=0.02, outlier_frac=1e-3)
    with StoreWriter(tmp_path) as sw:
        sw.add_compressed("w", compress_layer(W, chunk_size=1024))
        sw.add_tensor("norm", torch.ones(700, dtype=torch.bfloat16))
    with StoreReader(tmp_path) as rd, StoreReader(tmp_path, direct=True) as dd:
        # O_DIRECT where the file system takes it (tmpfs and overlay file
        # systems refuse it: the reader then reads buffered and says so).
        assert isinstance(dd.used_direct, bool)
        a, b = rd.layer("w", verify=True), dd.layer("w", verify=True)
        for f in ("packed", "chunk_offsets", "chunk_nbytes", "sym_lut", "len_lut"):
            assert np.array_equal(getattr(a.encoded, f), getattr(b.encoded, f))
        assert torch.equal(a.sign_mantissa, b.sign_mantissa)
        assert torch.equal(_bits(rd.raw("norm")), _bits(dd.raw("norm")))
        ha, hb = rd.host_block(["w"], pin=False, verify=True), dd.host_block(["w"], pin=False,
                                                                             verify=True)
        # The arrays' regions of the two pinned blocks (the padding between
        # them is not written).
        ba, bb = ha.buf.numpy(), hb.buf.numpy()
        for la, lb in zip(ha.layout, hb.layout):
            for f in ("packed", "chunk_offsets", "chunk_nbytes", "sign_mantissa"):
                (a0, an), (b0, bn) = getattr(la, f), getattr(lb, f)
                size = an * (4 if f.startswith("chunk") else 1)
                assert (a0, an) == (b0, bn) and np.array_equal(ba[a0:a0 + size], bb[b0:b0 + size])
        assert torch.equal(_bits(decompress_layer_gpu(b, device="cpu")), _bits(W))


def test_raw_bf16_bit_patterns_written_as_int16_read_back_as_bf16(tmp_path):
    # The reference writes force_raw_storage bf16 tensors and row-gather
    # embeddings as int16 bit patterns with dtype "bfloat16"
    # (streaming_engine.py:193, :237, :372-374) and reads them back by
    # reinterpreting the bytes (streaming_engine.py:1084-1095); a numeric
    # cast would turn the pattern 16256 (bf16 1.0) into 16256.0.
    W = torch.tensor([[1.0, -2.5, 3.0e-3], [0.0, 65280.0, -1.0e-30]], dtype=torch.bfloat16)
    bits = W.view(torch.int16).numpy()
    with StoreWriter(tmp_path) as sw:
        sw._entry("forced", {"orig_bytes": W.numel() * 2, "comp_bytes": W.numel() * 2,
                             "shape": list(W.shape), "compressed": False,
                             "dtype": "torch.bfloat16"}, {"raw": bits})
        sw._entry("embed", {"orig_bytes": W.numel() * 2, "comp_bytes": W.numel() * 2,
                            "shape": list(W.shape), "compressed": False, "row_gather": True,
                            "hidden_size": 3, "dtype": "bfloat16"}, {"raw": bits})
        sw.add_tensor("norm", torch.tensor([1.0, 0.5], dtype=torch.bfloat16))
    with StoreReader(tmp_path) as rd:
        got = rd.raw("forced", verify=True)
        assert got.dtype == torch.bfloat16 and torch.equal(got.view(torch.int16), W.view(torch.int16))
        assert float(got[0, 0]) == 1.0
        with pytest.raises(RuntimeError, match="row-gather-only"):
            rd.raw("embed")
        norm = rd.raw("norm")  # float32 copy cast back
        assert norm.dtype == torch.bfloat16 and norm.tolist() == [1.0, 0.5]
