"""The reference's compressed store on disk: one ``weights.bin`` holding every
tensor's arrays back to back, and a ``manifest.json`` that says where each
array lies (afterimage/runtime/binstore.py:41-247,
afterimage/runtime/streaming_engine.py:158-253, :352-428).

A store written here is read by the reference engine, and a store the
reference wrote is read here:

* manifest: ``schema_version`` 2 and ``tensors[key]`` = {orig_bytes,
  comp_bytes, shape, blobs, compressed, ...}; a compressed tensor adds
  max_bits, n_symbols and chunk_size, a raw one its dtype;
* blobs of a compressed tensor, written in this order: sign_mantissa,
  packed, chunk_offsets, chunk_nbytes, sym_lut, len_lut; each blob is
  {offset, nbytes, dtype, shape, crc32} (zlib CRC-32 of its bytes).

Reading. ``StoreReader.read_many`` merges nearby blobs into bounded extents
and returns non-owning, possibly unaligned views, as the reference's
``read_many`` does. ``StoreReader.host_block`` reads a decoder block's arrays
straight into one pinned buffer laid out for ``LayerRing`` (each array at an
alignment the kernel reads it with), so a streamed layer goes disk -> pinned
memory -> GPU with no intermediate copy.

``StoreReader(store_dir, direct=True)`` reads with O_DIRECT where the file
system takes it, as the reference's directio.py does for its weight reads
(afterimage/runtime/directio.py:1-107): the page cache is bypassed, so read
rates are the storage's own. O_DIRECT needs block-aligned offsets, lengths
and memory, so each read goes through a page-aligned bounce buffer that
holds the aligned span around it. Where O_DIRECT is refused the reader falls
back to buffered reads and says so (``used_direct``).
"""
from __future__ import annotations

import dataclasses
import json
import mmap
import os
import pathlib
import zlib

import numpy as np
import torch

from .compressed_store import CompressedLayer, compress_layer
from .huffman_chunked import ChunkedEncoded

SCHEMA_VERSION = 2
DIRECT_ALIGNMENT = 4096           # O_DIRECT offsets, lengths and addresses
DIRECT_BOUNCE_BYTES = 8 << 20     # the bounce buffer of one direct reader
_O_DIRECT = getattr(os, "O_DIRECT", None)
COMPRESSED_BLOBS = ("sign_mantissa", "packed", "chunk_offsets", "chunk_nbytes", "sym_lut",
                    "len_lut")


@dataclasses.dataclass
class BlobRef:
    """Where one array lies in weights.bin (binstore.py:41-47)."""

    offset: int
    nbytes: int
    dtype: str
    shape: tuple
    crc32: int = 0

    def to_dict(self) -> dict:
        return {"offset": self.offset, "nbytes": self.nbytes, "dtype": self.dtype,
                "shape": list(self.shape), "crc32": self.crc32}


class StoreError(ValueError):
    """A store that is truncated, corrupted or of another schema."""


def _crc_error(ref: dict, got: int) -> StoreError:
    return StoreError("checksum mismatch at offset %d (%d bytes): store is corrupted -- "
                      "got crc32=%d, manifest says %d"
                      % (ref["offset"], ref["nbytes"], got, ref.get("crc32", 0)))


class StoreWriter:
    """Writes weights.bin and, on close, manifest.json.

    ``add_tensor`` applies the reference's storage rule
    (streaming_engine.py:201-253): 2-D bf16 tensors of more than 65536
    elements are Huffman-coded with ``chunk_size`` / ``max_bits``, anything
    else is stored raw (float32 values, as the reference does for its small
    tensors). ``add_compressed`` stores an already-compressed layer (for
    example one of a ``compress_group`` that shares a codebook)."""

    def __init__(self, store_dir, model_id: str = "", chunk_size: int = 1024,
                 max_bits: int = 16):
        self.dir = pathlib.Path(store_dir)
        self.dir.mkdir(parents=True, exist_ok=True)
        self.chunk_size = int(chunk_size)
        self.max_bits = int(max_bits)
        self._fh = open(self.dir / "weights.bin", "wb")
        self._pos = 0
        self.manifest = {"schema_version": SCHEMA_VERSION, "model_id": model_id,
                         "revision": None, "quantize": None, "chunk_size": self.chunk_size,
                         "force_raw_storage": False, "tied": False, "tensors": {},
                         "expert_slices": {}}
        self._orig = 0
        self._comp = 0

    def _write(self, arr: np.ndarray) -> BlobRef:
        arr = np.ascontiguousarray(arr)
        data = memoryview(arr).cast("B")
        ref = BlobRef(offset=self._pos, nbytes=data.nbytes, dtype=str(arr.dtype),
                      shape=tuple(arr.shape), crc32=zlib.crc32(data))
        self._fh.write(data)
        self._pos += data.nbytes
        return ref

    def _entry(self, key: str, entry: dict, arrays: dict) -> None:
        if key in self.manifest["tensors"]:
            raise ValueError("tensor %r is already in the store" % key)
        entry["blobs"] = {name: self._write(a).to_dict() for name, a in arrays.items()}
        self.manifest["tensors"][key] = entry
        self._orig += entry["orig_bytes"]
        self._comp += entry["comp_bytes"]

    def add_compressed(self, key: str, layer: CompressedLayer) -> None:
        enc = layer.encoded
        arrays = {
            "sign_mantissa": np.ascontiguousarray(layer.sign_mantissa.numpy(), dtype=np.uint8),
            "packed": np.ascontiguousarray(enc.packed, dtype=np.uint8),
            "chunk_offsets": np.ascontiguousarray(enc.chunk_offsets, dtype=np.int32),
            "chunk_nbytes": np.ascontiguousarray(enc.chunk_nbytes, dtype=np.int32),
            "sym_lut": np.ascontiguousarray(enc.sym_lut, dtype=np.int32),
            "len_lut": np.ascontiguousarray(enc.len_lut, dtype=np.int8),
        }
        entry = {"orig_bytes": 2 * int(enc.n_symbols), "comp_bytes": int(layer.compressed_bytes),
                 "shape": [int(x) for x in layer.shape], "compressed": True,
                 "max_bits": int(enc.max_bits), "n_symbols": int(enc.n_symbols),
                 "chunk_size": int(enc.chunk_size)}
        self._entry(key, entry, arrays)

    def add_tensor(self, key: str, W: torch.Tensor) -> None:
        orig = W.numel() * W.element_size()
        if W.dtype == torch.bfloat16 and W.dim() == 2 and W.numel() > 65536:
            self.add_compressed(key, compress_layer(W, chunk_size=self.chunk_size,
                                                    max_bits=self.max_bits))
            return
        entry = {"orig_bytes": orig, "comp_bytes": orig, "shape": list(W.shape),
                 "compressed": False, "dtype": str(W.dtype)}
        self._entry(key, entry, {"raw": W.detach().cpu().to(torch.float32).numpy()})

    def close(self) -> None:
        if self._fh.closed:
            return
        self._fh.close()
        self.manifest["total_orig_bytes"] = self._orig
        self.manifest["total_comp_bytes"] = self._comp
        self.manifest["ratio"] = self._orig / max(self._comp, 1)
        (self.dir / "manifest.json").write_text(json.dumps(self.manifest, indent=2),
                                                 encoding="utf-8", newline="\n")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class StoreReader:
    """One open weights.bin for the store's lifetime, with the reference
    engine's always-on startup checks (streaming_engine.py:843-870): the
    schema version, and a file at least as long as every blob it lists."""

    def __init__(self, store_dir, direct: bool = False):
        self.dir = pathlib.Path(store_dir)
        self.manifest = json.loads((self.dir / "manifest.json").read_text())
        version = self.manifest.get("schema_version")
        if version != SCHEMA_VERSION:
            raise StoreError("store at %s has schema_version=%r, this code reads %d"
                             % (self.dir, version, SCHEMA_VERSION))
        path = self.dir / "weights.bin"
        if not path.exists():
            raise StoreError("no weights.bin found at %s" % self.dir)
        need = max((r["offset"] + r["nbytes"] for m in self.manifest["tensors"].values()
                    for r in m.get("blobs", {}).values()), default=0)
        size = path.stat().st_size
        if size < need:
            raise StoreError("weights.bin at %s is truncated: the manifest references bytes up "
                             "to offset %d but the file has %d" % (self.dir, need, size))
        self._fh = open(path, "rb", buffering=0)
        self._dfd = None
        self._bounce = None
        # True while reads go through O_DIRECT; False when not asked for, or
        # when the file system refused it (reads are then buffered).
        self.used_direct = False
        if direct and _O_DIRECT is not None:
            try:
                self._dfd = os.open(str(path), os.O_RDONLY | _O_DIRECT)
                self._bounce = mmap.mmap(-1, DIRECT_BOUNCE_BYTES)  # page-aligned
                self.used_direct = True
            except OSError:
                self._close_direct()

    @property
    def tensors(self) -> dict:
        return self.manifest["tensors"]

    def _close_direct(self) -> None:
        if self._dfd is not None:
            os.close(self._dfd)
        if self._bounce is not None:
            self._bounce.close()
        self._dfd = self._bounce = None
        self.used_direct = False

    def _readinto(self, offset: int, view: memoryview) -> None:
        if self._dfd is not None:
            try:
                direct_readinto(lambda b, at: os.preadv(self._dfd, [b], at),
                                self._bounce, offset, view)
                return
            except OSError:
                self._close_direct()  # this read and later ones go buffered
        self._fh.seek(offset)
        got = 0
        while got < view.nbytes:
            n = self._fh.readinto(view[got:])
            if not n:
                raise StoreError("short read at offset %d: wanted %d bytes, got %d"
                                 % (offset, view.nbytes, got))
            got += n

    def read(self, ref: dict, verify: bool = False) -> np.ndarray:
        """One blob as an owning, aligned array (binstore.py:84-107)."""
        out = np.empty(int(ref["nbytes"]), dtype=np.uint8)
        self._readinto(int(ref["offset"]), memoryview(out))
        if verify:
            got = zlib.crc32(out)
            if got != ref.get("crc32", 0):
                raise _crc_error(ref, got)
        return out.view(ref["dtype"]).reshape(ref["shape"])

    def read_many(self, refs: list[dict], *, max_gap_bytes: int = 0,
                  max_extent_bytes: int = 1 << 28, verify: bool = False
                  ) -> tuple[list[np.ndarray], int, int]:
        """Blobs in the caller's order, read through merged extents
        (binstore.py:109-192): blobs whose gap to the previous one is at most
        ``max_gap_bytes`` share one read while the extent stays within
        ``max_extent_bytes``. Returns (arrays, reads, bytes read); each array
        is a non-owning view into its extent's bytearray and need not be
        aligned to its dtype."""
        if max_gap_bytes < 0:
            raise ValueError("max_gap_bytes must be non-negative")
        if max_extent_bytes < 1:
            raise ValueError("max_extent_bytes must be positive")
        if not refs:
            return [], 0, 0
        order = sorted(range(len(refs)), key=lambda k: int(refs[k]["offset"]))
        extents: list[list] = []  # [start, end, [indices]]
        for k in order:
            start = int(refs[k]["offset"])
            end = start + int(refs[k]["nbytes"])
            if end < start:
                raise ValueError("blob extent overflows its offset")
            if extents:
                last = extents[-1]
                gap = start - last[1]
                merged = max(last[1], end)
                if 0 <= gap <= max_gap_bytes and merged - last[0] <= max_extent_bytes:
                    last[1] = merged
                    last[2].append(k)
                    continue
            extents.append([start, end, [k]])
        out: list = [None] * len(refs)
        total = 0
        for start, end, members in extents:
            buf = bytearray(end - start)
            view = memoryview(buf)
            self._readinto(start, view)
            total += end - start
            for k in members:
                ref = refs[k]
                rel = int(ref["offset"]) - start
                blob = view[rel: rel + int(ref["nbytes"])]
                if verify:
                    got = zlib.crc32(blob)
                    if got != ref.get("crc32", 0):
                        raise _crc_error(ref, got)
                out[k] = np.frombuffer(blob, dtype=ref["dtype"]).reshape(ref["shape"])
        return out, len(extents), total

    def layer(self, key: str, verify: bool = False) -> CompressedLayer:
        """A compressed tensor as a CompressedLayer over arrays read with
        read_many (the reference engine's _compressed_layer,
        streaming_engine.py:1149-1171)."""
        meta = self.tensors[key]
        if not meta.get("compressed"):
            raise ValueError("tensor %r is stored raw" % key)
        arrays, _, _ = self.read_many([meta["blobs"][b] for b in COMPRESSED_BLOBS],
                                      verify=verify)
        a = dict(zip(COMPRESSED_BLOBS, arrays))
        enc = ChunkedEncoded(packed=a["packed"], chunk_offsets=a["chunk_offsets"],
                             chunk_nbytes=a["chunk_nbytes"], sym_lut=a["sym_lut"],
                             len_lut=a["len_lut"], max_bits=int(meta["max_bits"]),
                             chunk_size=int(meta["chunk_size"]),
                             n_symbols=int(meta["n_symbols"]), shape=tuple(meta["shape"]))
        return CompressedLayer(sign_mantissa=torch.from_numpy(a["sign_mantissa"]), encoded=enc,
                               shape=tuple(meta["shape"]))

    def raw(self, key: str, verify: bool = False) -> torch.Tensor:
        """A raw tensor in its stored dtype, read as the reference's engine
        reads it (streaming_engine.py:1078-1105): an int16 blob of a bf16
        tensor holds its bit patterns (force_raw_storage and row-gather
        writes, streaming_engine.py:193, :237) and is reinterpreted; a float32
        blob of a bf16 tensor (the small-tensor rule) is cast back, which is
        exact. A row-gather tensor is never loaded whole."""
        meta = self.tensors[key]
        if meta.get("compressed"):
            raise ValueError("tensor %r is compressed" % key)
        if meta.get("row_gather"):
            raise RuntimeError("%s is stored row-gather-only and should never be loaded whole"
                               % key)
        t = torch.from_numpy(self.read(meta["blobs"]["raw"], verify=verify))
        dt = str(meta.get("dtype", "bfloat16")).replace("torch.", "")
        if t.dtype == torch.int16 and "bfloat16" in dt:
            return t.view(torch.bfloat16)
        dtype = getattr(torch, dt, None)
        return t.to(dtype) if isinstance(dtype, torch.dtype) else t

    def host_block(self, keys: list[str], pin: bool = True, verify: bool = False):
        """The compressed tensors ``keys`` (one decoder block) read from disk
        straight into one pinned HostBlock for LayerRing: per tensor, the
        sign/mantissa bytes and bitstreams in one read, the chunk offsets and
        lengths in another, each at the alignment the kernel reads it with;
        the LUTs go to host memory (they build the decode table). ``verify``
        checks every blob's CRC-32."""
        from .stream_ring import HostBlock

        metas = [self.tensors[k] for k in keys]
        for k, m in zip(keys, metas):
            if not m.get("compressed"):
                raise ValueError("tensor %r is stored raw; a HostBlock holds compressed tensors"
                                 % k)
        plan = HostBlock.plan([(int(m["blobs"]["sign_mantissa"]["nbytes"]),
                                int(m["blobs"]["packed"]["nbytes"]),
                                int(m["blobs"]["chunk_offsets"]["shape"][0]))
                               for m in metas])
        block = HostBlock.allocate(plan, pin=pin)
        host = block.buf.numpy()
        luts = []
        for (sm_at, pk_at, of_at, nb_at), m in zip(plan.spans, metas):
            b = m["blobs"]
            self._read_adjacent(host, [(b["sign_mantissa"], sm_at), (b["packed"], pk_at)], verify)
            self._read_adjacent(host, [(b["chunk_offsets"], of_at), (b["chunk_nbytes"], nb_at)],
                                verify)
            lut_arrays, _, _ = self.read_many([b["sym_lut"], b["len_lut"]], verify=verify)
            luts.append((np.ascontiguousarray(lut_arrays[0]), np.ascontiguousarray(lut_arrays[1]),
                         int(m["max_bits"])))
        block.describe([(int(m["chunk_size"]), int(m["n_symbols"]), tuple(m["shape"]))
                        for m in metas], luts)
        return block

    def _read_adjacent(self, host: np.ndarray, parts: list, verify: bool) -> None:
        """Blobs that lie back to back in weights.bin, read with one call
        when their places in ``host`` are back to back too."""
        (r0, at0), (r1, at1) = parts
        contiguous = (int(r0["offset"]) + int(r0["nbytes"]) == int(r1["offset"])
                      and at0 + int(r0["nbytes"]) == at1)
        if contiguous:
            n = int(r0["nbytes"]) + int(r1["nbytes"])
            self._readinto(int(r0["offset"]), memoryview(host[at0: at0 + n]))
        else:
            for ref, at in parts:
                self._readinto(int(ref["offset"]), memoryview(host[at: at + int(ref["nbytes"])]))
        if verify:
            for ref, at in parts:
                got = zlib.crc32(memoryview(host[at: at + int(ref["nbytes"])]))
                if got != ref.get("crc32", 0):
                    raise _crc_error(ref, got)

    def close(self) -> None:
        self._close_direct()
        self._fh.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def direct_readinto(pread, bounce: mmap.mmap, offset: int, view: memoryview,
                    alignment: int = DIRECT_ALIGNMENT) -> None:
    """view.nbytes bytes of the file from `offset` into `view`, through
    reads that are all aligned (offset, length and memory) to `alignment`:
    pread(buffer, file_offset) -> bytes read, as os.preadv on an O_DIRECT
    descriptor, into the page-aligned `bounce` buffer, whose part around
    each requested span is then copied out. A read that ends before the
    requested bytes (the end of the file) raises StoreError."""
    cap = (len(bounce) // alignment) * alignment
    n = view.nbytes
    got = 0
    with memoryview(bounce) as b:
        while got < n:
            pos = offset + got
            a0 = pos - pos % alignment
            lead = pos - a0
            want = min(n - got, cap - lead)
            span = -(-(lead + want) // alignment) * alignment
            r = pread(b[:span], a0)
            take = min(want, r - lead)
            if take <= 0:
                raise StoreError("short read at offset %d: wanted %d bytes, got %d"
                                 % (offset, n, got))
            view[got: got + take] = b[lead: lead + take]
            got += take


def verify_store(store_dir) -> tuple[bool, list[str]]:
    """Every blob against its manifest CRC-32 (binstore.py:222-247). Returns
    (ok, keys of the tensors with a bad blob)."""
    bad = []
    with StoreReader(store_dir) as reader:
        for key, meta in reader.tensors.items():
            for ref in meta.get("blobs", {}).values():
                if "crc32" not in ref:
                    continue
                try:
                    reader.read(ref, verify=True)
                except StoreError:
                    bad.append(key)
                    break
    return (not bad, bad)
