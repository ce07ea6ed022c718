"""Device-resident decode: the layer below the reference-shaped Python API.

``DeviceTensor`` holds one compressed tensor in HBM (bitstreams, chunk
offsets/lengths, sign/mantissa bytes and a decode-table blob).
``decode_bf16`` rebuilds any number of them with one kernel launch per
``MAX_TENSORS`` tensors, writing into caller-provided or fresh BF16 tensors,
on the current torch stream. No host synchronisation happens here.

Decode tables are keyed by codebook content (the stored LUT bytes and width),
so tensors that share a codebook share one device table, and a tensor can
never be decoded with another codebook's table.

A resident tensor may also carry a segment index (``build_index``): for each
168-bit segment its first codeword boundary, its chunk and its symbols' place
in a round of 512 segments, 4 bytes per segment, built once by the GPU from the
tensor itself. Decodes of a tensor with an index run in rounds of 512 segments
across chunk boundaries, with no speculative segment start, agreement check,
scan or compaction; the output is the same.
"""
from __future__ import annotations

import collections
import ctypes
import dataclasses
import hashlib
import threading
import weakref

import numpy as np
import torch

from .. import _native

MAX_TENSORS = _native.MAX_TENSORS


class DecodeTables(tuple):
    """Decode tables for one codebook.

    Unpacks like the reference's ``prepare_decode_tables`` result
    (afterimage/runtime/gpu_decode_v2.py:71-76): ``sym_lut, len_lut = tables``
    gives the flat LUTs as int32 tensors on the table's device (rebuilt from
    the blob, and only when read). The decoder itself reads ``blob``: the
    compact window table of ``aimg_build_table``, on the device (or on the
    host for the CPU decoder), shared by every tensor with this codebook.
    ``key`` is the SHA-256 of the codebook content; ``host_blob`` a host copy.
    """

    def __new__(cls, blob: torch.Tensor, max_bits: int, key: bytes, host_blob: np.ndarray):
        self = super().__new__(cls, ())
        self.blob = blob
        self.max_bits = int(max_bits)
        self.key = key
        self.host_blob = host_blob
        self._luts = None
        return self

    def _flat(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self._luts is None:
            sym, ln = flat_luts_from_blob(self.host_blob, self.max_bits)
            dev = self.blob.device
            self._luts = (torch.from_numpy(sym).to(dev), torch.from_numpy(ln).to(dev))
        return self._luts

    def __len__(self) -> int:
        return 2

    # A tuple built from () would compare and hash by that empty content:
    # tables are equal when they hold the same codebook on the same device.
    def __eq__(self, other) -> bool:
        if not isinstance(other, DecodeTables):
            return False
        return (self.key, self.max_bits, str(self.blob.device)) == \
            (other.key, other.max_bits, str(other.blob.device))

    def __ne__(self, other) -> bool:
        return not self.__eq__(other)

    def __hash__(self) -> int:
        return hash((self.key, self.max_bits, str(self.blob.device)))

    def __iter__(self):
        return iter(self._flat())

    def __getitem__(self, i):
        return self._flat()[i]

    def __repr__(self) -> str:
        return "DecodeTables(max_bits=%d, key=%s, device=%s)" % (
            self.max_bits, self.key.hex()[:12], self.blob.device)


def flat_luts_from_blob(blob: np.ndarray, max_bits: int) -> tuple[np.ndarray, np.ndarray]:
    """The flat (sym_lut, len_lut) of width ``max_bits`` that a table blob was
    built from, as int32 arrays (build_decode_lut's layout,
    afterimage/runtime/huffman.py:128-150: entry i is the codeword window i
    starts with; windows no codeword covers hold (0, 0))."""
    b = np.asarray(blob, dtype=np.uint8)
    hdr = b[:64].view(np.uint32)
    n_esc = int(hdr[6])
    wsyms = b[_SYMS_OFF:_META_OFF].view(np.uint32)
    wmeta = b[_META_OFF:_LEN_OFF]
    len_of = b[_LEN_OFF:_ESC_OFF].astype(np.int32)
    esc = b[_ESC_OFF:_ESC_OFF + 2 * 16 * n_esc].view(np.uint16).reshape(n_esc, 16)
    mb = int(max_bits)
    i = np.arange(1 << mb, dtype=np.int64)
    bits16 = (i << (16 - mb)) if mb <= 16 else i  # the window's first 16 bits
    w12 = (bits16 >> 4).astype(np.int64)
    meta = wmeta[w12]
    first = (wsyms[w12] & 0xFF).astype(np.int32)
    sym = np.where(meta != 0, first, 0).astype(np.int32)
    ln = np.where(meta != 0, len_of[first], 0).astype(np.int32)
    escw = meta == 0
    blk = (wsyms[w12] & 0xFFFF).astype(np.int64)
    use = escw & (blk != 0xFFFF) & (blk < n_esc)
    if use.any():
        v = esc[blk[use], (bits16[use] & 15)].astype(np.int32)
        sym[use] = np.where(v >> 8 != 0, v & 0xFF, 0)
        ln[use] = v >> 8
    return sym, ln


# Table blob layout (aimg_internal.h): 64-byte header, window symbols (uint32
# per 12-bit window), window meta (uint8), code length per symbol (256 B),
# escape blocks (16 uint16 entries each).
_SYMS_OFF = 64
_META_OFF = _SYMS_OFF + 4 * 4096
_LEN_OFF = _META_OFF + 4096
_ESC_OFF = _LEN_OFF + 256


def codebook_key(sym_lut: np.ndarray, len_lut: np.ndarray, max_bits: int) -> bytes:
    h = hashlib.sha256()
    h.update(np.int64(max_bits).tobytes())
    h.update(np.ascontiguousarray(sym_lut, dtype=np.int32).tobytes())
    h.update(np.ascontiguousarray(len_lut, dtype=np.int8).tobytes())
    return h.digest()


def build_table_blob(sym_lut: np.ndarray, len_lut: np.ndarray, max_bits: int) -> np.ndarray:
    """Host table blob for a stored LUT; raises NativeError on a bad LUT."""
    lib = _native.lib()
    size = 1 << int(max_bits) if 1 <= int(max_bits) <= 16 else 0
    sym = np.ascontiguousarray(sym_lut, dtype=np.int32)
    ln = np.ascontiguousarray(len_lut, dtype=np.int8)
    if sym.shape[0] < size or ln.shape[0] < size:
        raise ValueError("LUT has %d/%d entries, max_bits=%d needs %d"
                         % (sym.shape[0], ln.shape[0], max_bits, size))
    nbytes = ctypes.c_size_t(0)
    _native.check(lib.aimg_table_nbytes(int(max_bits), ctypes.byref(nbytes)))
    blob = np.zeros(nbytes.value, dtype=np.uint8)
    _native.check(lib.aimg_build_table(sym.ctypes.data, ln.ctypes.data, int(max_bits),
                                       blob.ctypes.data, blob.nbytes))
    return blob


class _TableCache:
    """LRU of decode tables keyed by (device, codebook content), bounded by the
    bytes of the tables it holds.

    A lookup first tries the LUT arrays' identity: the same pair of array
    objects (held by weak reference) at the same width returns its tables
    without reading the arrays again. Other arrays are keyed by a SHA-256 of
    their content, so equal codebooks share one table and different ones
    never collide. A LUT array changed in place after a lookup is not read
    again; pass a new array for a new codebook.

    Device tables are recorded on the current stream of every lookup, so an
    evicted table's memory is not reused while a launch queued on that
    stream may still read it.
    """

    def __init__(self, capacity_bytes: int = 64 << 20):
        self.capacity_bytes = capacity_bytes
        self._items: collections.OrderedDict = collections.OrderedDict()
        self._by_id: dict = {}
        self._lock = threading.Lock()
        self._bytes = 0
        self.builds = 0
        self.hashes = 0

    @staticmethod
    def _device(device) -> torch.device:
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        return dev

    def get(self, sym_lut, len_lut, max_bits: int, device) -> DecodeTables:
        dev = self._device(device)
        ident = (id(sym_lut), id(len_lut), int(max_bits), str(dev))
        with self._lock:
            hit = self._by_id.get(ident)
            if hit is not None:
                sref, lref, ckey = hit
                tables = self._items.get(ckey)
                if sref() is sym_lut and lref() is len_lut and tables is not None:
                    self._items.move_to_end(ckey)
                    self._record(tables, dev)
                    return tables
                del self._by_id[ident]
        key = codebook_key(sym_lut, len_lut, max_bits)
        ckey = (str(dev), key)
        with self._lock:
            self.hashes += 1
            tables = self._items.get(ckey)
        if tables is None:
            host = build_table_blob(sym_lut, len_lut, max_bits)
            blob = torch.from_numpy(host)
            if dev.type != "cpu":
                blob = blob.to(dev)
            tables = DecodeTables(blob, int(max_bits), key, host)
            with self._lock:
                self.builds += 1
                if ckey not in self._items:
                    self._items[ckey] = tables
                    self._bytes += blob.numel()
                tables = self._items[ckey]
                while self._bytes > self.capacity_bytes and len(self._items) > 1:
                    _, old = self._items.popitem(last=False)
                    self._bytes -= old.blob.numel()
        with self._lock:
            self._items.move_to_end(ckey)
            try:
                self._by_id[ident] = (weakref.ref(sym_lut), weakref.ref(len_lut), ckey)
            except TypeError:  # arrays without weak references: content key only
                pass
            if len(self._by_id) > 4 * max(1, len(self._items)) + 64:
                live = set(self._items)
                self._by_id = {k: v for k, v in self._by_id.items()
                               if v[2] in live and v[0]() is not None and v[1]() is not None}
        self._record(tables, dev)
        return tables

    @staticmethod
    def _record(tables: DecodeTables, dev: torch.device) -> None:
        if dev.type == "cuda":
            tables.blob.record_stream(torch.cuda.current_stream(dev))

    def clear(self) -> None:
        with self._lock:
            self._items.clear()
            self._by_id.clear()
            self._bytes = 0


TABLES = _TableCache()


@dataclasses.dataclass
class DeviceTensor:
    """One compressed tensor resident on the GPU."""

    packed: torch.Tensor          # uint8
    chunk_offsets: torch.Tensor   # int32
    chunk_nbytes: torch.Tensor    # int32
    sign_mantissa: torch.Tensor | None  # uint8[n_symbols] (None for exponent-only decode)
    tables: DecodeTables
    chunk_size: int
    n_symbols: int
    shape: tuple[int, ...]
    index: torch.Tensor | None = None  # uint8 segment index (build_index), or None
    # indexed_ranges' views, by their chunk ranges
    range_cache: dict = dataclasses.field(default_factory=dict, repr=False, compare=False)

    @property
    def n_chunks(self) -> int:
        return int(self.chunk_offsets.shape[0])

    @property
    def index_nbytes(self) -> int:
        """Bytes of this tensor's segment index (header, chunk bases and real
        ends, one 4-byte entry per segment, one 16-byte start per round of 512
        segments)."""
        n = ctypes.c_size_t(0)
        _native.check(_native.lib().aimg_index_nbytes(
            self.tables.host_blob.ctypes.data, int(self.packed.numel()), self.n_chunks,
            ctypes.byref(n)))
        return int(n.value)

    @property
    def index_bytes_read(self) -> int:
        """Index bytes a decode reads: the entries of the chunks' segments
        (4 bytes each), each chunk's first segment and real end, and the start
        of each round of 512 segments (0 without an index)."""
        if self.index is None:
            return 0
        seg = segment_bits(self.tables.host_blob)
        nb = self.chunk_nbytes.to(torch.int64)
        segments = int(((nb * 8 + seg - 1) // seg).sum().item())
        return 8 * self.n_chunks + 4 * segments + 16 * (segments // 512 + 1)

    @property
    def algorithmic_bytes(self) -> int:
        """Bytes one bf16 decode must move: chunk bitstreams, offsets and
        lengths, sign/mantissa read, window table, the segment index when the
        tensor has one, and the bf16 write."""
        return (int(self.chunk_nbytes.sum().item()) + 8 * self.n_chunks
                + self.n_symbols + (5 * 4096 + 256) + self.index_bytes_read
                + 2 * self.n_symbols)

    def build_index(self, keep_unusable: bool = False) -> "DeviceTensor":
        """Build this tensor's segment index on the current stream (one pass
        over its bitstreams, then a check of the result, which waits for
        it); later decodes use it. An index the build marks unusable (chunks
        not back to back in the packed buffer, or a chunk that does not hold
        its symbols) is dropped unless keep_unusable. Returns self."""
        build_indexes([self], keep_unusable)
        return self

    @property
    def index_usable(self) -> bool:
        return self.index is not None and \
            int(self.index[16:20].cpu().numpy().view(np.uint32)[0]) == 1

    def drop_index(self) -> None:
        """Free this tensor's segment index and the per-range indexes of
        indexed_ranges."""
        self.index = None
        self.range_cache.clear()

    def chunk_range(self, c0: int, c1: int) -> "DeviceTensor":
        """Chunks [c0, c1) as a tensor of their own, sharing this tensor's
        memory: chunk offsets point into the same packed buffer, and the
        sign/mantissa bytes are the range's slice. It holds the range's
        symbols, min(n_symbols, c1 * chunk_size) - c0 * chunk_size, and no
        segment index (an index covers a whole tensor)."""
        if not 0 <= c0 <= c1 <= self.n_chunks:
            raise ValueError("chunk range [%d, %d) outside [0, %d)" % (c0, c1, self.n_chunks))
        if c0 == 0 and c1 == self.n_chunks:
            return self
        base = c0 * self.chunk_size
        n = max(0, min(self.n_symbols, c1 * self.chunk_size) - base)
        sm = None if self.sign_mantissa is None else self.sign_mantissa[base: base + n]
        return DeviceTensor(packed=self.packed, chunk_offsets=self.chunk_offsets[c0:c1],
                            chunk_nbytes=self.chunk_nbytes[c0:c1], sign_mantissa=sm,
                            tables=self.tables, chunk_size=self.chunk_size, n_symbols=n,
                            shape=(n,))

    def indexed_ranges(self, ranges: list[tuple[int, int]]) -> list["DeviceTensor"]:
        """Chunk ranges as tensors that each carry a segment index of their
        own, built now (one batched build and one wait): each range's
        packed bytes are a view of this tensor's packed buffer that spans its
        chunks' bytes, starting on a 16-byte boundary, and its chunk offsets
        are rebased to that view (a new int32 array per range), so that an
        index holds only the range's segments. The views are cached
        on this tensor by their ranges. An index needs the range's chunks
        back to back in the packed buffer; a range whose index comes out
        unusable decodes without one."""
        key = tuple((int(a), int(b)) for a, b in ranges)
        hit = self.range_cache.get(key)
        if hit is not None:
            return hit
        offs = self.chunk_offsets.cpu().numpy().astype(np.int64)
        lens = self.chunk_nbytes.cpu().numpy().astype(np.int64)
        views = []
        for c0, c1 in key:
            v = self.chunk_range(c0, c1)
            if v is self or c1 <= c0:
                views.append(v)
                continue
            # The view spans every byte of the range's chunks (wherever they
            # lie in the buffer) and starts on the 16-byte boundary at or
            # before the first, so its base keeps the buffer's alignment.
            lo = int(offs[c0:c1].min()) & ~15
            hi = int((offs[c0:c1] + np.maximum(lens[c0:c1], 0)).max())
            if not 0 <= lo <= hi <= self.packed.numel():
                raise ValueError("chunks %d..%d lie outside the packed buffer" % (c0, c1 - 1))
            v.packed = self.packed[lo:hi]
            v.chunk_offsets = (self.chunk_offsets[c0:c1] - lo).contiguous()
            views.append(v)
        build_indexes([v for v in views if v is not self and v.n_chunks > 0])
        self.range_cache[key] = views
        return views

    @classmethod
    def from_encoded(cls, enc, sign_mantissa, device, tables: DecodeTables | None = None):
        """Upload a ChunkedEncoded (+ sign/mantissa bytes) to ``device``."""
        if tables is None:
            tables = TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, device)
        sm = None
        if sign_mantissa is not None:
            sm = torch.as_tensor(sign_mantissa).reshape(-1).to(device=device, dtype=torch.uint8)
        return cls(
            packed=_on_device(enc.packed, torch.uint8, device),
            chunk_offsets=_on_device(enc.chunk_offsets, torch.int32, device),
            chunk_nbytes=_on_device(enc.chunk_nbytes, torch.int32, device),
            sign_mantissa=sm, tables=tables, chunk_size=int(enc.chunk_size),
            n_symbols=int(enc.n_symbols), shape=tuple(enc.shape))


def _on_device(a, dtype: torch.dtype, device) -> torch.Tensor:
    """A 1-D contiguous ``dtype`` tensor on ``device`` with a's values: a
    tensor already there is used as it is (a layer kept resident in HBM is
    not copied again), a host array or tensor is copied."""
    if isinstance(a, torch.Tensor):
        return a.reshape(-1).to(device=device, dtype=dtype).contiguous()
    np_dtype = {torch.uint8: np.uint8, torch.int32: np.int32}[dtype]
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a).reshape(-1), dtype=np_dtype)).to(device)


def build_indexes(tensors: list[DeviceTensor], keep_unusable: bool = False) -> None:
    """Build the segment indexes of resident tensors on one device, up to
    MAX_TENSORS per aimg_build_index call, then wait once and drop (unless
    keep_unusable) every index the build marked unusable."""
    if not tensors:
        return
    dev = tensors[0].packed.device
    if dev.type != "cuda":
        raise RuntimeError("the segment index is built on the GPU; tensor is on %s" % dev)
    ixs = []
    lib = _native.lib()
    for i in range(0, len(tensors), MAX_TENSORS):
        group = tensors[i: i + MAX_TENSORS]
        d = (_native.AimgTensor * len(group))()
        for j, t in enumerate(group):
            if t.packed.device != dev:
                raise ValueError("tensors on %s and %s" % (dev, t.packed.device))
            ix = torch.empty(t.index_nbytes, dtype=torch.uint8, device=dev)
            d[j] = _descriptor(t, None, t.n_symbols)
            d[j].index = ix.data_ptr()
            d[j].index_nbytes = int(ix.numel())
            ixs.append(ix)
        with torch.cuda.device(dev):
            _native.check(lib.aimg_build_index(d, len(group), _stream_handle(dev)))
    ok = torch.stack([ix[16:20] for ix in ixs]).cpu().numpy().view(np.uint32).reshape(-1)
    for t, ix, flag in zip(tensors, ixs, ok):
        t.index = ix if flag == 1 or keep_unusable else None


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(torch.device(device)).cuda_stream


def segment_bits(host_blob: np.ndarray) -> int:
    """Bits per decode segment for a table blob: 84 codewords of its shortest
    length, at most 168, a whole number of bytes."""
    min_len = max(1, int(np.frombuffer(host_blob[12:16].tobytes(), np.uint32)[0]))
    return min(84 * min_len, 168) & ~7


def _descriptor(t: DeviceTensor, out: torch.Tensor | None, n_out: int) -> _native.AimgTensor:
    d = _native.AimgTensor()
    d.packed = t.packed.data_ptr()
    d.chunk_offsets = t.chunk_offsets.data_ptr()
    d.chunk_nbytes = t.chunk_nbytes.data_ptr()
    d.sign_mantissa = t.sign_mantissa.data_ptr() if t.sign_mantissa is not None else None
    d.out = out.data_ptr() if out is not None else None
    d.table = t.tables.blob.data_ptr()
    if t.index is not None:
        d.index = t.index.data_ptr()
        d.index_nbytes = int(t.index.numel())
    d.packed_nbytes = int(t.packed.numel())
    d.n_symbols = int(n_out)
    d.chunk_size = int(t.chunk_size)
    d.n_chunks = t.n_chunks
    return d


def _check_device(t: DeviceTensor, out: torch.Tensor) -> None:
    dev = out.device
    if dev.type != "cuda":
        raise RuntimeError("the decoder writes GPU memory only; got output on %s" % dev)
    for name in ("packed", "chunk_offsets", "chunk_nbytes"):
        x = getattr(t, name)
        if x.device != dev or not x.is_contiguous():
            raise ValueError("%s must be contiguous on %s" % (name, dev))
    if t.tables.blob.device != dev:
        raise ValueError("decode tables live on %s, output on %s" % (t.tables.blob.device, dev))


def decode_bf16(tensors: list[DeviceTensor], outs: list[torch.Tensor] | None = None,
                device=None) -> list[torch.Tensor]:
    """Rebuild bf16 tensors (flat, n_symbols each) on the current stream."""
    if not tensors:
        return []
    if outs is None:
        dev = device if device is not None else tensors[0].packed.device
        outs = [torch.empty(t.n_symbols, dtype=torch.bfloat16, device=dev) for t in tensors]
    lib = _native.lib()
    for i in range(0, len(tensors), MAX_TENSORS):
        group = tensors[i: i + MAX_TENSORS]
        gouts = outs[i: i + MAX_TENSORS]
        arr = (_native.AimgTensor * len(group))()
        for j, (t, o) in enumerate(zip(group, gouts)):
            _check_device(t, o)
            if o.dtype != torch.bfloat16 or not o.is_contiguous() or o.numel() < t.n_symbols:
                raise ValueError("output %d must be a contiguous bf16 tensor of >= %d elements"
                                 % (i + j, t.n_symbols))
            if t.sign_mantissa is None or t.sign_mantissa.numel() < t.n_symbols \
                    or t.sign_mantissa.device != o.device:
                raise ValueError("tensor %d needs sign_mantissa bytes on %s" % (i + j, o.device))
            arr[j] = _descriptor(t, o, t.n_symbols)
        with torch.cuda.device(gouts[0].device):
            _native.check(lib.aimg_decode_bf16(arr, len(group), _stream_handle(gouts[0].device)))
    return outs


def decode_u8(tensors: list[DeviceTensor], n_out: list[int] | None = None,
              outs: list[torch.Tensor] | None = None, device=None) -> list[torch.Tensor]:
    """Decode exponent bytes only; ``n_out[i]`` may extend into the padded
    tail of the last chunk (up to n_chunks * chunk_size)."""
    if not tensors:
        return []
    if n_out is None:
        n_out = [t.n_symbols for t in tensors]
    if outs is None:
        dev = device if device is not None else tensors[0].packed.device
        outs = [torch.empty(k, dtype=torch.uint8, device=dev) for k in n_out]
    lib = _native.lib()
    for i in range(0, len(tensors), MAX_TENSORS):
        group = tensors[i: i + MAX_TENSORS]
        gouts = outs[i: i + MAX_TENSORS]
        arr = (_native.AimgTensor * len(group))()
        for j, (t, o) in enumerate(zip(group, gouts)):
            _check_device(t, o)
            k = n_out[i + j]
            if o.dtype != torch.uint8 or not o.is_contiguous() or o.numel() < k:
                raise ValueError("output %d must be a contiguous uint8 tensor of >= %d elements"
                                 % (i + j, k))
            arr[j] = _descriptor(t, o, k)
        with torch.cuda.device(gouts[0].device):
            _native.check(lib.aimg_decode_u8(arr, len(group), _stream_handle(gouts[0].device)))
    return outs


GEMV_MAX_BATCH = 4
GEMM_MAX_ROWS = 16


def decode_gemv(t: DeviceTensor, x: torch.Tensor, rows: int, cols: int,
                y: torch.Tensor | None = None) -> torch.Tensor:
    """y += x @ W.T in fp32 for the rows x cols bf16 matrix W held by ``t``,
    decoded inside the kernel and never written. x: bf16 [b, cols] on the
    GPU (b <= GEMV_MAX_BATCH); y: fp32 [b, rows], zeros when not given.
    Returns y. The fp32 sums are added with atomics, so their order (and
    the last bits of y) can vary between calls."""
    return _fused(t, x, rows, cols, y, GEMV_MAX_BATCH, "aimg_decode_gemv_bf16")


def decode_gemm(t: DeviceTensor, x: torch.Tensor, rows: int, cols: int,
                y: torch.Tensor | None = None) -> torch.Tensor:
    """decode_gemv for 1..GEMM_MAX_ROWS rows of x (speculative-verify
    widths), on the matrix cores: bf16 products, fp32 sums, W decoded inside
    the kernel and never written. Needs cols % 8 == 0 and chunks of 1024 to
    2^24 symbols (a multiple of 8); other layers raise (the blocked
    decode_linear serves them)."""
    return _fused(t, x, rows, cols, y, GEMM_MAX_ROWS, "aimg_decode_gemm_bf16")


def _fused(t: DeviceTensor, x: torch.Tensor, rows: int, cols: int, y: torch.Tensor | None,
           max_b: int, entry: str) -> torch.Tensor:
    dev = x.device
    if dev.type != "cuda":
        raise RuntimeError("the decoder runs on the GPU only; got x on %s" % dev)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.shape[1] != cols or not x.is_contiguous():
        raise ValueError("x must be a contiguous bf16 [batch, %d] tensor" % cols)
    b = int(x.shape[0])
    if not 1 <= b <= max_b:
        raise ValueError("batch must be in 1..%d, got %d" % (max_b, b))
    if rows * cols != t.n_symbols:
        raise ValueError("rows * cols = %d, the tensor has %d weights" % (rows * cols, t.n_symbols))
    if y is None:
        y = torch.zeros((b, rows), dtype=torch.float32, device=dev)
    elif y.dtype != torch.float32 or tuple(y.shape) != (b, rows) or not y.is_contiguous():
        raise ValueError("y must be a contiguous fp32 [%d, %d] tensor" % (b, rows))
    if t.sign_mantissa is None or t.sign_mantissa.device != dev:
        raise ValueError("the tensor needs sign_mantissa bytes on %s" % dev)
    _check_device(t, y)
    d = (_native.AimgTensor * 1)()
    d[0] = _descriptor(t, y, t.n_symbols)
    d[0].out = None
    with torch.cuda.device(dev):
        _native.check(getattr(_native.lib(), entry)(
            d, rows, cols, x.data_ptr(), b, y.data_ptr(), _stream_handle(dev)))
    return y


def row_blocks(rows: int, cols: int, chunk_size: int, n_chunks: int, slice_rows: int):
    """The blocks of a blocked x @ W.T: (r0, r1, c0, c1) for each block of
    slice_rows rows (the last one shorter), with [c0, c1) the chunks that
    hold its elements [r0 * cols, r1 * cols). slice_rows <= 0: one block of
    all rows (no row blocking, as the reference's lm_head_slice_rows = 0)."""
    step = int(slice_rows) if int(slice_rows) > 0 else max(1, int(rows))
    out = []
    for r0 in range(0, rows, step):
        r1 = min(r0 + step, rows)
        c0 = (r0 * cols) // chunk_size
        c1 = min(n_chunks, -(-(r1 * cols) // chunk_size))
        out.append((r0, r1, c0, c1))
    return out


def decode_linear(t: DeviceTensor, x: torch.Tensor, rows: int, cols: int,
                  slice_rows: int, staging: torch.Tensor | None = None) -> torch.Tensor:
    """torch.nn.functional.linear(x, W) for the rows x cols bf16 weight W held
    by ``t``, slice_rows rows of W at a time: each block's chunks are decoded
    into one staging buffer, which every block reuses, the GEMM library
    multiplies x by the block, and the blocks' outputs are concatenated along
    the last dimension. This is the blocked lm_head projection of
    streaming_engine.py:2307-2332 (decompress_rows_gpu, F.linear, torch.cat):
    the same calls on the same bytes, at the same offsets from a buffer
    start, so the same result, with one buffer of about slice_rows * cols
    weights live instead of one per block. When ``t`` has a segment index,
    each block decodes through an index of its own (indexed_ranges, built on
    the first call for these blocks). Runs on the current stream."""
    dev = x.device
    if dev.type != "cuda":
        raise RuntimeError("the decoder runs on the GPU only; got x on %s" % dev)
    if x.dim() < 1 or x.shape[-1] != cols:
        raise ValueError("x must end in a dimension of %d, got shape %s" % (cols, tuple(x.shape)))
    if rows * cols != t.n_symbols:
        raise ValueError("rows * cols = %d, the tensor has %d weights" % (rows * cols, t.n_symbols))
    blocks = row_blocks(rows, cols, t.chunk_size, t.n_chunks, slice_rows)
    if not blocks:
        return torch.nn.functional.linear(
            x, torch.empty((0, cols), dtype=torch.bfloat16, device=dev))
    need = max(min(t.n_symbols, c1 * t.chunk_size) - c0 * t.chunk_size
               for _, _, c0, c1 in blocks)
    if staging is None:
        staging = torch.empty(need, dtype=torch.bfloat16, device=dev)
    elif staging.dtype != torch.bfloat16 or staging.device != dev or \
            not staging.is_contiguous() or staging.numel() < need:
        raise ValueError("staging must be a contiguous bf16 tensor of >= %d elements on %s"
                         % (need, dev))
    # A tensor with a segment index decodes its blocks through indexes of
    # their own (built on the first call for these blocks, then cached).
    ranges = [(c0, c1) for _, _, c0, c1 in blocks]
    views = t.indexed_ranges(ranges) if t.index is not None else \
        [t.chunk_range(c0, c1) for c0, c1 in ranges]
    parts = []
    for (r0, r1, c0, _), part in zip(blocks, views):
        decode_bf16([part], [staging])
        e0 = r0 * cols - c0 * t.chunk_size
        w = staging[e0: e0 + (r1 - r0) * cols].view(r1 - r0, cols)
        parts.append(torch.nn.functional.linear(x, w))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)



# ---------------------------------------------------------------------------
# Host (CPU) decode through the same library: aimg_cpu_decode_bf16 / _u8.
# ---------------------------------------------------------------------------

def host_array(a, dtype) -> np.ndarray:
    """A C-contiguous, aligned host array of ``dtype`` with a's values: ``a``
    itself when it already is one (for example a view into a store buffer),
    otherwise a copy. Accepts numpy arrays and CPU tensors."""
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.require(a, dtype=dtype, requirements=["C", "A"])


def default_threads() -> int:
    """Threads for a host decode: torch's intra-op thread count (which follows
    OMP_NUM_THREADS), so the decoder shares the CPU budget torch was given."""
    return max(1, torch.get_num_threads())


def cpu_decode(parts, n_threads: int | None = None, exponents_only: bool = False) -> None:
    """Decode on the CPU threads of the native library.

    ``parts``: (enc, sign_mantissa, out, n_out) per tensor, where ``enc`` is a
    ChunkedEncoded (host arrays), ``out`` a contiguous CPU tensor (bf16, or
    uint8 with ``exponents_only``) of at least n_out elements, and
    ``sign_mantissa`` the host bytes of elements [0, n_out) (ignored with
    ``exponents_only``). Returns when the outputs are written."""
    parts = list(parts)
    if not parts:
        return
    keep = []
    arr = (_native.AimgTensor * len(parts))()
    for j, (enc, sm, out, n_out) in enumerate(parts):
        if out.device.type != "cpu" or not out.is_contiguous() or out.numel() < n_out:
            raise ValueError("output %d must be a contiguous CPU tensor of >= %d elements" % (j, n_out))
        want = torch.uint8 if exponents_only else torch.bfloat16
        if out.dtype != want:
            raise ValueError("output %d must be %s" % (j, want))
        if n_out > int(enc.n_chunks) * int(enc.chunk_size):
            raise ValueError("tensor %d: %d outputs exceed its %d chunks" % (j, n_out, enc.n_chunks))
        tables = TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, "cpu")
        packed = host_array(enc.packed, np.uint8)
        offs = host_array(enc.chunk_offsets, np.int32)
        nbytes = host_array(enc.chunk_nbytes, np.int32)
        if offs.shape[0] < enc.n_chunks or nbytes.shape[0] < enc.n_chunks:
            raise ValueError("tensor %d: chunk tables shorter than n_chunks" % j)
        smh = None
        if not exponents_only:
            smh = host_array(sm, np.uint8).reshape(-1)
            if smh.shape[0] < n_out:
                raise ValueError("tensor %d needs %d sign/mantissa bytes, got %d"
                                 % (j, n_out, smh.shape[0]))
        keep.append((packed, offs, nbytes, smh, tables))
        d = arr[j]
        d.packed = packed.ctypes.data if packed.size else None
        d.chunk_offsets = offs.ctypes.data
        d.chunk_nbytes = nbytes.ctypes.data
        d.sign_mantissa = smh.ctypes.data if smh is not None else None
        d.out = out.data_ptr()
        d.table = tables.blob.data_ptr()
        d.packed_nbytes = int(packed.size)
        d.n_symbols = int(n_out)
        d.chunk_size = int(enc.chunk_size)
        d.n_chunks = int(enc.n_chunks)
    threads = default_threads() if n_threads is None else int(n_threads)
    fn = _native.lib().aimg_cpu_decode_u8 if exponents_only else _native.lib().aimg_cpu_decode_bf16
    _native.check(fn(arr, len(parts), threads))
    del keep


def recombine_bf16(exponent: torch.Tensor, sign_mantissa: torch.Tensor) -> torch.Tensor:
    """bf16 bits ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F) of two uint8
    tensors on one device (GPU: one kernel on the current stream; CPU: the
    library's host loop). Returns a flat bf16 tensor on that device."""
    e = exponent.reshape(-1)
    sm = sign_mantissa.reshape(-1)
    if e.dtype != torch.uint8 or sm.dtype != torch.uint8:
        raise ValueError("exponent and sign_mantissa must be uint8")
    if e.numel() != sm.numel():
        raise ValueError("exponent has %d elements, sign_mantissa %d" % (e.numel(), sm.numel()))
    if e.device != sm.device:
        raise ValueError("exponent on %s, sign_mantissa on %s" % (e.device, sm.device))
    e = e.contiguous()
    sm = sm.contiguous()
    out = torch.empty(e.numel(), dtype=torch.bfloat16, device=e.device)
    if e.numel() == 0:
        return out
    lib = _native.lib()
    if e.device.type == "cuda":
        with torch.cuda.device(e.device):
            _native.check(lib.aimg_recombine_bf16(e.data_ptr(), sm.data_ptr(), out.data_ptr(),
                                                  e.numel(), _stream_handle(e.device)))
    elif e.device.type == "cpu":
        _native.check(lib.aimg_cpu_recombine_bf16(e.data_ptr(), sm.data_ptr(), out.data_ptr(),
                                                  e.numel()))
    else:
        raise RuntimeError("recombine runs on a GPU or the CPU; got %s" % e.device)
    return out
