"""Device-resident decode: the layer below the reference-shaped Python API.

``DeviceTensor`` holds one compressed tensor in HBM (bitstreams, chunk
offsets/lengths, sign/mantissa bytes and a decode-table blob).
``decode_bf16`` rebuilds any number of them with one kernel launch per
``MAX_TENSORS`` tensors, writing into caller-provided or fresh BF16 tensors,
on the current torch stream. No host synchronisation happens here.

Decode tables are keyed by codebook content (the stored LUT bytes and width),
so tensors that share a codebook share one device table, and a tensor can
never be decoded with another codebook's table.
"""
from __future__ import annotations

import collections
import ctypes
import dataclasses
import hashlib
import threading

import numpy as np
import torch

from .. import _native

MAX_TENSORS = _native.MAX_TENSORS


class DecodeTables(tuple):
    """Device decode tables for one codebook: ``(blob, max_bits, key)``."""

    __slots__ = ()

    def __new__(cls, blob: torch.Tensor, max_bits: int, key: bytes):
        return super().__new__(cls, (blob, max_bits, key))

    @property
    def blob(self) -> torch.Tensor:
        return self[0]

    @property
    def max_bits(self) -> int:
        return self[1]

    @property
    def key(self) -> bytes:
        return self[2]


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
    """Small LRU of device tables keyed by (device, codebook content)."""

    def __init__(self, capacity: int = 64):
        self.capacity = capacity
        self._items: collections.OrderedDict = collections.OrderedDict()
        self._lock = threading.Lock()
        self.builds = 0

    def get(self, sym_lut, len_lut, max_bits: int, device) -> DecodeTables:
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        key = codebook_key(sym_lut, len_lut, max_bits)
        with self._lock:
            hit = self._items.get((str(dev), key))
            if hit is not None:
                self._items.move_to_end((str(dev), key))
                return hit
        blob = build_table_blob(sym_lut, len_lut, max_bits)
        tables = DecodeTables(torch.from_numpy(blob).to(dev), int(max_bits), key)
        with self._lock:
            self.builds += 1
            self._items[(str(dev), key)] = tables
            while len(self._items) > self.capacity:
                self._items.popitem(last=False)
        return tables

    def clear(self) -> None:
        with self._lock:
            self._items.clear()


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

    @property
    def n_chunks(self) -> int:
        return int(self.chunk_offsets.shape[0])

    @property
    def algorithmic_bytes(self) -> int:
        """Bytes one bf16 decode must move: chunk bitstreams, offsets and
        lengths, sign/mantissa read, window table, and the bf16 write."""
        return (int(self.chunk_nbytes.sum().item()) + 8 * self.n_chunks
                + self.n_symbols + (5 * 4096 + 256) + 2 * self.n_symbols)

    @classmethod
    def from_encoded(cls, enc, sign_mantissa, device, tables: DecodeTables | None = None):
        """Upload a ChunkedEncoded (+ sign/mantissa bytes) to ``device``."""
        if tables is None:
            tables = TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, device)
        sm = None
        if sign_mantissa is not None:
            sm = torch.as_tensor(sign_mantissa).reshape(-1).to(device=device, dtype=torch.uint8)
        return cls(
            packed=torch.from_numpy(np.ascontiguousarray(enc.packed)).to(device),
            chunk_offsets=torch.from_numpy(
                np.ascontiguousarray(enc.chunk_offsets, dtype=np.int32)).to(device),
            chunk_nbytes=torch.from_numpy(
                np.ascontiguousarray(enc.chunk_nbytes, dtype=np.int32)).to(device),
            sign_mantissa=sm, tables=tables, chunk_size=int(enc.chunk_size),
            n_symbols=int(enc.n_symbols), shape=tuple(enc.shape))


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(torch.device(device)).cuda_stream


def _descriptor(t: DeviceTensor, out: torch.Tensor, n_out: int) -> _native.AimgTensor:
    d = _native.AimgTensor()
    d.packed = t.packed.data_ptr()
    d.chunk_offsets = t.chunk_offsets.data_ptr()
    d.chunk_nbytes = t.chunk_nbytes.data_ptr()
    d.sign_mantissa = t.sign_mantissa.data_ptr() if t.sign_mantissa is not None else None
    d.out = out.data_ptr()
    d.table = t.tables.blob.data_ptr()
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


def decode_gemv(t: DeviceTensor, x: torch.Tensor, rows: int, cols: int,
                y: torch.Tensor | None = None) -> torch.Tensor:
    """y += x @ W.T in fp32 for the rows x cols bf16 matrix W held by ``t``,
    decoded inside the kernel and never written. x: bf16 [b, cols] on the
    GPU (b <= GEMV_MAX_BATCH); y: fp32 [b, rows], zeros when not given.
    Returns y. The fp32 sums are added with atomics, so their order (and
    the last bits of y) can vary between calls."""
    dev = x.device
    if dev.type != "cuda":
        raise RuntimeError("the decoder runs on the GPU only; got x on %s" % dev)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.shape[1] != cols or not x.is_contiguous():
        raise ValueError("x must be a contiguous bf16 [batch, %d] tensor" % cols)
    b = int(x.shape[0])
    if not 1 <= b <= GEMV_MAX_BATCH:
        raise ValueError("batch must be in 1..%d, got %d" % (GEMV_MAX_BATCH, b))
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
        _native.check(_native.lib().aimg_decode_gemv_bf16(
            d, rows, cols, x.data_ptr(), b, y.data_ptr(), _stream_handle(dev)))
    return y

