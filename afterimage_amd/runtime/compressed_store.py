"""BF16 tensor <-> (sign/mantissa bytes, chunked Huffman exponents), with the
reference's API (afterimage/runtime/compressed_store.py:28-303).

bf16 bit layout, MSB to LSB: [sign:1][exponent:8][mantissa:7]. The stored
sign/mantissa byte is (sign << 7) | mantissa; the exponent byte is
entropy-coded. Decompression runs one fused gfx950 kernel per slice: Huffman
decode of the exponents and the bit recombine
``((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F)`` write the bf16 output directly,
so no exponent scratch tensor and no chain of elementwise torch kernels exist.
With ``device="cpu"`` the same decode runs on the library's CPU threads, as the
reference decodes on the CPU for a CPU device (compressed_store.py:171-180).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch

from .device import (GEMM_MAX_ROWS, GEMV_MAX_BATCH, DeviceTensor, cpu_decode, decode_bf16,
                     decode_gemm, decode_gemv, decode_linear, recombine_bf16)
from .huffman_chunked import ChunkedEncoded, encode_chunked, lengths_from_counts, symbol_counts

EXPONENT_SHIFT = 7


@dataclasses.dataclass
class CompressedLayer:
    """(compressed_store.py:28-42)"""

    sign_mantissa: torch.Tensor  # uint8, flat, CPU
    encoded: ChunkedEncoded      # entropy-coded exponent field
    shape: tuple[int, ...]

    @property
    def compressed_bytes(self) -> int:
        return (self.sign_mantissa.numel() + self.encoded.packed.nbytes
                + self.encoded.sym_lut.nbytes + self.encoded.len_lut.nbytes)

    @property
    def original_bytes(self) -> int:
        return self.sign_mantissa.numel() * 2


def split_fields(bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(exponent, sign_mantissa) bytes of bf16 words given as uint16."""
    exponent = ((bits >> EXPONENT_SHIFT) & 0xFF).astype(np.uint8)
    sign_mantissa = (((bits >> 8) & 0x80) | (bits & 0x7F)).astype(np.uint8)
    return exponent, sign_mantissa


def _split_weight(W: torch.Tensor, work_chunk_elems: int) -> tuple[np.ndarray, np.ndarray]:
    assert W.dtype == torch.bfloat16, f"expected bfloat16, got {W.dtype}"
    if work_chunk_elems < 1:
        raise ValueError("work_chunk_elems must be positive")
    raw = W.detach().contiguous().cpu().view(torch.int16).reshape(-1).numpy().view(np.uint16)
    n = raw.shape[0]
    exponent = np.empty(n, dtype=np.uint8)
    sign_mantissa = np.empty(n, dtype=np.uint8)
    for start in range(0, n, work_chunk_elems):
        end = min(start + work_chunk_elems, n)
        exponent[start:end], sign_mantissa[start:end] = split_fields(raw[start:end])
    return exponent, sign_mantissa


def compress_layer(W: torch.Tensor, chunk_size: int = 1024, max_bits: int = 16,
                   work_chunk_elems: int = 1 << 24, *,
                   lengths: dict[int, int] | None = None) -> CompressedLayer:
    """Field split + chunked encode (compressed_store.py:48-91).

    The split runs in bounded pieces of ``work_chunk_elems`` so no full-size
    integer temporaries are built for large matrices. ``lengths``
    (keyword-only, not in the reference) encodes with a given codebook; see
    compress_group.
    """
    exponent, sign_mantissa = _split_weight(W, work_chunk_elems)
    encoded = encode_chunked(exponent, chunk_size=chunk_size, max_bits=max_bits,
                             lengths=lengths)
    return CompressedLayer(sign_mantissa=torch.from_numpy(sign_mantissa), encoded=encoded,
                           shape=tuple(W.shape))


def compress_group(weights: list[torch.Tensor], chunk_size: int = 1024, max_bits: int = 16,
                   work_chunk_elems: int = 1 << 24) -> list[CompressedLayer]:
    """Compress several tensors with one exponent codebook built from their
    pooled histogram (for example all tensors of one role in a decoder block),
    so they share one stored LUT and one device decode table. Each tensor's
    stream decodes exactly as if it had been encoded alone with that LUT."""
    split = [_split_weight(W, work_chunk_elems) for W in weights]
    counts = np.zeros(256, dtype=np.int64)
    for exponent, _ in split:
        counts += symbol_counts(exponent)
    lengths = lengths_from_counts(counts, max_bits)
    return [CompressedLayer(sign_mantissa=torch.from_numpy(sm),
                            encoded=encode_chunked(e, chunk_size=chunk_size, max_bits=max_bits,
                                                   lengths=lengths),
                            shape=tuple(W.shape))
            for W, (e, sm) in zip(weights, split)]


def _recombine(exponent: torch.Tensor, sign_mantissa: torch.Tensor,
               shape: tuple) -> torch.Tensor:
    """bf16 tensor of ``shape`` from decoded exponents and sign/mantissa bytes
    (the role of compressed_store.py:94-114), in one native pass: a gfx950
    kernel for GPU tensors, the library's host loop for CPU tensors. Exponents
    of another integer dtype are taken modulo 256 (they are bytes)."""
    e = exponent if exponent.dtype == torch.uint8 else exponent.to(torch.uint8)
    sm = sign_mantissa if sign_mantissa.dtype == torch.uint8 else sign_mantissa.to(torch.uint8)
    return recombine_bf16(e, sm).reshape(shape)


def recombine_exponent_and_sign_mantissa(exponent, sign_mantissa, shape: tuple,
                                         device: str) -> torch.Tensor:
    """Combine already-decoded exponents with sign/mantissa bytes
    (compressed_store.py:117-130): numpy arrays or tensors on any device are
    moved to ``device`` first, then combined there."""
    exp = torch.as_tensor(exponent, device=device)
    sm = torch.as_tensor(sign_mantissa, device=device)
    return _recombine(exp, sm, shape)


def _slice_encoded(enc: ChunkedEncoded, c0: int, c1: int) -> ChunkedEncoded:
    """Chunks [c0, c1) as a standalone ChunkedEncoded (compressed_store.py:133-158):
    the byte range plus up to 8 following bytes, offsets rebased, and
    ``n_symbols`` counting whole chunks."""
    byte_start = int(enc.chunk_offsets[c0])
    nbytes = enc.chunk_nbytes[c0:c1]
    byte_end = int(enc.chunk_offsets[c1 - 1]) + int(nbytes[-1])
    byte_end = min(byte_end + 8, enc.packed.shape[0])
    return ChunkedEncoded(
        packed=enc.packed[byte_start:byte_end],
        chunk_offsets=(enc.chunk_offsets[c0:c1] - byte_start),
        chunk_nbytes=nbytes,
        sym_lut=enc.sym_lut,
        len_lut=enc.len_lut,
        max_bits=enc.max_bits,
        chunk_size=enc.chunk_size,
        n_symbols=(c1 - c0) * enc.chunk_size,
        shape=((c1 - c0) * enc.chunk_size,),
    )


def _is_cpu(device) -> bool:
    return torch.device(device).type == "cpu"


def _gpu_device(device) -> torch.device:
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(
            "the gfx950 decoder runs on a GPU (device %r); use device='cpu' for the "
            "CPU decoder" % (str(device),))
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _decode_cpu_into(layer: CompressedLayer, c0: int, c1: int, out_flat: torch.Tensor,
                     take: int) -> None:
    """Decode chunks [c0, c1) of ``layer`` on the CPU into ``out_flat[:take]``."""
    enc = layer.encoded
    sub = enc if (c0 == 0 and c1 == enc.n_chunks) else _slice_encoded(enc, c0, c1)
    s0 = c0 * enc.chunk_size
    sm = layer.sign_mantissa.reshape(-1)[s0: s0 + take]
    cpu_decode([(sub, sm, out_flat, take)])


def _tables_for(enc: ChunkedEncoded, dev: torch.device):
    from . import gpu_decode_v2  # attribute looked up at call time

    return gpu_decode_v2.prepare_decode_tables(enc, dev)


def _decode_range_into(layer: CompressedLayer, c0: int, c1: int, out_flat: torch.Tensor,
                       take: int, dev: torch.device, tables) -> None:
    """Decode chunks [c0, c1) of ``layer`` into ``out_flat[:take]``."""
    enc = layer.encoded
    sub = enc if (c0 == 0 and c1 == enc.n_chunks) else _slice_encoded(enc, c0, c1)
    s0 = c0 * enc.chunk_size
    sm = layer.sign_mantissa.reshape(-1)[s0: s0 + take]
    dt = DeviceTensor.from_encoded(sub, sm, dev, tables=tables)
    dt.n_symbols = take
    decode_bf16([dt], [out_flat])


def decompress_layer_gpu(layer: CompressedLayer, device: str = "cuda",
                         max_slice_elems: int = 1 << 25, *,
                         reuse_decode_tables: bool = False) -> torch.Tensor:
    """The exact original bf16 tensor, decoded on ``device``
    (compressed_store.py:186-240).

    Tensors above ``max_slice_elems`` elements are processed in chunk-range
    slices, bounding the staged compressed input to one slice; the output is
    written in place slice by slice. With ``reuse_decode_tables`` the tables
    are prepared once for the whole call; otherwise once per slice (both go
    through the content-keyed table cache). Work is ordered on the current
    stream of ``device``. As in the reference, the call synchronises the
    device before it returns unless ``reuse_decode_tables`` is set
    (compressed_store.py:181-183 passes ``synchronize=tables is None`` to
    decode_gpu_v2, gpu_decode_v2.py:115-116), so a caller timing it with a
    host clock sees the decode. On a CPU device the library's CPU decoder
    writes the output directly (no slices are needed to bound memory there)
    and the call returns when it is done.
    """
    enc = layer.encoded
    n = enc.n_symbols
    if _is_cpu(device):
        out = torch.empty(n, dtype=torch.bfloat16)
        if n:
            _decode_cpu_into(layer, 0, enc.n_chunks, out, n)
        return out.reshape(layer.shape)
    dev = _gpu_device(device)
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    if n == 0:
        return out.reshape(layer.shape)
    tables = _tables_for(enc, dev) if reuse_decode_tables else None
    if n <= max_slice_elems:
        _decode_range_into(layer, 0, enc.n_chunks, out, n,
                           dev, tables if tables is not None else _tables_for(enc, dev))
    else:
        chunks_per_slice = max(1, max_slice_elems // enc.chunk_size)
        for c0 in range(0, enc.n_chunks, chunks_per_slice):
            c1 = min(c0 + chunks_per_slice, enc.n_chunks)
            s0 = c0 * enc.chunk_size
            s1 = min(c1 * enc.chunk_size, n)
            _decode_range_into(layer, c0, c1, out[s0:s1], s1 - s0, dev,
                               tables if tables is not None else _tables_for(enc, dev))
    if not reuse_decode_tables:
        torch.cuda.synchronize(dev)
    return out.reshape(layer.shape)


def decompress_rows_gpu(layer: CompressedLayer, row_start: int, row_end: int,
                        device: str = "cuda") -> torch.Tensor:
    """Rows [row_start, row_end) of a 2-D compressed tensor
    (compressed_store.py:254-303): the covering chunk range is decoded and
    the exact element range returned as a (rows, cols) view. On the GPU the
    call synchronises the device after the decode, as the reference's does
    (its _decode_exponent runs decode_gpu_v2 with synchronize=True)."""
    if len(layer.shape) != 2:
        raise ValueError("decompress_rows_gpu needs a 2D tensor, got shape %r"
                         % (layer.shape,))
    cpu = _is_cpu(device)
    dev = torch.device("cpu") if cpu else _gpu_device(device)
    rows, cols = layer.shape
    row_start = max(0, row_start)
    row_end = min(rows, row_end)
    if row_end <= row_start:
        return torch.empty((0, cols), dtype=torch.bfloat16, device=dev)
    enc = layer.encoded
    cs = enc.chunk_size
    e0, e1 = row_start * cols, row_end * cols
    c0 = e0 // cs
    c1 = min(enc.n_chunks, -(-e1 // cs))
    base = c0 * cs
    avail = min(enc.n_symbols, c1 * cs) - base
    flat = torch.empty(avail, dtype=torch.bfloat16, device=dev)
    if cpu:
        _decode_cpu_into(layer, c0, c1, flat, avail)
    else:
        _decode_range_into(layer, c0, c1, flat, avail, dev, _tables_for(enc, dev))
        torch.cuda.synchronize(dev)
    return flat[e0 - base:e1 - base].reshape(row_end - row_start, cols)


def decompress_layer_cpu_reference(layer: CompressedLayer) -> torch.Tensor:
    """The exact original bf16 tensor decoded on the CPU
    (compressed_store.py:243-251). The reference uses its pure-Python reader
    here; this package decodes with the library's CPU decoder, whose output is
    the same on every valid stream (it reads the same validated table as the
    GPU kernel and is checked against the reference's decoded vectors)."""
    return decompress_layer_gpu(layer, device="cpu")


def decompress_matvec_gpu(layer: CompressedLayer, x: torch.Tensor,
                          device: str | torch.device = "cuda") -> torch.Tensor:
    """x @ W.T for the layer's 2-D bf16 weight W [rows, cols] without
    materialising W: the exponents are decoded and multiplied in one kernel
    (fp32 accumulation, bf16 result). x: [cols] or [b, cols] with b <= 16
    (a speculative-verify width), any float dtype; it is rounded to bf16.
    Up to 4 rows take the fused GEMV, 5 to 16 the fused GEMM on the matrix
    cores (which needs cols % 8 == 0 and chunks of at least 1024 symbols).
    Returns [b, rows] (or [rows] for a 1-D x) in bf16. The reference forms
    the same product as decompress_rows_gpu (compressed_store.py:254-303)
    followed by a matmul (streaming_engine.py:2271-2335)."""
    dev = _gpu_device(device)
    if len(layer.shape) != 2:
        raise ValueError("decompress_matvec_gpu needs a 2-D layer, got shape %s" % (layer.shape,))
    rows, cols = (int(v) for v in layer.shape)
    squeeze = x.dim() == 1
    xb = x.reshape(1, -1) if squeeze else x
    xb = xb.to(device=dev, dtype=torch.bfloat16).contiguous()
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, dev,
                                  tables=_tables_for(layer.encoded, dev))
    fn = decode_gemv if int(xb.shape[0]) <= GEMV_MAX_BATCH else decode_gemm
    y = fn(t, xb, rows, cols).to(torch.bfloat16)
    return y.reshape(rows) if squeeze else y


def decompress_linear_gpu(layer: CompressedLayer, x: torch.Tensor, slice_rows: int = 8192,
                          device: str | torch.device = "cuda",
                          fused: bool = False) -> torch.Tensor:
    """x @ W.T for the layer's 2-D bf16 weight W [rows, cols], as the
    reference's chunked lm_head computes it (streaming_engine.py:2307-2332):
    x [..., cols] times W a block of slice_rows rows at a time, each block
    decoded (decompress_rows_gpu's chunk range) and multiplied with
    torch.nn.functional.linear, the outputs concatenated along the last
    dimension. x must be bf16, the weight's dtype (F.linear refuses mixed
    dtypes). Returns [..., rows] in bf16.

    The blocked path (the default) gives the reference's own result: the
    same weights, bit for bit, in the same F.linear calls. Its blocks reuse
    one staging buffer. slice_rows <= 0 takes all rows as one block (the
    reference installs no chunked head then).

    fused=True multiplies inside the decode kernel (decompress_matvec_gpu;
    fp32 sums added with atomics in no fixed order, rounded once to bf16)
    without decoding any block to memory, for at most 16 rows of x (single
    tokens and the speculative-verify widths: up to 4 rows on the fused GEMV,
    5 to 16 on the fused GEMM, which needs cols % 8 == 0 and chunks of at
    least 1024 symbols). It is neither bit-identical to the blocked path nor
    reproducible from call to call; it is held to rel 1e-2 / abs 1e-3 of the
    fp32 product. Neither path is bit-identical to one unblocked F.linear:
    the reference marks its blocked head lossy for that reason (its
    tests/test_chunked_lm_head_gpu.py:1-27).

    The layer's arrays may be host arrays (copied to the GPU on each call,
    as the reference reads them for each token) or tensors already on the
    GPU (used in place)."""
    dev = _gpu_device(device)
    if len(layer.shape) != 2:
        raise ValueError("decompress_linear_gpu needs a 2-D layer, got shape %s" % (layer.shape,))
    rows, cols = (int(v) for v in layer.shape)
    if x.dim() < 1 or x.shape[-1] != cols:
        raise ValueError("x must end in a dimension of %d, got shape %s" % (cols, tuple(x.shape)))
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bf16, the weight's dtype; got %s" % x.dtype)
    lead = tuple(x.shape[:-1])
    tokens = int(np.prod(lead)) if lead else 1
    if fused and not 1 <= tokens <= GEMM_MAX_ROWS:
        raise ValueError("the fused product takes 1..%d rows of x, got %d"
                         % (GEMM_MAX_ROWS, tokens))
    x = x.to(dev)
    if rows == 0:
        return x.new_zeros(lead + (0,))
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, dev,
                                  tables=_tables_for(layer.encoded, dev))
    if fused:
        xb = x.reshape(tokens, cols).contiguous()
        fn = decode_gemv if tokens <= GEMV_MAX_BATCH else decode_gemm
        y = fn(t, xb, rows, cols).to(torch.bfloat16)
        return y.reshape(lead + (rows,))
    return decode_linear(t, x, rows, cols, slice_rows)

