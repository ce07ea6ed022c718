"""Exponent-stream GPU decode with the reference's API
(afterimage/runtime/gpu_decode_v2.py:71-117), served by the gfx950 kernel in
``libafterimage_decode`` instead of a Triton program.

``block_chunks`` keeps its validation (a power of 2, checked before ``enc`` is
touched) so callers and configs behave the same, but it does not shape the
launch: the HIP kernel runs persistent 512-thread workgroups that split into
sub-groups of 16 to 512 threads, one chunk per sub-group, sized from the
chunk length, and each sub-group splits its chunk's bitstream across its
threads.
"""
from __future__ import annotations

import torch

from .device import TABLES, DecodeTables, DeviceTensor, decode_u8

_SYMBOL_MSG = "decoder output is uint8; symbol alphabet must fit in a byte"


def _require_gpu(device) -> torch.device:
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(
            "decode_gpu_v2 runs on a GPU (device %r); CPU decoding goes through "
            "decompress_layer_gpu(..., device='cpu')" % (str(device),))
    return dev


def prepare_decode_tables(enc, device: str = "cuda") -> DecodeTables:
    """Decode tables for ``enc``'s codebook on ``device`` (gpu_decode_v2.py:71-76).

    ``sym_lut, len_lut = tables`` unpacks as the reference's int32 LUT pair;
    the decoder reads the compact table blob the same object carries. Tables
    are cached by codebook content, so tensors that share a codebook share
    one table, and different codebooks never collide.
    """
    if int(enc.sym_lut.max(initial=0)) > 255:
        raise AssertionError(_SYMBOL_MSG)
    return TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, torch.device(device))


def decode_gpu_v2(enc, block_chunks: int = 32, device: str = "cuda", *,
                  tables: DecodeTables | None = None, synchronize: bool = True) -> torch.Tensor:
    """uint8 exponents of ``enc`` (length ``enc.n_symbols``) on ``device``."""
    if block_chunks < 1 or block_chunks & (block_chunks - 1) != 0:
        raise ValueError(f"block_chunks must be a power of 2, got {block_chunks}")
    dev = _require_gpu(device)
    if tables is None:
        tables = prepare_decode_tables(enc, dev)
    if enc.n_symbols == 0:
        return torch.empty(0, dtype=torch.uint8, device=dev)
    dt = DeviceTensor.from_encoded(enc, None, dev, tables=tables)
    (out,) = decode_u8([dt], [enc.n_symbols], device=dev)
    if synchronize:
        torch.cuda.synchronize(dev)
    return out
