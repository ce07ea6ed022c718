"""Exponent-stream GPU decode with the reference's API
(afterimage/runtime/gpu_decode_v2.py:71-117), served by the gfx950 kernel in
``libafterimage_decode`` instead of a Triton program.

``block_chunks`` keeps its validation (a power of 2, checked before ``enc`` is
touched) so callers and configs behave the same, but it does not shape the
launch: the HIP kernel assigns a 256-thread workgroup per chunk and splits
each chunk's bitstream across the threads itself.
"""
from __future__ import annotations

import torch

from .device import TABLES, DecodeTables, DeviceTensor, decode_u8

_SYMBOL_MSG = "decoder output is uint8; symbol alphabet must fit in a byte"


def _require_gpu(device) -> torch.device:
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(
            "afterimage_amd decodes on the GPU only (device %r); there is no CPU "
            "decode path in this package" % (str(device),))
    return dev


def prepare_decode_tables(enc, device: str = "cuda") -> DecodeTables:
    """Device decode tables for ``enc``'s codebook (gpu_decode_v2.py:71-76).

    Tables are cached by codebook content, so tensors that share a codebook
    share one device table; different codebooks never collide.
    """
    if int(enc.sym_lut.max(initial=0)) > 255:
        raise AssertionError(_SYMBOL_MSG)
    return TABLES.get(enc.sym_lut, enc.len_lut, enc.max_bits, _require_gpu(device))


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
