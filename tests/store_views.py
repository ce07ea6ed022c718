"""Compressed layers rebuilt from non-owning numpy views into one bytearray at
unaligned offsets: the form in which the reference's store reader hands blobs
to its engine (afterimage/runtime/binstore.py:115-133)."""
import numpy as np
import torch

from afterimage_amd.runtime import compressed_store as cs
from afterimage_amd.runtime.huffman_chunked import ChunkedEncoded


def store_views(layer, misalign):
    """The layer's arrays as non-owning numpy views into one bytearray at
    unaligned offsets, the way the reference's read_many returns blobs
    (afterimage/runtime/binstore.py:115-133)."""
    enc = layer.encoded
    parts = [np.ascontiguousarray(layer.sign_mantissa.numpy()), enc.packed,
             np.ascontiguousarray(enc.chunk_offsets, np.int32),
             np.ascontiguousarray(enc.chunk_nbytes, np.int32),
             np.ascontiguousarray(enc.sym_lut, np.int32), np.ascontiguousarray(enc.len_lut, np.int8)]
    buf = bytearray(sum(p.nbytes + misalign for p in parts) + 16)
    views = []
    pos = misalign
    for p in parts:
        buf[pos:pos + p.nbytes] = p.tobytes()
        views.append(np.frombuffer(buf, dtype=p.dtype, count=p.size, offset=pos))
        pos += p.nbytes + misalign
    sm, packed, offs, nbytes, sym, ln = views
    enc2 = ChunkedEncoded(packed=packed, chunk_offsets=offs, chunk_nbytes=nbytes, sym_lut=sym,
                          len_lut=ln, max_bits=enc.max_bits, chunk_size=enc.chunk_size,
                          n_symbols=enc.n_symbols, shape=enc.shape)
    return cs.CompressedLayer(sign_mantissa=torch.from_numpy(sm), encoded=enc2,
                              shape=layer.shape), views
