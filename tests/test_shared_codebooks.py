"""Shared per-role codebooks (one stored LUT and one decode table for all
tensors of a role): encoding with a given code, checked on the CPU by the
oracle against the original weights."""
import numpy as np
import pytest
import torch

import oracle
from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import compress_group, compress_layer
from afterimage_amd.runtime.huffman_chunked import encode_chunked


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def test_group_shares_one_lut_and_round_trips():
    ws = [workloads.bf16_normal((64, 96), 50 + i, 0.02) for i in range(3)]
    layers = compress_group(ws, chunk_size=512)
    luts = {(l.encoded.sym_lut.tobytes(), l.encoded.len_lut.tobytes()) for l in layers}
    assert len(luts) == 1
    for w, l in zip(ws, layers):
        assert torch.equal(_bits(oracle.decompress_layer_reference(l)), _bits(w))


def test_group_code_is_the_code_of_the_pooled_data():
    """The shared code equals encode_chunked's own code for the concatenation."""
    ws = [workloads.bf16_normal((32, 64), 7 + i, 0.02 * (i + 1)) for i in range(2)]
    layers = compress_group(ws, chunk_size=256)
    pooled = compress_layer(torch.cat([w.reshape(-1) for w in ws]), chunk_size=256)
    assert np.array_equal(layers[0].encoded.sym_lut, pooled.encoded.sym_lut)
    assert np.array_equal(layers[0].encoded.len_lut, pooled.encoded.len_lut)


def test_given_lengths_must_cover_every_symbol():
    with pytest.raises(ValueError, match="no code"):
        encode_chunked(np.array([1, 2, 3], dtype=np.uint8), chunk_size=4, lengths={1: 1, 2: 1})


def test_small_block_roles_share_codebooks():
    blk = workloads.block_14b(scale=0.01, chunk_size=4096)
    by_role = {}
    for (name, w, layer), (_, _, role) in zip(blk, workloads.BLOCK_14B):
        by_role.setdefault(role, set()).add(layer.encoded.sym_lut.tobytes())
        exps = oracle.decode_chunked_reference(layer.encoded)
        ref = oracle.recombine(exps, layer.sign_mantissa.numpy())
        assert np.array_equal(ref, _bits(w).numpy().reshape(-1).view(np.uint16)), name
    assert all(len(v) == 1 for v in by_role.values())
    assert len(by_role) == 5
