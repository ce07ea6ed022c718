"""Host side of the blocked x @ W.T (chunked lm_head): the row blocks and the
chunk ranges that hold them, and chunk-range views of a resident tensor,
checked on CPU tensors (no decode)."""
import numpy as np
import pytest
import torch

from afterimage_amd.runtime.compressed_store import compress_layer
from afterimage_amd.runtime.device import DeviceTensor, row_blocks


@pytest.mark.parametrize("rows,cols,chunk,step", [(300, 64, 32, 7), (301, 100, 256, 64),
                                                  (1500, 200, 65536, 128), (9496, 5120, 1024, 2374),
                                                  (5, 3, 4, 1), (10, 10, 1000, 3)])
def test_row_blocks_cover_the_rows_and_their_chunks(rows, cols, chunk, step):
    n_chunks = -(-rows * cols // chunk)
    blocks = row_blocks(rows, cols, chunk, n_chunks, step)
    assert [b[0] for b in blocks] == list(range(0, rows, step))
    assert blocks[-1][1] == rows
    for r0, r1, c0, c1 in blocks:
        assert 0 < r1 - r0 <= step
        # the chunks hold the block's elements, and no chunk more than needed
        assert c0 * chunk <= r0 * cols and r1 * cols <= min(rows * cols, c1 * chunk)
        assert (c0 + 1) * chunk > r0 * cols and (c1 - 1) * chunk < r1 * cols
        assert 0 <= c0 < c1 <= n_chunks
    assert row_blocks(0, cols, chunk, 0, step) == []


@pytest.mark.parametrize("step", [0, -5])
def test_row_blocks_without_slicing_are_one_block(step):
    # lm_head_slice_rows = 0 means no chunked head: the whole tensor at once,
    # not 1-row blocks.
    assert row_blocks(151936, 5120, 1024, 759680, step) == [(0, 151936, 0, 759680)]
    assert row_blocks(7, 3, 4, 6, step) == [(0, 7, 0, 6)]


def _cpu_tensor(layer):
    enc = layer.encoded
    return DeviceTensor(packed=torch.from_numpy(enc.packed.copy()),
                        chunk_offsets=torch.from_numpy(enc.chunk_offsets.astype(np.int32)),
                        chunk_nbytes=torch.from_numpy(enc.chunk_nbytes.astype(np.int32)),
                        sign_mantissa=layer.sign_mantissa.reshape(-1), tables=None,
                        chunk_size=enc.chunk_size, n_symbols=enc.n_symbols, shape=enc.shape)


def test_chunk_range_views_share_memory():
    torch.manual_seed(3)
    W = torch.randn(37, 50, dtype=torch.float32).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=64)
    t = _cpu_tensor(layer)
    n = t.n_symbols
    assert t.chunk_range(0, t.n_chunks) is t
    for c0, c1 in [(0, 1), (3, 9), (t.n_chunks - 1, t.n_chunks), (5, 5)]:
        v = t.chunk_range(c0, c1)
        assert v.index is None and v.packed is t.packed
        assert v.n_chunks == c1 - c0
        assert v.n_symbols == max(0, min(n, c1 * 64) - c0 * 64)
        assert torch.equal(v.chunk_offsets, t.chunk_offsets[c0:c1])
        if v.n_symbols:
            assert v.sign_mantissa.data_ptr() == t.sign_mantissa.data_ptr() + c0 * 64
        assert v.sign_mantissa.numel() == v.n_symbols
    t.range_cache[((0, 1),)] = [t.chunk_range(0, 1)]
    t.drop_index()
    assert t.index is None and not t.range_cache
    with pytest.raises(ValueError):
        t.chunk_range(2, 1)
    with pytest.raises(ValueError):
        t.chunk_range(0, t.n_chunks + 1)
