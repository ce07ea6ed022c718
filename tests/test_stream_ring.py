"""The streamed-block ring's host side: one pinned buffer per block holding
every tensor's compressed arrays."""
import numpy as np
import pytest

from afterimage_amd import workloads
from afterimage_amd.runtime.stream_ring import ALIGN, HostBlock, LayerRing


def test_host_block_holds_every_array_at_aligned_offsets():
    blk = workloads.block_14b(scale=0.01, chunk_size=4096)
    hb = HostBlock([l for _, _, l in blk], pin=False)
    buf = hb.buf.numpy()
    for (_, _, layer), t in zip(blk, hb.layout):
        enc = layer.encoded
        # Sign/mantissa bytes and chunk offsets start aligned; the bitstream
        # and the chunk lengths follow them directly (one store read each).
        s0, sn = t.sign_mantissa
        o0, on = t.chunk_offsets
        assert s0 % ALIGN == 0 and o0 % ALIGN == 0
        assert t.packed[0] == s0 + sn and t.chunk_nbytes[0] == o0 + 4 * on
        p0, pn = t.packed
        assert np.array_equal(buf[p0:p0 + pn], enc.packed)
        o0, on = t.chunk_offsets
        assert np.array_equal(buf[o0:o0 + 4 * on].view(np.int32), enc.chunk_offsets)
        b0, bn = t.chunk_nbytes
        assert np.array_equal(buf[b0:b0 + 4 * bn].view(np.int32), enc.chunk_nbytes)
        s0, sn = t.sign_mantissa
        assert np.array_equal(buf[s0:s0 + sn], layer.sign_mantissa.numpy())
    assert hb.decoded_nbytes >= 2 * sum(l.encoded.n_symbols for _, _, l in blk)


def test_ring_refuses_a_cpu_device_and_one_slot():
    hb = HostBlock([workloads.small_layer(rows=8, cols=64, chunk_size=128)[1]], pin=False)
    with pytest.raises(RuntimeError, match="GPU"):
        LayerRing([hb], device="cpu")
    with pytest.raises(ValueError, match="2 slots"):
        LayerRing([hb], device="cpu", slots=1)
