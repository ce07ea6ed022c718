"""CodecConfig (the reference EngineConfig's codec fields) and the reference's
size claims for compress_layer (its tests/test_compressed_store.py:47-75)."""
import pytest
import torch

from afterimage_amd.runtime.compressed_store import compress_layer
from afterimage_amd.runtime.config import CodecConfig


def test_defaults_match_the_reference():
    c = CodecConfig()
    assert (c.chunk_size, c.block_chunks, c.max_bits) == (1024, 32, 16)
    assert c.decode_slice_elems == 1 << 25 and c.reuse_decode_tables is False
    assert c.lm_head_slice_rows == 0 and c.is_lossless


@pytest.mark.parametrize("kw", [{"block_chunks": 24}, {"max_bits": 0}, {"max_bits": 17},
                                {"chunk_size": 0}, {"decode_slice_elems": 0},
                                {"lm_head_slice_rows": -1}])
def test_invalid_settings_raise(kw):
    with pytest.raises(ValueError):
        CodecConfig(**kw)


def test_blocked_head_is_not_lossless():
    assert not CodecConfig(lm_head_slice_rows=8192).is_lossless


def test_compression_reduces_size_at_real_layer_scale():
    torch.manual_seed(2)
    W = (torch.randn(8960, 1536) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W)
    assert layer.compressed_bytes / layer.original_bytes < 0.75


def test_lut_fixed_cost_dominates_below_a_scale_threshold():
    # The stored LUT (2^16 int32 + int8 entries at max_bits 16) outweighs a
    # 256-weight tensor.
    torch.manual_seed(9)
    tiny = (torch.randn(16, 16) * 0.02).to(torch.bfloat16)
    layer = compress_layer(tiny)
    assert layer.compressed_bytes > layer.original_bytes
