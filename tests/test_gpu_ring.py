"""Streamed blocks through the double-buffered ring: every layer bit-exact."""
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.stream_ring import HostBlock, LayerRing

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.fixture(scope="module")
def two_blocks():
    return [workloads.block_14b(seed=s, scale=0.05, chunk_size=4096) for s in (4, 5)]


@pytest.mark.parametrize("slots", [2, 3])
def test_ring_streams_layers_bit_exact(two_blocks, slots):
    hbs = [HostBlock([l for _, _, l in blk]) for blk in two_blocks]
    ref = [[_bits(w.cuda()) for _, w, _ in blk] for blk in two_blocks]
    ring = LayerRing(hbs, device="cuda", slots=slots)
    seen = 0
    for k, tensors in ring.stream(7):
        want = ref[k % 2]
        assert len(tensors) == len(want)
        for got, w in zip(tensors, want):
            assert got.shape == w.shape
            assert torch.equal(_bits(got), w), "layer %d" % k
        seen += 1
    assert seen == 7


def test_ring_respects_the_vram_budget(two_blocks):
    hbs = [HostBlock([l for _, _, l in blk]) for blk in two_blocks]
    with pytest.raises(ValueError, match="budget"):
        LayerRing(hbs, device="cuda", vram_budget=1 << 20)
