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


@pytest.fixture(scope="module")
def store_two_full_blocks(tmp_path_factory):
    """Two full 14B-class blocks (config-3 shapes, 65536-symbol chunks, seeds
    3 and 4) written to a store on disk."""
    from afterimage_amd.runtime.store import StoreWriter

    d = tmp_path_factory.mktemp("store_14b")
    keys, refs = [], []
    with StoreWriter(d, model_id="block14b-x2", chunk_size=65536) as sw:
        for b, seed in enumerate((3, 4)):
            blk = workloads.block_14b(seed=seed)
            names = []
            for name, _, layer in blk:
                sw.add_compressed("layers.%d.%s" % (b, name), layer)
                names.append("layers.%d.%s" % (b, name))
            keys.append(names)
            refs.append([w.reshape(-1).view(torch.int16) for _, w, _ in blk])
            del blk
    return d, keys, refs


def test_streamed_full_blocks_from_the_store_under_4gb(store_two_full_blocks):
    """The streamed ring at its real shapes: full 14B-class blocks read from the store
    straight into pinned buffers (CRC-32 checked), then streamed through a
    2-slot ring under a 4 GiB device budget for 6 layers; every tensor of
    every layer bit-exact against the seeded originals."""
    from afterimage_amd.runtime.store import StoreReader

    d, keys, refs = store_two_full_blocks
    with StoreReader(d) as rd:
        hbs = [rd.host_block(k, pin=True, verify=True) for k in keys]
    ring = LayerRing(hbs, device="cuda", slots=2, vram_budget=4 << 30)
    assert ring.ring_bytes <= 4 << 30
    want = [[r.cuda() for r in blk] for blk in refs]
    seen = 0
    for k, tensors in ring.stream(6):
        for t, (got, w) in enumerate(zip(tensors, want[k % 2])):
            assert torch.equal(_bits(got).reshape(-1), w), "layer %d tensor %d" % (k, t)
        seen += 1
    assert seen == 6
