"""Split chunks on the GPU. When the last pass of a chunk-by-chunk launch
would leave some CUs with more whole-workgroup chunks than others (the
5120x17408 layer: 1360 chunks on 512 workgroups), the last chunks are decoded
in two halves of their rounds on different workgroups, the first half handing
its state to the second through a device record.

On MI355X (256 CUs, a grid of 512) the layer's last 336 chunks are split
(the busiest CU's rounds 12 -> 11). Checked: bit-exact against the seeded originals (the reference decoder is
lossless) and against the same launch with splitting off (AIMG_CHUNK_SPLIT=0);
back-to-back launches of different data of one shape (no record of one
launch is taken by the next); launches on two streams at once (records of
overlapping launches are told apart by their tags, and a second half that
cannot take its record decodes its chunk whole).
"""
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import compress_layer
from afterimage_amd.runtime.device import DeviceTensor, decode_bf16, decode_u8

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).reshape(-1)


@pytest.fixture(scope="module")
def layers():
    """Two 5120x17408 layers (1360 chunks of 65536 symbols each), different
    seeds, with 0.1% outliers."""
    out = []
    for seed in (2, 7):
        W, layer = workloads.single_layer(seed=seed)
        assert layer.encoded.n_chunks == 1360
        out.append((W, layer, DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")))
    return out


def test_split_matches_unsplit_and_original(layers, monkeypatch):
    W, layer, dt = layers[0]
    (a,) = decode_bf16([dt])
    monkeypatch.setenv("AIMG_CHUNK_SPLIT", "0")
    (b,) = decode_bf16([dt])
    monkeypatch.delenv("AIMG_CHUNK_SPLIT")
    torch.cuda.synchronize()
    assert torch.equal(_bits(a), _bits(W))
    assert torch.equal(_bits(b), _bits(W))


def test_split_exponent_bytes(layers, monkeypatch):
    W, layer, dt = layers[1]
    want = ((W.contiguous().view(torch.int16).reshape(-1).to(torch.int32) >> 7) & 0xFF).to(torch.uint8)
    (a,) = decode_u8([dt])
    monkeypatch.setenv("AIMG_CHUNK_SPLIT", "0")
    (b,) = decode_u8([dt])
    monkeypatch.delenv("AIMG_CHUNK_SPLIT")
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), want)
    assert torch.equal(b.cpu(), want)


def test_back_to_back_launches_of_one_shape(layers):
    # A, B, A, B, ... on one stream with no host synchronisation: every
    # launch's second halves read only their own launch's records.
    outs = []
    for k in range(6):
        W, layer, dt = layers[k % 2]
        (o,) = decode_bf16([dt])
        outs.append((W, o))
    torch.cuda.synchronize()
    for W, o in outs:
        assert torch.equal(_bits(o), _bits(W))


def test_launches_on_two_streams_at_once(layers):
    # Two launches that may overlap on the GPU and share the record array:
    # each decodes its own layer exactly, whichever halves hand over or fall
    # back to whole chunks.
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for _ in range(4):
        with torch.cuda.stream(s1):
            (o1,) = decode_bf16([layers[0][2]])
        with torch.cuda.stream(s2):
            (o2,) = decode_bf16([layers[1][2]])
        outs.append((o1, o2))
    torch.cuda.synchronize()
    for o1, o2 in outs:
        assert torch.equal(_bits(o1), _bits(layers[0][0]))
        assert torch.equal(_bits(o2), _bits(layers[1][0]))


@pytest.mark.parametrize("rows", [3081, 3335])
def test_ragged_split_layers(rows):
    # 16384 columns: 771 and 834 chunks, the last one ragged (770.25 and
    # 833.75 chunks' worth of symbols); on a 512-workgroup grid the last 259
    # and 322 are split (the busiest CU's rounds 8 -> 7).
    W = workloads.bf16_normal((rows, 16384), rows, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=65536)
    dt = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    (o,) = decode_bf16([dt])
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(W))


def test_records_reused_by_a_smaller_launch_next(layers, monkeypatch):
    # Two split launches in a row through the C-ABI, the second smaller (771
    # chunks: the last 259 split): the records the first leaves empty serve
    # the second, and both equal the same launches with splitting off.
    W1, _, dt1 = layers[0]
    W2 = workloads.bf16_normal((3081, 16384), 31, 0.02, outlier_frac=1e-3)
    l2 = compress_layer(W2, chunk_size=65536)
    assert l2.encoded.n_chunks == 771
    dt2 = DeviceTensor.from_encoded(l2.encoded, l2.sign_mantissa, "cuda")
    (a1,) = decode_bf16([dt1])
    (a2,) = decode_bf16([dt2])
    monkeypatch.setenv("AIMG_CHUNK_SPLIT", "0")
    (b1,) = decode_bf16([dt1])
    (b2,) = decode_bf16([dt2])
    monkeypatch.delenv("AIMG_CHUNK_SPLIT")
    torch.cuda.synchronize()
    assert torch.equal(_bits(a1), _bits(b1)) and torch.equal(_bits(a1), _bits(W1))
    assert torch.equal(_bits(a2), _bits(b2)) and torch.equal(_bits(a2), _bits(W2))
