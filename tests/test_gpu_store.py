"""Full BF16 reconstruction on the GPU (decompress_layer_gpu and friends),
bit-exact against the original weights and the oracle.

Mirrors the reference's tests/test_compressed_store.py, test_sliced_decompress.py,
test_decode_table_reuse.py and test_chunked_lm_head_gpu.py decode cases.
"""
import dataclasses

import numpy as np
import pytest
import torch

import oracle
from afterimage_amd import workloads
from afterimage_amd.runtime import device as devmod
from afterimage_amd.runtime import gpu_decode_v2 as gd
from afterimage_amd.runtime.compressed_store import (
    compress_layer,
    decompress_layer_gpu,
    decompress_rows_gpu,
)
from afterimage_amd.runtime.device import DeviceTensor, decode_bf16

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def test_full_weight_reconstruction_bit_exact():
    torch.manual_seed(0)
    W = (torch.randn(128, 512) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=256)
    out = decompress_layer_gpu(layer)
    assert out.dtype == torch.bfloat16 and out.shape == W.shape and out.is_cuda
    assert torch.equal(_bits(out), _bits(W))
    assert torch.equal(_bits(out), _bits(oracle.decompress_layer_reference(layer)))


def test_bounded_work_chunks_preserve_every_bit():
    torch.manual_seed(40)
    W = (torch.randn(37, 59) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=31, work_chunk_elems=17)
    assert torch.equal(_bits(decompress_layer_gpu(layer)), _bits(W))


@pytest.mark.parametrize("scale", [0.001, 0.02, 0.5, 3.0])
def test_realistic_weight_scales(scale):
    torch.manual_seed(1)
    W = (torch.randn(64, 256) * scale).to(torch.bfloat16)
    layer = compress_layer(W)
    assert torch.equal(_bits(decompress_layer_gpu(layer)), _bits(W))


def test_zero_negative_and_extreme_values():
    W = torch.tensor([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30, 1e30, -1e30, 3.14159],
                     dtype=torch.bfloat16).reshape(3, 3)
    layer = compress_layer(W, chunk_size=9)
    assert torch.equal(_bits(decompress_layer_gpu(layer)), _bits(W))


def test_every_bf16_bit_pattern():
    W = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    layer = compress_layer(W.reshape(256, 256), chunk_size=1024)
    assert torch.equal(_bits(decompress_layer_gpu(layer)).reshape(-1), W.view(torch.int16))


@pytest.mark.parametrize("shape", [(1, 100), (100, 1), (7, 13), (8960, 1536)])
def test_shapes(shape):
    torch.manual_seed(3)
    W = (torch.randn(*shape) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=512)
    out = decompress_layer_gpu(layer)
    assert out.shape == shape
    assert torch.equal(_bits(out), _bits(W))


def test_sliced_matches_unsliced():
    torch.manual_seed(1)
    W = (torch.randn(4096, 512) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=1024)
    big = decompress_layer_gpu(layer, max_slice_elems=1 << 30)
    small = decompress_layer_gpu(layer, max_slice_elems=1 << 17)
    assert torch.equal(_bits(big), _bits(small))
    assert torch.equal(_bits(small), _bits(W))


@pytest.mark.parametrize("slice_elems", [97, 1 << 20])
def test_reused_tables_are_bit_exact_and_built_once_per_call(monkeypatch, slice_elems):
    original = gd.prepare_decode_tables
    seen = []

    def prepare(enc, device="cuda"):
        seen.append(id(enc))
        return original(enc, device)

    monkeypatch.setattr(gd, "prepare_decode_tables", prepare)
    keys = []
    for seed, scale in [(1, .01), (2, 10.)]:
        torch.manual_seed(seed)
        weight = (torch.randn(31, 59) * scale).to(torch.bfloat16)
        layer = compress_layer(weight, chunk_size=31)
        before = len(seen)
        out = decompress_layer_gpu(layer, max_slice_elems=slice_elems, reuse_decode_tables=True)
        assert torch.equal(_bits(out), _bits(weight))
        assert len(seen) - before == 1
        keys.append(original(layer.encoded, "cuda").key)
    # Different codebooks never share a table.
    assert keys[0] != keys[1]


def test_reused_tables_on_nondefault_stream_and_special_bit_patterns():
    bits = torch.tensor([0, -32768, 32640, -128, 32705, -63, 1, 127, 128,
                         16256, -16512, 32767], dtype=torch.int16).reshape(3, 4)
    layer = compress_layer(bits.view(torch.bfloat16), chunk_size=5)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        out = decompress_layer_gpu(layer, max_slice_elems=7, reuse_decode_tables=True)
    stream.synchronize()
    assert torch.equal(_bits(out), bits)


def test_decompress_rows_matches_full_decode():
    torch.manual_seed(17)
    W = torch.randn(300, 64, dtype=torch.float32).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=32)
    full = decompress_layer_gpu(layer, device="cuda")
    assert torch.equal(full, W.to("cuda"))
    for step in (300, 128, 64, 7, 1):
        parts = [decompress_rows_gpu(layer, r0, min(r0 + step, 300), device="cuda")
                 for r0 in range(0, 300, step)]
        assert torch.equal(torch.cat(parts, dim=0), full), "step=%d" % step
    assert decompress_rows_gpu(layer, 5, 5, device="cuda").shape == (0, 64)


def test_calls_return_after_the_decode_as_the_reference_does():
    # The reference synchronises when tables are not reused
    # (compressed_store.py:181-183, gpu_decode_v2.py:115-116): an engine that
    # times decompress_layer_gpu with a host clock sees the whole decode. On a
    # stream kept busy beforehand, the call's return means every launch on
    # the stream is done; with reuse_decode_tables it need not be.
    W, layer = workloads.single_layer(seed=5, rows=1024, cols=17408, chunk_size=65536)
    dev = torch.device("cuda")
    junk = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    for _ in range(20):
        junk.mul_(1.0001)  # about 20 ms of queued work before the call
    out = decompress_layer_gpu(layer, device="cuda")
    assert torch.cuda.current_stream(dev).query(), "decompress_layer_gpu returned before its work"
    rows = decompress_rows_gpu(layer, 10, 700, device="cuda")
    assert torch.cuda.current_stream(dev).query(), "decompress_rows_gpu returned before its work"
    again = decompress_layer_gpu(layer, device="cuda", reuse_decode_tables=True)
    torch.cuda.synchronize(dev)
    assert torch.equal(out.view(torch.int16), W.to(dev).view(torch.int16))
    assert torch.equal(again, out) and torch.equal(rows, out[10:700])


def test_unaligned_output_view_uses_elementwise_stores():
    torch.manual_seed(5)
    W = (torch.randn(64, 96) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=256)
    dt = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    buf = torch.zeros(W.numel() + 3, dtype=torch.bfloat16, device="cuda")
    decode_bf16([dt], [buf[3:]])
    assert torch.equal(_bits(buf[3:]).reshape(W.shape), _bits(W))
    assert torch.equal(_bits(buf[:3]), torch.zeros(3, dtype=torch.int16))


@pytest.mark.parametrize("shape,chunk,tiny", [((3,), 3, True), ((7, 5), 16, False),
                                              ((64, 1000), 4096, False), ((40, 4096), 65536, False),
                                              ((30,), 65536, False), ((23,), 65536, False),
                                              ((20,), 65536, False)])
def test_packed_buffer_without_slack_bytes(shape, chunk, tiny):
    """A packed buffer that ends at the last chunk's last byte: the final
    words come from the buffer's last whole word, or byte by byte when the
    whole buffer is shorter than 4 bytes. At 65536-symbol chunks (whole
    workgroups) (30,) packs into 10 bytes, (23,) into 8 and (20,) into 7."""
    W = workloads.bf16_normal(shape, 123, 0.02)
    layer = compress_layer(W, chunk_size=chunk)
    enc = layer.encoded
    used = int(enc.chunk_offsets[-1]) + int(enc.chunk_nbytes[-1])
    assert (used < 4) == tiny
    trimmed = dataclasses.replace(enc, packed=enc.packed[:used].copy())
    dt = DeviceTensor.from_encoded(trimmed, layer.sign_mantissa, "cuda")
    assert dt.packed.numel() == used
    (out,) = decode_bf16([dt])
    assert torch.equal(_bits(out), _bits(W).reshape(-1))
    exps = gd.decode_gpu_v2(trimmed).cpu().numpy()
    assert np.array_equal(exps, oracle.decode_chunked_reference(enc))


def test_batched_block_launch_with_shared_codebooks():
    """Several tensors in one launch; same-role tensors share one codebook
    (encoded from the pooled histogram) and therefore one device table."""
    shapes = [(512, 640), (128, 640), (128, 640), (512, 640), (640, 1088), (5120,)]
    ws = [workloads.bf16_normal(s, 10 + i, 0.02, outlier_frac=1e-3) for i, s in enumerate(shapes)]
    ws[-1] = workloads.bf16_normal((5120,), 99, 0.05, center=1.0)
    layers = [compress_layer(w, chunk_size=4096) for w in ws]
    dts = [DeviceTensor.from_encoded(l.encoded, l.sign_mantissa, "cuda") for l in layers]
    outs = decode_bf16(dts)
    for w, o in zip(ws, outs):
        assert torch.equal(_bits(o), _bits(w).reshape(-1))
    # Same LUT content -> same cached table object.
    t0 = devmod.TABLES.get(layers[1].encoded.sym_lut, layers[1].encoded.len_lut,
                           layers[1].encoded.max_bits, "cuda")
    t1 = devmod.TABLES.get(layers[1].encoded.sym_lut.copy(), layers[1].encoded.len_lut.copy(),
                           layers[1].encoded.max_bits, "cuda")
    assert t0.blob.data_ptr() == t1.blob.data_ptr()


def test_cpu_device_decodes_the_same_bits():
    torch.manual_seed(20)
    W = (torch.randn(160, 96) * 0.02).to(torch.bfloat16)
    layer = compress_layer(W, chunk_size=512)
    cpu = decompress_layer_gpu(layer, device="cpu")
    gpu = decompress_layer_gpu(layer, device="cuda")
    assert cpu.device.type == "cpu"
    assert torch.equal(_bits(cpu), _bits(gpu)) and torch.equal(_bits(cpu), _bits(W))


@pytest.mark.parametrize("name", ["single_symbol", "skewed_2sym", "dirichlet_6", "bf16_outliers_64k",
                                  "scales_3p0", "uniform256"])
@pytest.mark.parametrize("chunk_size", [64, 4096, 65536])
def test_cpu_and_gpu_decoders_agree_on_random_bytes(name, chunk_size):
    """Arbitrary bytes under real codebooks, including ones with windows that
    start no codeword (single_symbol, whose code is '0'): the host and GPU
    decoders read one table blob and must agree on every position."""
    from tests.golden_data import case

    from afterimage_amd.runtime.huffman_chunked import ChunkedEncoded

    base = case(name)["encoded"]
    g = np.random.default_rng(chunk_size)
    n_chunks = 5
    nbytes = g.integers(0, chunk_size // 2 + 8, n_chunks).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(nbytes)[:-1]]).astype(np.int32)
    packed = g.integers(0, 256, int(nbytes.sum()) + 8, dtype=np.uint8)
    enc = ChunkedEncoded(packed=packed, chunk_offsets=offsets, chunk_nbytes=nbytes,
                         sym_lut=base.sym_lut, len_lut=base.len_lut, max_bits=base.max_bits,
                         chunk_size=chunk_size, n_symbols=n_chunks * chunk_size - 3,
                         shape=(n_chunks * chunk_size - 3,))
    gpu = gd.decode_gpu_v2(enc).cpu().numpy()
    cpu = torch.empty(enc.n_symbols, dtype=torch.uint8)
    devmod.cpu_decode([(enc, None, cpu, enc.n_symbols)], exponents_only=True)
    assert np.array_equal(gpu, cpu.numpy())


def test_recombine_kernel_on_every_byte_pair_and_offsets():
    from afterimage_amd.runtime.compressed_store import recombine_exponent_and_sign_mantissa

    e = np.repeat(np.arange(256, dtype=np.uint8), 256)
    sm = np.tile(np.arange(256, dtype=np.uint8), 256)
    want = oracle.recombine(e, sm).view(np.int16)
    got = recombine_exponent_and_sign_mantissa(e, sm, (256, 256), "cuda")
    assert got.is_cuda and got.dtype == torch.bfloat16 and tuple(got.shape) == (256, 256)
    assert np.array_equal(_bits(got).numpy().reshape(-1), want)
    # Unaligned starts and ragged lengths take the element-wise kernel.
    et = torch.from_numpy(e).cuda()
    st = torch.from_numpy(sm).cuda()
    for a, b in [(1, 65536), (3, 1000), (16, 65531), (0, 15), (7, 8)]:
        out = devmod.recombine_bf16(et[a:b], st[a:b])
        assert np.array_equal(_bits(out).numpy(), want[a:b]), (a, b)


@pytest.mark.parametrize("misalign", [1, 3])
def test_decode_from_store_views_small_layer(misalign):
    """Config-1 layer from non-owning unaligned views, as read_many returns
    them (afterimage/runtime/binstore.py:115-133)."""
    from tests.store_views import store_views

    W, layer = workloads.small_layer()
    view_layer, views = store_views(layer, misalign)
    assert all(not v.flags.owndata for v in views)
    out = decompress_layer_gpu(view_layer)
    assert torch.equal(_bits(out), _bits(W))
    rows = decompress_rows_gpu(view_layer, 100, 357)
    assert torch.equal(_bits(rows), _bits(W[100:357]))


def test_small_layer_1024x3072_chunk4096():
    W, layer = workloads.small_layer()
    out = decompress_layer_gpu(layer)
    assert torch.equal(_bits(out), _bits(W))
    exps = oracle.decode_chunked_reference(layer.encoded)
    ref = oracle.recombine(exps, layer.sign_mantissa.numpy())
    assert np.array_equal(_bits(out).numpy().reshape(-1).view(np.uint16), ref)


def test_single_layer_5120x17408_chunk65536():
    """The full-size layer: bit-exact against the seeded original (the
    reference decoder is lossless, so its output is the original)."""
    W, layer = workloads.single_layer()
    assert layer.encoded.n_chunks == 1360
    dt = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    (out,) = decode_bf16([dt])
    assert torch.equal(_bits(out), _bits(W).reshape(-1))
    # And the oracle agrees on a sample of chunks (the whole tensor is
    # checked against W above).
    exps = oracle.decode_chunks(layer.encoded, 0, 8, n_threads=4)
    sm = layer.sign_mantissa.numpy()[: exps.size]
    assert np.array_equal(_bits(out).numpy()[: exps.size].view(np.uint16), oracle.recombine(exps, sm))


@pytest.fixture(scope="module")
def block14b():
    return workloads.block_14b()


def test_block_14b_decodes_in_one_launch_with_shared_tables(block14b):
    """The full 14B-class block (330M weights, 9 tensors) in one decode call:
    same-role tensors share one device table; every tensor bit-exact."""
    dts = [DeviceTensor.from_encoded(l.encoded, l.sign_mantissa, "cuda") for _, _, l in block14b]
    assert len(dts) <= devmod.MAX_TENSORS  # decode_bf16 issues a single launch
    tables = {}
    for dt, (_, _, role) in zip(dts, workloads.BLOCK_14B):
        tables.setdefault(role, set()).add(dt.tables.blob.data_ptr())
    assert len(tables) == 5 and all(len(v) == 1 for v in tables.values())
    outs = decode_bf16(dts)
    for (name, w, _), o in zip(block14b, outs):
        assert torch.equal(_bits(o), _bits(w).reshape(-1)), name



def test_block_14b_decodes_from_store_views(block14b):
    """Every tensor of the 14B-class block through the reference API from
    non-owning unaligned views of one buffer per tensor."""
    from tests.store_views import store_views

    for name, w, layer in block14b:
        view_layer, _ = store_views(layer, 5)
        out = decompress_layer_gpu(view_layer, reuse_decode_tables=True)
        assert torch.equal(_bits(out), _bits(w)), name
