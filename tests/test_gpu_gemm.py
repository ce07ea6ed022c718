"""Fused decode -> GEMM on the matrix cores (Y = X @ W.T for 5 to 16 rows of
X, W decoded inside the kernel and never written), the speculative-verify
widths of the chunked lm_head (ref streaming_engine.py:2307-2332, called with
step_k + 1 positions at :2554-2556). The weights decode bit-exact, so the
reference product is the fp32 matmul of the original bf16 weights; the
result must agree within rel 1e-2 / abs 1e-3 (bf16 products, fp32 sums in
no fixed order, then bf16 for the API's result)."""
import numpy as np
import pytest
import torch

from afterimage_amd import _native, workloads
from afterimage_amd.runtime.compressed_store import (compress_layer, decompress_linear_gpu,
                                                     decompress_matvec_gpu)
from afterimage_amd.runtime.device import GEMM_MAX_ROWS, DeviceTensor, decode_gemm

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _x(n, cols, seed):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.standard_normal((n, cols), dtype=np.float32)).to(torch.bfloat16)


def _ref(W, x):
    # fp32 on the GPU, both operands contiguous (no transposed-view products).
    Wf = W.to("cuda").float().contiguous()
    xf = x.to("cuda").float().contiguous()
    return torch.matmul(xf, Wf.t().contiguous())


def _check(y, ref):
    err = (y.float() - ref).abs()
    bound = ATOL + RTOL * ref.abs()
    assert bool((err <= bound).all()), "max excess %.3g" % float((err - bound).max())


@pytest.fixture(scope="module")
def down_proj():
    return workloads.single_layer()


@pytest.mark.parametrize("n_x", [5, 8, 16])
def test_down_proj_5120x17408(down_proj, n_x):
    """The 5120x17408 layer (64Ki-symbol chunks): rows of 17408 weights, each
    16-row tile of W spread over several rounds and workgroups."""
    W, layer = down_proj
    x = _x(n_x, W.shape[1], 50 + n_x)
    y = decompress_matvec_gpu(layer, x)
    assert tuple(y.shape) == (n_x, W.shape[0]) and y.dtype == torch.bfloat16
    _check(y, _ref(W, x))


@pytest.mark.parametrize("n_x", [5, 8, 16])
@pytest.mark.parametrize("shape,chunk", [((2000, 5120), 1024), ((96, 4104), 65536),
                                         ((300, 200), 1024), ((1500, 1000), 4096),
                                         ((64, 32768), 8192), ((33, 1032), 2048)])
def test_shapes(shape, chunk, n_x):
    """Head-like rows at the reference store's 1024-symbol chunks; a last
    32-column slice cut short (cols % 32 != 0: 4104, 200, 1000, 1032); rows
    too short for the bank padding (200: 25 groups); many rows a round
    (200, 1000); rows longer than a round (32768)."""
    W = workloads.bf16_normal(shape, 60 + shape[1] % 97, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=chunk)
    x = _x(n_x, shape[1], shape[0] + n_x)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    y = decode_gemm(t, x.cuda(), shape[0], shape[1])
    assert y.dtype == torch.float32 and tuple(y.shape) == (n_x, shape[0])
    _check(y, _ref(W, x))


@pytest.mark.parametrize("tokens", [5, 8, 16])
def test_decompress_linear_fused_head(tokens):
    """decompress_linear_gpu(fused=True) at verify widths: x [1, tokens, cols]
    -> [1, tokens, rows] bf16, no weight block decoded to memory; the layer's
    arrays once on the host (copied per call) and once resident on the GPU
    (used in place)."""
    W = workloads.bf16_normal((3000, 1536), 70 + tokens, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=1024)
    x = _x(tokens, 1536, tokens).reshape(1, tokens, 1536).cuda()
    ref = _ref(W, x.reshape(tokens, 1536)).reshape(1, tokens, 3000)
    y = decompress_linear_gpu(layer, x, fused=True)
    assert y.shape == (1, tokens, 3000) and y.dtype == torch.bfloat16
    _check(y, ref)
    enc = layer.encoded
    resident = type(layer)(
        encoded=type(enc)(packed=torch.from_numpy(enc.packed).cuda(),
                          chunk_offsets=torch.from_numpy(enc.chunk_offsets).cuda(),
                          chunk_nbytes=torch.from_numpy(enc.chunk_nbytes).cuda(),
                          sym_lut=enc.sym_lut, len_lut=enc.len_lut, max_bits=enc.max_bits,
                          chunk_size=enc.chunk_size, n_symbols=enc.n_symbols, shape=enc.shape),
        sign_mantissa=layer.sign_mantissa.cuda(), shape=layer.shape)
    _check(decompress_linear_gpu(resident, x, fused=True), ref)


def test_accumulates_into_given_y_repeatedly():
    """y is added to, not overwritten; calls in a row give the same sums
    within fp32 rounding (the order of the additions is not fixed)."""
    W = workloads.bf16_normal((257, 2048), 11, 0.02)
    layer = compress_layer(W, chunk_size=2048)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    x = _x(GEMM_MAX_ROWS, 2048, 3).cuda()
    ref = _ref(W, x)
    y = torch.full((GEMM_MAX_ROWS, 257), 2.0, dtype=torch.float32, device="cuda")
    decode_gemm(t, x, 257, 2048, y)
    _check(y - 2.0, ref)
    for _ in range(3):
        y2 = decode_gemm(t, x, 257, 2048)
        assert bool(((y2 - ref).abs() <= 1e-4 + 1e-4 * ref.abs()).all())


def test_rejects_what_it_does_not_serve():
    W = workloads.bf16_normal((40, 256), 2, 0.02)
    small = compress_layer(W, chunk_size=512)
    t = DeviceTensor.from_encoded(small.encoded, small.sign_mantissa, "cuda")
    x = _x(6, 256, 1).cuda()
    with pytest.raises(_native.NativeError, match="1024"):
        decode_gemm(t, x, 40, 256)                               # chunks below 1024 symbols
    with pytest.raises(ValueError, match="batch"):
        decode_gemm(t, _x(17, 256, 1).cuda(), 40, 256)           # more than 16 rows of x
    with pytest.raises(ValueError, match="rows"):
        decode_gemm(t, x, 20, 256)
    with pytest.raises(_native.NativeError, match="1024"):
        decompress_linear_gpu(small, x.reshape(1, 6, 256), fused=True)
    # The blocked path serves the same layer.
    y = decompress_linear_gpu(small, x.reshape(1, 6, 256))
    _check(y.reshape(6, 40), _ref(W, x))
