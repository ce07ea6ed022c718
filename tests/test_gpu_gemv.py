"""Fused decode -> GEMV (y = x @ W.T, W decoded inside the kernel) against
decode-then-matmul: the weights are bit-exact, so the reference product is
the fp32 matmul of the original bf16 weights; the bf16 result must agree
within rel 1e-2 / abs 1e-3."""
import numpy as np
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import compress_layer, decompress_matvec_gpu
from afterimage_amd.runtime.device import DeviceTensor, decode_gemv

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _x(batch, cols, seed):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.standard_normal((batch, cols), dtype=np.float32)).to(torch.bfloat16)


def _ref(W, x):
    # fp32 on the GPU, both operands contiguous (no transposed-view products).
    Wf = W.to("cuda").float().contiguous()
    xf = x.to("cuda").float().contiguous()
    return torch.matmul(xf, Wf.t().contiguous())


def _check(y, ref):
    assert y.dtype == torch.bfloat16
    err = (y.float() - ref).abs()
    bound = ATOL + RTOL * ref.abs()
    assert bool((err <= bound).all()), "max excess %.3g" % float((err - bound).max())


@pytest.fixture(scope="module")
def down_proj():
    return workloads.single_layer()


@pytest.mark.parametrize("batch", [1, 4])
def test_down_proj_5120x17408(down_proj, batch):
    W, layer = down_proj
    x = _x(batch, W.shape[1], 17 + batch)
    y = decompress_matvec_gpu(layer, x)
    assert tuple(y.shape) == (batch, W.shape[0])
    _check(y, _ref(W, x))


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("shape,chunk", [((64, 96), 256), ((40, 1000), 4096), ((7, 1024), 16),
                                         ((33, 1001), 512), ((96, 4104), 65536),
                                         ((1500, 200), 65536), ((260, 512), 65536),
                                         ((130, 1032), 65536)])
def test_small_shapes(shape, chunk, batch):
    """Sub-group chunks (16 symbols), rows shorter and longer than a chunk,
    cols % 8 != 0 (element-wise products), and 512-thread chunks whose
    64-group wave steps span several rows (cols 200), exactly one (512) or
    cross a row boundary now and then (1032)."""
    W = workloads.bf16_normal(shape, 5 + shape[1], 0.02, outlier_frac=1e-2)
    layer = compress_layer(W, chunk_size=chunk)
    x = _x(batch, shape[1], shape[0])
    _check(decompress_matvec_gpu(layer, x), _ref(W, x))


def test_vector_x_and_float_input():
    W = workloads.bf16_normal((48, 256), 9, 0.05)
    layer = compress_layer(W, chunk_size=1024)
    x = torch.randn(256)  # float32, 1-D
    y = decompress_matvec_gpu(layer, x)
    assert tuple(y.shape) == (48,)
    _check(y.reshape(1, -1), _ref(W, x.to(torch.bfloat16).reshape(1, -1)))


def test_accumulates_into_given_y_and_rejects_bad_shapes():
    W = workloads.bf16_normal((16, 64), 3, 0.02)
    layer = compress_layer(W, chunk_size=128)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, "cuda")
    x = _x(2, 64, 1).cuda()
    y = torch.full((2, 16), 1.0, dtype=torch.float32, device="cuda")
    decode_gemv(t, x, 16, 64, y)
    ref = _ref(W, x) + 1.0
    assert bool(((y - ref).abs() <= 1e-4 + 1e-4 * ref.abs()).all())
    with pytest.raises(ValueError, match="batch"):
        decode_gemv(t, _x(5, 64, 1).cuda(), 16, 64)
    with pytest.raises(ValueError, match="rows"):
        decode_gemv(t, x, 8, 64)
    with pytest.raises(ValueError, match="2-D"):
        decompress_matvec_gpu(compress_layer(W.reshape(-1)), x[0])
