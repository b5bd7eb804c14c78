"""GPU parity of the model-side entries behind the native decoder loop:
GEMM with the tanh-GELU epilogue (hipBLASLt's fused epilogue and the
separate pass), residual add fused with LayerNorm, and the strided head split
that reads one column block of a fused QKV projection. References are numpy
float64 restatements of the same math (tanh GELU of minitorch/nn.py:222-226,
one-pass LayerNorm of src/layernorm_kernel.cu:37-99)."""
import numpy as np
import pytest

from minitorch_amd.model import model_library, DecoderLM
from minitorch_amd.runtime import DeviceTensor, call, P, I, F
from minitorch_amd.dtypes import dtype_code

pytestmark = pytest.mark.gpu


def gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def to_host(t):
    a = t.to_numpy()
    return np.asarray(a, np.float64)


def round_to(a, dtype):
    return np.asarray(DeviceTensor.from_numpy(np.asarray(a, np.float32), dtype).to_numpy(), np.float64)


@pytest.mark.parametrize('fused', [1, 0])
@pytest.mark.parametrize('dtype', ['float32', 'bfloat16', 'float16'])
def test_gemm_gelu_epilogue(dtype, fused):
    rng = np.random.default_rng(3)
    m, k, n = 37, 256, 384
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((k, n)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(n) * 0.5).astype(np.float32)
    A, W, B = (DeviceTensor.from_numpy(x, dtype) for x in (a, w, b))
    out = DeviceTensor((m, n), dtype)
    blas = DecoderLM(n_vocab=16, n_embd=16, n_head=1, n_layer=1, n_positions=4).blas()
    call(model_library(), 'mt_gemm_epilogue', [P] * 5 + [I] * 6, blas.handle, out.ptr, A.ptr, W.ptr, B.ptr,
         m, n, k, dtype_code(dtype), 1, fused)
    got = to_host(out)
    # reference on the rounded operands; the pre-activation is the fp32 GEMM
    pre = round_to(a, dtype) @ round_to(w, dtype) + round_to(b, dtype)
    ref = gelu64(pre)
    if dtype == 'float32':
        tol = 2e-5 * np.abs(ref).max()
    else:
        # one rounding of the output plus fp32-accumulation noise of the GEMM
        tol = (2 ** -7 if dtype == 'bfloat16' else 2 ** -10) * np.maximum(np.abs(ref), 0.05) + 1e-3
    assert np.all(np.abs(got - ref) <= tol), float(np.max(np.abs(got - ref) / np.maximum(tol, 1e-30)))


@pytest.mark.parametrize('width', [1000, 768, 1024, 2048])
@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_residual_layernorm(dtype, width):
    # widths that are multiples of 256 (up to 2048) take the one-wave-per-row
    # kernel, others the workgroup-per-row kernel
    rng = np.random.default_rng(4)
    rows = 9
    x = (rng.standard_normal((rows, width)) * 3 + 1).astype(np.float32)
    y = rng.standard_normal((rows, width)).astype(np.float32)
    g = rng.standard_normal(width).astype(np.float32)
    be = rng.standard_normal(width).astype(np.float32)
    X = DeviceTensor.from_numpy(x, 'float32')
    Y = DeviceTensor.from_numpy(y, dtype)
    G, Bt = DeviceTensor.from_numpy(g, 'float32'), DeviceTensor.from_numpy(be, 'float32')
    out = DeviceTensor((rows, width), dtype)
    call(model_library(), 'mt_residual_layernorm', [P, P, P, P, P, I, I, F, I], out.ptr, X.ptr, Y.ptr,
         G.ptr, Bt.ptr, rows, width, 1e-5, dtype_code(dtype))
    xs = x.astype(np.float64) + round_to(y, dtype)
    assert np.allclose(to_host(X), xs, rtol=1e-6, atol=1e-6)
    mean = xs.mean(axis=1, keepdims=True)
    var = np.maximum((xs ** 2).mean(axis=1, keepdims=True) - mean ** 2, 0) + 1e-5
    ref = g * ((xs - mean) / np.sqrt(var)) + be
    got = to_host(out)
    if dtype == 'float32':
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    else:
        unit = 2 ** -7 if dtype == 'bfloat16' else 2 ** -10
        assert np.all(np.abs(got - ref) <= unit * np.abs(ref) + 1e-3)


@pytest.mark.parametrize('width', [1000, 768])
@pytest.mark.parametrize('dtype', ['float32', 'bfloat16'])
def test_layernorm_typed(dtype, width):
    rng = np.random.default_rng(5)
    rows = 7
    x = (rng.standard_normal((rows, width)) * 2 - 1).astype(np.float32)
    g = rng.standard_normal(width).astype(np.float32)
    be = rng.standard_normal(width).astype(np.float32)
    X = DeviceTensor.from_numpy(x, 'float32')
    G, Bt = DeviceTensor.from_numpy(g, 'float32'), DeviceTensor.from_numpy(be, 'float32')
    out = DeviceTensor((rows, width), dtype)
    call(model_library(), 'mt_layernorm_typed', [P, P, P, P, I, I, F, I], out.ptr, X.ptr, G.ptr, Bt.ptr,
         rows, width, 1e-5, dtype_code(dtype))
    assert np.array_equal(to_host(X), x)  # the input is not written
    xs = x.astype(np.float64)
    mean = xs.mean(axis=1, keepdims=True)
    var = np.maximum((xs ** 2).mean(axis=1, keepdims=True) - mean ** 2, 0) + 1e-5
    ref = g * ((xs - mean) / np.sqrt(var)) + be
    got = to_host(out)
    if dtype == 'float32':
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    else:
        assert np.all(np.abs(got - ref) <= 2 ** -7 * np.abs(ref) + 1e-3)


@pytest.mark.parametrize('dtype', ['float32', 'float16'])
def test_heads_split_of_fused_qkv_block(dtype):
    rng = np.random.default_rng(5)
    b, n, h, d = 3, 5, 4, 16
    qkv = rng.standard_normal((b, n, 3 * h * d)).astype(np.float32)
    t = DeviceTensor.from_numpy(qkv.reshape(b * n, 3 * h * d), dtype)
    item = 4 if dtype == 'float32' else 2
    host = t.to_numpy().reshape(b, n, 3, h, d)
    for column in range(3):
        out = DeviceTensor((b, h, n, d), dtype)
        call(model_library(), 'mt_heads', [P, P, I, I, I, I, I, I, I], out.ptr, t.ptr + column * h * d * item,
             b, n, h, d, 1, 3 * h * d, dtype_code(dtype))
        assert np.array_equal(out.to_numpy(), host[:, :, column].transpose(0, 2, 1, 3))

