"""GPU parity of the decode projection kernel (mt_decode_projection) and of
the residual + LayerNorm that reduces its split partial sums
(mt_residual_layernorm_partials), against float64 numpy on the same rounded
operands.

Tolerances: the fp32 partial sums may differ from the fp64 product by the fp32
accumulation error, bounded here by 1e-5 * sum_k |x||w| (a dropped or doubled
term is of order |x||w| and fails it at these k); a rounded output may differ
by half a unit in the last place of its type at |ref| + that bound, plus the
bound itself. The decoder-level effect (tokens of the captured and eager
steps, logits against the fp64 GPT-2 oracle) is covered by the model tests.
"""
import numpy as np
import pytest

from minitorch_amd.model import model_library
from minitorch_amd.runtime import DeviceTensor, call, P, I, F
from minitorch_amd.dtypes import dtype_code

pytestmark = pytest.mark.gpu

PROJ = [P, P, P, P, I, I, I, I, I, I, I]
LN_PARTIALS = [P, P, P, I, P, P, P, I, I, F, I, I]
MANT = {'bfloat16': 7, 'float16': 10}


def host(t):
    return np.asarray(t.to_numpy(), np.float64)


def rounded(a, dtype):
    t = DeviceTensor.from_numpy(np.asarray(a, np.float32), dtype)
    return t, host(t)


def half_ulp(v, dtype):
    """Half the spacing of dtype's values at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14)))
    return 0.5 * 2.0 ** (e - MANT[dtype])


def gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


CASES = [
    # m, n, k, splits, epilogue
    (1, 64, 128, 1, 0),
    (16, 256, 256, 1, 1),
    (17, 768, 768, 2, 2),
    (37, 384, 256, 1, 1),
    (64, 128, 1024, 8, 2),
    (128, 3072, 1024, 1, 0),
    (128, 1024, 1024, 4, 2),
    (128, 4096, 1024, 1, 1),
    (128, 1024, 4096, 8, 2),
    (200, 2304, 768, 1, 0),
    (256, 768, 3072, 4, 2),
    (150, 1024, 4096, 4, 2),
    # more than 32 rows with 8 splits
    (150, 1024, 4096, 8, 2),
    (40, 768, 3072, 8, 2),
    (128, 1024, 1024, 8, 2),
]


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('m,n,k,splits,epilogue', CASES)
def test_decode_projection(dtype, m, n, k, splits, epilogue):
    rng = np.random.default_rng([m, n, k, splits, epilogue])
    x = rng.standard_normal((m, k))
    w = rng.standard_normal((n, k)) * 0.05
    b = rng.standard_normal(n) * 0.5
    X, xr = rounded(x, dtype)
    W, wr = rounded(w, dtype)
    B, br = rounded(b, dtype)
    bound = 1e-5 * (np.abs(xr) @ np.abs(wr).T) + 1e-7
    prod = xr @ wr.T
    if epilogue == 2:
        out = DeviceTensor((splits, m, n), 'float32')
        call(model_library(), 'mt_decode_projection', PROJ, out.ptr, X.ptr, W.ptr, 0, m, n, k, splits, 2,
             dtype_code(dtype), 0)
        got = host(out)
        kc = k // splits
        for s in range(splits):
            ref = xr[:, s * kc:(s + 1) * kc] @ wr[:, s * kc:(s + 1) * kc].T
            assert np.all(np.abs(got[s] - ref) <= bound), f'split {s}: {np.max(np.abs(got[s] - ref) / bound)}'
        assert np.all(np.abs(got.sum(axis=0) - prod) <= bound)
        return
    out = DeviceTensor((m, n), dtype)
    call(model_library(), 'mt_decode_projection', PROJ, out.ptr, X.ptr, W.ptr, B.ptr, m, n, k, 1, epilogue,
         dtype_code(dtype), 0)
    pre = prod + br
    if epilogue == 1:
        ref = gelu64(pre)
        err = bound * 1.2 + 1e-6   # |gelu'| <= 1.13
    else:
        ref = pre
        err = bound
    got = host(out)
    tol = half_ulp(np.abs(ref) + err, dtype) + err
    assert np.all(np.abs(got - ref) <= tol), float(np.max(np.abs(got - ref) / tol))


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
def test_decode_projection_without_bias(dtype):
    rng = np.random.default_rng(7)
    m, n, k = 5, 512, 384
    X, xr = rounded(rng.standard_normal((m, k)), dtype)
    W, wr = rounded(rng.standard_normal((n, k)) * 0.05, dtype)
    out = DeviceTensor((m, n), dtype)
    call(model_library(), 'mt_decode_projection', PROJ, out.ptr, X.ptr, W.ptr, 0, m, n, k, 1, 0, dtype_code(dtype), 0)
    ref = xr @ wr.T
    err = 1e-5 * (np.abs(xr) @ np.abs(wr).T) + 1e-7
    assert np.all(np.abs(host(out) - ref) <= half_ulp(np.abs(ref) + err, dtype) + err)


def test_decode_projection_rejects_unsupported_shapes():
    X = DeviceTensor((300, 1024), 'bfloat16')
    W = DeviceTensor((1024, 1024), 'bfloat16')
    out = DeviceTensor((8, 300, 1024), 'float32')
    lib, bf = model_library(), dtype_code('bfloat16')
    bad = [
        (257, 1024, 1024, 1, 0, bf),    # more rows than the kernel takes
        (4, 40, 1024, 1, 0, bf),        # n not a multiple of 16
        (4, 1024, 100, 1, 0, bf),       # k not a multiple of 32
        (4, 1024, 1024, 3, 2, bf),      # splits not a power of two
        (4, 1024, 1024, 16, 2, bf),     # more than 8 splits
        (4, 1024, 96, 2, 2, bf),        # a split's k range not a whole number of 32-wide steps
        (128, 1024, 4096, 1, 0, bf),    # k range too long for the waves of one workgroup
        (4, 1024, 1024, 2, 0, bf),      # a split needs the partial-sum epilogue
        (4, 1024, 1024, 1, 3, bf),      # no such epilogue
        (4, 1024, 1024, 1, 0, 0),       # fp32 is not taken
        (0, 1024, 1024, 1, 0, bf),
    ]
    for m, n, k, s, e, d in bad:
        with pytest.raises(RuntimeError):
            call(lib, 'mt_decode_projection', PROJ, out.ptr, X.ptr, W.ptr, 0, m, n, k, s, e, d, 0)
    with pytest.raises(RuntimeError):  # misaligned activations
        call(lib, 'mt_decode_projection', PROJ, out.ptr, X.ptr + 2, W.ptr, 0, 4, 1024, 1024, 1, 0, bf, 0)
    for m, n, k, s, e, layout in [(4, 1024, 1024, 2, 2, 2),   # split partials are written row-major
                                  (4, 1024, 1024, 2, 2, 3),
                                  (4, 48, 1024, 1, 0, 2),     # a tiled output needs n a multiple of 32
                                  (4, 1024, 1024, 1, 0, 8),   # no such layout bit
                                  (4, 1024, 1024, 1, 0, -1)]:
        with pytest.raises(RuntimeError):
            call(lib, 'mt_decode_projection', PROJ, out.ptr, X.ptr, W.ptr, 0, m, n, k, s, e, bf, layout)


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('width,splits,bias', [(1024, 4, True), (768, 1, True), (2048, 8, False), (1024, 2, False),
                                               (768, 3, True)])
def test_residual_layernorm_partials(dtype, width, splits, bias):
    rng = np.random.default_rng([width, splits])
    rows = 37
    x = (rng.standard_normal((rows, width)) * 3 + 1).astype(np.float32)
    part = rng.standard_normal((splits, rows, width)).astype(np.float32)
    g = rng.standard_normal(width).astype(np.float32)
    be = rng.standard_normal(width).astype(np.float32)
    X = DeviceTensor.from_numpy(x, 'float32')
    Pt = DeviceTensor.from_numpy(part, 'float32')
    Bv, bv = rounded(rng.standard_normal(width), dtype)
    G, Bt = DeviceTensor.from_numpy(g, 'float32'), DeviceTensor.from_numpy(be, 'float32')
    out = DeviceTensor((rows, width), dtype)
    call(model_library(), 'mt_residual_layernorm_partials', LN_PARTIALS, out.ptr, X.ptr, Pt.ptr, splits,
         Bv.ptr if bias else 0, G.ptr, Bt.ptr, rows, width, 1e-5, dtype_code(dtype), 0)
    xs = x.astype(np.float64) + part.astype(np.float64).sum(axis=0) + (bv if bias else 0.0)
    assert np.allclose(host(X), xs, rtol=1e-6, atol=1e-5)
    mean = xs.mean(axis=1, keepdims=True)
    var = np.maximum((xs ** 2).mean(axis=1, keepdims=True) - mean ** 2, 0) + 1e-5
    ref = g * ((xs - mean) / np.sqrt(var)) + be
    err = 1e-5 * (np.abs(g) * np.abs((xs - mean) / np.sqrt(var)) + 1)
    assert np.all(np.abs(host(out) - ref) <= half_ulp(np.abs(ref) + err, dtype) + err)


def test_residual_layernorm_partials_rejects():
    X = DeviceTensor((4, 1000), 'float32')
    Pt = DeviceTensor((9, 4, 1000), 'float32')
    G = DeviceTensor((1000,), 'float32')
    out = DeviceTensor((4, 1000), 'bfloat16')
    lib = model_library()
    for rows, width, splits, d in [(4, 1000, 1, 2), (4, 768, 9, 2), (4, 768, 0, 2), (4, 768, 1, 0), (0, 768, 1, 2),
                                   (4, 2304, 1, 2)]:
        with pytest.raises(RuntimeError):
            call(lib, 'mt_residual_layernorm_partials', LN_PARTIALS, out.ptr, X.ptr, Pt.ptr, splits, 0, G.ptr,
                 G.ptr, rows, width, 1e-5, d, 0)
    with pytest.raises(RuntimeError):  # layout 1 (tiled input) means nothing here
        call(lib, 'mt_residual_layernorm_partials', LN_PARTIALS, out.ptr, X.ptr, Pt.ptr, 1, 0, G.ptr,
             G.ptr, 4, 768, 1e-5, 2, 1)


PROJ_LN = [P, P, P, P, I, P, P, P, F, P, P, I, I, I, I, I, I]


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('m,n,k,splits,epilogue', [(1, 2304, 768, 0, 0), (2, 3072, 768, 4, 1), (8, 4096, 1024, 2, 1),
                                                    (5, 3072, 1024, 1, 0), (16, 256, 256, 4, 0)])
def test_decode_projection_layernorm_prologue(dtype, m, n, k, splits, epilogue):
    run_layernorm_prologue(dtype, m, n, k, splits, epilogue, 0)


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('m,n,k,splits,epilogue', [(1, 2304, 768, 0, 0), (2, 4096, 1024, 4, 1), (8, 3072, 1024, 2, 0)])
def test_decode_projection_layernorm_prologue_tiled_weights(dtype, m, n, k, splits, epilogue):
    """layout 4 (tiled weights) gives bit for bit the row-major result."""
    got = run_layernorm_prologue(dtype, m, n, k, splits, epilogue, 4)
    assert np.array_equal(got, run_layernorm_prologue(dtype, m, n, k, splits, epilogue, 0))


def run_layernorm_prologue(dtype, m, n, k, splits, epilogue, layout):
    rng = np.random.default_rng([m, n, k, splits, epilogue, 1])
    x = (rng.standard_normal((m, k)) * 2 + 0.5).astype(np.float32)
    part = rng.standard_normal((max(splits, 1), m, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    be = (0.1 * rng.standard_normal(k)).astype(np.float32)
    X, Xo = DeviceTensor.from_numpy(x, 'float32'), DeviceTensor((m, k), 'float32')
    Pt = DeviceTensor.from_numpy(part, 'float32')
    PB, pb = rounded(rng.standard_normal(k) * 0.5, dtype)
    G, Bt = DeviceTensor.from_numpy(g, 'float32'), DeviceTensor.from_numpy(be, 'float32')
    W, wr = rounded(rng.standard_normal((n, k)) * 0.05, dtype)
    if layout & 4:
        W = DeviceTensor.from_numpy(tiled(wr).astype(np.float32), dtype)
    B, br = rounded(rng.standard_normal(n) * 0.5, dtype)
    out = DeviceTensor((m, n), dtype)
    call(model_library(), 'mt_decode_projection_ln', PROJ_LN, out.ptr, X.ptr, Xo.ptr, Pt.ptr if splits else 0,
         splits, PB.ptr if splits else 0, G.ptr, Bt.ptr, 1e-5, W.ptr, B.ptr, m, n, k, epilogue, dtype_code(dtype),
         layout)
    v = x.astype(np.float64) + (part.astype(np.float64).sum(axis=0) + pb if splits else 0.0)
    assert np.allclose(host(Xo), v, rtol=1e-6, atol=1e-5)
    assert np.array_equal(X.to_numpy(), x)
    mean = v.mean(axis=1, keepdims=True)
    var = np.maximum((v ** 2).mean(axis=1, keepdims=True) - mean ** 2, 0) + 1e-5
    hn = g * ((v - mean) / np.sqrt(var)) + be
    # h is rounded to dtype from an fp32 computation: within one unit in the
    # last place of the fp64 value; that unit, carried through |w|, plus the
    # fp32 accumulation bound
    h_err = 2 * half_ulp(np.abs(hn) + 1e-4, dtype) + 1e-5
    pre = hn @ wr.T + br
    err = np.abs(h_err) @ np.abs(wr).T + 1e-5 * (np.abs(hn) @ np.abs(wr).T) + 1e-6
    if epilogue == 1:
        ref, err = gelu64(pre), err * 1.2 + 1e-6
    else:
        ref = pre
    got = host(out)
    tol = half_ulp(np.abs(ref) + err, dtype) + err
    assert np.all(np.abs(got - ref) <= tol), float(np.max(np.abs(got - ref) / tol))
    return got


def test_decode_projection_layernorm_prologue_rejects():
    X, Xo = DeviceTensor((16, 1280), 'float32'), DeviceTensor((16, 1280), 'float32')
    Pt = DeviceTensor((4, 16, 1280), 'float32')
    G = DeviceTensor((1280,), 'float32')
    W = DeviceTensor((1024, 1280), 'bfloat16')
    out = DeviceTensor((16, 1024), 'bfloat16')
    lib, bf = model_library(), dtype_code('bfloat16')

    def run(x_out=Xo.ptr, part=Pt.ptr, splits=4, part_bias=0, m=4, n=1024, k=1024, epi=0, d=bf, layout=0):
        call(lib, 'mt_decode_projection_ln', PROJ_LN, out.ptr, X.ptr, x_out, part, splits, part_bias, G.ptr, G.ptr,
             1e-5, W.ptr, 0, m, n, k, epi, d, layout)
    run()  # valid
    for kw in [dict(x_out=X.ptr), dict(k=1280), dict(k=640), dict(splits=3), dict(splits=0), dict(part=0),
               dict(part=0, splits=0, part_bias=G.ptr), dict(m=17), dict(m=0), dict(n=40), dict(epi=2), dict(d=0),
               dict(layout=1), dict(layout=2), dict(layout=5)]:
        with pytest.raises(RuntimeError):
            run(**kw)


def tiled(a, fill=np.nan):
    """[rows, width] -> the fragment-tiled layout of mt_decode_projection
    (flat, ceil(rows / 16) * 16 rows, padding rows set to `fill`): block
    (R, K) of 16 rows x 32 columns at (R * width / 32 + K) * 512, element
    (r, c) of the block at ((c // 8) * 16 + r) * 8 + c % 8."""
    rows, width = a.shape
    mp = -(-rows // 16) * 16
    p = np.full((mp, width), fill, np.float64)
    p[:rows] = a
    # [R, r, K, g, e] -> [R, K, g, r, e]
    return p.reshape(mp // 16, 16, width // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)


def untiled(flat, rows, width):
    mp = -(-rows // 16) * 16
    return np.asarray(flat, np.float64).reshape(mp // 16, width // 32, 4, 16, 8).transpose(
        0, 3, 1, 2, 4).reshape(mp, width)[:rows]


def test_tiled_layout_helpers_invert():
    a = np.arange(37 * 64, dtype=np.float64).reshape(37, 64)
    t = tiled(a)
    assert t.size == 48 * 64
    # element (r, c) sits where the layout's formula puts it
    for r, c in [(0, 0), (5, 9), (16, 31), (17, 32), (36, 63)]:
        assert t[((r // 16) * 2 + c // 32) * 512 + (((c // 8) % 4) * 16 + r % 16) * 8 + c % 8] == a[r, c]
    assert np.array_equal(untiled(t, 37, 64), a)


TILED_CASES = [
    # m, n, k, splits, epilogue, layout
    (1, 64, 128, 1, 0, 1),
    (9, 2304, 768, 1, 0, 3),
    (17, 768, 768, 2, 2, 1),
    (37, 3072, 768, 1, 1, 3),
    (128, 3072, 1024, 1, 0, 1),
    (128, 4096, 1024, 1, 1, 3),
    (128, 1024, 4096, 4, 2, 1),
    (128, 1024, 4096, 8, 2, 1),
    (150, 1024, 1024, 1, 1, 2),
    (150, 4096, 1024, 1, 1, 3),
    (150, 1024, 4096, 4, 2, 1),
    (256, 768, 3072, 4, 2, 1),
    # tiled weights (layout bit 2)
    (1, 64, 128, 1, 0, 4),
    (2, 2304, 768, 1, 1, 4),
    (9, 2304, 768, 1, 0, 7),
    (17, 768, 768, 2, 2, 5),
    (16, 1024, 4096, 4, 2, 4),
    (128, 3072, 1024, 1, 0, 5),
    (128, 4096, 1024, 1, 1, 7),
    (128, 1024, 4096, 4, 2, 5),
    (150, 1024, 1024, 1, 1, 6),
]


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('m,n,k,splits,epilogue,layout', TILED_CASES)
def test_decode_projection_tiled_layouts(dtype, m, n, k, splits, epilogue, layout):
    """The tiled layouts give bit for bit the row-major results (the same
    products summed in the same order), with NaN in the padding rows of a
    tiled input, and match the float64 product."""
    rng = np.random.default_rng([m, n, k, splits, epilogue, layout])
    x = rng.standard_normal((m, k))
    X, xr = rounded(x, dtype)
    XT = DeviceTensor.from_numpy(tiled(xr).astype(np.float32), dtype) if layout & 1 else X
    W, wr = rounded(rng.standard_normal((n, k)) * 0.05, dtype)
    WT = DeviceTensor.from_numpy(tiled(wr).astype(np.float32), dtype) if layout & 4 else W
    B, br = rounded(rng.standard_normal(n) * 0.5, dtype)
    lib, code = model_library(), dtype_code(dtype)
    if epilogue == 2:
        ref_out, out = DeviceTensor((splits, m, n), 'float32'), DeviceTensor((splits, m, n), 'float32')
        call(lib, 'mt_decode_projection', PROJ, ref_out.ptr, X.ptr, W.ptr, 0, m, n, k, splits, 2, code, 0)
        call(lib, 'mt_decode_projection', PROJ, out.ptr, XT.ptr, WT.ptr, 0, m, n, k, splits, 2, code, layout)
        got, want = host(out), host(ref_out)
        assert np.array_equal(got, want)
        bound = 1e-5 * (np.abs(xr) @ np.abs(wr).T) + 1e-7
        assert np.all(np.abs(got.sum(axis=0) - xr @ wr.T) <= bound)
        return
    ref_out = DeviceTensor((m, n), dtype)
    call(lib, 'mt_decode_projection', PROJ, ref_out.ptr, X.ptr, W.ptr, B.ptr, m, n, k, 1, epilogue, code, 0)
    mp = -(-m // 16) * 16
    out = DeviceTensor((mp * n,) if layout & 2 else (m, n), dtype)
    call(lib, 'mt_decode_projection', PROJ, out.ptr, XT.ptr, WT.ptr, B.ptr, m, n, k, 1, epilogue, code, layout)
    got = untiled(host(out), m, n) if layout & 2 else host(out)
    want = host(ref_out)
    assert np.array_equal(got, want)
    pre = xr @ wr.T + br
    ref = gelu64(pre) if epilogue == 1 else pre
    err = (1e-5 * (np.abs(xr) @ np.abs(wr).T) + 1e-7) * (1.2 if epilogue == 1 else 1.0) + 1e-6 * epilogue
    assert np.all(np.abs(got - ref) <= half_ulp(np.abs(ref) + err, dtype) + err)


@pytest.mark.parametrize('dtype', ['bfloat16', 'float16'])
@pytest.mark.parametrize('rows,width,splits', [(37, 1024, 4), (128, 768, 8), (5, 2048, 1)])
def test_residual_layernorm_partials_tiled_output(dtype, rows, width, splits):
    """layout 2 writes the same rounded values as layout 0, in the tiled
    order; the residual stream is updated the same way."""
    rng = np.random.default_rng([rows, width, splits, 2])
    x = (rng.standard_normal((rows, width)) * 3 + 1).astype(np.float32)
    part = rng.standard_normal((splits, rows, width)).astype(np.float32)
    Pt = DeviceTensor.from_numpy(part, 'float32')
    Bv, _ = rounded(rng.standard_normal(width), dtype)
    G = DeviceTensor.from_numpy((1 + 0.1 * rng.standard_normal(width)).astype(np.float32), 'float32')
    Bt = DeviceTensor.from_numpy((0.1 * rng.standard_normal(width)).astype(np.float32), 'float32')
    lib, code = model_library(), dtype_code(dtype)
    outs = []
    for layout in (0, 2):
        X = DeviceTensor.from_numpy(x, 'float32')
        out = DeviceTensor((-(-rows // 16) * 16 * width,) if layout else (rows, width), dtype)
        call(lib, 'mt_residual_layernorm_partials', LN_PARTIALS, out.ptr, X.ptr, Pt.ptr, splits, Bv.ptr, G.ptr,
             Bt.ptr, rows, width, 1e-5, code, layout)
        outs.append((host(X), untiled(host(out), rows, width) if layout else host(out)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
