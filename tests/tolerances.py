"""Parity tolerances for attention outputs, stated once for every test.

* float32: per (request, head) row, max |out - ref| <= 1e-5 * max(|ref|)
  (1e-5 relative error, normwise over the head_dim vector), with NaN exactly
  where the reference has NaN. ``ref`` is the float64 oracle.
* float16 / bfloat16: |out - ref| <= 2e-3 absolute (the north star's bound),
  or, where that is larger, the representation limit of the output type: half
  a unit in the last place at |ref| + eps, plus eps, where eps = 2e-5 times the
  row's max |ref| bounds the fp32 accumulation error (a bfloat16 value of
  magnitude >= 1 cannot be stored closer than half an ulp >= 3.9e-3; a result
  within eps of a rounding midpoint may round to either side). NaN exactly
  where the reference has NaN. Against a reference that is itself rounded to
  the output type (the C oracle's output, ``ref_rounded``), two roundings of
  values within eps of each other may differ by one unit in the last place:
  the bound is then one ulp at |ref| + eps, plus eps.
"""
import numpy as np


def ulp(ref, dtype):
    a = np.abs(np.asarray(ref, np.float64))
    if dtype == 'float16':
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    if dtype == 'bfloat16':
        with np.errstate(divide='ignore'):
            e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
        return np.where(a > 0, 2.0 ** (np.maximum(e, -126) - 7), 2.0 ** -133)
    return np.zeros_like(a)


def assert_attention_close(out, ref, dtype, context='', ref_rounded=False):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    nan_out, nan_ref = np.isnan(out), np.isnan(ref)
    assert np.array_equal(nan_out, nan_ref), f'{context}: NaN pattern differs at {np.argwhere(nan_out != nan_ref)[:5]}'
    o = np.where(nan_ref, 0, out)
    r = np.where(nan_ref, 0, ref)
    if dtype == 'float32':
        d = o.shape[-1]
        rows_o, rows_r = o.reshape(-1, d), r.reshape(-1, d)
        err = np.abs(rows_o - rows_r).max(axis=1)
        scale = np.abs(rows_r).max(axis=1)
        bad = err > 1e-5 * np.maximum(scale, 1e-30)
        assert not bad.any(), f'{context}: fp32 rel err {(err / np.maximum(scale, 1e-30))[bad].max():.3e} at rows {np.nonzero(bad)[0][:5]}'
    else:
        d = o.shape[-1]
        eps = 2e-5 * np.abs(r.reshape(-1, d)).max(axis=1, keepdims=True)
        eps = np.broadcast_to(eps, (eps.shape[0], d)).reshape(r.shape)
        tol = np.maximum(2e-3, (1.0 if ref_rounded else 0.5) * ulp(np.abs(r) + eps, dtype) + eps)
        err = np.abs(o - r)
        bad = err > tol
        assert not bad.any(), f'{context}: {dtype} abs err {err[bad].max():.3e} (tol {tol[bad].min():.3e}) at {np.argwhere(bad)[:5]}'
