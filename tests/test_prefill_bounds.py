"""The bounds of the far-below-block-maximum GEMM test, checked on the CPU for what they catch: a model of the E4M3
hi + lo activation rows (OCP E4M3: round to nearest even on a 4-significant-bit grid down to 2^-6, multiples of 2^-9
below) stays inside both bounds, and the same model without the lo row (a kernel that drops it) breaks both.
"""
import numpy as np

import far_below
from oracle import mxfp4_oracle as mo


def _e4m3(v):
    a = np.abs(v)
    q = np.where(a >= 2.0 ** -6, np.exp2(np.floor(np.log2(np.maximum(a, 2.0 ** -300))) - 3), 2.0 ** -9)
    return np.round(v / q) * q


def _scale(m):
    return np.exp2(np.maximum(np.floor(np.log2(np.maximum(m, 2.0 ** -300))) - 7, -126))


def _quantised(x, with_lo):
    xb = np.asarray(x, np.float64).reshape(x.shape[0], -1, 32)
    s_hi = _scale(np.abs(xb).max(-1, keepdims=True))
    q = _e4m3(xb / s_hi) * s_hi
    if with_lo:
        r = xb - q
        s_lo = _scale(np.abs(r).max(-1, keepdims=True))
        q = q + _e4m3(r / s_lo) * s_lo
    return q.reshape(x.shape)


def test_far_below_bounds_catch_a_dropped_lo_row():
    slot, x = far_below.case(M=8)
    W = mo.expert_weights(slot)[0].astype(np.float64)
    want, bound, rms = far_below.bounds(x, W)
    good = np.abs(_quantised(x, True) @ W.T - want)
    assert (good <= bound).all() and (good <= 2.0 ** -2 * rms).all()
    bad = np.abs(_quantised(x, False) @ W.T - want)
    assert (bad > bound).any() and (bad > 2.0 ** -2 * rms).any()


def test_far_below_case_shape():
    slot, x = far_below.case(M=4)
    xb = np.abs(x).reshape(4, 90, 32)
    m = xb[:, :, 0]
    assert (xb[:, :, 1:].max(-1) < m * 2.0 ** -15).all() and (xb[:, :, 1:].min(-1) >= m * 2.0 ** -21).all()
    assert not mo.expert_weights(slot)[0][:, ::32].any()
