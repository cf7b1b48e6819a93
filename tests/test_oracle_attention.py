"""Pins of the CPU attention oracle (oracle/attention_oracle.py) by brute force and closed forms.

ref64 (the fp64 closed form of reference tests/test_attention.py:89-99) is checked against an element-by-element
loop on a tiny cache, and both ref64 and attn_bf16 (k_attn's bf16 rounding points, fused_core.py:145-208) against
closed forms that fix the sink term, the window, the ring addressing and the softmax: one key, equal scores, a sink
at -inf (plain softmax attention, computed with scipy), and a ring cache holding the same window as a linear one.
A planted mistake (the sink dropped) fails the one-key closed form.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax

from oracle import attention_oracle as ao
from oracle.bf16 import rb

NKV, REP, HD = ao.NKV, ao.REP, ao.HD


def _case(rng, S, scale=1.0):
    q = rb(rng.standard_normal(ao.NQ * HD).astype(np.float32))
    k = rb((rng.standard_normal((NKV, S, HD)) * scale).astype(np.float32))
    v = rb((rng.standard_normal((NKV, S, HD)) * scale).astype(np.float32))
    sinks = rb(rng.standard_normal(ao.NQ).astype(np.float32))
    return q, k, v, sinks


def _loop_attention(q, k, v, sinks, pos, scaling, sliding):
    """Element by element: for every (kv head, row), score every key in the window, softmax with the sink."""
    out = np.zeros((NKV, REP, HD))
    lo = max(pos - sliding + 1, 0) if sliding else 0
    for h in range(NKV):
        for r in range(REP):
            qi = q.reshape(NKV, REP, HD)[h, r].astype(np.float64)
            scores = [float(np.dot(qi, k[h, j].astype(np.float64))) * scaling for j in range(lo, pos + 1)]
            sink = float(sinks[h * REP + r])
            m = max(scores + [sink])
            w = [math.exp(s - m) for s in scores]
            den = sum(w) + math.exp(sink - m)
            for t, j in enumerate(range(lo, pos + 1)):
                out[h, r] += w[t] / den * v[h, j].astype(np.float64)
    return out.reshape(-1)


@pytest.mark.parametrize("pos,sliding", [(0, 0), (5, 0), (9, 4), (3, 4)])
def test_ref64_equals_loop(pos, sliding):
    rng = np.random.default_rng(pos + 10 * sliding)
    q, k, v, sinks = _case(rng, 12)
    got = ao.ref64(q, k, v, sinks, pos, 0.125, sliding=sliding)
    want = _loop_attention(q, k, v, sinks, pos, 0.125, sliding)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def _one_key_closed_form(q, k, v, sinks, scaling):
    s = np.einsum("hrd,hd->hr", q.reshape(NKV, REP, HD).astype(np.float64), k[:, 0].astype(np.float64)) * scaling
    sk = sinks.reshape(NKV, REP).astype(np.float64)
    wgt = 1.0 / (1.0 + np.exp(sk - s))                     # exp(s) / (exp(s) + exp(sink))
    return (wgt[:, :, None] * v[:, 0][:, None, :].astype(np.float64)).reshape(-1)


def test_one_key_closed_form_and_planted_mistake():
    rng = np.random.default_rng(1)
    q, k, v, sinks = _case(rng, 4)
    want = _one_key_closed_form(q, k, v, sinks, 0.125)
    assert np.allclose(ao.ref64(q, k, v, sinks, 0, 0.125), want, rtol=1e-12, atol=1e-12)
    assert np.abs(ao.attn_bf16(q, k, v, sinks, 0, 0.125) - want).max() < 2e-2
    # planted mistake: attention without the sink term is v0 itself, far from the closed form
    no_sink = np.broadcast_to(v[:, 0][:, None, :], (NKV, REP, HD)).reshape(-1).astype(np.float64)
    assert np.abs(no_sink - want).max() > 0.1


def test_equal_scores_give_the_window_mean_scaled_by_the_sink():
    rng = np.random.default_rng(2)
    _, k, v, sinks = _case(rng, 40)
    q = np.zeros(ao.NQ * HD, np.float32)                   # every score 0
    for pos, sliding in ((29, 0), (29, 8)):
        lo = max(pos - sliding + 1, 0) if sliding else 0
        n = pos - lo + 1
        mean = v[:, lo:pos + 1].astype(np.float64).mean(axis=1)          # [NKV, HD]
        sk = sinks.reshape(NKV, REP).astype(np.float64)
        m = np.maximum(sk, 0.0)
        frac = n * np.exp(-m) / (n * np.exp(-m) + np.exp(sk - m))        # share of the keys vs the sink
        want = (frac[:, :, None] * mean[:, None, :]).reshape(-1)
        assert np.allclose(ao.ref64(q, k, v, sinks, pos, 0.125, sliding), want, rtol=1e-12, atol=1e-12)
        assert np.abs(ao.attn_bf16(q, k, v, sinks, pos, 0.125, sliding) - want).max() < 2e-2


def test_sink_at_minus_infinity_is_plain_softmax_attention():
    rng = np.random.default_rng(3)
    q, k, v, _ = _case(rng, 50)
    sinks = np.full(ao.NQ, -1e30, np.float32)
    pos = 37
    s = np.einsum("hrd,hnd->hrn", q.reshape(NKV, REP, HD).astype(np.float64), k[:, :pos + 1].astype(np.float64))
    want = np.einsum("hrn,hnd->hrd", softmax(s * 0.125, axis=-1), v[:, :pos + 1].astype(np.float64)).reshape(-1)
    assert np.allclose(ao.ref64(q, k, v, sinks, pos, 0.125), want, rtol=1e-10, atol=1e-12)


def test_ring_cache_equals_linear_cache():
    rng = np.random.default_rng(4)
    q, k, v, sinks = _case(rng, 400)
    R, W = 128, 128
    for pos in (0, 100, 127, 128, 300, 399):
        kr = rb(rng.standard_normal((NKV, R, HD)).astype(np.float32) * 3)       # stale slots hold garbage
        vr = rb(rng.standard_normal((NKV, R, HD)).astype(np.float32) * 3)
        js = np.arange(max(0, pos - W + 1), pos + 1)
        kr[:, js % R] = k[:, js]
        vr[:, js % R] = v[:, js]
        assert np.array_equal(ao.ref64(q, k, v, sinks, pos, 0.125, W), ao.ref64(q, kr, vr, sinks, pos, 0.125, W, R))
        assert np.array_equal(ao.attn_bf16(q, k, v, sinks, pos, 0.125, W),
                              ao.attn_bf16(q, kr, vr, sinks, pos, 0.125, W, R))


def test_bf16_rounding_variant_stays_within_tolerance_of_fp64():
    rng = np.random.default_rng(5)
    q, k, v, sinks = _case(rng, 2048)
    for pos, sliding in ((2047, 0), (1000, 128), (64, 0)):
        d = np.abs(ao.attn_bf16(q, k, v, sinks, pos, 0.125, sliding) - ao.ref64(q, k, v, sinks, pos, 0.125, sliding))
        assert d.max() < 2e-2, (pos, sliding, d.max())
