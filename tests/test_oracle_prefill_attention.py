"""Pins of the prompt-attention oracle (oracle/attention_oracle.py: prefill_attn_tiled, prefill_ref64).

prefill_ref64 is the decode closed form ``ref64`` (pinned against an element-by-element loop in
test_oracle_attention.py) applied at every query's own position; here it is checked against that loop directly.
prefill_attn_tiled (k_prefill_attn's tile loop, reference fused_core.py:684-759) is checked against prefill_ref64 on
the north-star tolerance at several tilings, against closed forms (one key, equal keys), and with planted mistakes
(sink dropped, one key past the diagonal, a window one key too wide) that each fail on inputs built to expose them.
"""
import math

import numpy as np
import pytest

from oracle import attention_oracle as ao
from oracle.bf16 import rb

NQ, NKV, REP, HD = ao.NQ, ao.NKV, ao.REP, ao.HD
SC = 0.125
ATOL, RTOL = 2e-2, 1e-2          # expert / attention output tolerance of the north star


def _rn(rng, *shape, scale=1.0):
    return rb((rng.standard_normal(shape) * scale).astype(np.float32))


def _case(rng, T, S):
    return _rn(rng, T, NQ, HD), _rn(rng, NKV, S, HD), _rn(rng, NKV, S, HD), _rn(rng, NQ)


def _within(got, want):
    return bool(np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want)))


def _loop_query(qt, K, V, sinks, qp, sliding):
    """One prompt query (all 64 heads) by an element-by-element loop."""
    out = np.zeros((NQ, HD))
    lo = max(qp - sliding + 1, 0) if sliding else 0
    for hq in range(NQ):
        h = hq // REP
        sc = [float(np.dot(qt[hq].astype(np.float64), K[h, j].astype(np.float64))) * SC for j in range(lo, qp + 1)]
        m = max(sc + [float(sinks[hq])])
        w = [math.exp(s - m) for s in sc]
        den = sum(w) + math.exp(float(sinks[hq]) - m)
        for t, j in enumerate(range(lo, qp + 1)):
            out[hq] += w[t] / den * V[h, j].astype(np.float64)
    return out


@pytest.mark.parametrize("p0,T,W", [(0, 3, 0), (5, 4, 0), (9, 3, 4), (2, 5, 3)])
def test_prefill_ref64_equals_loop(p0, T, W):
    rng = np.random.default_rng(100 * p0 + 10 * T + W)
    q, K, V, sinks = _case(rng, T, p0 + T + 2)
    got = ao.prefill_ref64(q, K, V, sinks, p0, SC, W)
    for t in range(T):
        assert np.allclose(got[t], _loop_query(q[t], K, V, sinks, p0 + t, W), rtol=1e-12, atol=1e-12)


# the reference's prompt-attention cases (tests/test_attention.py:245-246), the small ones
CASES = [(0, 1), (0, 7), (0, 128), (50, 1), (50, 300), (300, 64), (127, 1), (128, 2), (129, 255)]


@pytest.mark.parametrize("p0,T", CASES)
@pytest.mark.parametrize("W", [0, 128])
def test_tiled_oracle_within_tolerance_of_exact(p0, T, W):
    rng = np.random.default_rng(7 * p0 + T + W)
    q, K, V, sinks = _case(rng, T, p0 + T)
    got = ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, W)
    want = ao.prefill_ref64(q, K, V, sinks, p0, SC, W)
    assert _within(got, want)
    assert np.abs(got - want).mean() < 1e-3            # bf16 output rounding and bf16 P only


@pytest.mark.parametrize("bm,bn", [(32, 32), (128, 64), (16, 16), (64, 128)])
def test_tilings_agree_to_rounding(bm, bn):
    """The reference accepts many BM/BN tilings (tests/test_attention.py:322-323); they differ by rounding only."""
    rng = np.random.default_rng(bm + bn)
    q, K, V, sinks = _case(rng, 150, 250)
    a = ao.prefill_attn_tiled(q, K, V, sinks, 100, SC, 128)
    b = ao.prefill_attn_tiled(q, K, V, sinks, 100, SC, 128, BM=bm, BN=bn)
    want = ao.prefill_ref64(q, K, V, sinks, 100, SC, 128)
    assert _within(a, want) and _within(b, want)
    assert np.abs(a - b).max() <= 4 * 2.0 ** -8 * max(1.0, np.abs(want).max())


def test_one_key_closed_form_and_dropped_sink():
    """T = 1 at p0 = 0: one key, o = v0 / (1 + exp(sink - s0)).  Dropping the sink gives o = v0 and fails."""
    rng = np.random.default_rng(3)
    q, K, V, sinks = _case(rng, 1, 1)
    s = np.einsum("hd,hd->h", q[0].astype(np.float64), K[np.arange(NQ) // REP, 0].astype(np.float64)) * SC
    want = V[np.arange(NQ) // REP, 0].astype(np.float64) / (1.0 + np.exp(sinks.astype(np.float64) - s))[:, None]
    assert _within(ao.prefill_attn_tiled(q, K, V, sinks, 0, SC)[0], want)
    assert not _within(ao.prefill_attn_tiled(q, K, V, sinks, 0, SC, sink=False)[0], want)


def test_equal_keys_give_the_window_mean_scaled_by_the_sink():
    """All keys equal (score s for every key): o = mean(V over the window) * n e^s / (n e^s + e^sink)."""
    rng = np.random.default_rng(4)
    T, p0, W = 40, 30, 16
    q, _, V, sinks = _case(rng, T, p0 + T)
    K = np.broadcast_to(_rn(rng, NKV, 1, HD), (NKV, p0 + T, HD)).copy()
    got = ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, W)
    for t in (0, 17, T - 1):
        qp = p0 + t
        lo = max(qp - W + 1, 0)
        n = qp - lo + 1
        for hq in (0, 9, 63):
            h = hq // REP
            s = float(np.dot(q[t, hq].astype(np.float64), K[h, 0].astype(np.float64))) * SC
            wgt = n / (n + math.exp(float(sinks[hq]) - s))
            want = V[h, lo:qp + 1].astype(np.float64).mean(0) * wgt
            assert _within(got[t, hq], want)


def _spike(rng, T, S, j_star, value=4.0):
    """All queries equal to one vector u; every key small except key j_star = 2u (a dominant score, ~16) whose value
    row is ``value``: a query that attends j_star returns about ``value``, any other about 0."""
    u = _rn(rng, HD)
    q = np.broadcast_to(u, (T, NQ, HD)).copy()
    K = _rn(rng, NKV, S, HD, scale=0.05)
    V = _rn(rng, NKV, S, HD, scale=0.05)
    K[:, j_star] = rb(2 * u)
    V[:, j_star] = value
    return q, K, V, _rn(rng, NQ)


def test_planted_causal_mistake_fails():
    rng = np.random.default_rng(5)
    p0, T, t0 = 20, 30, 11
    q, K, V, sinks = _spike(rng, T, p0 + T, p0 + t0 + 1)
    want = ao.prefill_ref64(q, K, V, sinks, p0, SC)
    assert _within(ao.prefill_attn_tiled(q, K, V, sinks, p0, SC), want)
    assert not _within(ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, causal_shift=1), want)


def test_planted_window_mistake_fails():
    rng = np.random.default_rng(6)
    p0, T, W, t0 = 40, 30, 16, 20
    q, K, V, sinks = _spike(rng, T, p0 + T, p0 + t0 - W)
    want = ao.prefill_ref64(q, K, V, sinks, p0, SC, W)
    assert _within(ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, W), want)
    assert not _within(ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, W, window_shift=1), want)


def test_empty_prompt():
    rng = np.random.default_rng(8)
    q, K, V, sinks = _case(rng, 0, 4)
    assert ao.prefill_attn_tiled(q, K, V, sinks, 3, SC).shape == (0, NQ, HD)
