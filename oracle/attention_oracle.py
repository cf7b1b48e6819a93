"""GQA decode attention with learned sinks, restated on the CPU (test infrastructure; see oracle/__init__.py).

Shapes (reference fused_core.py:63): NQ = 64 query heads, NKV = 8 KV heads, HD = 64, REP = 8 query heads per KV head.
q [NQ*HD] (RoPE and the attention scale handling are the caller's), K/V caches [NKV, S, HD] per sequence, sinks [NQ].
"""
import numpy as np

from .bf16 import rb

NQ, NKV, HD = 64, 8, 64
REP = NQ // NKV


def key_range(pos: int, sliding: int):
    """Keys attended by the query at ``pos``: [lo, pos] with lo = max(pos - sliding + 1, 0) on sliding layers
    (reference fused_core.py:153-156)."""
    lo = max(pos - sliding + 1, 0) if sliding else 0
    return lo, pos


def cache_rows(j: np.ndarray, ring: int) -> np.ndarray:
    """Cache row of absolute key position j: j itself (linear cache) or j % ring (rolling cache, fused_core.py:174-177)."""
    return j % ring if ring else j


def ref64(q, kc, vc, sinks, pos, scaling, sliding=0, ring=0):
    """Exact-math fp64 sink attention of one decode query (the closed form of reference tests/test_attention.py:89-99):
    s = scaling * q.k ; m = max(sink, max s) ; out = sum_j exp(s_j - m) v_j / (sum_j exp(s_j - m) + exp(sink - m))."""
    lo, hi = key_range(pos, sliding)
    j = np.arange(lo, hi + 1)
    rows = cache_rows(j, ring)
    qd = np.asarray(q, np.float64).reshape(NKV, REP, HD)
    k = np.asarray(kc, np.float64)[:, rows]                 # [NKV, n, HD]
    v = np.asarray(vc, np.float64)[:, rows]
    s = np.einsum("hrd,hnd->hrn", qd, k) * scaling
    sk = np.asarray(sinks, np.float64).reshape(NKV, REP, 1)
    m = np.maximum(s.max(-1, keepdims=True), sk)
    e = np.exp(s - m)
    den = e.sum(-1, keepdims=True) + np.exp(sk - m)
    return np.einsum("hrn,hnd->hrd", e / den, v).reshape(-1)


def attn_bf16(q, kc, vc, sinks, pos, scaling, sliding=0, ring=0):
    """k_attn's rounding points (reference fused_core.py:145-208): s = bf16(bf16(q.k) * scaling) with q.k accumulated
    in fp32; m = max(sink, max_j s_j); S = exp(bf16(sink - m)) + sum_j exp(bf16(s_j - m)); p_j = bf16(exp(bf16(s_j - m))
    / S); out = bf16(sum_j p_j v_j).  Sums are taken in fp64 here (the reference's fp32 summation order is
    layout-dependent and not reproducible); every rounding point above is reproduced exactly."""
    lo, hi = key_range(pos, sliding)
    j = np.arange(lo, hi + 1)
    rows = cache_rows(j, ring)
    qf = np.asarray(q, np.float32).reshape(NKV, REP, HD).astype(np.float64)
    k = np.asarray(kc, np.float32)[:, rows].astype(np.float64)
    v = np.asarray(vc, np.float32)[:, rows].astype(np.float64)
    dot = np.einsum("hrd,hnd->hrn", qf, k).astype(np.float32)
    s = rb(rb(dot) * np.float32(scaling))
    sink = np.asarray(sinks, np.float32).reshape(NKV, REP, 1)
    m = np.maximum(s.max(-1, keepdims=True), sink)
    e = np.exp(rb(s - m).astype(np.float64))
    S = np.exp(rb(sink - m).astype(np.float64)) + e.sum(-1, keepdims=True)
    p = rb((e / S).astype(np.float32)).astype(np.float64)
    out = np.einsum("hrn,hnd->hrd", p, v)
    return rb(out.astype(np.float32)).reshape(-1)
