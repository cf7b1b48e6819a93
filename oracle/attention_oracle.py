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


# ------------------------------------------------------------------------------------------ prompt (prefill) attention
def prefill_ref64(q, K, V, sinks, p0, scaling, sliding=0):
    """Exact-math fp64 sink attention of T prompt queries at positions p0 .. p0+T-1 over a linear cache: each query is
    the decode closed form ``ref64`` at its own position (keys [lo(qp), qp]).  q [T, NQ, HD]; K, V [NKV, S, HD] with
    S >= p0 + T; returns [T, NQ, HD] fp64."""
    q = np.asarray(q, np.float64)
    T = q.shape[0]
    return np.stack([ref64(q[t].reshape(-1), K, V, sinks, p0 + t, scaling, sliding).reshape(NQ, HD)
                     for t in range(T)]) if T else np.zeros((0, NQ, HD))


def prefill_attn_tiled(q, K, V, sinks, p0, scaling, sliding=0, BM=64, BN=64, sink=True, causal_shift=0,
                       window_shift=0):
    """k_prefill_attn's algorithm (reference fused_core.py:684-759), fp32, over a linear cache K, V [NKV, S, HD]:
    query blocks of BM rows; per block keys walk [lo, hi) in tiles of BN, lo = max(first query - sliding + 1, 0)
    rounded down to BN (0 on full layers), hi = one past the block's last query; per tile s = (q . k) * scaling,
    masked to -inf outside j <= qp (and j > qp - sliding); m_new = max(m, max s); alpha = exp(m - m_new);
    p = exp(s - m_new); l = l alpha + sum p; acc = acc alpha + bf16(p) . v; the running state starts at m = sink,
    l = 1.  Output bf16(acc / l) [T, NQ, HD] (fp32 values on the bf16 grid).

    ``sink``, ``causal_shift`` and ``window_shift`` exist only to plant mistakes in tests (drop the sink, attend one
    key past the diagonal, widen the window by one); the defaults are the reference's algorithm."""
    q = np.asarray(q, np.float32)
    T = q.shape[0]
    K = np.asarray(K, np.float32)
    V = np.asarray(V, np.float32)
    kvh = np.arange(NQ) // REP
    sk = np.asarray(sinks, np.float32)
    out = np.zeros((T, NQ, HD), np.float32)
    sc = np.float32(scaling)
    for mb in range((T + BM - 1) // BM):
        offs = mb * BM + np.arange(BM)
        mm = offs < T
        qpos = p0 + offs
        qb = np.where(mm[:, None, None], q[np.minimum(offs, T - 1)], 0).astype(np.float32)   # [BM, NQ, HD]
        qh = qb.transpose(1, 0, 2)                                                           # [NQ, BM, HD]
        m = np.broadcast_to(sk[:, None] if sink else np.float32(-np.inf), (NQ, BM)).astype(np.float32).copy()
        lsum = np.full((NQ, BM), 1.0 if sink else 0.0, np.float32)
        acc = np.zeros((NQ, BM, HD), np.float32)
        hi = min(p0 + mb * BM + BM, p0 + T)
        lo = max(p0 + mb * BM - sliding + 1, 0) if sliding else 0
        lo = (lo // BN) * BN
        for s0 in range(lo, hi, BN):
            j = s0 + np.arange(BN)
            jm = j < hi
            rows = np.minimum(j, hi - 1)
            k = np.where(jm[None, :, None], K[:, rows], 0)[kvh]                                # [NQ, BN, HD]
            v = np.where(jm[None, :, None], V[:, rows], 0)[kvh]
            s = np.matmul(qh, k.transpose(0, 2, 1)) * sc                                      # [NQ, BM, BN]
            ok = (j[None, :] <= qpos[:, None] + causal_shift) & jm[None, :]
            if sliding:
                ok &= j[None, :] > qpos[:, None] - sliding - window_shift
            s = np.where(ok[None], s, -np.inf).astype(np.float32)
            m_new = np.maximum(m, s.max(-1))
            with np.errstate(invalid="ignore"):
                alpha = np.where(m == m_new, 1.0, np.exp(m - m_new)).astype(np.float32)
                p = np.exp(s - m_new[..., None]).astype(np.float32)
            p = np.where(np.isneginf(m_new)[..., None], 0, p).astype(np.float32)
            lsum = lsum * alpha + p.sum(-1, dtype=np.float32)
            acc = acc * alpha[..., None] + np.matmul(rb(p), v).astype(np.float32)
            m = m_new
        with np.errstate(invalid="ignore", divide="ignore"):
            o = acc / lsum[..., None]
        out[offs[mm]] = rb(o.transpose(1, 0, 2)[mm].astype(np.float32))
    return out
