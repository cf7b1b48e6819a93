"""Prompt (prefill) attention on the GPU (neural_amd.attention.prefill_attention -> na_prefill_attention, ring_write ->
na_ring_write) against the CPU oracle.

Mirrors the reference's prompt-attention tests (reference tests/test_attention.py:240-311): q/k/v ~ N(0,1) bf16,
sinks ~ N(0,1) bf16, scaling 1/8, window 128, ring 128.  Bars: every output within 2e-2 + 1e-2 |want| of the oracle's
k_prefill_attn restatement and of the fp64 closed form, mean error no worse than the oracle's own against fp64 plus
a bf16 rounding; ring mode (keys < p0 from the rolling cache, the block's own K/V from a strided view) bit-identical
to linear mode; ring_write stores exactly the last min(T, ring) positions; a chained multi-block prompt plus a decode
continuation equal between ring and linear caches; rows past T untouched.
"""
import numpy as np
import pytest

from oracle import attention_oracle as ao
from oracle.bf16 import rb

pytestmark = pytest.mark.gpu

NQ, NKV, HD = ao.NQ, ao.NKV, ao.HD
SC, W, RING = 0.125, 128, 128
ATOL, RTOL = 2e-2, 1e-2


def _dev():
    import torch
    return torch.device("cuda", 0)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(dev)


def _np(t):
    import torch
    return t.to(torch.float32).cpu().numpy()


def _rn(rng, *shape, scale=1.0):
    return rb((rng.standard_normal(shape) * scale).astype(np.float32))


CASES = [(0, 1), (0, 7), (0, 128), (0, 700), (50, 1), (50, 300), (300, 64), (1000, 129), (127, 1), (128, 2),
         (129, 255), (4000, 1100)]


@pytest.mark.parametrize("p0,T", CASES)
@pytest.mark.parametrize("sliding", [0, W])
def test_prefill_attention_vs_oracle(p0, T, sliding):
    import torch
    from neural_amd import attention as A
    dev = _dev()
    rng = np.random.default_rng(p0 * 7 + T + sliding)
    S = p0 + T + 5
    K, V = _rn(rng, NKV, S, HD), _rn(rng, NKV, S, HD)
    q, sinks = _rn(rng, T, NQ, HD), _rn(rng, NQ)
    print(f"prefill attention p0={p0} T={T} window={sliding}", flush=True)
    o = A.prefill_attention(_t(q, dev), _t(K[None], dev), _t(V[None], dev), _t(sinks, dev), p0, SC, sliding, S)
    torch.cuda.synchronize()
    got = _np(o)
    want = ao.prefill_attn_tiled(q, K, V, sinks, p0, SC, sliding)
    rows = np.arange(T) if T <= 300 else np.linspace(0, T - 1, 64).astype(int)
    exact = np.stack([ao.ref64(q[t].reshape(-1), K, V, sinks, p0 + t, SC, sliding).reshape(NQ, HD) for t in rows])
    assert np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want)), np.abs(got - want).max()
    assert np.all(np.abs(got[rows] - exact) <= ATOL + RTOL * np.abs(exact))
    e_gpu = np.abs(got[rows] - exact).mean()
    e_orc = np.abs(want[rows] - exact).mean()
    assert e_gpu <= 1.25 * e_orc + 2e-4, (e_gpu, e_orc)


def _ring_from_linear(rng, K, V, p0):
    """A rolling cache holding positions max(0, p0 - RING) .. p0 - 1 of the linear cache, stale values elsewhere."""
    kr, vr = _rn(rng, NKV, RING, HD, scale=5.0), _rn(rng, NKV, RING, HD, scale=5.0)
    js = np.arange(max(0, p0 - RING), p0)
    kr[:, js % RING] = K[:, js]
    vr[:, js % RING] = V[:, js]
    return kr, vr


@pytest.mark.parametrize("p0,T", CASES)
def test_ring_mode_equals_linear_and_ring_write(p0, T):
    """reference tests/test_attention.py:240-280: ring == linear (torch.equal) with the block's V a strided view of a
    wider row, then ring_write leaves the last min(T, ring) positions in their slots."""
    import torch
    from neural_amd import attention as A
    dev = _dev()
    rng = np.random.default_rng(p0 + 3 * T)
    S = p0 + T
    K, V = _rn(rng, NKV, S, HD), _rn(rng, NKV, S, HD)
    q, sinks = _t(_rn(rng, T, NQ, HD), dev), _t(_rn(rng, NQ), dev)
    kl, vl = _t(K[None], dev), _t(V[None], dev)
    kn = kl[0, :, p0:p0 + T].transpose(0, 1).contiguous()                      # [T, 8, 64]
    vwide = torch.zeros(T, NKV * HD + 512, dtype=torch.bfloat16, device=dev)
    vwide[:, 256:256 + NKV * HD] = vl[0, :, p0:p0 + T].transpose(0, 1).reshape(T, -1)
    vn = vwide[:, 256:256 + NKV * HD].view(T, NKV, HD)                          # row stride 1024 elements
    kr_np, vr_np = _ring_from_linear(rng, K, V, p0)
    kr, vr = _t(kr_np[None], dev), _t(vr_np[None], dev)
    print(f"ring vs linear p0={p0} T={T}", flush=True)
    ol = A.prefill_attention(q, kl, vl, sinks, p0, SC, W, S)
    orr = A.prefill_attention(q, kr, vr, sinks, p0, SC, W, S, k_new=kn, v_new=vn, ring=RING)
    A.ring_write(kr, vr, kn, vn, p0, RING)
    torch.cuda.synchronize()
    assert torch.equal(ol, orr)
    jw = torch.arange(max(0, p0 + T - RING), p0 + T, device=dev)
    assert torch.equal(kr[0, :, jw % RING], kl[0, :, jw]) and torch.equal(vr[0, :, jw % RING], vl[0, :, jw])
    # slots the block did not reach keep their old contents
    keep = np.setdiff1d(np.arange(RING), (np.arange(max(0, p0 + T - RING), p0 + T) % RING))
    if keep.size:
        assert np.array_equal(_np(kr)[0][:, keep], kr_np[:, keep])


def test_chained_blocks_and_decode_continuation_ring_equals_linear():
    """reference tests/test_attention.py:282-307: a prompt in blocks, the ring only updated by ring_write, then 300
    decode steps with the ring row written per step: equal to the linear path at every block and step."""
    import torch
    from neural_amd import attention as A
    dev = _dev()
    rng = np.random.default_rng(11)
    S = 1600
    K, V = _rn(rng, NKV, S, HD), _rn(rng, NKV, S, HD)
    Kf, Vf = _t(K[None], dev), _t(V[None], dev)
    sinks = _t(_rn(rng, NQ), dev)
    kr = torch.zeros(1, NKV, RING, HD, dtype=torch.bfloat16, device=dev)
    vr = torch.zeros_like(kr)
    for p0, T in [(0, 300), (300, 64), (364, 1), (365, 129), (494, 700), (1194, 3)]:
        q = _t(_rn(rng, T, NQ, HD), dev)
        kn = Kf[0, :, p0:p0 + T].transpose(0, 1).contiguous()
        vn = Vf[0, :, p0:p0 + T].transpose(0, 1).contiguous()
        a = A.prefill_attention(q, Kf, Vf, sinks, p0, SC, W, S)
        b = A.prefill_attention(q, kr, vr, sinks, p0, SC, W, S, k_new=kn, v_new=vn, ring=RING)
        A.ring_write(kr, vr, kn, vn, p0, RING)
        torch.cuda.synchronize()
        assert torch.equal(a, b), (p0, T)
    pos_dev = torch.zeros(1, dtype=torch.int64, device=dev)
    o_l = torch.empty(NQ * HD, dtype=torch.bfloat16, device=dev)
    o_r = torch.empty_like(o_l)
    for pos in range(1197, 1197 + 300):
        kr[0, :, pos % RING] = Kf[0, :, pos]
        vr[0, :, pos % RING] = Vf[0, :, pos]
        q = _t(_rn(rng, NQ * HD), dev)
        pos_dev.fill_(pos)
        A.decode_attention(q, Kf, Vf, sinks, pos_dev, o_l, SC, W, S)
        A.decode_attention(q, kr, vr, sinks, pos_dev, o_r, SC, W, S, ring=RING)
    torch.cuda.synchronize()
    assert torch.equal(o_l, o_r)


def test_rows_past_t_untouched_and_empty_prompt():
    import torch
    from neural_amd import attention as A
    dev = _dev()
    rng = np.random.default_rng(12)
    T, S = 45, 64
    K, V = _t(_rn(rng, NKV, S, HD)[None], dev), _t(_rn(rng, NKV, S, HD)[None], dev)
    q, sinks = _t(_rn(rng, T, NQ, HD), dev), _t(_rn(rng, NQ), dev)
    big = torch.full((T + 3, NQ, HD), 7.0, dtype=torch.bfloat16, device=dev)
    A.prefill_attention(q, K, V, sinks, 10, SC, 0, S, out=big[:T])
    torch.cuda.synchronize()
    assert bool((big[T:] == 7.0).all())
    assert torch.isfinite(big[:T].float()).all()
    e = A.prefill_attention(q[:0], K, V, sinks, 3, SC, W, S)
    torch.cuda.synchronize()
    assert e.shape == (0, NQ, HD)


def test_long_prompt_sampled_rows_vs_exact():
    """A 4096-token prompt at p0 = 0 (configuration 4's context), full and sliding: 96 sampled query rows against the
    fp64 closed form, and the sliding-layer ring mode bit-identical to the linear mode."""
    import torch
    from neural_amd import attention as A
    dev = _dev()
    rng = np.random.default_rng(13)
    T = 4096
    K, V = _rn(rng, NKV, T, HD), _rn(rng, NKV, T, HD)
    q, sinks = _rn(rng, T, NQ, HD), _rn(rng, NQ)
    qd, Kd, Vd, sd = _t(q, dev), _t(K[None], dev), _t(V[None], dev), _t(sinks, dev)
    rows = np.unique(np.concatenate([np.arange(4), np.linspace(0, T - 1, 92).astype(int)]))
    for sliding in (0, W):
        print(f"long prompt T={T} window={sliding}", flush=True)
        got = _np(A.prefill_attention(qd, Kd, Vd, sd, 0, SC, sliding, T))
        exact = np.stack([ao.ref64(q[t].reshape(-1), K, V, sinks, t, SC, sliding).reshape(NQ, HD) for t in rows])
        assert np.all(np.abs(got[rows] - exact) <= ATOL + RTOL * np.abs(exact))
        assert np.abs(got[rows] - exact).mean() < 2e-3
    kr = torch.zeros(1, NKV, RING, HD, dtype=torch.bfloat16, device=dev)
    vr = torch.zeros_like(kr)
    kn, vn = Kd[0].transpose(0, 1).contiguous(), Vd[0].transpose(0, 1).contiguous()
    a = A.prefill_attention(qd, Kd, Vd, sd, 0, SC, W, T)
    b = A.prefill_attention(qd, kr, vr, sd, 0, SC, W, T, k_new=kn, v_new=vn, ring=RING)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
