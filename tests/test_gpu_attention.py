"""Decode attention on the GPU (neural_amd.attention -> na_decode_attention) against the CPU oracle.

Mirrors the reference's attention tests (reference tests/test_attention.py): q/k/v ~ N(0,1) bf16, sinks ~ N(0,1) bf16,
scaling 1/8.  Bars: every output within 2e-2 + 1e-2 * max|want| of the oracle's k_attn rounding-point restatement and
within 2e-2 of the fp64 closed form (the reference's own bar, test_attention.py:148); chunked (split) vs one chunk
per head: rounding flips only (<= 2 bf16 ulps at the output's scale, the reference's criterion :198-203); rolling
(ring) cache vs linear cache: bit-identical (:147); graph replays with pos changed on the device == eager.
"""
import math

import numpy as np
import pytest

from oracle import attention_oracle as ao
from oracle.bf16 import rb

pytestmark = pytest.mark.gpu

NQ, NKV, HD = ao.NQ, ao.NKV, ao.HD
SC = 0.125


def _dev():
    import torch
    return torch.device("cuda", 0)


def _cache(rng, B, S, scale=1.0):
    k = rb((rng.standard_normal((B, NKV, S, HD)) * scale).astype(np.float32))
    v = rb((rng.standard_normal((B, NKV, S, HD)) * scale).astype(np.float32))
    return k, v


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(dev)


def _check_vs_oracle(got, q, k, v, sinks, pos, sliding=0, ring=0, tag=""):
    want = ao.attn_bf16(q, k, v, sinks, pos, SC, sliding, ring)
    ref = ao.ref64(q, k, v, sinks, pos, SC, sliding, ring)
    d = np.abs(got - want)
    assert d.max() <= 2e-2 + 1e-2 * np.abs(want).max(), (tag, pos, d.max())
    assert np.abs(got - ref).max() < 2e-2, (tag, pos, np.abs(got - ref).max())


def _out_scale_ulp(o):
    return 2.0 ** (math.floor(math.log2(float(np.abs(o).max()))) - 7)


@pytest.mark.parametrize("ns", [1, 8, 32])
def test_full_layer_matches_oracle(ns):
    import torch
    from neural_amd import attention as A
    dev = _dev()
    S = 8192
    rng = np.random.default_rng(100 + ns)
    k, v = _cache(rng, 1, S)
    sinks = rb(rng.standard_normal(NQ).astype(np.float32))
    kd, vd, sd = _t(k, dev), _t(v, dev), _t(sinks, dev)
    split = A.SplitAttn(ns, S, dev) if ns > 1 else None
    pos_dev = torch.zeros(1, dtype=torch.int64, device=dev)
    out = torch.empty(NQ * HD, dtype=torch.bfloat16, device=dev)
    for pos in (0, 1, 63, 64, 65, 1000, 4095, 8191):
        print(f"case attention full ns={ns} pos={pos}", flush=True)
        q = rb(rng.standard_normal(NQ * HD).astype(np.float32))
        pos_dev.fill_(pos)
        A.decode_attention(_t(q, dev), kd, vd, sd, pos_dev, out, SC, 0, S, split=split)
        got = out.float().cpu().numpy()
        _check_vs_oracle(got, q, k[0], v[0], sinks, pos, tag=f"ns={ns}")
    if split is not None:
        assert int(split.counters.abs().sum().item()) == 0, "counters must be left at zero"


def test_split_vs_single_is_rounding_only():
    import torch
    from neural_amd import attention as A
    dev = _dev()
    S = 8192
    rng = np.random.default_rng(7)
    k, v = _cache(rng, 1, S)
    sinks = rb(rng.standard_normal(NQ).astype(np.float32))
    kd, vd, sd = _t(k, dev), _t(v, dev), _t(sinks, dev)
    pos_dev = torch.zeros(1, dtype=torch.int64, device=dev)
    o1 = torch.empty(NQ * HD, dtype=torch.bfloat16, device=dev)
    o2 = torch.empty_like(o1)
    for pos in (0, 63, 255, 256, 4095, 8191):
        q = _t(rng.standard_normal(NQ * HD), dev)
        pos_dev.fill_(pos)
        A.decode_attention(q, kd, vd, sd, pos_dev, o1, SC, 0, S)
        for ns in (4, 16, 64):
            print(f"case attention split-vs-single pos={pos} ns={ns}", flush=True)
            A.decode_attention(q, kd, vd, sd, pos_dev, o2, SC, 0, S, split=A.SplitAttn(ns, S, dev))
            a, b = o1.float().cpu().numpy(), o2.float().cpu().numpy()
            if pos < 64:                                    # one 64-key block: every other chunk is empty
                assert np.array_equal(a, b), (pos, ns)
            assert np.abs(a - b).max() <= 2 * _out_scale_ulp(a), (pos, ns, np.abs(a - b).max())


def test_sliding_ring_equals_linear_and_oracle():
    import torch
    from neural_amd import attention as A
    dev = _dev()
    S, R, W = 4096, 128, 128
    rng = np.random.default_rng(11)
    k, v = _cache(rng, 1, S)
    sinks = rb(rng.standard_normal(NQ).astype(np.float32))
    kd, vd, sd = _t(k, dev), _t(v, dev), _t(sinks, dev)
    kr = _t(rng.standard_normal((1, NKV, R, HD)) * 3.0, dev)       # stale slots hold garbage
    vr = _t(rng.standard_normal((1, NKV, R, HD)) * 3.0, dev)
    pos_dev = torch.zeros(1, dtype=torch.int64, device=dev)
    ol = torch.empty(NQ * HD, dtype=torch.bfloat16, device=dev)
    orr = torch.empty_like(ol)
    bad = []
    positions = list(range(0, 300)) + [1000, 2047, 2048, 4000, 4095]
    for pos in positions:
        js = torch.arange(max(0, pos - R + 1), pos + 1, device=dev)
        kr[0, :, js % R] = kd[0, :, js]
        vr[0, :, js % R] = vd[0, :, js]
        q = rng.standard_normal(NQ * HD).astype(np.float32)
        qd = _t(q, dev)
        pos_dev.fill_(pos)
        A.decode_attention(qd, kd, vd, sd, pos_dev, ol, SC, W, S)
        A.decode_attention(qd, kr, vr, sd, pos_dev, orr, SC, W, S, ring=R)
        if not torch.equal(ol, orr):
            bad.append(pos)
        if pos in (0, 127, 128, 299, 4095):
            print(f"case attention sliding pos={pos}", flush=True)
            _check_vs_oracle(ol.float().cpu().numpy(), rb(q), k[0], v[0], sinks, pos, sliding=W, tag="sliding")
    assert not bad, bad[:10]


@pytest.mark.parametrize("S,sliding,ns", [(4096, 0, 16), (4096, 128, 1), (8192, 0, 16), (8192, 0, 32),
                                          (8192, 128, 1)])
def test_batched_sequences(S, sliding, ns):
    """Configuration 3's batch of 4 sequences, each at its own position (up to the last row of an 8192-row cache)."""
    import torch
    from neural_amd import attention as A
    dev = _dev()
    B = 4
    rng = np.random.default_rng(21 + ns + S)
    k, v = _cache(rng, B, S)
    sinks = rb(rng.standard_normal(NQ).astype(np.float32))
    q = rb(rng.standard_normal((B, NQ * HD)).astype(np.float32))
    pos = np.array([4095, 17, 1024, 3000] if S == 4096 else [8191, 63, 5000, 8128], np.int64)
    print(f"case attention batched B={B} S={S} sliding={sliding} ns={ns}", flush=True)
    out = torch.empty(B, NQ * HD, dtype=torch.bfloat16, device=dev)
    split = A.SplitAttn(ns, S, dev, batch=B) if ns > 1 else None
    A.decode_attention_batched(_t(q, dev), _t(k, dev), _t(v, dev), _t(sinks, dev), torch.from_numpy(pos).to(dev),
                               out, SC, sliding, split=split)
    got = out.float().cpu().numpy()
    for b in range(B):
        _check_vs_oracle(got[b], q[b], k[b], v[b], sinks, int(pos[b]), sliding=sliding, tag=f"b={b}")


def test_graph_replay_with_device_pos():
    import torch
    from neural_amd import attention as A
    dev = _dev()
    S = 4096
    rng = np.random.default_rng(31)
    k, v = _cache(rng, 1, S)
    sinks = _t(rng.standard_normal(NQ), dev)
    kd, vd = _t(k, dev), _t(v, dev)
    q = _t(rng.standard_normal(NQ * HD), dev)
    split = A.SplitAttn(16, S, dev)
    pos_dev = torch.full((1,), 100, dtype=torch.int64, device=dev)
    out = torch.empty(NQ * HD, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        A.decode_attention(q, kd, vd, sinks, pos_dev, out, SC, 0, S, split=split)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.decode_attention(q, kd, vd, sinks, pos_dev, out, SC, 0, S, split=split)
    eager = torch.empty_like(out)
    for p in (5, 700, 4095, 64, 2000):
        print(f"case attention graph pos={p}", flush=True)
        pos_dev.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        A.decode_attention(q, kd, vd, sinks, pos_dev, eager, SC, 0, S, split=split)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), p
    assert int(split.counters.abs().sum().item()) == 0
