"""GPU parity: decode GEMV, masked GEMV, fused decode expert body and router through the C-ABI library, against
the CPU oracle on seeded synthetic slots (configuration 0 shapes).

Tolerance (north star: 1e-2 relative / 2e-2 absolute against the fp32-accumulate result), with "relative" measured
the way the reference's own GEMV check does (tools/scale_pack_gpu_test.py:183-189: max|d| / max|ref|):
    max|got - want| <= 2e-2 + 1e-2 * max|want|,
plus mean|got - want| <= 1e-3 * max|want| so that a systematic error cannot hide under the max.  Per element, bf16
outputs of magnitude ~300 carry an ulp of 2, so an element-wise 1% bound would reject one-ulp rounding flips.
raw == PS4 and graph replay == eager are bit-exact."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as mo
from oracle.bf16 import rb
from neural_amd import scale_pack as sp
from neural_amd import synth
from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, mxfp4_pool_views
from tolerance import ulp_profile

pytestmark = pytest.mark.gpu

NSLOT = 12
RTOL, ATOL = 1e-2, 2e-2


def within_tol(got, want, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = np.abs(got - want)
    scale = float(np.abs(want).max())
    ok = d.max() <= atol + rtol * scale and d.mean() <= 1e-3 * scale + 1e-6
    return bool(ok), float(d.mean()), float(d.max()), scale


@pytest.fixture(scope="module")
def dev():
    from neural_amd import _native as N
    N.lib()
    return torch.device("cuda", 0)


@pytest.fixture(scope="module")
def host_slots():
    rng = np.random.default_rng(1001)
    return [synth.slot_raw(rng) for _ in range(NSLOT)]


@pytest.fixture(scope="module")
def pools(dev, host_slots):
    raw = torch.from_numpy(np.stack(host_slots)).to(dev)
    pk = torch.from_numpy(np.stack([sp.pack_slot(s) for s in host_slots])).to(dev)
    return raw, pk


@pytest.fixture(scope="module")
def weights_cache(host_slots):
    return {}


def _weights(cache, host_slots, i):
    if i not in cache:
        cache[i] = mo.expert_weights(host_slots[i])
    return cache[i]


def test_fp4_conversion_builtin_layout(dev):
    from neural_amd import _native as N
    out = torch.zeros(768, dtype=torch.int16, device=dev)
    N.call("na_selftest_fp4", out.data_ptr(), N.stream(dev))
    o = out.cpu().numpy().view(np.uint16)
    vals = (o[:512].astype(np.uint32) << 16).view(np.float32).reshape(256, 2)
    b = np.arange(256)
    assert np.array_equal(vals[:, 0], mo.E2M1[b & 15].astype(np.float32))
    assert np.array_equal(vals[:, 1], mo.E2M1[b >> 4].astype(np.float32))
    assert np.array_equal(np.signbit(vals[:, 0]), np.signbit(mo.E2M1[b & 15]))
    assert (o[512:] == 1).all()


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("which", ["gate", "down"])
def test_mxfp4_gemv_matches_oracle(dev, pools, host_slots, weights_cache, packed, which):
    from neural_amd.q80.mxfp4_kernels import mxfp4_gemv
    L = GPTOSS_LAYOUT_PS4 if packed else GPTOSS_LAYOUT
    gb, db, gs, ds = mxfp4_pool_views(pools[1] if packed else pools[0], L)
    blocks, scales = (gb, gs) if which == "gate" else (db, ds)
    rng = np.random.default_rng(5)
    sl = [3, 0, 7, 11]
    slots = torch.tensor(sl, dtype=torch.int64, device=dev)
    per = which == "down"
    x = synth.bf16_normal(rng, (4 if per else 1, 2880)).to(dev)
    print(f"case gemv which={which} packed={packed} slots={sl}", flush=True)
    out = mxfp4_gemv(x, blocks, scales, slots, per_expert_x=per)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    xs = x.float().cpu().numpy()
    for i, s in enumerate(sl):
        w = _weights(weights_cache, host_slots, s)[0 if which == "gate" else 1]
        want = rb(mo.gemv_f64(xs[i:i + 1] if per else xs, w).astype(np.float32))[0]
        ok, *info = within_tol(got[i], want)
        assert ok, (i, info)
        prof = ulp_profile(got[i], want)        # exact products, fp32 sums, one rounding: within one bf16 ulp
        assert prof[0] >= 0.999 and prof[1] == 1.0, (i, prof)


def test_gemv_raw_equals_ps4_bitwise(dev, pools):
    from neural_amd.q80.mxfp4_kernels import mxfp4_gemv
    rng = np.random.default_rng(6)
    slots = torch.tensor([1, 2, 5, 9], dtype=torch.int64, device=dev)
    x = synth.bf16_normal(rng, (1, 2880)).to(dev)
    a = mxfp4_gemv(x, *[mxfp4_pool_views(pools[0], GPTOSS_LAYOUT)[i] for i in (0, 2)], slots)
    b = mxfp4_gemv(x, *[mxfp4_pool_views(pools[1], GPTOSS_LAYOUT_PS4)[i] for i in (0, 2)], slots)
    assert torch.equal(a, b)


def test_masked_gemv(dev, pools):
    from neural_amd.q80.mxfp4_kernels import mxfp4_gemv, mxfp4_gemv_masked
    gb, _, gs, _ = mxfp4_pool_views(pools[0], GPTOSS_LAYOUT)
    rng = np.random.default_rng(8)
    slots = torch.tensor([4, 6, 8, 10], dtype=torch.int64, device=dev)
    x = synth.bf16_normal(rng, (1, 2880)).to(dev)
    stock = mxfp4_gemv(x, gb, gs, slots)
    for dt in (torch.bfloat16, torch.float32):
        act = torch.tensor([0.5, 0.0, float("nan"), -0.0], dtype=dt, device=dev)
        got = mxfp4_gemv_masked(x, gb, gs, slots, act)
        assert torch.equal(got[0], stock[0]) and torch.equal(got[2], stock[2])
        assert (got[1] == 0).all() and (got[3] == 0).all()
        assert not torch.signbit(got[1].float()).any()
    with pytest.raises(ValueError):
        mxfp4_gemv_masked(x, gb, gs, slots, torch.ones(3, device=dev))


def _decode_case(dev, B, seed, bias):
    from neural_amd.moe.experts import ResidentExperts
    rng = np.random.default_rng(seed)
    x = synth.bf16_normal(rng, (B, 2880))
    # top-4 distinct ids per token from 128 experts, folded onto the NSLOT physical slots by the slot table
    ids = np.stack([rng.choice(128, 4, replace=False) for _ in range(B)]).astype(np.int64)
    if B >= 2:
        ids[1, 2] = ids[0, 0]          # force a shared expert across tokens
    logits = rng.standard_normal((B, 4)).astype(np.float32)
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    w = rb(w.astype(np.float32))
    n = 36 * 128
    tab = (np.arange(n) % NSLOT).astype(np.int64)
    if bias:
        bgu = synth.bf16_normal(rng, (n, 5760), 0.02)
        bdn = synth.bf16_normal(rng, (n, 2880), 0.02)
    else:
        bgu = bdn = None
    return x, ids, w, tab, bgu, bdn


@pytest.mark.parametrize("B", [1, 2, 4, 8])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_decode_matches_oracle(dev, pools, host_slots, weights_cache, B, bias):
    from neural_amd.moe.experts import ResidentExperts
    layer = 5
    x, ids, w, tab, bgu, bdn = _decode_case(dev, B, 100 + B + 10 * bias, bias)
    print(f"case moe_decode B={B} bias={bias} ids={ids.tolist()}", flush=True)
    rx = ResidentExperts(pools[0], GPTOSS_LAYOUT, None if bgu is None else bgu.to(dev),
                         None if bdn is None else bdn.to(dev), torch.from_numpy(tab).to(dev))
    out = rx.forward_decode(layer, x.to(dev), torch.from_numpy(ids).to(dev),
                            torch.from_numpy(w).to(torch.bfloat16).to(dev))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    xs = x.float().numpy()
    for b in range(B):
        ys = []
        for k in range(4):
            g = layer * 128 + int(ids[b, k])
            wts = _weights(weights_cache, host_slots, int(tab[g]))
            bg = np.zeros(5760, np.float32) if bgu is None else bgu[g].float().numpy()
            bd = np.zeros(2880, np.float32) if bdn is None else bdn[g].float().numpy()
            ys.append(mo.expert_forward_bf16(xs[b:b + 1], None, bg, bd, weights=wts)[0])
        want = mo.combine_bf16(np.stack(ys), w[b])
        ok, *info = within_tol(got[b], want)
        assert ok, (b, info)
        prof = ulp_profile(got[b], want)        # per element: rounding flips at the body's bf16 points only
        assert prof[1] >= 0.99 and prof[2] >= 0.995, (b, prof)


def test_moe_decode_raw_equals_ps4_and_graph_replay(dev, pools):
    from neural_amd.moe.experts import ResidentExperts
    B = 4
    x, ids, w, tab, bgu, bdn = _decode_case(dev, B, 77, True)
    args = (torch.from_numpy(tab).to(dev),)
    ra = ResidentExperts(pools[0], GPTOSS_LAYOUT, bgu.to(dev), bdn.to(dev), *args)
    rp = ResidentExperts(pools[1], GPTOSS_LAYOUT_PS4, bgu.to(dev), bdn.to(dev), *args)
    xd, idd = x.to(dev), torch.from_numpy(ids).to(dev)
    wd = torch.from_numpy(w).to(torch.bfloat16).to(dev)
    a = ra.forward_decode(3, xd, idd, wd)
    b = rp.forward_decode(3, xd, idd, wd)
    assert torch.equal(a, b)
    # hipGraph: capture once, replay with new inputs written in place; each replay equals eager
    out = torch.empty_like(a)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ra.forward_decode(3, xd, idd, wd, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ra.forward_decode(3, xd, idd, wd, out=out)
    rng = np.random.default_rng(9)
    for rep in range(3):
        xd.copy_(synth.bf16_normal(rng, (B, 2880)).to(dev))
        idd.copy_(torch.from_numpy(np.stack([rng.choice(128, 4, replace=False) for _ in range(B)])).to(dev))
        g.replay()
        torch.cuda.synchronize()
        eager = ra.forward_decode(3, xd, idd, wd)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep


def test_router_topk_matches_oracle(dev):
    from neural_amd.moe.experts import Router
    rng = np.random.default_rng(12)
    B = 4
    xn = synth.bf16_normal(rng, (B, 2880))
    wr = synth.bf16_normal(rng, (128, 2880), 0.02)
    br = synth.bf16_normal(rng, (128,), 0.02)
    r = Router(dev)
    ids = torch.zeros(B, 4, dtype=torch.int64, device=dev)
    wo = torch.zeros(B, 4, dtype=torch.bfloat16, device=dev)
    for rep in range(2):                     # the last-block counter must reset itself
        r(xn.to(dev), wr.to(dev), br.to(dev), ids, wo)
        torch.cuda.synchronize()
        for b in range(B):
            lg = mo.router_logits_bf16(xn[b].float().numpy(), wr.float().numpy(), br.float().numpy())[0]
            want_i, want_w = mo.router_top4(lg)
            got_i = ids[b].cpu().numpy()
            srt = np.sort(lg)[::-1]
            if srt[3] - srt[4] > 0.05:       # no near-tie at the top-4 boundary
                assert set(got_i.tolist()) == set(want_i.tolist())
            if got_i.tolist() == want_i.tolist():
                assert np.allclose(wo[b].float().cpu().numpy(), want_w, rtol=1e-2, atol=1e-3)
    assert int(r.counter.item()) == 0
