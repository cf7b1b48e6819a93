"""neural_amd.fused_core, the drop-in for the reference's fused_core module (FusedCore.run, fused_core.py:505-629; the
direct launches k_qkv[grid] / k_prefill_attn[grid] of tests/test_attention.py:331-335, 412), on the GPU.

- A 2-layer model (sliding window 16 on a 16-row ring + full attention with split-K, vocab 4096) decodes through the
  mirror the way the reference's token loop drives it (embed, per layer FusedCore.run then the expert body on bx /
  idx_o / bw, the tail) and through DecodeModel: every step's K/V rows, mid, expert output and token are bit-equal.
- run()'s serving outputs: bx == h_norm; pack = h_norm | weights | ids | resident flags; bslots / bgids / bw from
  the slot table, with a non-resident expert (slot -1) giving slot 0 and weight +0; near misses = ranks 5-8 of the
  kernel's own router logits by repeated argmax (lowest index on ties); a wrong kc layout is refused.
- k_qkv[grid]: the ring slot pos % 16 holds what the linear row pos holds, q and xbuf equal, the other ring slots
  untouched (the reference's test (d) invariant); k_prefill_attn[grid] equals prefill_attention bit for bit in
  linear and ring mode and reports its LDS bytes.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, NE, NQ, NKV, HD, K = 2880, 128, 64, 8, 64, 4
VOCAB, WIN, N_SLOTS, SMAX = 4096, 16, 8, 64


@pytest.fixture(scope="module")
def tiny():
    import torch
    from neural_amd import synth
    from neural_amd.model import random_weights
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case fused core fixture: 2 layers, vocab 4096, window 16 on a 16-row ring", flush=True)
    w = random_weights(n_layers=2, vocab=VOCAB, device="cpu", seed=5, window=WIN, norm_std=0.1).to(dev)
    pool = synth.t950_pool_device(2 * N_SLOTS, dev, seed=44)
    n = LT.n_layers * LT.n_experts
    tab = np.zeros(n, np.int64)
    for li in range(2):
        tab[li * NE:(li + 1) * NE] = li * N_SLOTS + np.arange(NE) % N_SLOTS
    tab = torch.from_numpy(tab).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    bgu = (torch.randn(n, LT.gate_up_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(n, LT.down_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    rx = ResidentExperts(pool, LT, bgu, bdn, tab, max_batch=1)
    return dict(dev=dev, w=w, rx=rx, tab=tab)


def _bufs(dev, near_miss=False):
    import torch
    bf = torch.bfloat16
    return dict(mid=torch.zeros(1, H, dtype=bf, device=dev), g_out=torch.zeros(1, H, dtype=bf, device=dev),
                c_out=torch.zeros(1, H, dtype=torch.float32, device=dev), bx=torch.zeros(1, H, dtype=bf, device=dev),
                bslots=torch.zeros(K, dtype=torch.int64, device=dev), bgids=torch.zeros(K, dtype=torch.int64, device=dev),
                bw=torch.zeros(K, dtype=bf, device=dev), pack=torch.zeros(H + 4 * K, dtype=torch.float32, device=dev))


def test_mirror_decode_equals_decode_model(tiny):
    import torch
    from neural_amd import _native as N
    from neural_amd import fused_core as fc
    from neural_amd.model import DecodeModel
    dev, w, rx = tiny["dev"], tiny["w"], tiny["rx"]
    print("case fused core mirror vs DecodeModel, 2 layers, 24 steps", flush=True)
    cg = fc.core_graphs(w, SMAX, dev)
    core = fc.FusedCore(cg, dev, ring=WIN, split_k=4)
    assert [core.layer_ring(L) for L in range(2)] == [WIN, 0] and cg.layers[0].k.shape == (1, NKV, WIN, HD)
    m = DecodeModel(w, rx, smax=SMAX, n_split=4, sliding_split=1, ring=WIN)
    prompt = np.random.default_rng(6).integers(0, VOCAB, 10)
    m.reset(prompt)
    b = _bufs(dev)
    seq = torch.zeros(SMAX, dtype=torch.int64, device=dev)
    seq[:len(prompt)] = torch.from_numpy(prompt).to(dev)
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    hn = torch.zeros(1, H, dtype=torch.bfloat16, device=dev)
    part = torch.empty(N.lib().na_core_lm_partials(VOCAB), dtype=torch.int64, device=dev)
    s = N.stream(dev)
    for p in range(24):
        cg.pos.fill_(p)
        N.call("na_core_embed", w.embed.data_ptr(), VOCAB, seq.data_ptr(), SMAX, cg.pos.data_ptr(),
               b["mid"].data_ptr(), s)
        for L in range(2):
            core.run(L, b["mid"], b["g_out"], b["c_out"], tiny["tab"], b["bx"], b["bslots"], b["bgids"], b["bw"],
                     b["pack"])
            lg = cg.layers[L]
            rx.forward_decode(L, b["bx"], lg.r_idx, b["bw"].view(1, K), out=b["g_out"])
        N.call("na_core_lm_tail", b["mid"].data_ptr(), b["g_out"].data_ptr(), b["c_out"].data_ptr(),
               w.final_w.data_ptr(), 1e-5, w.lm_head.data_ptr(), VOCAB, hn.data_ptr(), None, part.data_ptr(),
               tok.data_ptr(), None, 0, None, None, None, 0, s)
        if p + 1 >= len(prompt):
            seq[p + 1] = tok[0]
        m.step()
        torch.cuda.synchronize()
        assert torch.equal(b["mid"], m.mid) and torch.equal(b["g_out"], m.g), p
        assert int(tok.item()) == int(m.pred[p + 1].item()), p
        for L in range(2):
            assert torch.equal(cg.layers[L].k, m.kc[L]) and torch.equal(cg.layers[L].v, m.vc[L]), (p, L)
    assert torch.equal(seq[:25], m.seq[:25])
    assert int(core.counter.item()) == 0 and int(core.split.counters.abs().sum()) == 0


def test_run_serving_outputs_and_near_misses(tiny):
    import torch
    from neural_amd import fused_core as fc
    dev, w = tiny["dev"], tiny["w"]
    print("case fused core serving outputs, near misses, layout check", flush=True)
    cg = fc.core_graphs(w, SMAX, dev)
    core = fc.FusedCore(cg, dev, ring=WIN, near_miss=True)
    b = _bufs(dev, near_miss=True)
    rng = np.random.default_rng(12)
    b["mid"].copy_(torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32) * 2).to(torch.bfloat16))
    b["g_out"].copy_(torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32) * 20).to(torch.bfloat16))
    b["c_out"].copy_(torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)))
    cg.pos.fill_(37)
    tab = tiny["tab"].clone()
    mid0 = b["mid"].clone()
    core.run(1, b["mid"], b["g_out"], b["c_out"], tab, b["bx"], b["bslots"], b["bgids"], b["bw"], b["pack"])
    torch.cuda.synchronize()
    lg = cg.layers[1]
    ids = lg.r_idx.cpu().numpy().reshape(-1)
    wts = lg.r_scores.float().cpu().numpy().reshape(-1)
    hn = lg.h_norm.float().cpu().numpy().reshape(-1)
    pk = b["pack"].cpu().numpy()
    assert torch.equal(b["bx"], lg.h_norm)
    assert np.array_equal(pk[:H], hn)
    assert np.array_equal(pk[H:H + 4], wts) and np.array_equal(pk[H + 4:H + 8], ids.astype(np.float32))
    assert np.array_equal(pk[H + 8:H + 12], np.ones(4, np.float32))
    t = tab.cpu().numpy()
    assert np.array_equal(b["bslots"].cpu().numpy(), t[NE + ids]) and np.array_equal(b["bgids"].cpu().numpy(), NE + ids)
    assert torch.equal(b["bw"], lg.r_scores.view(-1))
    lgt = core.logits.cpu().numpy().astype(np.float64)
    order = []
    for _ in range(8):                          # repeated argmax, lowest index first
        i = int(np.argmax(lgt))
        order.append(i)
        lgt[i] = -np.inf
    assert order[:4] == ids.tolist() and pk[H + 12:H + 16].astype(np.int64).tolist() == order[4:]
    # an expert that is not resident: slot 0, weight +0, flag 0 (the rest unchanged)
    tab[NE + int(ids[2])] = -1
    b["mid"].copy_(mid0)                              # run() updated mid in place: same inputs, same routing
    core.run(1, b["mid"], b["g_out"], b["c_out"], tab, b["bx"], b["bslots"], b["bgids"], b["bw"], b["pack"])
    torch.cuda.synchronize()
    assert np.array_equal(lg.r_idx.cpu().numpy().reshape(-1), ids)
    assert b["bslots"][2].item() == 0 and b["bw"][2].item() == 0 and b["pack"][H + 10].item() == 0
    assert b["bw"][0].item() != 0 and b["pack"][H + 8].item() == 1
    with pytest.raises(AssertionError):
        core.run(0, b["mid"], b["g_out"], b["c_out"], tab, b["bx"], b["bslots"], b["bgids"], b["bw"], b["pack"],
                 kc=cg.layers[1].k)                   # a linear cache on the ring layer


def test_named_kernel_launches(tiny):
    import torch
    from neural_amd import fused_core as fc
    from neural_amd.model import yarn_inv_freq
    dev, w = tiny["dev"], tiny["w"]
    print("case fused core k_qkv[grid] / k_prefill_attn[grid]", flush=True)
    bf = torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    rnd = lambda *s, sc=1.0: (torch.randn(*s, generator=g, device=dev) * sc).to(bf)  # noqa: E731
    ly = w.layers[0]
    inv, att = yarn_inv_freq()
    inv = inv.to(dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    R = 128
    kl = torch.zeros(1, NKV, 512, HD, dtype=bf, device=dev)
    vl = torch.zeros_like(kl)
    for first in (True, False):
        for p in (0, 1, 127, 128, 300, 511):
            mid, gout = rnd(H), rnd(H, sc=0.3)
            cout = torch.randn(H, generator=g, device=dev) * 0.3
            kr, vr = rnd(1, NKV, R, HD), rnd(1, NKV, R, HD)
            kr0, vr0 = kr.clone(), vr.clone()
            xa, xb = torch.empty(H, dtype=bf, device=dev), torch.empty(H, dtype=bf, device=dev)
            qa, qb = torch.empty(NQ * HD, dtype=bf, device=dev), torch.empty(NQ * HD, dtype=bf, device=dev)
            pos.fill_(p)
            for kc_, vc_, xb_, qo_, ring, rows in ((kl, vl, xa, qa, 0, 512), (kr, vr, xb, qb, R, R)):
                fc.k_qkv[(2 * (NQ + 2 * NKV),)](mid, gout, cout, xb_, ly.in_w, ly.Wqkv, ly.bqkv, pos, inv, kc_, vc_,
                                                qo_, 1e-5, att, SMAX=rows, FIRST=first, H=H, HP=fc.HP, BK=128,
                                                NQ=NQ, NKV=NKV, RING=ring, num_warps=4)
            torch.cuda.synchronize()
            sl = p % R
            assert torch.equal(kl[0, :, p], kr[0, :, sl]) and torch.equal(vl[0, :, p], vr[0, :, sl]), (first, p)
            assert torch.equal(qa, qb) and torch.equal(xa, xb), (first, p)
            other = torch.ones(R, dtype=torch.bool, device=dev)
            other[sl] = False
            assert torch.equal(kr[0, :, other], kr0[0, :, other]) and torch.equal(vr[0, :, other], vr0[0, :, other])
            assert bool(kl[0, :, p].abs().sum() > 0)
    with pytest.raises(AssertionError):
        fc.k_qkv[(1,)](mid, gout, cout, xa, ly.in_w, ly.Wqkv, ly.bqkv, pos, inv, kl, vl, qa, 1e-5, att, SMAX=512,
                       FIRST=True, H=4096, NQ=NQ, NKV=NKV)
    # prompt attention: the named launch equals prefill_attention, linear and ring
    T, p0, W = 40, 150, 128
    sinks = rnd(NQ)
    q = rnd(T, NQ, HD)
    Kf, Vf = rnd(1, NKV, 256, HD), rnd(1, NKV, 256, HD)
    o1, o2 = torch.empty_like(q), torch.empty_like(q)
    ck = fc.k_prefill_attn[(T, NQ)](q, Kf, Vf, Kf, Vf, 0, 0, 0, 0, sinks, o1, p0, T, 0.125, SLIDING=W, SMAX=256,
                                    REP=8, NQ=NQ, BM=64, BN=64, num_warps=4)
    fc.prefill_attention(q, Kf, Vf, sinks, p0, 0.125, W, 256, out=o2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and ck.metadata.shared > 0
    kr = torch.zeros(1, NKV, R, HD, dtype=bf, device=dev)
    vr = torch.zeros_like(kr)
    js = np.arange(p0 - R, p0)
    kr[0, :, torch.from_numpy(js % R).to(dev)] = Kf[0, :, p0 - R:p0]
    vr[0, :, torch.from_numpy(js % R).to(dev)] = Vf[0, :, p0 - R:p0]
    kn = Kf[0, :, p0:p0 + T].transpose(0, 1).contiguous()
    vn = Vf[0, :, p0:p0 + T].transpose(0, 1).contiguous()
    o3 = torch.empty_like(q)
    fc.k_prefill_attn[(T, NQ)](q, kr, vr, kn, vn, NKV * HD, HD, NKV * HD, HD, sinks, o3, p0, T, 0.125, SLIDING=W,
                               SMAX=R, REP=8, NQ=NQ, BM=64, BN=64, RING=R, num_warps=4)
    torch.cuda.synchronize()
    assert torch.equal(o3, o1)
