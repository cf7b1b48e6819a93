"""Dense decode core and the whole greedy decode step on the GPU (neural_amd.model -> na_core_*, na_decode_attention,
na_moe_decode_t950) against the CPU oracle (oracle/model_oracle.py, itself pinned against transformers' gpt-oss
modules in test_oracle_model.py).

Kernel bars (fp32 sums on the GPU vs fp64 in the oracle, the same bf16 rounding points): outputs differ from the
oracle by rounding flips only, i.e. on a small fraction of elements by at most one bf16 ulp (or, where rounded terms
cancel, one ulp of the vector's largest element); integer outputs (token ids, expert ids, cache positions) exactly,
except between logits that are equal in bf16 or within 2 ulps of each other (the near-tie rule).
Model bars: a 2-layer model (sliding + full attention, window 16 on a 16-row rolling cache, 8 distinct expert slots
per layer, vocab 4096) decodes a prompt and then greedily; teacher-forced on the GPU's own sequence, the oracle's
logits agree with the GPU's within 1e-2 relative / 2e-2 absolute of the logit range and its argmax is the GPU's token
or a near tie; graph replays give the same tokens as eager steps, bit for bit.
"""
import numpy as np
import pytest

from oracle.bf16 import rb
from oracle.model_oracle import DecodeOracle, argmax_first, near_tie, residual

pytestmark = pytest.mark.gpu

H, NE = 2880, 128
VOCAB, WIN, N_SLOTS = 4096, 16, 8


def _flips_only(got, ref, frac=0.02):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    unit = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    d = np.abs(got - ref)
    ok = (d <= unit) | (d <= 2.0 ** -8 * np.abs(ref).max())
    return bool(ok.all()) and float(np.mean(d > 0)) < frac, (float(d.max()), float(np.mean(d > 0)))


@pytest.fixture(scope="module")
def tiny():
    import torch
    from neural_amd import synth, tiles
    from neural_amd.model import DecodeModel, random_weights, yarn_inv_freq
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case model fixture: 2 layers, vocab 4096, window 16", flush=True)
    w_cpu = random_weights(n_layers=2, vocab=VOCAB, device="cpu", seed=3, window=WIN, norm_std=0.1, sink_std=1.0)
    rng = np.random.default_rng(21)
    slots = [synth.slot_raw(rng) for _ in range(2 * N_SLOTS)]
    raw = torch.from_numpy(np.stack(slots)).to(dev)
    pool = torch.empty(raw.shape[0], LT.slot_bytes, dtype=torch.uint8, device=dev)
    tiles.repack_to_t950(raw, pool)
    del raw
    n = LT.n_layers * LT.n_experts
    tab = np.zeros(n, np.int64)
    for li in range(2):
        tab[li * NE:(li + 1) * NE] = li * N_SLOTS + np.arange(NE) % N_SLOTS
    g = torch.Generator().manual_seed(9)
    bgu = (torch.randn(n, LT.gate_up_n, generator=g) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(n, LT.down_n, generator=g) * 0.02).to(torch.bfloat16)
    rx = ResidentExperts(pool, LT, bgu.to(dev), bdn.to(dev), torch.from_numpy(tab).to(dev), max_batch=1)
    w = w_cpu.to(dev)
    model = DecodeModel(w, rx, smax=64, n_split=4, keep_logits=True)
    torch.cuda.synchronize()

    f = lambda t: t.float().numpy()  # noqa: E731
    ol = [dict(in_w=f(ly.in_w), Wqkv=f(ly.Wqkv), bqkv=f(ly.bqkv), Wo=f(ly.Wo), bo=f(ly.bo), sinks=f(ly.sinks),
               post_w=f(ly.post_w), Wr=f(ly.Wr), br=f(ly.br), sliding=ly.sliding) for ly in w_cpu.layers]
    bgu_np, bdn_np = f(bgu), f(bdn)
    inv, att = yarn_inv_freq()

    def oracle():
        return DecodeOracle(f(w_cpu.embed), ol, f(w_cpu.final_w), f(w_cpu.lm_head),
                            lambda li, e: (slots[tab[li * NE + e]], bgu_np[li * NE + e], bdn_np[li * NE + e]),
                            inv.numpy(), att, smax=64)
    return dict(model=model, w=w, w_cpu=w_cpu, oracle=oracle, dev=dev)


def _np(t):
    return t.float().cpu().numpy().reshape(-1)


def _bf(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).to(dev)


# ------------------------------------------------------------------------------------------------ single kernels
@pytest.mark.parametrize("li,pos", [(0, 0), (0, 37), (1, 5), (1, 63)])
def test_qkv_rope_cache_write(tiny, li, pos):
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print(f"case core qkv layer={li} pos={pos}", flush=True)
    rng = np.random.default_rng(40 + pos)
    mid = rb(rng.standard_normal(H).astype(np.float32) * 3)
    g = rb(rng.standard_normal(H).astype(np.float32) * 50)
    m.mid.copy_(_bf(mid, dev).view(1, H))
    m.g.copy_(_bf(g, dev).view(1, H))
    m.pos.fill_(pos)
    for c in m.kc + m.vc:
        c.zero_()
    first = li == 0 and pos == 0                  # also cover the first layer's form (no expert input)
    ly = m.w.layers[li]
    ring = m.ring if ly.sliding else 0
    kc, vc = m.kc[li], m.vc[li]
    N.call("na_core_qkv", m.mid.data_ptr(), None if first else m.g.data_ptr(), None, m.xbuf.data_ptr(),
           ly.in_w.data_ptr(), ly.Wqkv.data_ptr(), ly.bqkv.data_ptr(), m.pos.data_ptr(), m.inv_freq.data_ptr(),
           kc.data_ptr(), vc.data_ptr(), kc.shape[2], ring, m.q.data_ptr(), 1e-5, float(m.att_scale), N.stream(dev))
    torch.cuda.synchronize()
    orc = tiny["oracle"]()
    x = residual(mid) if first else residual(mid, g)
    assert np.array_equal(_np(m.xbuf), x)
    q, k, v = orc.qkv(li, x, pos)
    row = pos % ring if ring else pos
    ok, info = _flips_only(_np(m.q), q)
    assert ok, ("q", info)
    ok, info = _flips_only(kc[0, :, row].float().cpu().numpy().reshape(-1), k)
    assert ok, ("k", info)
    ok, info = _flips_only(vc[0, :, row].float().cpu().numpy().reshape(-1), v)
    assert ok, ("v", info)
    # nothing else of the caches was written
    for c in (kc, vc):
        rest = c.clone()
        rest[0, :, row] = 0
        assert not bool(rest.any())


def test_oproj_residual(tiny):
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print("case core oproj", flush=True)
    rng = np.random.default_rng(50)
    att = rb(rng.standard_normal(4096).astype(np.float32))
    x = rb(rng.standard_normal(H).astype(np.float32) * 30)
    m.att.copy_(_bf(att, dev))
    m.xbuf.copy_(_bf(x, dev).view(1, H))
    ly = m.w.layers[1]
    N.call("na_core_oproj", m.att.data_ptr(), ly.Wo.data_ptr(), ly.bo.data_ptr(), m.xbuf.data_ptr(),
           m.mid.data_ptr(), N.stream(dev))
    torch.cuda.synchronize()
    ok, info = _flips_only(_np(m.mid), tiny["oracle"]().oproj(1, att, x))
    assert ok, info


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_router_norm_top4(tiny, seed):
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print(f"case core router seed={seed}", flush=True)
    rng = np.random.default_rng(60 + seed)
    mid = rb(rng.standard_normal(H).astype(np.float32) * 10)
    m.mid.copy_(_bf(mid, dev).view(1, H))
    ly = m.w.layers[0]
    for rep in range(2):                       # the second call checks the counter was left at zero
        N.call("na_core_router", m.mid.data_ptr(), ly.post_w.data_ptr(), 1e-5, ly.Wr.data_ptr(), ly.br.data_ptr(),
               m.hn.data_ptr(), m.r_logits.data_ptr(), m.r_counter.data_ptr(), m.ids.data_ptr(), m.wts.data_ptr(),
               N.stream(dev))
        torch.cuda.synchronize()
        assert int(m.r_counter.item()) == 0
    hn, lg, ids, wts = tiny["oracle"]().route(0, mid)
    ok, info = _flips_only(_np(m.hn), hn)
    assert ok, info
    g_lg = m.r_logits.cpu().numpy()
    ok, info = _flips_only(g_lg, lg, frac=0.05)
    assert ok, info
    g_ids = m.ids.cpu().numpy().reshape(-1)
    # the kernel's own choice from its own logits is exact: repeated argmax, lowest index first
    order = []
    v = g_lg.astype(np.float64).copy()
    for _ in range(4):
        i = int(np.argmax(v))
        order.append(i)
        v[i] = -np.inf
    assert g_ids.tolist() == order
    for k in range(4):
        assert g_ids[k] == ids[k] or near_tie(lg, int(g_ids[k]), int(ids[k])), (k, g_ids, ids)
    if np.array_equal(g_ids, ids):
        ok, info = _flips_only(_np(m.wts), wts, frac=0.5)
        assert ok, info


@pytest.mark.parametrize("vocab", [4096, 1000])
def test_lm_tail_argmax(tiny, vocab):
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print(f"case core lm tail vocab={vocab}", flush=True)
    rng = np.random.default_rng(70 + vocab)
    mid = rb(rng.standard_normal(H).astype(np.float32) * 3)
    g = rb(rng.standard_normal(H).astype(np.float32) * 30)
    m.mid.copy_(_bf(mid, dev).view(1, H))
    m.g.copy_(_bf(g, dev).view(1, H))
    Wl = m.w.lm_head[:vocab].contiguous()
    logits = torch.empty(vocab, dtype=torch.bfloat16, device=dev)
    part = torch.empty(N.lib().na_core_lm_partials(vocab), dtype=torch.int64, device=dev)
    tok = torch.full((1,), -1, dtype=torch.int64, device=dev)
    pos = torch.full((1,), 5, dtype=torch.int64, device=dev)
    seq = torch.zeros(16, dtype=torch.int64, device=dev)
    pred = torch.full((16,), -1, dtype=torch.int64, device=dev)
    nf = torch.full((1,), 7, dtype=torch.int64, device=dev)
    for step in range(3):                      # positions 5, 6 (forced: 6 < 7), 7
        N.call("na_core_lm_tail", m.mid.data_ptr(), m.g.data_ptr(), None, m.w.final_w.data_ptr(), 1e-5,
               Wl.data_ptr(), vocab, m.hn.data_ptr(), logits.data_ptr(), part.data_ptr(), tok.data_ptr(),
               pos.data_ptr(), 1, seq.data_ptr(), nf.data_ptr(), pred.data_ptr(), 16, N.stream(dev))
    torch.cuda.synchronize()
    gl = _np(logits)
    t = int(tok.item())
    assert t == argmax_first(gl)                           # exact: first index of the kernel's own maximum
    assert int(pos.item()) == 8
    p_ = pred.cpu().numpy()
    s_ = seq.cpu().numpy()
    assert p_[6] == p_[7] == p_[8] == t and p_[5] == -1 and p_[9] == -1
    assert s_[6] == 0 and s_[7] == t and s_[8] == t        # position 6 < n_forced keeps its token
    orc = tiny["oracle"]()
    orc.lm_head = orc.lm_head[:vocab]
    want = orc.tail(mid, g)
    d = np.abs(gl - want)
    assert d.max() <= 1e-2 * np.abs(want).max() + 2e-2, d.max()
    a = argmax_first(want)
    assert t == a or near_tie(want, t, a), (t, a)


def test_lm_tail_tie_takes_first_index(tiny):
    """Rows of lm_head that are equal give equal logits: the argmax must return the first (as torch.argmax)."""
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print("case core lm tail ties", flush=True)
    vocab = 3000
    Wl = m.w.lm_head[:vocab].clone()
    m.mid.copy_(_bf(np.ones(H, np.float32), dev).view(1, H))
    torch.cuda.synchronize()
    N.call("na_core_lm_tail", m.mid.data_ptr(), None, None, m.w.final_w.data_ptr(), 1e-5, Wl.data_ptr(), vocab,
           m.hn.data_ptr(), None, m.part.data_ptr(), m.tok.data_ptr(), None, 0, None, None, None, 0, N.stream(dev))
    torch.cuda.synchronize()
    best = int(m.tok.item())
    # copy the winning row to two places before it (different workgroups and lanes) and after it
    for r in (best // 3, 17, best + 1) if best + 1 < vocab else (best // 3, 17):
        if r != best:
            Wl[r] = Wl[best]
    N.call("na_core_lm_tail", m.mid.data_ptr(), None, None, m.w.final_w.data_ptr(), 1e-5, Wl.data_ptr(), vocab,
           m.hn.data_ptr(), None, m.part.data_ptr(), m.tok.data_ptr(), None, 0, None, None, None, 0, N.stream(dev))
    torch.cuda.synchronize()
    assert int(m.tok.item()) == min(best // 3, 17, best)


def test_embed_lookup_and_clamp(tiny):
    import torch
    from neural_amd import _native as N
    m, dev = tiny["model"], tiny["dev"]
    print("case core embed", flush=True)
    seq = torch.tensor([5, 4095, -3, 99999], dtype=torch.int64, device=dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    emb = m.w.embed
    for p, want in ((0, 5), (1, 4095), (2, 0), (3, VOCAB - 1), (9, VOCAB - 1), (-1, 5)):
        pos.fill_(p)
        N.call("na_core_embed", emb.data_ptr(), VOCAB, seq.data_ptr(), 4, pos.data_ptr(), m.mid.data_ptr(),
               N.stream(dev))
        torch.cuda.synchronize()
        assert torch.equal(m.mid.view(-1), emb[want]), p


# ------------------------------------------------------------------------------------------------ whole model
PROMPT, NEW = 20, 12


def test_greedy_decode_teacher_forced_against_oracle(tiny):
    """A prompt then greedy tokens, step by step and layer by layer: every stage of the oracle runs on the GPU's own
    inputs of that stage (its residual, q/k/v, attention output, normed hidden state and routing), so rounding flips
    do not compound across stages, layers or positions (random-init experts produce outputs in the thousands, where
    one bf16 ulp is 8 or 16).  Each generated token must be the oracle's argmax of the same final state, or a near
    tie."""
    import torch
    m = tiny["model"]
    print("case model greedy 2 layers, eager steps, stage by stage", flush=True)
    prompt = np.random.default_rng(80).integers(0, VOCAB, PROMPT)
    m.reset(prompt)
    orc = tiny["oracle"]()
    emb = tiny["w_cpu"].embed.float().numpy()
    exact = 0
    steps = PROMPT - 1 + NEW
    for p in range(steps):
        m.embed()
        torch.cuda.synchronize()
        tok = int(m.seq[p].item())
        mid, g = _np(m.mid), None
        assert np.array_equal(mid, rb(emb[tok])), p
        for li in range(2):
            m.layer(li)
            torch.cuda.synchronize()
            tag = (p, li)
            x = residual(mid, g)
            assert np.array_equal(_np(m.xbuf), x), tag
            ring = m.ring if m.w.layers[li].sliding else 0
            row = p % ring if ring else p
            q_g = _np(m.q)
            k_g = m.kc[li][0, :, row].float().cpu().numpy().reshape(-1)
            v_g = m.vc[li][0, :, row].float().cpu().numpy().reshape(-1)
            q, k, v = orc.qkv(li, x, p)
            for nm, got, want in (("q", q_g, q), ("k", k_g, k), ("v", v_g, v)):
                ok, info = _flips_only(got, want)
                assert ok, (tag, nm, info)
            att = orc.attend(li, q_g, k_g, v_g, p)                # the oracle's caches hold the GPU's K/V rows
            att_g = _np(m.att)
            assert np.abs(att_g - att).max() <= 2e-2 + 1e-2 * np.abs(att).max(), (tag, "att")
            mid_g = _np(m.mid)
            ok, info = _flips_only(mid_g, orc.oproj(li, att_g, x))
            assert ok, (tag, "mid", info)
            hn, lg, ids, wts = orc.route(li, mid_g)
            hn_g, ids_g, wts_g = _np(m.hn), m.ids.cpu().numpy().reshape(-1), _np(m.wts)
            ok, info = _flips_only(hn_g, hn)
            assert ok, (tag, "hn", info)
            for k_ in range(4):
                assert ids_g[k_] == ids[k_] or near_tie(lg, int(ids_g[k_]), int(ids[k_])), (tag, ids_g, ids)
            g_g = _np(m.g)
            g_o = orc.moe(li, hn_g, ids_g, wts_g)
            assert np.abs(g_g - g_o).max() <= 1e-2 * np.abs(g_o).max() + 2e-2, (tag, "experts")
            mid, g = mid_g, g_g
        m.tail()
        torch.cuda.synchronize()
        want = orc.tail(mid, g)
        got = _np(m.logits)
        assert np.abs(got - want).max() <= 1e-2 * np.abs(want).max() + 2e-2, (p, "logits")
        t = int(m.pred[p + 1].item())
        assert t == argmax_first(got), p
        a = argmax_first(want)
        assert t == a or near_tie(want, t, a), (p, t, a)
        exact += int(t == a)
        assert int(m.pos.item()) == p + 1
    seq = m.seq[:PROMPT + NEW].cpu().numpy()
    pred = m.pred[:PROMPT + NEW].cpu().numpy()
    assert np.array_equal(seq[:PROMPT], prompt) and np.array_equal(seq[PROMPT:], pred[PROMPT:])
    assert bool((m.kc[0].float().abs().sum(-1) > 0).all())          # the 16-row ring wrapped: every row written
    print(f"tokens equal to the oracle's argmax: {exact} / {steps}", flush=True)


def test_graph_replay_matches_eager(tiny):
    import torch
    m = tiny["model"]
    print("case model graph replay vs eager", flush=True)
    prompt = np.random.default_rng(81).integers(0, VOCAB, PROMPT)
    eager = m.generate(prompt, NEW, graph=False)
    m.graph = None
    first = m.generate(prompt, NEW, graph=True)
    again = m.generate(prompt, NEW, graph=True)          # replays of the same graph from a reset state
    assert torch.equal(eager, first) and torch.equal(first, again)
    assert int(m.attn_counters.abs().sum()) == 0 and int(m.r_counter.item()) == 0


def test_generate_redoes_a_flagged_decode(tiny):
    """An error word raised by a bounded wait makes generate() decode again with the multi-launch path; the words
    are planted from the host (no kernel is made to give up a wait), and the tokens equal the unflagged run's."""
    import torch
    m = tiny["model"]
    print("case generate with a planted error word", flush=True)
    prompt = np.random.default_rng(82).integers(0, VOCAB, PROMPT)
    want = m.generate(prompt, NEW, graph=True)
    assert not m.sync_error() and m.sync_redos == 0
    for words in (m.sync, m.rx.sync):
        words[:1].fill_(1)
        got = m.generate(prompt, NEW, graph=True)
        assert torch.equal(got, want)
        assert not m.sync_error() and m.fused_attn and m.rx.one
    assert m.sync_redos == 2
