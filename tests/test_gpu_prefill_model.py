"""Whole-model prompt processing on the GPU (DecodeModel.prefill -> na_rows_*, F.linear, na_prefill_attention,
na_ring_write, na_moe_prefill, na_core_lm_tail) against the CPU oracle (DecodeOracle stages and prefill_attn_tiled,
pinned in test_oracle_prefill_model.py / test_oracle_prefill_attention.py).

A 2-layer model (sliding window 16 + full attention; the sliding layer on a 16-row rolling cache or on a linear
cache; 8 distinct expert slots per layer; vocab 4096) prefills a 150-token prompt in one block and in 64-token
blocks.  Every stage of every (block, layer) is recomputed by the oracle from the GPU's own input to that stage
(teacher forcing, so rounding flips do not compound): row kernels and GEMMs to rounding flips, the prompt attention
within 1e-2 relative / 2e-2 absolute, the routing from the GPU's logits exactly, the experts within the expert
tolerance.  Then the cache contents, the tail (the greedy token of the last position, or a near tie) and one decode
step that reads the prefilled caches.
"""
import numpy as np
import pytest

from oracle.attention_oracle import attn_bf16, prefill_attn_tiled
from oracle.bf16 import rb
from oracle.model_oracle import DecodeOracle, argmax_first, near_tie, rms_bf16, linear_bf16, rope_bf16, rope_tables
from oracle.mxfp4_oracle import router_top4

pytestmark = pytest.mark.gpu

H, NE, NQ, NKV, HD = 2880, 128, 64, 8, 64
VOCAB, WIN, N_SLOTS, T = 4096, 16, 8, 150


def _flips_only(got, ref, frac=0.02):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    unit = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    d = np.abs(got - ref)
    ok = (d <= unit) | (d <= 2.0 ** -8 * np.abs(ref).max())
    return bool(ok.all()) and float(np.mean(d > 0)) < frac, (float(d.max()), float(np.mean(d > 0)))


def _f(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def tiny():
    import torch
    from neural_amd import synth, tiles
    from neural_amd.model import random_weights, yarn_inv_freq
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case prefill model fixture: 2 layers, vocab 4096, window 16", flush=True)
    w_cpu = random_weights(n_layers=2, vocab=VOCAB, device="cpu", seed=13, window=WIN, norm_std=0.1, sink_std=1.0)
    rng = np.random.default_rng(31)
    slots = [synth.slot_raw(rng) for _ in range(2 * N_SLOTS)]
    raw = torch.from_numpy(np.stack(slots)).to(dev)
    pool = torch.empty(raw.shape[0], LT.slot_bytes, dtype=torch.uint8, device=dev)
    tiles.repack_to_t950(raw, pool)
    del raw
    n = LT.n_layers * LT.n_experts
    tab = np.zeros(n, np.int64)
    for li in range(2):
        tab[li * NE:(li + 1) * NE] = li * N_SLOTS + np.arange(NE) % N_SLOTS
    g = torch.Generator().manual_seed(19)
    bgu = (torch.randn(n, LT.gate_up_n, generator=g) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(n, LT.down_n, generator=g) * 0.02).to(torch.bfloat16)
    rx = ResidentExperts(pool, LT, bgu.to(dev), bdn.to(dev), torch.from_numpy(tab).to(dev), max_batch=1)
    w = w_cpu.to(dev)
    torch.cuda.synchronize()
    ol = [dict(in_w=_f(ly.in_w), Wqkv=_f(ly.Wqkv), bqkv=_f(ly.bqkv), Wo=_f(ly.Wo), bo=_f(ly.bo), sinks=_f(ly.sinks),
               post_w=_f(ly.post_w), Wr=_f(ly.Wr), br=_f(ly.br), sliding=ly.sliding) for ly in w_cpu.layers]
    bgu_np, bdn_np = _f(bgu), _f(bdn)
    inv, att = yarn_inv_freq()
    orc = DecodeOracle(_f(w_cpu.embed), ol, _f(w_cpu.final_w), _f(w_cpu.lm_head),
                       lambda li, e: (slots[tab[li * NE + e]], bgu_np[li * NE + e], bdn_np[li * NE + e]),
                       inv.numpy(), att, smax=T + 8)
    prompt = np.random.default_rng(90).integers(0, VOCAB, T)
    return dict(w=w, rx=rx, orc=orc, dev=dev, prompt=prompt, inv=inv.numpy(), att=att)


def _model(tiny, ring):
    from neural_amd.model import DecodeModel
    return DecodeModel(tiny["w"], tiny["rx"], smax=T + 8, n_split=4, ring=ring, keep_logits=True)


@pytest.mark.parametrize("chunk,ring", [(4096, None), (64, None), (64, 0)])
def test_prefill_teacher_forced_against_oracle(tiny, chunk, ring):
    import torch
    print(f"case prefill model chunk={chunk} ring={ring}", flush=True)
    m = _model(tiny, ring)
    trace = []
    m.prefill(tiny["prompt"], chunk=chunk, trace=trace)
    torch.cuda.synchronize()
    orc, emb = tiny["orc"], tiny["orc"].embed
    keys = {0: [], 1: []}                                   # per layer: the K / V rows of every position so far
    vals = {0: [], 1: []}
    for rec in trace:
        li, p0 = rec["layer"], rec["p0"]
        ly = orc.layers[li]
        Tb = rec["x"].shape[0]
        x_in = _f(rec["x_in"])
        if li == 0:
            assert np.array_equal(x_in, rb(emb[tiny["prompt"][p0:p0 + Tb]]))
        x = rb(x_in + _f(rec["m_in"])) if rec["m_in"] is not None else x_in
        assert np.array_equal(_f(rec["x"]), x), (p0, li)
        ok, info = _flips_only(_f(rec["h"]), rms_bf16(x, ly["in_w"], orc.eps))
        assert ok, ("h", p0, li, info)
        h = _f(rec["h"])
        ok, info = _flips_only(_f(rec["qkv"]), linear_bf16(h, ly["Wqkv"], ly["bqkv"]), 0.05)
        assert ok, ("qkv", p0, li, info)
        y = _f(rec["qkv"])
        cs, sn = rope_tables(p0 + np.arange(Tb), tiny["inv"], tiny["att"])
        q = rope_bf16(y[:, :4096].reshape(Tb, NQ, HD), cs[:, None], sn[:, None])
        k = rope_bf16(y[:, 4096:4608].reshape(Tb, NKV, HD), cs[:, None], sn[:, None])
        v = y[:, 4608:].reshape(Tb, NKV, HD)
        ok, info = _flips_only(_f(rec["q"]), q)
        assert ok, ("q", p0, li, info)
        if rec["k_new"] is not None:
            gk, gv = _f(rec["k_new"]), _f(rec["v_new"])
        else:
            gk, gv = _f(rec["k_cache"]).transpose(1, 0, 2), _f(rec["v_cache"]).transpose(1, 0, 2)
        ok, info = _flips_only(gk, k)
        assert ok, ("k", p0, li, info)
        assert np.array_equal(gv, v), ("v", p0, li)
        keys[li].append(gk)
        vals[li].append(gv)
        K = np.concatenate(keys[li]).transpose(1, 0, 2)
        V = np.concatenate(vals[li]).transpose(1, 0, 2)
        want_o = prefill_attn_tiled(_f(rec["q"]), K, V, ly["sinks"], p0, HD ** -0.5, ly["sliding"])
        go = _f(rec["o"])
        assert np.all(np.abs(go - want_o) <= 2e-2 + 1e-2 * np.abs(want_o)), ("attention", p0, li)
        ok, info = _flips_only(_f(rec["att"]), linear_bf16(go.reshape(Tb, 4096), ly["Wo"], ly["bo"]), 0.05)
        assert ok, ("o_proj", p0, li, info)
        mid = rb(x + _f(rec["att"]))
        assert np.array_equal(_f(rec["mid"]), mid), ("mid", p0, li)
        ok, info = _flips_only(_f(rec["hn"]), rms_bf16(mid, ly["post_w"], orc.eps))
        assert ok, ("hn", p0, li, info)
        hn = _f(rec["hn"])
        lg = _f(rec["logits"])
        ok, info = _flips_only(lg, linear_bf16(hn, ly["Wr"], ly["br"]), 0.05)
        assert ok, ("router logits", p0, li, info)
        gids, gw = rec["ids"].cpu().numpy(), _f(rec["wts"])
        for t in range(Tb):
            ids, wts = router_top4(lg[t])
            assert np.array_equal(gids[t], ids), ("ids", p0, li, t)
            assert np.all(np.abs(gw[t] - wts) <= 2.0 ** -8 * np.abs(wts)), ("weights", p0, li, t)
        want_m = orc.moe_rows(li, hn, gids, gw)
        gm = _f(rec["m"])
        assert np.all(np.abs(gm - want_m) <= 2e-2 + 1e-2 * np.abs(want_m).max()), ("experts", p0, li)
    # the tail: greedy successor of the last prompt token, written at position T; pos advanced to T
    last = trace[-1]
    want = orc.tail(_f(last["mid"])[-1], _f(last["m"])[-1])
    gl = _f(m.logits)
    assert np.abs(gl - want).max() <= 1e-2 * np.abs(want).max() + 2e-2
    tok = int(m.tok.item())
    a = argmax_first(want)
    assert tok == argmax_first(gl) and (tok == a or near_tie(want, tok, a)), (tok, a)
    assert int(m.pos.item()) == T and int(m.seq[T].item()) == tok
    assert np.array_equal(m.seq[:T].cpu().numpy(), tiny["prompt"])
    # caches: full layer rows 0..T-1 hold every position's K/V; the sliding layer's ring the last 16 positions
    K1 = np.concatenate(keys[1])
    assert np.array_equal(_f(m.kc[1])[0][:, :T], K1.transpose(1, 0, 2))
    K0, V0 = np.concatenate(keys[0]), np.concatenate(vals[0])
    if m.ring:
        js = np.arange(T - m.ring, T)
        assert np.array_equal(_f(m.kc[0])[0][:, js % m.ring], K0[js].transpose(1, 0, 2))
        assert np.array_equal(_f(m.vc[0])[0][:, js % m.ring], V0[js].transpose(1, 0, 2))
    else:
        assert np.array_equal(_f(m.kc[0])[0][:, :T], K0.transpose(1, 0, 2))
    # one decode step at position T reads the prefilled caches: its attention output against the oracle's over the
    # same keys (the step's own K/V included)
    m.embed()
    for li in range(2):
        m.layer(li)
        torch.cuda.synchronize()
        ly = orc.layers[li]
        Kp = np.concatenate(keys[li] + [np.zeros((1, NKV, HD), np.float32)]).transpose(1, 0, 2).copy()
        Vp = np.concatenate(vals[li] + [np.zeros((1, NKV, HD), np.float32)]).transpose(1, 0, 2).copy()
        row = T % m.ring if (ly["sliding"] and m.ring) else T
        Kp[:, T] = _f(m.kc[li])[0][:, row]
        Vp[:, T] = _f(m.vc[li])[0][:, row]
        want_att = attn_bf16(_f(m.q), Kp, Vp, ly["sinks"], T, HD ** -0.5, ly["sliding"])
        ga = _f(m.att)
        assert np.all(np.abs(ga - want_att) <= 2e-2 + 1e-2 * np.abs(want_att).max()), ("decode after prefill", li)


def test_prefill_then_graph_decode_is_deterministic(tiny):
    """Prefill, then greedy decode by graph replays; the same again from a fresh prefill gives the same tokens."""
    import torch
    print("case prefill + graph decode determinism", flush=True)
    toks = []
    for _ in range(2):
        m = _model(tiny, None)
        m.prefill(tiny["prompt"][:100])
        m.run(5)
        torch.cuda.synchronize()
        toks.append(m.seq[:106].cpu().numpy())
    assert np.array_equal(toks[0], toks[1])
    assert np.array_equal(toks[0][:100], tiny["prompt"][:100])
