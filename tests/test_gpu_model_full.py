"""Configuration 4 at its real size on the GPU: the 36-layer GPT-OSS-120B-shaped model (vocab 201,088, sliding layers
on 128-row rolling caches, all 36 x 128 MXFP4 experts resident in the t950 layout and distinct, expert biases
N(0, 0.02)), a 4096-token random prompt prefilled by DecodeModel.prefill, then 256 greedy decode steps by replays of
one captured step graph (reference token loop server.py:453-545; tail server.py:521-525).

Bars (the oracle is oracle/model_oracle.py, pinned against transformers' gpt-oss modules):
- every generated token (the prefill's successor of the prompt and each of the 256 steps) is the argmax of the
  oracle's tail (combine + final RMSNorm + full-vocabulary lm_head in fp64, one bf16 rounding) over the GPU's own
  final state of that step, or a near tie (within 2 bf16 ulps; reference near-tie rule tests/test_attention.py:
  597-610).  The GPU's choice is teacher-forced: the next step reads the GPU's token, as the reference's greedy loop
  reads its own;
- at sampled (layer, position) pairs of the decode (layers 0, 1, 17, 34, 35 at positions 4096, 4223 and 4351, and
  every one of the 36 layers at 4224: the first decode position, both sides of a ring wrap and the last) every stage of the layer is recomputed by the
  oracle from the GPU's own input of that stage, as in the 2-layer model test: q / k / v and o_proj to rounding
  flips, attention over the GPU's own 4352-position (full) or 128-row ring (sliding) cache within 1e-2 relative /
  2e-2 absolute, the routing exactly or a near tie, the experts within the expert tolerance;
- at sampled rows of the 4096-token prefill (layers 0, 1, 34, 35) the same stage checks on the prompt path, the
  attention against the fp64 closed form at the row's position; the prefill runs its library GEMMs as the bench
  does, with the committed TunableOp choices (model.use_tuned_prompt_gemms);
- the decode tail alone at the full vocabulary: logits against the oracle, the first index among tied rows planted
  more than 1024 partial keys apart (the argmax reduces 12,568 partial keys in several passes), and the sampling
  tail's draw against the oracle's Gumbel-max over the kernel's own logits;
- no bounded wait of the one-launch attention blocks or expert bodies gave up, in the prefill or the 256 steps (the
  error words stay clear).
"""
import numpy as np
import pytest

from oracle.attention_oracle import attn_bf16, prefill_ref64
from oracle.bf16 import rb
from oracle.model_oracle import (DecodeOracle, argmax_first, gumbel_scores, linear_bf16, near_tie, residual,
                                 rms_bf16, rope_bf16, rope_tables, sample_token, uniform_draws)
from oracle.mxfp4_oracle import router_top4

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

H, NE, NQ, NKV, HD, NL = 2880, 128, 64, 8, 64, 36
CTX, NEW = 4096, 256
DECODE_LAYERS = (0, 1, 17, 34, 35)
DECODE_POS = (4096, 4223, 4224, 4351)
ALL_LAYERS_AT = 4224                      # a ring wrap (4224 % 128 == 0): every layer is stage-checked there
PREFILL_LAYERS = (0, 1, 34, 35)
PREFILL_ROWS = (0, 127, 128, 2047, 4095)


def _flips_only(got, ref, frac=0.02):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    unit = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    d = np.abs(got - ref)
    ok = (d <= unit) | (d <= 2.0 ** -8 * np.abs(ref).max())
    return bool(ok.all()) and float(np.mean(d > 0)) < frac, (float(d.max()), float(np.mean(d > 0)))


def _f(t):
    return t.float().cpu().numpy()


class Experts:
    """The oracle's view of the resident pool: raw store bytes of a slot (read back through the device inverse
    repack, which is bit-exact) and its biases, cached per slot so the oracle's dequantisation cache hits."""

    def __init__(self, pool, bgu, bdn):
        self.pool, self.bgu, self.bdn, self.raw = pool, bgu, bdn, {}

    def slot(self, s):
        import torch
        from neural_amd import tiles
        from neural_amd.moe.layout import GPTOSS_LAYOUT
        if s not in self.raw:
            buf = torch.empty(1, GPTOSS_LAYOUT.slot_bytes, dtype=torch.uint8, device=self.pool.device)
            tiles.repack_from_t950(self.pool[s:s + 1], buf)
            self.raw[s] = buf.cpu().numpy()[0]
        return self.raw[s]

    def layer_fn(self, li):
        return lambda _l, e: (self.slot(li * NE + e), _f(self.bgu[li * NE + e]), _f(self.bdn[li * NE + e]))


@pytest.fixture(scope="module")
def full():
    import torch
    from neural_amd import synth
    from neural_amd.model import DecodeModel, random_weights, use_tuned_prompt_gemms, yarn_inv_freq
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case full model fixture: 36 layers x 128 distinct experts (t950, 61.2 GB), vocab 201088, ring 128",
          flush=True)
    pool = synth.t950_pool_device(NL * NE, dev, seed=4343)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    bgu = (torch.randn(NL * NE, LT.gate_up_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(NL * NE, LT.down_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    rx = ResidentExperts(pool, LT, bgu, bdn, max_batch=1)
    w = random_weights(device=dev, seed=78)
    model = DecodeModel(w, rx, smax=CTX + NEW + 8)          # the bench's key split: auto_split(4360) = 18 chunks
    assert model.n_split == 18
    prompt = np.random.default_rng(4096).integers(0, w.vocab, CTX)
    # the bench's prompt GEMMs: the committed hipBLASLt choices for these shapes (the stage checks below pin them)
    assert use_tuned_prompt_gemms(), "the committed TunableOp results do not match this PyTorch / ROCm build"
    trace = []
    model.prefill(prompt, trace=trace)
    torch.cuda.synchronize()
    trace = [r for r in trace if r["layer"] in PREFILL_LAYERS]
    torch.cuda.empty_cache()
    inv, att = yarn_inv_freq()
    state = dict(model=model, w=w, dev=dev, prompt=prompt, trace=trace, experts=Experts(pool, bgu, bdn),
                 inv=inv.numpy(), att=att, first_state=(_f(model.mid)[0], _f(model.g)[0]),
                 first_tok=int(model.seq[CTX].item()))
    print("full model prefilled", flush=True)
    use_tuned_prompt_gemms(False)
    yield state
    state.clear()
    del model, rx, pool, w, bgu, bdn, trace
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _layer_dict(ly):
    return dict(in_w=_f(ly.in_w), Wqkv=_f(ly.Wqkv), bqkv=_f(ly.bqkv), Wo=_f(ly.Wo), bo=_f(ly.bo), sinks=_f(ly.sinks),
                post_w=_f(ly.post_w), Wr=_f(ly.Wr), br=_f(ly.br), sliding=ly.sliding)


def _layer_oracle(full, li, smax):
    """An oracle of the single layer li (index 0 inside it); the embedding and lm_head are not needed there."""
    w = full["w"]
    z = np.zeros((1, H), np.float32)
    return DecodeOracle(z, [_layer_dict(w.layers[li])], _f(w.final_w), z, full["experts"].layer_fn(li),
                        full["inv"], full["att"], smax=smax)


def _tail_oracle(full):
    w = full["w"]
    return DecodeOracle(np.zeros((1, H), np.float32), [], _f(w.final_w), _f(w.lm_head), None, full["inv"],
                        full["att"], smax=1)


def _check_tokens(logits, toks, tag):
    """Each row's token is the argmax of the oracle's logits or a near tie; returns the count of exact matches."""
    exact = 0
    for i, (lg, t) in enumerate(zip(logits, toks)):
        a = argmax_first(lg)
        assert t == a or near_tie(lg, int(t), a), (tag, i, int(t), a, float(lg[t]), float(lg[a]))
        exact += int(t == a)
    return exact


# ------------------------------------------------------------------------------------------------ prompt path
def test_prefill_4096_sampled_rows_against_oracle(full):
    """Stage checks on sampled prompt rows of layers 0, 1, 34, 35 (each stage from the GPU's own stage input), and the
    prompt's greedy successor against the oracle's tail of the GPU's final state of the last prompt token."""
    m = full["model"]
    rows = np.array(PREFILL_ROWS)
    print(f"case full model prefill rows {PREFILL_ROWS} at layers {PREFILL_LAYERS}", flush=True)
    cs, sn = rope_tables(rows, full["inv"], full["att"])
    for rec in full["trace"]:
        li = rec["layer"]
        orc = _layer_oracle(full, li, smax=1)
        ly = orc.layers[0]
        x_in = _f(rec["x_in"][rows])
        x = rb(x_in + _f(rec["m_in"][rows])) if rec["m_in"] is not None else x_in
        assert np.array_equal(_f(rec["x"][rows]), x), li
        ok, info = _flips_only(_f(rec["h"][rows]), rms_bf16(x, ly["in_w"], orc.eps))
        assert ok, ("h", li, info)
        h = _f(rec["h"][rows])
        ok, info = _flips_only(_f(rec["qkv"][rows]), linear_bf16(h, ly["Wqkv"], ly["bqkv"]), 0.05)
        assert ok, ("qkv", li, info)
        y = _f(rec["qkv"][rows])
        q = rope_bf16(y[:, :4096].reshape(-1, NQ, HD), cs[:, None], sn[:, None])
        k = rope_bf16(y[:, 4096:4608].reshape(-1, NKV, HD), cs[:, None], sn[:, None])
        ok, info = _flips_only(_f(rec["q"][rows]), q)
        assert ok, ("q", li, info)
        if rec["k_new"] is not None:                          # sliding layer: the block's own K / V [T, 8, 64]
            K, V = _f(rec["k_new"]).transpose(1, 0, 2), _f(rec["v_new"]).transpose(1, 0, 2)
        else:                                                 # full layer: the linear cache rows 0 .. T-1
            K, V = _f(rec["k_cache"]), _f(rec["v_cache"])
        ok, info = _flips_only(K[:, rows].transpose(1, 0, 2), k)
        assert ok, ("k", li, info)
        assert np.array_equal(V[:, rows].transpose(1, 0, 2), y[:, 4608:].reshape(-1, NKV, HD)), ("v", li)
        go = _f(rec["o"][rows])
        for i, p in enumerate(rows):
            want = prefill_ref64(_f(rec["q"][p:p + 1]), K, V, ly["sinks"], int(p), HD ** -0.5, ly["sliding"])[0]
            assert np.all(np.abs(go[i] - want) <= 2e-2 + 1e-2 * np.abs(want)), ("attention", li, int(p))
        ok, info = _flips_only(_f(rec["att"][rows]), linear_bf16(go.reshape(-1, 4096), ly["Wo"], ly["bo"]), 0.05)
        assert ok, ("o_proj", li, info)
        mid = rb(x + _f(rec["att"][rows]))
        assert np.array_equal(_f(rec["mid"][rows]), mid), ("mid", li)
        ok, info = _flips_only(_f(rec["hn"][rows]), rms_bf16(mid, ly["post_w"], orc.eps))
        assert ok, ("hn", li, info)
        hn, lg = _f(rec["hn"][rows]), _f(rec["logits"][rows])
        ok, info = _flips_only(lg, linear_bf16(hn, ly["Wr"], ly["br"]), 0.05)
        assert ok, ("router logits", li, info)
        gids, gw = rec["ids"][rows].cpu().numpy(), _f(rec["wts"][rows])
        for i in range(len(rows)):
            ids, wts = router_top4(lg[i])
            assert np.array_equal(gids[i], ids), ("ids", li, i)
            assert np.all(np.abs(gw[i] - wts) <= 2.0 ** -8 * np.abs(wts)), ("weights", li, i)
        want_m = orc.moe_rows(0, hn, gids, gw)
        gm = _f(rec["m"][rows])
        assert np.all(np.abs(gm - want_m) <= 2e-2 + 1e-2 * np.abs(want_m).max()), ("experts", li)
        del orc
        print(f"  prefill stage checks at layer {li} passed", flush=True)
    assert not m.sync_error()
    mid, g = full["first_state"]
    want = _tail_oracle(full).tail(mid[None], g[None])
    _check_tokens(want, [full["first_tok"]], "prefill tail")
    assert np.array_equal(m.seq[:CTX].cpu().numpy(), full["prompt"])


# ------------------------------------------------------------------------------------------------ decode
def _decode_stage_checks(full, p, li, mid_prev, g_prev):
    """After the eager m.layer(li) at position p: each stage against the oracle on the GPU's own stage inputs."""
    m = full["model"]
    ly_w = m.w.layers[li]
    ring = m.ring if ly_w.sliding else 0
    rows = m.kc[li].shape[2]
    orc = _layer_oracle(full, li, smax=1)
    ly = orc.layers[0]
    tag = (p, li)
    x = residual(mid_prev, g_prev)
    assert np.array_equal(_f(m.xbuf).reshape(-1), x), tag
    row = p % ring if ring else p
    kc, vc = _f(m.kc[li])[0], _f(m.vc[li])[0]
    q_g, k_g, v_g = _f(m.q).reshape(-1), kc[:, row].reshape(-1), vc[:, row].reshape(-1)
    q, k, v = orc.qkv(0, x, p)
    for nm, got, want in (("q", q_g, q), ("k", k_g, k), ("v", v_g, v)):
        ok, info = _flips_only(got, want)
        assert ok, (tag, nm, info)
    assert rows == (ring if ring else m.smax)
    want_att = attn_bf16(q_g, kc, vc, ly["sinks"], p, HD ** -0.5, ly["sliding"], ring=ring)
    att_g = _f(m.att).reshape(-1)
    assert np.abs(att_g - want_att).max() <= 2e-2 + 1e-2 * np.abs(want_att).max(), (tag, "att")
    mid_g = _f(m.mid).reshape(-1)
    ok, info = _flips_only(mid_g, orc.oproj(0, att_g, x))
    assert ok, (tag, "mid", info)
    hn, lg, ids, wts = orc.route(0, mid_g)
    hn_g, ids_g, wts_g = _f(m.hn).reshape(-1), m.ids.cpu().numpy().reshape(-1), _f(m.wts).reshape(-1)
    ok, info = _flips_only(hn_g, hn)
    assert ok, (tag, "hn", info)
    for k_ in range(4):
        assert ids_g[k_] == ids[k_] or near_tie(lg, int(ids_g[k_]), int(ids[k_])), (tag, ids_g, ids)
    g_g = _f(m.g).reshape(-1)
    g_o = orc.moe(0, hn_g, ids_g, wts_g)
    assert np.abs(g_g - g_o).max() <= 1e-2 * np.abs(g_o).max() + 2e-2, (tag, "experts")
    return mid_g, g_g


def test_greedy_256_graph_steps_against_oracle(full):
    """256 greedy steps after the 4096-token prefill: replays of one captured step graph, eager layer-by-layer steps
    with stage checks at the sampled positions; every token against the oracle's tail of the GPU's final state."""
    import torch
    m, dev = full["model"], full["dev"]
    print(f"case full model greedy decode {NEW} steps from position {CTX}", flush=True)
    assert int(m.pos.item()) == CTX
    hist_mid = torch.empty(NEW, H, dtype=torch.bfloat16, device=dev)
    hist_g = torch.empty(NEW, H, dtype=torch.bfloat16, device=dev)
    m.capture()
    checked = 0
    for i in range(NEW):
        p = CTX + i
        if p in DECODE_POS:
            m.embed()
            mid_prev, g_prev = _f(m.mid).reshape(-1), None
            for li in range(NL):
                m.layer(li)
                if li in DECODE_LAYERS or p == ALL_LAYERS_AT:
                    torch.cuda.synchronize()
                    mid_prev, g_prev = _decode_stage_checks(full, p, li, mid_prev, g_prev)
                    checked += 1
                else:
                    torch.cuda.synchronize()
                    mid_prev, g_prev = _f(m.mid).reshape(-1), _f(m.g).reshape(-1)
            m.tail()
            print(f"  stage checks at position {p} passed", flush=True)
        else:
            m.graph.replay()
        hist_mid[i].copy_(m.mid[0])
        hist_g[i].copy_(m.g[0])
    torch.cuda.synchronize()
    assert checked == len(DECODE_LAYERS) * (len(DECODE_POS) - 1) + NL
    assert not m.sync_error(), "a bounded wait of the attention block or the expert body gave up"
    assert int(m.pos.item()) == CTX + NEW
    seq = m.seq[:CTX + NEW + 1].cpu().numpy()
    pred = m.pred[:CTX + NEW + 1].cpu().numpy()
    assert np.array_equal(seq[:CTX], full["prompt"])
    assert np.array_equal(seq[CTX + 1:], pred[CTX + 1:])
    logits = _tail_oracle(full).tail(_f(hist_mid), _f(hist_g))
    exact = _check_tokens(logits, seq[CTX + 1:CTX + 1 + NEW], "decode")
    assert int(m.attn_counters.abs().sum()) == 0 and int(m.r_counter.item()) == 0
    print(f"greedy tokens equal to the oracle's argmax: {exact} / {NEW} (the rest near ties)", flush=True)


# ------------------------------------------------------------------------------------------------ tail alone
def test_lm_tail_full_vocab_ties_and_sampling(full):
    import torch
    from neural_amd import _native as N
    m, dev = full["model"], full["dev"]
    vocab = m.w.vocab
    print(f"case lm tail vocab={vocab}: logits, planted ties, sampling", flush=True)
    assert vocab == 201088 and N.lib().na_core_lm_partials(vocab) == 64 + 2 * 768   # 768 workgroups' two words
    rng = np.random.default_rng(201088)
    mid = rb(rng.standard_normal(H).astype(np.float32) * 3)
    g = rb(rng.standard_normal(H).astype(np.float32) * 30)
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(dev)  # noqa: E731
    mid_d, g_d = bf(mid), bf(g)
    Wl = m.w.lm_head.clone()
    logits = torch.empty(vocab, dtype=torch.bfloat16, device=dev)
    part = torch.empty(N.lib().na_core_lm_partials(vocab), dtype=torch.int64, device=dev)
    tok = torch.full((1,), -1, dtype=torch.int64, device=dev)
    hn = torch.empty(H, dtype=torch.bfloat16, device=dev)

    def greedy(with_residual=True):
        N.call("na_core_lm_tail", mid_d.data_ptr(), g_d.data_ptr() if with_residual else None, None,
               m.w.final_w.data_ptr(), 1e-5, Wl.data_ptr(), vocab, hn.data_ptr(), logits.data_ptr(), part.data_ptr(),
               tok.data_ptr(), None, 0, None, None, None, 0, N.stream(dev))
        torch.cuda.synchronize()
        return int(tok.item())

    best = greedy()
    gl = _f(logits)
    assert best == argmax_first(gl)
    want = _tail_oracle(full).tail(mid, g)
    assert np.abs(gl - want).max() <= 1e-2 * np.abs(want).max() + 2e-2
    _check_tokens(want[None], [best], "tail")
    # copies of the winning row in other workgroups' 16-row blocks (blocks 12000, 12567, 6000, 2000: workgroups 480,
    # 279, 624, 464 of 768), which the last workgroup's threads 224, 23, 112, 208 read
    far = [r for r in (16 * 12000 + 15, vocab - 1, 16 * 6000 + 4, 16 * 2000 + 1) if abs(r - best) >= 16]
    for r in far:
        Wl[r] = Wl[best]
    assert greedy() == min([best] + far)
    low = 16 * 5 + 7
    if best - low >= 16 * 1100:
        Wl[low] = Wl[best]
        assert greedy() == low
    # the sampling tail over the same logits: the oracle's Gumbel-max draw on the kernel's own logits
    Wl.copy_(m.w.lm_head)
    temp = torch.full((1,), 0.8, dtype=torch.float32, device=dev)
    seed = torch.full((1,), 12345, dtype=torch.int64, device=dev)
    pos = torch.full((1,), 4100, dtype=torch.int64, device=dev)
    N.call("na_core_lm_tail_sample", mid_d.data_ptr(), g_d.data_ptr(), None, m.w.final_w.data_ptr(), 1e-5,
           Wl.data_ptr(), vocab, hn.data_ptr(), logits.data_ptr(), part.data_ptr(), tok.data_ptr(), pos.data_ptr(), 0,
           None, None, None, 0, temp.data_ptr(), None, seed.data_ptr(), N.stream(dev))
    torch.cuda.synchronize()
    got = int(tok.item())
    lg = _f(logits)
    u = uniform_draws(12345, 4100, vocab)
    want_tok = sample_token(lg, 0.8, u)
    sc = gumbel_scores(lg, 0.8, u)
    assert got == want_tok or abs(float(sc[got]) - float(sc[want_tok])) <= \
        4 * np.finfo(np.float32).eps * max(1.0, abs(float(sc[want_tok]))), (got, want_tok)
