"""The prompt-processing oracle (DecodeOracle.prefill, oracle/model_oracle.py) pinned against the decode oracle.

The decode stages (DecodeOracle.qkv / attend / oproj / route / moe / tail) are pinned against transformers' gpt-oss
modules in test_oracle_model.py, and prefill_attn_tiled against closed forms in test_oracle_prefill_attention.py.
Here every stage of a 2-layer prefill (sliding window 8 + full attention, 30 prompt tokens) is recomputed at each
position by the decode stage functions from the prefill's own input to that stage (teacher forcing), which pins how
the prefill composes them: positions of RoPE and of the K/V rows, the causal and window ranges, the residual order,
the per-row routing and the top-k combine.  Equal up to fp64 summation order, except the attention: the decode form
rounds scores to bf16 (k_attn) where the prompt kernel keeps them in fp32 (k_prefill_attn), which at these scores
(|s| up to ~30, a bf16 ulp of 0.125) is a different result, so the prompt attention of every position is held to the
fp64 closed form (attention_oracle.ref64) over the same cache instead, within the attention tolerance.
"""
import numpy as np
import pytest

from neural_amd import synth
from neural_amd.model import yarn_inv_freq
from oracle.attention_oracle import ref64
from oracle.bf16 import rb
from oracle.model_oracle import DecodeOracle

H, NE, VOCAB, T, WIN = 2880, 128, 300, 30, 8


def _rn(rng, *shape, s=0.02, mean=0.0):
    return rb((rng.standard_normal(shape) * s + mean).astype(np.float32))


@pytest.fixture(scope="module")
def pair():
    rng = np.random.default_rng(5)
    layers = [dict(in_w=_rn(rng, H, s=0.1, mean=1.0), Wqkv=_rn(rng, 5120, H), bqkv=_rn(rng, 5120), Wo=_rn(rng, H, 4096),
                   bo=_rn(rng, H), sinks=_rn(rng, 64, s=1.0), post_w=_rn(rng, H, s=0.1, mean=1.0), Wr=_rn(rng, NE, H),
                   br=_rn(rng, NE), sliding=WIN if li == 0 else 0) for li in range(2)]
    slots = [synth.slot_raw(rng) for _ in range(8)]
    bgu, bdn = _rn(rng, 8, 5760), _rn(rng, 8, H)
    experts = lambda li, e: (slots[4 * li + e % 4], bgu[4 * li + e % 4], bdn[4 * li + e % 4])  # noqa: E731
    inv, att = yarn_inv_freq()
    embed, final_w, lm_head = _rn(rng, VOCAB, H), _rn(rng, H, s=0.1, mean=1.0), _rn(rng, VOCAB, H)

    def make():
        return DecodeOracle(embed, layers, final_w, lm_head, experts, inv.numpy(), att, smax=64)
    tokens = rng.integers(0, VOCAB, T)
    pre = make()
    trace = []
    logits = pre.prefill(tokens, 0, trace)
    return dict(make=make, pre=pre, trace=trace, logits=logits, tokens=tokens, embed=embed)


def _close(a, b, frac=0.02):
    """Equal up to fp64 summation order: a few elements may differ by one bf16 ulp."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    unit = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(b), 2.0 ** -126))) - 7)
    d = np.abs(a - b)
    return bool(np.all(d <= unit)) and float(np.mean(d > 0)) <= frac


def test_prefill_stages_equal_decode_stages(pair):
    dec = pair["make"]()
    tr, tok = pair["trace"], pair["tokens"]
    assert np.array_equal(tr[0]["x"], rb(pair["embed"][tok]))
    for li in range(2):
        L = tr[li]
        if li:
            assert np.array_equal(L["x"], rb(tr[li - 1]["mid"] + tr[li - 1]["m"]))
        for t in range(T):
            q, k, v = dec.qkv(li, L["x"][t], t)
            assert _close(q, L["q"][t].reshape(-1)) and _close(k, L["k"][t].reshape(-1))
            assert _close(v, L["v"][t].reshape(-1))
        # the prefill's K/V rows are where decode reads them: rows 0..T-1 of the layer's cache
        assert np.array_equal(pair["pre"].kc[li][:, :T], L["k"].transpose(1, 0, 2))
        assert np.array_equal(pair["pre"].vc[li][:, :T], L["v"].transpose(1, 0, 2))
        dec.kc[li][:, :T] = L["k"].transpose(1, 0, 2)
        dec.vc[li][:, :T] = L["v"].transpose(1, 0, 2)
        for t in range(T):
            o = L["o"][t].reshape(-1)
            exact = ref64(L["q"][t].reshape(-1), dec.kc[li], dec.vc[li], dec.layers[li]["sinks"], t, 0.125,
                          dec.layers[li]["sliding"])
            assert np.all(np.abs(o - exact) <= 2e-2 + 1e-2 * np.abs(exact)), (li, t)
            assert _close(dec.oproj(li, o, L["x"][t]), L["mid"][t])
            hn, logits, ids, wts = dec.route(li, L["mid"][t])
            assert _close(hn, L["hn"][t]) and _close(logits, L["logits"][t], 0.05)
            hn_p, ids_p, wts_p = L["hn"][t], L["ids"][t], L["wts"][t]
            g = dec.moe(li, hn_p, ids_p, wts_p)
            assert _close(g, L["m"][t], 0.05), (li, t)


def test_prefill_window_and_causality_reach(pair):
    """Position t of the sliding layer attends exactly [t - 7, t]: changing a key outside that range (and every key
    after t) leaves its output unchanged, changing one inside moves it."""
    from oracle.attention_oracle import prefill_attn_tiled
    L = pair["trace"][0]
    pre = pair["pre"]
    K, V = pre.kc[0][:, :T].copy(), pre.vc[0][:, :T].copy()
    sinks = pre.layers[0]["sinks"]
    base = prefill_attn_tiled(L["q"], K, V, sinks, 0, 0.125, WIN)
    t = 20
    for j, moved in ((t - WIN, False), (t + 1, False), (t - WIN + 1, True), (t, True)):
        K2 = K.copy()
        K2[:, j] = K2[:, j] * 3 + 1
        V2 = V.copy()
        V2[:, j] = V2[:, j] + 5
        out = prefill_attn_tiled(L["q"], K2, V2, sinks, 0, 0.125, WIN)
        assert (not np.array_equal(out[t], base[t])) == moved, j


def test_prefill_tail_is_the_decode_tail_of_the_last_token(pair):
    dec = pair["make"]()
    L = pair["trace"][-1]
    assert np.array_equal(dec.tail(L["mid"][-1], L["m"][-1]), pair["logits"])
