"""The decode-step oracle (oracle/model_oracle.py) pinned on the CPU.

The pieces against closed forms (RMSNorm of a constant vector, RoPE at position 0 and at a quarter turn, the residual
combine, the argmax tie rule) and against transformers' own gpt-oss modules (the model the reference's eager core
copies op for op, neural/moe/gptoss_core_graphs.py:10-16): RMSNorm, the YaRN rotary table, RoPE, and a whole
2-layer model (sliding + full attention, 8 MXFP4 experts per layer dequantised into transformers' bf16 expert
tensors) whose logits at every position of a prompt must agree with the oracle's step-by-step decode.
"""
import math

import numpy as np
import pytest
import torch

from oracle.bf16 import rb
from oracle.attention_oracle import attn_bf16
from oracle.model_oracle import (DecodeOracle, argmax_first, near_tie, residual, rms_bf16, rope_bf16,
                                 rope_tables)
from oracle.mxfp4_oracle import expert_weights
from neural_amd import synth
from neural_amd.model import yarn_inv_freq

transformers = pytest.importorskip("transformers")
from transformers import GptOssConfig  # noqa: E402
from transformers.models.gpt_oss import modeling_gpt_oss as hf  # noqa: E402

H = 2880


def bf(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def test_rms_constant_vector_closed_form():
    x = np.full(H, 3.0, np.float32)
    w = np.ones(H, np.float32)
    out = rms_bf16(x, w, 1e-5)
    assert np.all(out == rb(np.float32(3.0 / math.sqrt(9.0 + 1e-5))))
    # the weight multiplies after the normalisation: w = 2 doubles the output exactly
    assert np.all(rms_bf16(x, 2 * w, 1e-5) == rb(2 * out))


def test_rms_matches_transformers():
    rng = np.random.default_rng(1)
    for scale in (1.0, 1e-3, 40.0):
        x = rb(rng.standard_normal(H).astype(np.float32) * scale)
        w = rb(1 + 0.1 * rng.standard_normal(H).astype(np.float32))
        m = hf.GptOssRMSNorm(H, eps=1e-5)
        m.weight.data = bf(w)
        with torch.no_grad():
            ref = m(bf(x)[None]).float().numpy()[0]
        got = rms_bf16(x, w, 1e-5)
        # fp32 summation order of the mean may move r by an ulp: allow one bf16 ulp on a few elements
        diff = np.abs(got - ref)
        assert np.mean(diff > 0) < 0.01
        assert np.all(diff <= np.abs(ref) * 2.0 ** -7 + 1e-30)


def test_yarn_table_matches_transformers():
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    inv, att = ROPE_INIT_FUNCTIONS["yarn"](GptOssConfig(), "cpu")
    mine, matt = yarn_inv_freq()
    assert torch.equal(inv, mine) and att == matt


def test_rope_closed_forms():
    inv, att = yarn_inv_freq()
    y = rb(np.random.default_rng(2).standard_normal((3, 64)).astype(np.float32))
    cs, sn = rope_tables(0, inv.numpy(), att)
    assert np.all(sn == 0) and np.all(cs == rb(np.float32(att)))
    out = rope_bf16(y, cs, sn)
    assert np.array_equal(out, rb(y * np.concatenate([cs, cs])))      # position 0: a pure (bf16) scaling
    # a rotation by a quarter turn maps (a, b) -> (-b, a) (with cos = 0 exactly: inv_freq * pos = pi/2 has no exact
    # fp32 form, so the table is built by hand here)
    cs0, sn1 = np.zeros(32, np.float32), np.ones(32, np.float32)
    out = rope_bf16(y, cs0, sn1)
    assert np.array_equal(out[:, :32], -y[:, 32:]) and np.array_equal(out[:, 32:], y[:, :32])


def test_rope_matches_transformers():
    cfg = GptOssConfig()
    rot = hf.GptOssRotaryEmbedding(cfg)
    inv, att = yarn_inv_freq()
    rng = np.random.default_rng(3)
    q = rb(rng.standard_normal((1, 64, 1, 64)).astype(np.float32))
    k = rb(rng.standard_normal((1, 8, 1, 64)).astype(np.float32))
    for pos in (0, 1, 127, 4095, 4097, 77777, 131071):
        cos, sin = rot(bf(q), torch.tensor([[pos]]))
        qr, kr = hf.apply_rotary_pos_emb(bf(q), bf(k), cos, sin)
        cs, sn = rope_tables(pos, inv.numpy(), att)
        assert np.array_equal(cs, cos.float().numpy().reshape(-1)), pos
        assert np.array_equal(sn, sin.float().numpy().reshape(-1)), pos
        assert np.array_equal(rope_bf16(q, cs, sn), qr.float().numpy()), pos
        assert np.array_equal(rope_bf16(k, cs, sn), kr.float().numpy()), pos


def test_residual_combine_rounding():
    mid = rb(np.float32([1.0, 256.0, -3.0]))
    g = rb(np.float32([2.0 ** -9, 1.0, 3.0]))
    # 1 + 2^-9 rounds back to 1 in bf16; 256 + 1 rounds to 256 (ulp 2); -3 + 3 = 0
    assert np.array_equal(residual(mid, g), np.float32([1.0, 256.0, 0.0]))
    assert np.array_equal(residual(mid), mid)
    # the CPU-side expert output c is rounded to bf16 before it joins g
    c = np.float32([0.0, 2.0 ** -10, 0.0])
    assert np.array_equal(residual(mid, g, c), residual(mid, g))


def test_argmax_tie_rule_and_near_tie():
    lg = rb(np.float32([1.0, 3.0, 3.0, 2.0]))
    assert argmax_first(lg) == 1
    assert near_tie(lg, 1, 2)
    assert not near_tie(lg, 1, 3)
    assert near_tie(np.float32([1.0, 1.0 + 2 * 2.0 ** -7]), 0, 1)
    assert not near_tie(np.float32([1.0, 1.0 + 4 * 2.0 ** -7]), 0, 1)


# ------------------------------------------------------------------------------------ whole model vs transformers
N_EXP, VOCAB, WIN, T = 8, 256, 8, 14


def _tiny_model():
    rng = np.random.default_rng(11)
    slots = [synth.slot_raw(rng) for _ in range(2 * N_EXP)]
    g = torch.Generator().manual_seed(5)

    def rn(*s, std=0.02, mean=0.0):
        return (torch.randn(*s, generator=g) * std + mean).to(torch.bfloat16)

    layers = []
    for li in range(2):
        layers.append(dict(in_w=rn(H, mean=1.0), Wqkv=rn(5120, H), bqkv=rn(5120), Wo=rn(H, 4096), bo=rn(H),
                           sinks=rn(64, std=1.0), post_w=rn(H, mean=1.0), Wr=rn(N_EXP, H, std=0.2), br=rn(N_EXP),
                           sliding=WIN if li % 2 == 0 else 0))
    embed, final_w, lm_head = rn(VOCAB, H), rn(H, mean=1.0), rn(VOCAB, H)
    bgu, bdn = rn(2 * N_EXP, 2 * H), rn(2 * N_EXP, H)
    return slots, layers, embed, final_w, lm_head, bgu, bdn


def _hf_model(slots, layers, embed, final_w, lm_head, bgu, bdn):
    cfg = GptOssConfig(num_hidden_layers=2, num_local_experts=N_EXP, vocab_size=VOCAB, sliding_window=WIN,
                       layer_types=["sliding_attention", "full_attention"])
    cfg._attn_implementation = "eager"
    m = hf.GptOssForCausalLM(cfg).to(torch.bfloat16).eval()
    # .to(bfloat16) also casts the rotary table; a checkpoint load keeps it in fp32 (the model computes it in fp32)
    m.model.rotary_emb.inv_freq = hf.GptOssRotaryEmbedding(cfg).inv_freq.float()
    assert m.model.rotary_emb.inv_freq.dtype is torch.float32
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(embed)
        m.model.norm.weight.copy_(final_w)
        m.lm_head.weight.copy_(lm_head)
        for li, ly in enumerate(layers):
            d = m.model.layers[li]
            a = d.self_attn
            a.q_proj.weight.copy_(ly["Wqkv"][:4096]); a.q_proj.bias.copy_(ly["bqkv"][:4096])
            a.k_proj.weight.copy_(ly["Wqkv"][4096:4608]); a.k_proj.bias.copy_(ly["bqkv"][4096:4608])
            a.v_proj.weight.copy_(ly["Wqkv"][4608:]); a.v_proj.bias.copy_(ly["bqkv"][4608:])
            a.o_proj.weight.copy_(ly["Wo"]); a.o_proj.bias.copy_(ly["bo"])
            a.sinks.copy_(ly["sinks"])
            d.input_layernorm.weight.copy_(ly["in_w"])
            d.post_attention_layernorm.weight.copy_(ly["post_w"])
            d.mlp.router.weight.copy_(ly["Wr"]); d.mlp.router.bias.copy_(ly["br"])
            ex = d.mlp.experts
            for e in range(N_EXP):
                wg, wd = expert_weights(slots[li * N_EXP + e])          # [5760, 2880] (gate | up rows), [2880, 2880]
                gu = torch.from_numpy(wg).to(torch.bfloat16)            # exact: E2M1 x 2^k fits bf16
                # transformers interleaves gate / up columns of gate_up_proj [H, 2I]
                ex.gate_up_proj[e, :, 0::2] = gu[:H].T
                ex.gate_up_proj[e, :, 1::2] = gu[H:].T
                b = bgu[li * N_EXP + e]
                ex.gate_up_proj_bias[e, 0::2] = b[:H]
                ex.gate_up_proj_bias[e, 1::2] = b[H:]
                ex.down_proj[e] = torch.from_numpy(wd).to(torch.bfloat16).T
                ex.down_proj_bias[e] = bdn[li * N_EXP + e]
    return m


def _flips_only(got, ref, frac=0.01):
    """got and ref (bf16 values) differ only by rounding flips: on fewer than ``frac`` of the elements, each by at most
    one bf16 ulp of the element or, where a difference of rounded terms cancels, of the vector's largest element."""
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    unit = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    d = np.abs(got - ref)
    ok = (d <= unit) | (d <= 2.0 ** -8 * np.abs(ref).max())
    return bool(ok.all()) and float(np.mean(d > 0)) < frac


@pytest.mark.timeout(600)
def test_decode_oracle_matches_transformers_stage_by_stage():
    """transformers' model decoding a prompt one token at a time (with its KV cache, as the reference's decode loop
    does) against the oracle.  Each stage of the oracle gets transformers' input of that stage: RMSNorm + QKV + RoPE,
    the sink attention over transformers' own K/V cache, o_proj + residual, post norm + router + top-4, the experts
    with their weighted sum, and the tail.  Stage outputs must agree up to rare one-ulp flips (fp64 here vs fp32 sums
    there); the expert sum, which transformers forms in bf16 in expert-index order and the reference in fp32 in top-k
    order, to a few ulps.  A second oracle instance runs whole layers (teacher-forced on transformers' layer inputs)
    to pin the wiring between the stages."""
    slots, layers, embed, final_w, lm_head, bgu, bdn = _tiny_model()
    m = _hf_model(slots, layers, embed, final_w, lm_head, bgu, bdn)
    toks = np.random.default_rng(12).integers(0, VOCAB, T)
    cap = {}
    hooks = []
    for li in range(2):
        d = m.model.layers[li]
        for nm, mod in (("layer", d), ("post", d.post_attention_layernorm), ("router", d.mlp.router),
                        ("experts", d.mlp.experts)):
            hooks.append(mod.register_forward_hook(
                lambda mod, inp, out, key=(li, nm): cap.__setitem__(key, (inp, out))))
    hooks.append(m.model.norm.register_forward_hook(lambda mod, inp, out: cap.__setitem__("final", inp[0])))
    eager = hf.eager_attention_forward

    def spy(module, q, k, v, mask, scaling, **kw):
        out, w = eager(module, q, k, v, mask, scaling, **kw)
        cap[(module.layer_idx, "attn")] = (q, k, v, mask, out)
        return out, w

    hf.eager_attention_forward = spy
    try:
        inv, att = yarn_inv_freq()
        f = lambda t: t.detach().float().numpy()  # noqa: E731
        ol = [{k: (f(v) if isinstance(v, torch.Tensor) else v) for k, v in ly.items()} for ly in layers]
        mk = lambda: DecodeOracle(  # noqa: E731
            f(embed), ol, f(final_w), f(lm_head),
            lambda li, e: (slots[li * N_EXP + e], f(bgu[li * N_EXP + e]), f(bdn[li * N_EXP + e])),
            inv.numpy(), att, smax=T)
        orc, whole = mk(), mk()
        past = None
        for p in range(T):
            with torch.no_grad():
                o = m(torch.tensor([[int(toks[p])]]), past_key_values=past, use_cache=True)
            past = o.past_key_values
            ref_logits = f(o.logits).reshape(-1)
            for li in range(2):
                x = f(cap[(li, "layer")][0][0]).reshape(-1)
                lo = cap[(li, "layer")][1]
                x_out = f(lo[0] if isinstance(lo, tuple) else lo).reshape(-1)
                if li == 0:
                    assert np.array_equal(x, rb(f(embed)[toks[p]]))
                q_h, k_h, v_h, mask, a_h = cap[(li, "attn")]
                q_h, k_h, v_h = f(q_h).reshape(-1), f(k_h)[0], f(v_h)[0]      # k_h, v_h [8, n, 64]
                # 1. norm + QKV + RoPE: this position's q, k, v
                q, k, v = orc.qkv(li, x, p)
                for got, ref in ((q, q_h), (k, k_h[:, -1].reshape(-1)), (v, v_h[:, -1].reshape(-1))):
                    assert _flips_only(got, ref), (li, p)
                # 2. attention over transformers' cache (the keys it keeps are the last n positions, all valid)
                n = k_h.shape[1]
                assert bool((f(mask) == 0).all()) and n == (min(p + 1, WIN) if li % 2 == 0 else p + 1), (li, p, n)
                a = attn_bf16(q_h, k_h, v_h, ol[li]["sinks"], n - 1, 0.125)
                a_ref = f(a_h).reshape(-1)
                assert _flips_only(a, a_ref), (li, p)
                # 3. o_proj + bias + residual
                mid_h = f(cap[(li, "post")][0][0]).reshape(-1)
                mid = orc.oproj(li, a_ref, x)
                assert _flips_only(mid, mid_h), (li, p)
                # 4. post norm + router + top-4 + softmax
                hn_h = f(cap[(li, "post")][1]).reshape(-1)
                lg_h, sc_h, ids_h = (f(t_) for t_ in cap[(li, "router")][1])
                lg_h, sc_h, ids_h = lg_h.reshape(-1), sc_h.reshape(-1), ids_h.reshape(-1).astype(np.int64)
                hn, lg, ids, wts = orc.route(li, mid_h)
                assert _flips_only(hn, hn_h), (li, p)
                assert _flips_only(lg, lg_h, frac=0.05), (li, p)
                # torch.topk orders equal logits arbitrarily; the reference's k_topk (and the oracle) take the lowest
                # index first
                for k_ in range(4):
                    assert ids[k_] == ids_h[k_] or lg_h[ids[k_]] == lg_h[ids_h[k_]], (li, p, ids, ids_h)
                assert _flips_only(wts, sc_h, frac=0.5), (li, p)
                # 5. experts and their weighted sum
                g_h = f(cap[(li, "experts")][1]).reshape(-1)
                g = orc.moe(li, hn_h, ids_h, sc_h)
                top = np.abs(g_h).max()
                assert np.abs(g - g_h).max() <= 2.0 ** -6 * top and np.abs(g - g_h).mean() <= 2.0 ** -11 * top
                # 6. the layer output is bf16(mid + experts)
                assert np.array_equal(x_out, rb(mid_h + g_h))
                # whole layer, teacher-forced on the layer input
                wm, wg = whole.layer(li, x, None, p)
                got = residual(wm, wg)
                top = np.abs(x_out).max()
                assert np.abs(got - x_out).max() <= 2.0 ** -5 * top, (li, p)
                assert np.abs(got - x_out).mean() <= 2.0 ** -9 * top, (li, p)
            # 7. tail
            lg = orc.tail(f(cap["final"]).reshape(-1), None)
            assert np.abs(lg - ref_logits).max() <= 1e-2 * np.abs(ref_logits).max() + 2e-2, p
            a, b = argmax_first(lg), argmax_first(ref_logits)
            assert a == b or near_tie(ref_logits, a, b), (p, a, b)
    finally:
        hf.eager_attention_forward = eager
        for h in hooks:
            h.remove()
