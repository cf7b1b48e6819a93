"""GPT-OSS decode step restated on the CPU in numpy (test infrastructure; see oracle/__init__.py).

The eager decode core of the reference (neural/moe/gptoss_core_graphs.py:55-109, an op-for-op copy of transformers'
gpt-oss forward in bf16) with its fused twin's residual combine (fused_core.py:72-79), the expert body (server.py:
508-518, through mxfp4_oracle) and the decode tail (server.py:521-525).  Every bf16 rounding point is reproduced;
dot products are summed in fp64 and rounded once (the reference's fp32 summation order is not reproducible).

Weights are passed as numpy arrays of bf16 values held in fp32 (the dense matrices are widened to fp64 once).
"""
from __future__ import annotations

import numpy as np

from .attention_oracle import attn_bf16
from .bf16 import rb
from .mxfp4_oracle import combine_bf16, expert_forward_bf16, expert_weights, router_logits_bf16, router_top4

H, NQ, NKV, HD, NE = 2880, 64, 8, 64, 128
HQ = NQ * HD


def rms_bf16(x, w, eps):
    """RMSNorm at the reference's rounding points (gptoss_core_graphs.py:48-53; fused_core.py:95-109):
    r = rsqrt(mean(x^2) + eps) in fp32, out = bf16(w * (x * r)), over the last axis (one row or [T, H] rows).
    x, w: bf16 values."""
    x = np.asarray(x, np.float32)
    var = (np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True) / x.shape[-1]).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    return rb(np.asarray(w, np.float32) * (x * r))


def linear_bf16(x, W64, b=None):
    """F.linear in bf16: bf16(x . W^T (+ b)), one rounding (fp64 sum here); x one row or [T, K] rows."""
    y = np.asarray(np.asarray(x, np.float64) @ W64.T)
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return rb(y.astype(np.float32))


def rope_tables(pos, inv_freq, att_scale):
    """cos/sin of one position, or [T, 32] of an array of positions (gptoss_core_graphs.py:68-73, server.py:2357-2364):
    freqs = inv_freq * pos in fp32; bf16(cos(f) * s), bf16(sin(f) * s)."""
    p = np.asarray(pos, np.float32)
    f = (np.asarray(inv_freq, np.float32) * (p[..., None] if p.ndim else p)).astype(np.float32)
    cs = rb((np.cos(f.astype(np.float64)).astype(np.float32) * np.float32(att_scale)).astype(np.float32))
    sn = rb((np.sin(f.astype(np.float64)).astype(np.float32) * np.float32(att_scale)).astype(np.float32))
    return cs, sn


def rope_bf16(y, cs, sn):
    """Rotate-half RoPE in bf16 ops (gptoss_core_graphs.py:74-77): [y1 cs - y2 sn, y2 cs + y1 sn] with every product
    and sum rounded.  y [..., 64]."""
    y = np.asarray(y, np.float32)
    y1, y2 = y[..., :HD // 2], y[..., HD // 2:]
    return np.concatenate([rb(rb(y1 * cs) - rb(y2 * sn)), rb(rb(y2 * cs) + rb(y1 * sn))], axis=-1)


def residual(mid, g=None, c=None):
    """x = mid, or bf16(mid + bf16(g + bf16(c))) (fused_core.py:72-79; server.py:522 for the tail)."""
    mid = np.asarray(mid, np.float32)
    if g is None:
        return mid
    cc = rb(np.asarray(c, np.float32)) if c is not None else np.float32(0.0)
    return rb(mid + rb(np.asarray(g, np.float32) + cc))


class DecodeOracle:
    """Greedy decode of one sequence.  ``layers``: list of dicts with bf16-valued numpy arrays in_w, Wqkv, bqkv, Wo,
    bo, sinks, post_w, Wr, br and int ``sliding``; ``experts(li, e)`` -> (raw slot bytes, bias_gu, bias_dn) of expert
    e of layer li.  K/V caches are linear (position j in row j)."""

    def __init__(self, embed, layers, final_w, lm_head, experts, inv_freq, att_scale, eps=1e-5, smax=256):
        f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
        self.embed = f32(embed)
        self.layers = []
        for ly in layers:
            d = {k: f32(ly[k]) for k in ("in_w", "bqkv", "bo", "sinks", "post_w", "br")}
            d["Wqkv"] = np.asarray(ly["Wqkv"], np.float64)
            d["Wo"] = np.asarray(ly["Wo"], np.float64)
            d["Wr"] = f32(ly["Wr"])
            d["sliding"] = int(ly["sliding"])
            self.layers.append(d)
        self.final_w = f32(final_w)
        self.lm_head = np.asarray(lm_head, np.float64)
        self.experts = experts
        self.inv_freq, self.att_scale, self.eps = f32(inv_freq), float(att_scale), float(eps)
        self.kc = [np.zeros((NKV, smax, HD), np.float32) for _ in layers]
        self.vc = [np.zeros((NKV, smax, HD), np.float32) for _ in layers]
        self._wcache = {}

    def _expert(self, li, e):
        slot, bgu, bdn = self.experts(li, e)
        key = id(slot)
        w = self._wcache.get(key)
        if w is None:
            wg, wd = expert_weights(slot)
            w = (np.asarray(wg, np.float64), np.asarray(wd, np.float64))
            self._wcache[key] = w
        return w, bgu, bdn

    # -- the stages of one layer (each restates one kernel of the reference's fused core)
    def qkv(self, li, x, pos):
        """Input RMSNorm + Q|K|V + bias + RoPE (fused_core.py:82-142): returns q [4096], k [512], v [512]."""
        ly = self.layers[li]
        h = rms_bf16(x, ly["in_w"], self.eps)
        y = linear_bf16(h, ly["Wqkv"], ly["bqkv"])
        q = y[:HQ].reshape(NQ, HD)
        k = y[HQ:HQ + NKV * HD].reshape(NKV, HD)
        v = y[HQ + NKV * HD:].reshape(NKV, HD)
        cs, sn = rope_tables(pos, self.inv_freq, self.att_scale)
        return rope_bf16(q, cs, sn).reshape(-1), rope_bf16(k, cs, sn).reshape(-1), v.reshape(-1)

    def attend(self, li, q, k, v, pos):
        """Store K/V at pos, then sink attention over the layer's key range (fused_core.py:145-208)."""
        ly = self.layers[li]
        self.kc[li][:, pos] = np.asarray(k, np.float32).reshape(NKV, HD)
        self.vc[li][:, pos] = np.asarray(v, np.float32).reshape(NKV, HD)
        return attn_bf16(q, self.kc[li], self.vc[li], ly["sinks"], pos, HD ** -0.5, ly["sliding"])

    def oproj(self, li, att, x):
        """mid = bf16(x + bf16(att . Wo^T + bo)) (fused_core.py:401-414)."""
        ly = self.layers[li]
        return rb(np.asarray(x, np.float32) + linear_bf16(att, ly["Wo"], ly["bo"]))

    def route(self, li, mid):
        """Post-attention RMSNorm, router logits, top-4 and their softmax (fused_core.py:417-502)."""
        ly = self.layers[li]
        hn = rms_bf16(mid, ly["post_w"], self.eps)
        logits = router_logits_bf16(hn, ly["Wr"], ly["br"])[0]
        ids, wts = router_top4(logits)
        return hn, logits, ids, wts

    def moe(self, li, hn, ids, wts):
        """Expert body of one token: the top-4 experts and their weighted sum (server.py:508-518)."""
        ys = []
        for e in ids:
            (wg, wd), bgu, bdn = self._expert(li, int(e))
            ys.append(expert_forward_bf16(hn, None, bgu, bdn, weights=(wg, wd))[0])
        return combine_bf16(np.stack(ys), wts)

    def layer(self, li, mid, g, pos, trace=None):
        """One layer at position pos: returns (mid, g) for the next layer.  trace: optional dict filled with the
        layer's intermediates (x, q, k, v, att, mid, hn, logits, ids, wts, g)."""
        x = residual(mid, g)
        q, k, v = self.qkv(li, x, pos)
        att = self.attend(li, q, k, v, pos)
        mid = self.oproj(li, att, x)
        hn, logits, ids, wts = self.route(li, mid)
        gout = self.moe(li, hn, ids, wts)
        if trace is not None:
            trace.update(x=x, q=q, k=k, v=v, att=att, mid=mid, hn=hn, logits=logits, ids=ids, wts=wts, g=gout)
        return mid, gout

    def moe_rows(self, li, hn, ids, wts):
        """Expert layer over prompt rows (server.py:1837-1936 moe_prefill): every (token, rank) pair through its
        expert, then per token bf16(sum_k fp32(bf16(y_k * w_k))) in top-k order (server.py:2340-2341).  An id outside
        [0, 128) (no expert; the masked contract of the GPU path) contributes +0."""
        hn = np.asarray(hn, np.float32)
        ids = np.asarray(ids, np.int64)
        T, K = ids.shape
        y = np.zeros((T, K, H), np.float32)
        for e in np.unique(ids):
            if not 0 <= e < NE:
                continue
            tt, kk = np.nonzero(ids == e)
            (wg, wd), bgu, bdn = self._expert(li, int(e))
            y[tt, kk] = expert_forward_bf16(hn[tt], None, bgu, bdn, weights=(wg, wd))
        prod = rb(y * np.asarray(wts, np.float32)[:, :, None])
        acc = np.zeros((T, H), np.float32)
        for k in range(K):
            acc = (acc + prod[:, k]).astype(np.float32)
        return rb(acc)

    def prefill(self, tokens, p0=0, trace=None):
        """Prompt processing of ``tokens`` at positions p0 .. p0+T-1 (server.py:2366-2418: _attn_router and the
        experts, layer by layer over the whole block): x = embed; per layer x = bf16(x + m), h = RMSNorm, Q|K|V =
        F.linear, RoPE, K/V stored at their positions, prompt attention (attention_oracle.prefill_attn_tiled, the
        k_prefill_attn algorithm), x = bf16(x + F.linear(o, Wo, bo)), post RMSNorm, router top-4, experts.  Returns the
        bf16 logits of the last token (the tail).  trace: optional list receiving per layer dict(x (the residual
        input), h, q, k, v, o, mid, hn, logits, ids, wts, m)."""
        from .attention_oracle import prefill_attn_tiled

        tok = np.asarray(tokens, np.int64).reshape(-1)
        T = tok.size
        x = rb(self.embed[tok])
        m = None
        cs, sn = rope_tables(p0 + np.arange(T), self.inv_freq, self.att_scale)      # [T, 32]
        cs, sn = cs[:, None, :], sn[:, None, :]
        for li, ly in enumerate(self.layers):
            if m is not None:
                x = rb(x + m)
            x_res = x
            h = rms_bf16(x, ly["in_w"], self.eps)
            y = linear_bf16(h, ly["Wqkv"], ly["bqkv"])
            q = rope_bf16(y[:, :HQ].reshape(T, NQ, HD), cs, sn)
            k = rope_bf16(y[:, HQ:HQ + NKV * HD].reshape(T, NKV, HD), cs, sn)
            v = y[:, HQ + NKV * HD:].reshape(T, NKV, HD)
            self.kc[li][:, p0:p0 + T] = k.transpose(1, 0, 2)
            self.vc[li][:, p0:p0 + T] = v.transpose(1, 0, 2)
            o = prefill_attn_tiled(q, self.kc[li], self.vc[li], ly["sinks"], p0, HD ** -0.5, ly["sliding"])
            x = rb(x + linear_bf16(o.reshape(T, HQ), ly["Wo"], ly["bo"]))
            hn = rms_bf16(x, ly["post_w"], self.eps)
            logits = router_logits_bf16(hn, ly["Wr"], ly["br"])
            sel = [router_top4(r) for r in logits]
            ids = np.array([a for a, _ in sel], np.int64)
            wts = np.array([b for _, b in sel], np.float32)
            m = self.moe_rows(li, hn, ids, wts)
            if trace is not None:
                trace.append(dict(x=x_res, h=h, q=q, k=k, v=v, o=o, mid=x, hn=hn, logits=logits, ids=ids, wts=wts,
                                  m=m))
        return self.tail(x[-1], m[-1] if m is not None else None)

    def tail(self, mid, g):
        """Final norm + lm_head: bf16 logits [vocab] (server.py:521-525)."""
        h = residual(mid, g)
        hn = rms_bf16(h, self.final_w, self.eps)
        return linear_bf16(hn, self.lm_head)

    def step(self, tok, pos, trace=None):
        """One decode step: token tok at position pos -> bf16 logits of the next token."""
        mid = rb(self.embed[int(tok)])
        g = None
        for li in range(len(self.layers)):
            t = {} if trace is not None else None
            mid, g = self.layer(li, mid, g, pos, t)
            if trace is not None:
                trace.append(t)
        return self.tail(mid, g)


_GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix64(z):
    """SplitMix64's output function (Steele, Lea and Flood, OOPSLA 2014) on uint64 values, wrapping arithmetic."""
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = z + _GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniform_draws(seed: int, pos: int, n: int) -> np.ndarray:
    """The tail's on-device uniforms for (seed, position): top 24 bits of splitmix64(splitmix64(seed ^ pos) ^ v),
    times 2^-24, for v < n (fp32, exact)."""
    z = splitmix64(np.uint64(seed) ^ np.uint64(pos))
    return (splitmix64(z ^ np.arange(n, dtype=np.uint64)) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)


def gumbel_scores(logits, temp, u) -> np.ndarray:
    """The sampling tail's fp32 scores (reference server.py:1576-1583): logits / temp + (-log(-log(clamp(u, 1e-12,
    1 - 1e-7))))."""
    uc = np.clip(np.asarray(u, np.float32), np.float32(1e-12), np.float32(1.0 - 1e-7)).astype(np.float32)
    g = (-np.log(-np.log(uc))).astype(np.float32)
    return (np.asarray(logits, np.float32) / np.float32(temp)).astype(np.float32) + g


def sample_token(logits, temp, u) -> int:
    """Gumbel-max draw: argmax of gumbel_scores (first index on ties); temp <= 0 is the greedy argmax."""
    if temp <= 0:
        return argmax_first(logits)
    return int(np.argmax(gumbel_scores(logits, temp, u)))


def argmax_first(logits) -> int:
    """First index of the maximum (torch.argmax's documented tie rule; server.py:525)."""
    return int(np.argmax(np.asarray(logits, np.float32)))


def near_tie(logits, a: int, b: int, ulps: float = 2.0) -> bool:
    """Whether tokens a and b are within ``ulps`` bf16 units (at the larger logit's magnitude) of each other: the rule
    for accepting a different greedy choice between two implementations whose fp32 sums differ in order."""
    la, lb = float(logits[a]), float(logits[b])
    m = max(abs(la), abs(lb), 1e-30)
    ulp = 2.0 ** (np.floor(np.log2(m)) - 7)
    return abs(la - lb) <= ulps * ulp
