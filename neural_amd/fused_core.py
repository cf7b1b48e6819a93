"""Drop-in for the reference's fused_core.py on MI355X: the module a serving loop imports as ``fc``.

It keeps the reference module's call surface (fused_core.py:63, 336-398, 505-629, 684-820):
  constants        H, HP, NQ, NKV, HD, NE, K, REP
  attention        decode_attention, SplitAttn, prefill_attention, ring_write, ring_reuse_ok (neural_amd.attention)
  FusedCore        the per-layer launcher: FusedCore(cg, dev, ..., ring=0, split_k=1, near_miss=False)
                   .run(L, mid, g_out, c_out, slot_tab, bx, bslots, bgids, bw, pack, kc=None, vc=None, hn_o=None,
                   sc_o=None, idx_o=None), layer_ring, snapshot_rings, restore_rings
  k_qkv, k_prefill_attn
                   the two kernels the reference's tests launch directly as ``kernel[grid](...)``
                   (tests/test_attention.py:331-335, 412): named wrappers with the same positional arguments and
                   keyword constants, launching this package's kernels (the grid and the tiling constants are
                   accepted; the model constants are checked)

``cg`` is the reference's GptOssCoreGraphs (neural/moe/gptoss_core_graphs.py:113-140), or any object with the same
attributes: ``layers`` (each with ``layer`` -- a gpt-oss decoder layer: self_attn.{q,k,v,o}_proj.{weight,bias},
self_attn.sinks, input_layernorm / post_attention_layernorm .weight and .variance_epsilon, mlp.router.{weight,bias} --
and ``k``, ``v``, ``sliding``, ``smax``, ``scaling``, ``h_norm``, ``r_scores``, ``r_idx``), ``pos`` (int64 [1] on the
device), ``inv_freq`` (fp32 [32]) and ``att_scale``.  ``core_graphs(weights, smax, dev)`` builds such an object from a
neural_amd.model.DecodeWeights, for callers without the reference's eager core.

Per layer, run() is five launches on the current stream (no host synchronisation, nothing read on the host, so it
can be captured): na_core_qkv (residual combine + RMSNorm + Q|K|V + bias + RoPE + K/V write), na_decode_attention,
na_core_oproj, na_core_router (post RMSNorm + router + top-4 + softmax), na_core_route_pack (bx, pack, bslots, bgids,
bw: the expert body's inputs and the host pack).
"""
from __future__ import annotations

import types

import torch

from . import _native as N
from .attention import (H, HD, HP, K, MAX_SPLIT, NE, NKV, NQ, REP, SplitAttn, decode_attention,  # noqa: F401
                        prefill_attention, ring_reuse_ok, ring_write)

_PACK_BASE = H + 3 * K        # h_norm | 4 weights | 4 ids | 4 resident flags (server.py:471), + 4 near-miss ids


# Rows of the fused Q|K|V product that each projection owns (q: 64 heads, k and v: 8 heads each, 64 dims per head).
_QKV_ROWS = (("q_proj", 0, NQ * HD), ("k_proj", NQ * HD, (NQ + NKV) * HD),
             ("v_proj", (NQ + NKV) * HD, (NQ + 2 * NKV) * HD))
# The reference's Triton tiling knobs: accepted and recorded in FusedCore.cfg, no meaning for these kernels.
_TILING_KNOBS = ("qkv_bk", "qkv_warps", "o_rows", "o_bk", "o_warps", "r_rows", "r_bk", "attn_bn")


def _fuse_projections(attn):
    """Gather attn.{q,k,v}_proj into one weight buffer [5120, 2880] and one bias buffer [5120] (rows in _QKV_ROWS
    order), then point each projection's weight and bias at its rows: the module computes exactly what it did, on
    storage the fused QKV kernel reads in one pass."""
    n_rows = _QKV_ROWS[-1][2]
    w_like, b_like = attn.q_proj.weight, attn.q_proj.bias
    if w_like.dtype is not torch.bfloat16:
        raise AssertionError(f"q/k/v weights must be bf16 and stack to [{n_rows}, {H}]")
    W = torch.empty(n_rows, H, dtype=w_like.dtype, device=w_like.device)
    Bv = torch.empty(n_rows, dtype=b_like.dtype, device=b_like.device)
    with torch.no_grad():
        for name, lo, hi in _QKV_ROWS:
            proj = getattr(attn, name)
            if tuple(proj.weight.shape) != (hi - lo, H) or proj.weight.dtype is not torch.bfloat16:
                raise AssertionError(f"q/k/v weights must be bf16 and stack to [{n_rows}, {H}]")
            W[lo:hi].copy_(proj.weight)
            Bv[lo:hi].copy_(proj.bias)
            proj.weight.data, proj.bias.data = W[lo:hi], Bv[lo:hi]
    return W, Bv


class FusedCore:
    """Per-layer decode launcher with the reference's constructor and run() signature (fused_core.py:505-629).

    Side effects of construction on ``cg`` (the drop-in contract; construct before any graph capture):
      * every layer's q/k/v projection weights and biases are re-pointed at row ranges of one fused buffer per
        layer (``self.W[L]`` [5120, 2880] bf16, ``self.B[L]`` [5120]); the module's own forward is unchanged;
      * ``lg.ring`` is set on every layer: ``ring`` for sliding layers when ring > 0, else 0;
      * with ring > 0, each sliding layer's ``lg.k`` / ``lg.v`` become new zeroed rolling caches [1, NKV, ring, HD]
        (position p in slot p % ring); ring must cover the layer's window;
      * with split_k = NS > 1, the full-attention layers share one chunked-attention workspace (SplitAttn over NS
        chunks); they must then share one smax.
    The Triton tiling knobs are accepted and recorded in ``cfg``; the kernels' tilings are their own."""

    def __init__(self, cg, dev, qkv_bk=128, qkv_warps=4, o_rows=16, o_bk=256, o_warps=4, r_rows=8, r_bk=256,
                 attn_bn=64, ring=0, split_k=1, split_bn=64, split_cache_s=True, near_miss=False):
        self.cg, self.dev = cg, torch.device(dev)
        self.ring, self.split_k, self.near_miss = int(ring), int(split_k), bool(near_miss)
        if not 1 <= self.split_k <= MAX_SPLIT:
            raise AssertionError(f"split_k must be in [1, {MAX_SPLIT}]")
        knobs = (qkv_bk, qkv_warps, o_rows, o_bk, o_warps, r_rows, r_bk, attn_bn)
        self.cfg = {**dict(zip(_TILING_KNOBS, knobs)), "ring": self.ring, "split_k": self.split_k,
                    "split_bn": split_bn, "split_cache_s": bool(split_cache_s), "near_miss": self.near_miss}
        fused = [_fuse_projections(lg.layer.self_attn) for lg in cg.layers]
        self.W = [w for w, _ in fused]
        self.B = [b for _, b in fused]
        self._install_rings()
        self.xbuf, self.q, self.att = (torch.zeros(n, dtype=torch.bfloat16, device=self.dev)
                                       for n in (H, NQ * HD, NQ * HD))
        self.logits = torch.zeros(NE, dtype=torch.float32, device=self.dev)
        self.counter = torch.zeros(1, dtype=torch.int32, device=self.dev)
        full_rows = sorted({int(lg.smax) for lg in cg.layers if not lg.sliding})
        if self.split_k > 1 and len(full_rows) > 1:
            raise AssertionError(f"full-attention layers with different smax {set(full_rows)}")
        self.split = (SplitAttn(self.split_k, full_rows[0], self.dev, bn=split_bn, cache_s=split_cache_s)
                      if self.split_k > 1 and full_rows else None)

    def _install_rings(self):
        for lg in self.cg.layers:
            r = self.ring if (self.ring and lg.sliding) else 0
            if r and r < int(lg.sliding):
                raise AssertionError(f"ring {r} is smaller than the sliding window {lg.sliding}")
            if r:
                lg.k, lg.v = (torch.zeros(1, NKV, r, HD, dtype=torch.bfloat16, device=self.dev) for _ in "kv")
            lg.ring = r

    def layer_ring(self, L):
        """Ring size of layer L's cache (0 = linear)."""
        return int(self.cg.layers[L].ring)

    def snapshot_rings(self):
        """Per layer, a copy (k, v) of its rolling cache, or None for a linear layer: the state to resume a prompt
        at this position (ring_reuse_ok says when that is valid)."""
        return [None if not lg.ring else (lg.k.clone(), lg.v.clone()) for lg in self.cg.layers]

    def restore_rings(self, snap):
        """Copy a snapshot_rings() result back into the same cache tensors (addresses unchanged, so captured graphs
        stay valid)."""
        for lg, saved in zip(self.cg.layers, snap):
            for dst, src in zip((lg.k, lg.v), saved or ()):
                dst.copy_(src)

    def _cache(self, L, name, override, default, rows, ring):
        t = default if override is None else override
        if not (tuple(t.shape) == (1, NKV, rows, HD) and t.dtype == torch.bfloat16 and t.is_contiguous()):
            raise AssertionError(f"layer {L}: {name} must be a contiguous bf16 [1, {NKV}, {rows}, {HD}] "
                                 f"({'ring' if ring else 'linear'} layout), got {tuple(t.shape)} {t.dtype} "
                                 f"stride {t.stride()}")
        return t

    def run(self, L, mid, g_out, c_out, slot_tab, bx, bslots, bgids, bw, pack, kc=None, vc=None, hn_o=None,
            sc_o=None, idx_o=None):
        """One layer at the device position cg.pos.  Reads mid (and for L > 0 the previous layer's expert outputs
        g_out bf16 and c_out fp32: x = bf16(mid + bf16(g_out + bf16(c_out)))); writes K/V at pos (or pos % ring),
        mid <- x + o_proj(attention), hn_o <- post RMSNorm(mid), sc_o / idx_o <- top-4 weights / ids, and the expert
        body's inputs: bx <- hn, bslots / bgids / bw (slot_tab[L * 128 + id], -1 = not resident: slot 0, weight 0),
        pack <- hn | weights | ids | resident flags (| ranks 5-8 with near_miss).  kc / vc overrides must have the
        layer's layout, contiguous bf16 [1, NKV, rows, HD] (AssertionError otherwise, checked on the host)."""
        cg = self.cg
        lg = cg.layers[L]
        ly = lg.layer
        a = ly.self_attn
        ring = self.layer_ring(L)
        rows = ring or int(lg.smax)
        kc = self._cache(L, "kc", kc, lg.k, rows, ring)
        vc = self._cache(L, "vc", vc, lg.v, rows, ring)
        hn_o, sc_o, idx_o = (d if o is None else o for o, d in ((hn_o, lg.h_norm), (sc_o, lg.r_scores),
                                                                 (idx_o, lg.r_idx)))
        _need(mid, H, torch.bfloat16, "mid")
        _need(bx, H, torch.bfloat16, "bx")
        _need(hn_o, H, torch.bfloat16, "hn_o")
        _need(sc_o, K, torch.bfloat16, "sc_o")
        _need(idx_o, K, torch.int64, "idx_o")
        _need(bslots, K, torch.int64, "bslots")
        _need(bgids, K, torch.int64, "bgids")
        _need(bw, K, torch.bfloat16, "bw")
        _need(pack, _PACK_BASE + (K if self.near_miss else 0), torch.float32, "pack", at_least=True)
        if L:
            _need(g_out, H, torch.bfloat16, "g_out")
            if c_out is not None:
                _need(c_out, H, torch.float32, "c_out")
        if slot_tab is not None and (slot_tab.dtype is not torch.int64 or slot_tab.numel() < (L + 1) * NE):
            raise AssertionError("slot_tab must be int64 with an entry per (layer, expert)")
        s = N.stream(self.dev)
        N.call("na_core_qkv", mid.data_ptr(), g_out.data_ptr() if L else None,
               c_out.data_ptr() if (L and c_out is not None) else None, self.xbuf.data_ptr(),
               ly.input_layernorm.weight.data_ptr(), self.W[L].data_ptr(), self.B[L].data_ptr(), cg.pos.data_ptr(),
               cg.inv_freq.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, ring, self.q.data_ptr(),
               float(ly.input_layernorm.variance_epsilon), float(cg.att_scale), s)
        if self.split is not None and not lg.sliding:
            self.split.launch(self.q, kc, vc, a.sinks, cg.pos, self.att, float(lg.scaling))
        else:
            N.call("na_decode_attention", self.q.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, a.sinks.data_ptr(),
                   cg.pos.data_ptr(), self.att.data_ptr(), 1, float(lg.scaling), int(lg.sliding or 0), ring, 1, None,
                   None, None, s)
        N.call("na_core_oproj", self.att.data_ptr(), a.o_proj.weight.data_ptr(), a.o_proj.bias.data_ptr(),
               self.xbuf.data_ptr(), mid.data_ptr(), s)
        r = ly.mlp.router
        N.call("na_core_router", mid.data_ptr(), ly.post_attention_layernorm.weight.data_ptr(),
               float(ly.post_attention_layernorm.variance_epsilon), r.weight.data_ptr(), r.bias.data_ptr(),
               hn_o.data_ptr(), self.logits.data_ptr(), self.counter.data_ptr(), idx_o.data_ptr(), sc_o.data_ptr(), s)
        N.call("na_core_route_pack", hn_o.data_ptr(), self.logits.data_ptr(), idx_o.data_ptr(), sc_o.data_ptr(),
               N.ptr(slot_tab), L * NE, bx.data_ptr(), pack.data_ptr(), int(self.near_miss), bslots.data_ptr(),
               bgids.data_ptr(), bw.data_ptr(), s)


def _need(t, n, dtype, name, at_least=False):
    ok = t is not None and t.dtype is dtype and t.is_contiguous() and (t.numel() >= n if at_least else t.numel() == n)
    if not ok:
        what = f"at least {n}" if at_least else f"{n}"
        raise AssertionError(f"{name} must be a contiguous {dtype} tensor of {what} elements")


# ------------------------------------------------------------------------------------------ core graphs stand-in
def _ns(**kw):
    return types.SimpleNamespace(**kw)


class _CoreLayer:
    """One layer as FusedCore reads it from the reference's _LayerGraph (gptoss_core_graphs.py:26-45)."""

    def __init__(self, lw, pos, smax, dev, eps):
        lin = lambda w, b: _ns(weight=w, bias=b)  # noqa: E731
        q, k = NQ * HD, NKV * HD
        attn = _ns(q_proj=lin(lw.Wqkv[:q], lw.bqkv[:q]), k_proj=lin(lw.Wqkv[q:q + k], lw.bqkv[q:q + k]),
                   v_proj=lin(lw.Wqkv[q + k:], lw.bqkv[q + k:]), o_proj=lin(lw.Wo, lw.bo), sinks=lw.sinks,
                   head_dim=HD, scaling=HD ** -0.5, sliding_window=lw.sliding or None)
        self.layer = _ns(self_attn=attn, input_layernorm=_ns(weight=lw.in_w, variance_epsilon=eps),
                         post_attention_layernorm=_ns(weight=lw.post_w, variance_epsilon=eps),
                         mlp=_ns(router=lin(lw.Wr, lw.br)))
        self.pos, self.smax, self.sliding, self.scaling = pos, smax, lw.sliding or None, HD ** -0.5
        z = lambda *s, dt=torch.bfloat16: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
        self.k = z(1, NKV, smax, HD)
        self.v = z(1, NKV, smax, HD)
        self.h_norm = z(1, H)
        self.r_scores = z(1, K)
        self.r_idx = z(1, K, dt=torch.int64)
        self.ring = 0


def core_graphs(weights, smax, dev, eps=1e-5):
    """A stand-in for the reference's GptOssCoreGraphs over a neural_amd.model.DecodeWeights: the attributes
    FusedCore reads (layers, pos, inv_freq, att_scale), the per-layer linear K/V caches of ``smax`` rows and the
    router output buffers.  The weights are shared, not copied (FusedCore re-points the q/k/v views)."""
    from .model import yarn_inv_freq

    dev = torch.device(dev)
    inv, att = yarn_inv_freq()
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    return _ns(layers=[_CoreLayer(ly, pos, int(smax), dev, eps) for ly in weights.layers], pos=pos,
               inv_freq=inv.to(dev), att_scale=att, smax=int(smax), dev=dev)


# ------------------------------------------------------------------------------------------ direct kernel launches
class _Launched:
    """What a ``kernel[grid](...)`` call returns: metadata.shared = LDS bytes of the launched kernel."""

    def __init__(self, shared):
        self.metadata = _ns(shared=int(shared), num_warps=None)


class _Kernel:
    def __init__(self, fn, name):
        self._fn, self.__name__ = fn, name

    def __getitem__(self, grid):
        return lambda *args, **kw: self._fn(*args, **kw)


def _model_constants(**kw):
    want = dict(H=H, HP=HP, NQ=NQ, NKV=NKV, REP=REP)
    for k, v in kw.items():
        if v is not None and k in want and int(v) != want[k]:
            raise AssertionError(f"{k}={v}: these kernels are built for GPT-OSS-120B ({k}={want[k]})")


def _qkv(mid, gout, cout, xbuf, in_w, W, Bq, pos_ptr, inv_freq, kc, vc, qout, eps, att_scale, SMAX, FIRST,
         H=None, HP=None, BK=None, NQ=None, NKV=None, RING=0, num_warps=None):
    """k_qkv[grid](...) (reference fused_core.py:82-142): x = mid if FIRST else bf16(mid + bf16(gout + bf16(cout)));
    xbuf <- x; RMSNorm(in_w); Q|K|V GEMV of W [5120, 2880] + Bq; RoPE at *pos_ptr; K/V into kc, vc [1, NKV, SMAX, 64]
    at row pos (RING = 0) or slot pos % RING; qout <- q."""
    _model_constants(H=H, HP=HP, NQ=NQ, NKV=NKV)
    ring = int(RING or 0)
    if ring and int(SMAX) != ring:
        raise AssertionError("RING > 0 needs SMAX == RING")
    N.call("na_core_qkv", mid.data_ptr(), None if FIRST else gout.data_ptr(),
           None if (FIRST or cout is None) else cout.data_ptr(), xbuf.data_ptr(), in_w.data_ptr(), W.data_ptr(),
           Bq.data_ptr(), pos_ptr.data_ptr(), inv_freq.data_ptr(), kc.data_ptr(), vc.data_ptr(), int(SMAX), ring,
           qout.data_ptr(), float(eps), float(att_scale), N.stream(mid.device))
    return _Launched(0)


_PREFILL_ATTN_LDS = 2 * 64 * (64 * 2 + 16) + 2 * 64 * (64 * 2 + 8)   # K and V^T tiles, two of each (bytes)


def _prefill_attn(Q, Kc, Vc, Kn, Vn, sk_t, sk_h, sv_t, sv_h, sinks, O, p0, T, scaling, SLIDING, SMAX, REP=None,
                  NQ=None, BM=None, BN=None, RING=0, num_warps=None):
    """k_prefill_attn[grid](...) (reference fused_core.py:684-759): prompt attention of T queries Q [T, NQ, 64] at
    positions p0 .. p0+T-1 into O; linear cache Kc / Vc of SMAX rows (RING = 0; Kn / Vn unused), or a rolling cache
    of RING rows plus the block's own K / V in Kn / Vn with element strides (sk_t, sk_h), (sv_t, sv_h)."""
    _model_constants(REP=REP, NQ=NQ)
    ring = int(RING or 0)
    N.call("na_prefill_attention", Q.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), int(SMAX),
           Kn.data_ptr() if ring else None, Vn.data_ptr() if ring else None, int(sk_t) if ring else 0,
           int(sk_h) if ring else 0, int(sv_t) if ring else 0, int(sv_h) if ring else 0, sinks.data_ptr(),
           O.data_ptr(), int(p0), int(T), float(scaling), int(SLIDING or 0), ring, None, N.stream(Q.device))
    return _Launched(_PREFILL_ATTN_LDS)


k_qkv = _Kernel(_qkv, "k_qkv")
k_prefill_attn = _Kernel(_prefill_attn, "k_prefill_attn")
