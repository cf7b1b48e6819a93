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


class FusedCore:
    """Per-layer decode launcher (reference fused_core.py:505-629).  Concatenates each layer's q/k/v weights and
    biases into one buffer and re-points the modules' tensors at views of it; with ring=R > 0 replaces every sliding
    layer's K/V cache by a rolling [1, NKV, R, HD] cache (slot = pos % R) and sets lg.ring on every layer; with
    split_k = NS > 1 full-attention layers run chunked attention (NS chunks) on one shared workspace.  The Triton
    tiling arguments (qkv_bk, qkv_warps, o_rows, o_bk, o_warps, r_rows, r_bk, attn_bn, split_bn, split_cache_s) are
    accepted and recorded; the kernels' tilings are their own.  Construct before any graph capture."""

    def __init__(self, cg, dev, qkv_bk=128, qkv_warps=4, o_rows=16, o_bk=256, o_warps=4, r_rows=8, r_bk=256,
                 attn_bn=64, ring=0, split_k=1, split_bn=64, split_cache_s=True, near_miss=False):
        self.cg, self.dev = cg, torch.device(dev)
        self.ring, self.split_k = int(ring), int(split_k)
        self.near_miss = bool(near_miss)
        if not 1 <= self.split_k <= MAX_SPLIT:
            raise AssertionError(f"split_k must be in [1, {MAX_SPLIT}]")
        self.cfg = dict(qkv_bk=qkv_bk, qkv_warps=qkv_warps, o_rows=o_rows, o_bk=o_bk, o_warps=o_warps,
                        r_rows=r_rows, r_bk=r_bk, attn_bn=attn_bn, ring=self.ring, split_k=self.split_k,
                        split_bn=split_bn, split_cache_s=bool(split_cache_s), near_miss=self.near_miss)
        self.W, self.B = [], []
        for lg in cg.layers:
            a = lg.layer.self_attn
            with torch.no_grad():
                W = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).contiguous()
                B = torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]).contiguous()
                a.q_proj.weight.data = W[:NQ * HD]
                a.k_proj.weight.data = W[NQ * HD:(NQ + NKV) * HD]
                a.v_proj.weight.data = W[(NQ + NKV) * HD:]
                a.q_proj.bias.data = B[:NQ * HD]
                a.k_proj.bias.data = B[NQ * HD:(NQ + NKV) * HD]
                a.v_proj.bias.data = B[(NQ + NKV) * HD:]
            if W.dtype is not torch.bfloat16 or tuple(W.shape) != ((NQ + 2 * NKV) * HD, H):
                raise AssertionError(f"q/k/v weights must be bf16 and stack to [{(NQ + 2 * NKV) * HD}, {H}]")
            self.W.append(W)
            self.B.append(B)
        for lg in cg.layers:
            if self.ring and lg.sliding:
                if self.ring < int(lg.sliding):
                    raise AssertionError(f"ring {self.ring} is smaller than the sliding window {lg.sliding}")
                lg.k = torch.zeros(1, NKV, self.ring, HD, dtype=torch.bfloat16, device=self.dev)
                lg.v = torch.zeros_like(lg.k)
                lg.ring = self.ring
            else:
                lg.ring = 0
        z = lambda *s, dt=torch.bfloat16: torch.zeros(*s, dtype=dt, device=self.dev)  # noqa: E731
        self.xbuf = z(H)
        self.q = z(NQ * HD)
        self.att = z(NQ * HD)
        self.logits = z(NE, dt=torch.float32)
        self.counter = z(1, dt=torch.int32)
        self.split = None
        if self.split_k > 1:
            full = {int(lg.smax) for lg in cg.layers if not lg.sliding}
            if len(full) > 1:
                raise AssertionError(f"full-attention layers with different smax {full}")
            if full:
                self.split = SplitAttn(self.split_k, full.pop(), self.dev, bn=split_bn, cache_s=split_cache_s)

    def layer_ring(self, L):
        """Ring size of layer L's cache (0 = linear)."""
        return self.ring if (self.ring and self.cg.layers[L].sliding) else 0

    def snapshot_rings(self):
        """Copy of every sliding layer's ring (None for the other layers), to resume a prompt at this position."""
        return [(lg.k.clone(), lg.v.clone()) if (self.ring and lg.sliding) else None for lg in self.cg.layers]

    def restore_rings(self, snap):
        """In-place restore of snapshot_rings() (addresses unchanged: captured graphs stay valid)."""
        for lg, kv in zip(self.cg.layers, snap):
            if kv is not None:
                lg.k.copy_(kv[0])
                lg.v.copy_(kv[1])

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
        kc = lg.k if kc is None else kc
        vc = lg.v if vc is None else vc
        hn_o = lg.h_norm if hn_o is None else hn_o
        sc_o = lg.r_scores if sc_o is None else sc_o
        idx_o = lg.r_idx if idx_o is None else idx_o
        ring = self.layer_ring(L)
        rows = ring or int(lg.smax)
        for t, nm in ((kc, "kc"), (vc, "vc")):
            assert tuple(t.shape) == (1, NKV, rows, HD) and t.dtype == torch.bfloat16 and t.is_contiguous(), (
                f"layer {L}: {nm} must be a contiguous bf16 [1, {NKV}, {rows}, {HD}] "
                f"({'ring' if ring else 'linear'} layout), got {tuple(t.shape)} {t.dtype} stride {t.stride()}")
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
