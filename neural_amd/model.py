"""GPT-OSS-120B single-sequence greedy decode on one MI355X: the per-token decode loop of the reference server
(server.py:453-545: embed -> 36 x [core layer, expert body] -> tail), with every launch a HIP kernel of this package
and the whole step capturable in one hipGraph.

Per layer (reference fused_core.py:581-629, FusedCore.run, plus the expert body server.py:508-518):
    na_core_qkv        residual combine + input RMSNorm + Q|K|V GEMV + bias + YaRN RoPE + K/V cache write
    na_decode_attention   GQA sink attention (sliding layers: 128-key window over a rolling cache)
    na_core_oproj      o_proj + bias + residual -> mid
    na_core_router     post RMSNorm -> hn, router GEMV + top-4 + softmax -> ids / weights
    ResidentExperts    gate_up + bias + clamped SwiGLU, down + bias + weight, top-4 combine -> g
and the tail (server.py:521-525): combine + final RMSNorm + lm_head + argmax, which also advances the position and
appends the token to the device-side sequence.  The input token of each step is read on the device from that
sequence at the current position, so replaying a captured step graph runs greedy decode with no host involvement;
positions below ``n_forced`` keep their preset tokens (a prompt read token by token, or a teacher-forced sequence).

Shapes (reference neural/moe/layout.py and the model config): hidden 2880, 64 query / 8 KV heads of 64, q|k|v rows
5120, o_proj [2880, 4096], router [128, 2880], vocab 201088, RMSNorm eps 1e-5, layers alternate sliding (even, window
128) and full attention, YaRN RoPE (theta 150000, factor 32, beta_fast 32, beta_slow 1, original context 4096).
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass, field

import torch

from . import _native as N
from .attention import auto_split, prefill_attention, ring_write
from .moe.experts import ResidentExperts

H, NQ, NKV, HD, NE, TOP_K = 2880, 64, 8, 64, 128, 4
HQ = NQ * HD                      # 4096
QKV_ROWS = (NQ + 2 * NKV) * HD    # 5120
N_LAYERS, VOCAB, EPS, WINDOW = 36, 201088, 1e-5, 128
ROPE_THETA = 150000.0
YARN = dict(factor=32.0, beta_fast=32.0, beta_slow=1.0, original_max_position_embeddings=4096, truncate=False)


def yarn_inv_freq(head_dim: int = HD, theta: float = ROPE_THETA, factor: float = 32.0, beta_fast: float = 32.0,
                  beta_slow: float = 1.0, original_max_position_embeddings: int = 4096, truncate: bool = False):
    """YaRN rotary frequencies (Peng et al. 2023, "YaRN: Efficient Context Window Extension of Large Language Models",
    sections 3.2-3.4) as the model's rotary embedding computes them in fp32: dimension pair i has the base frequency
    theta^(-2i/d); pairs that complete fewer than beta_slow rotations over the original context are interpolated
    (frequency / factor), pairs that complete more than beta_fast keep it, with a linear ramp over the pair index in
    between.  Returns (inv_freq fp32 [head_dim / 2] on the CPU, attention factor 0.1 ln(factor) + 1 that scales cos and
    sin).  The reference reads the same table from the checkpoint's rotary module (gptoss_core_graphs.py:126-127)."""
    d = head_dim

    def corr_dim(n_rot):               # pair index at which a pair makes n_rot full turns over the original context
        return (d * math.log(original_max_position_embeddings / (n_rot * 2 * math.pi))) / (2 * math.log(theta))

    lo, hi = corr_dim(beta_fast), corr_dim(beta_slow)
    if truncate:
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, d - 1)
    if lo == hi:
        hi += 0.001
    pos_freqs = theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d)
    extrap = 1.0 / pos_freqs
    interp = 1.0 / (factor * pos_freqs)
    ramp = torch.clamp((torch.arange(d // 2, dtype=torch.float32) - lo) / (hi - lo), 0, 1)
    keep = 1 - ramp                    # 1: keep the base frequency, 0: interpolate
    inv_freq = interp * (1 - keep) + extrap * keep
    return inv_freq, 0.1 * math.log(factor) + 1.0


@dataclass
class LayerWeights:
    in_w: torch.Tensor        # [2880] input RMSNorm
    Wqkv: torch.Tensor        # [5120, 2880]  q | k | v rows
    bqkv: torch.Tensor        # [5120]
    Wo: torch.Tensor          # [2880, 4096]
    bo: torch.Tensor          # [2880]
    sinks: torch.Tensor       # [64]
    post_w: torch.Tensor      # [2880] post-attention RMSNorm
    Wr: torch.Tensor          # [128, 2880] router
    br: torch.Tensor          # [128]
    sliding: int              # window (0: full attention)

    def to(self, dev):
        kw = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return LayerWeights(**kw)


@dataclass
class DecodeWeights:
    embed: torch.Tensor       # [vocab, 2880]
    layers: list = field(default_factory=list)
    final_w: torch.Tensor = None
    lm_head: torch.Tensor = None  # [vocab, 2880]

    @property
    def vocab(self) -> int:
        return self.embed.shape[0]

    def to(self, dev):
        return DecodeWeights(self.embed.to(dev), [ly.to(dev) for ly in self.layers], self.final_w.to(dev),
                             self.lm_head.to(dev))


TUNED_PROMPT_GEMMS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tunableop_mi355x.csv")


def use_tuned_prompt_gemms(enable: bool = True) -> bool:
    """Let the prompt path's library GEMMs (F.linear: Q|K|V, o_proj, router logits) take the hipBLASLt algorithms
    measured fastest on MI355X for configuration 4's 4,096-token prompt instead of the library's default choice.
    This is PyTorch's TunableOp with tuning off: the choices come from ``TUNED_PROMPT_GEMMS``, whose validator lines
    name the PyTorch, HIP, hipBLASLt and rocBLAS versions and the gfx950 target.  On a mismatch, and for a shape the
    file does not hold, the library's default algorithm runs.  The setting is process-wide, like every TunableOp
    setting.  TunableOp's own results file is pointed at the temp directory, so the committed file is only read.
    Returns whether the file's results were taken; with enable=False, TunableOp is switched off and it returns
    False."""
    import tempfile

    import torch.cuda.tunable as tun
    if not enable:
        tun.enable(False)
        return False
    tun.enable(True)
    tun.tuning_enable(False)
    tun.set_filename(os.path.join(tempfile.gettempdir(), "neural_amd_tunableop.csv"))
    return bool(tun.read_file(TUNED_PROMPT_GEMMS))


def random_weights(n_layers: int = N_LAYERS, vocab: int = VOCAB, device="cpu", seed: int = 0, std: float = 0.02,
                   bias_std: float = 0.02, norm_std: float = 0.02, sink_std: float = 1.0,
                   window: int = WINDOW) -> DecodeWeights:
    """Random-init weights of the model's shapes, bf16: matrices and embeddings N(0, std), biases N(0, bias_std), norm
    weights 1 + N(0, norm_std), sinks N(0, sink_std).  Layer L is a sliding-window layer when L is even.  Drawn with a
    torch generator on ``device`` (a function of the seed on a given device type)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    bf = torch.bfloat16

    def rn(*shape, s=std, mean=0.0):
        t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
        return (t * s + mean).to(bf)

    layers = []
    for li in range(n_layers):
        layers.append(LayerWeights(
            in_w=rn(H, s=norm_std, mean=1.0), Wqkv=rn(QKV_ROWS, H), bqkv=rn(QKV_ROWS, s=bias_std),
            Wo=rn(H, HQ), bo=rn(H, s=bias_std), sinks=rn(NQ, s=sink_std), post_w=rn(H, s=norm_std, mean=1.0),
            Wr=rn(NE, H), br=rn(NE, s=bias_std), sliding=window if li % 2 == 0 else 0))
    return DecodeWeights(rn(vocab, H), layers, rn(H, s=norm_std, mean=1.0), rn(vocab, H))


class DecodeModel:
    """Greedy single-sequence decode over ``weights`` (a DecodeWeights on the device) and ``experts`` (a
    ResidentExperts over the same number of layers or more).

    smax:       positions the full-attention K/V caches hold (the sequence buffer holds smax tokens)
    n_split:    key chunks of full-attention layers (1..64; None: attention.auto_split(smax)); sliding layers use
                ``sliding_split``
    ring:       rows of a sliding layer's rolling K/V cache (>= its window; 0: linear caches of smax rows)
    fused_attn: run each layer's QKV, attention, o_proj and router as one launch (na_core_attn_block) instead of four

    The step reads its input token from ``seq[pos]`` and writes the argmax to ``pred[pos + 1]`` and, unless
    ``pos + 1 < n_forced``, to ``seq[pos + 1]``; it then advances ``pos``.  All of that state lives on the device."""

    def __init__(self, weights: DecodeWeights, experts: ResidentExperts, smax: int, n_split: int | None = None,
                 sliding_split: int = 1, ring: int | None = None, keep_logits: bool = False, sample: bool = False,
                 fused_attn: bool = True):
        dev = weights.embed.device
        if dev.type != "cuda":
            raise ValueError("weights must be on a CUDA device")
        self.w, self.rx, self.dev = weights, experts, dev
        self.n_layers = len(weights.layers)
        if self.n_layers > experts.layout.n_layers:
            raise ValueError("the expert pool holds fewer layers than the model")
        self._check_weights()
        self.smax = int(smax)
        self.n_split = auto_split(self.smax) if n_split is None else int(n_split)
        self.sliding_split = int(sliding_split)
        windows = {ly.sliding for ly in weights.layers if ly.sliding}
        self.ring = (max(windows) if windows else 0) if ring is None else int(ring)
        for win in windows:
            if self.ring and self.ring < win:
                raise ValueError(f"ring {self.ring} is smaller than a sliding window {win}")
        bf = torch.bfloat16
        z = lambda *s, dt=bf: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
        # every layer's K and V cache is a view of one buffer, so that reset() clears them with one launch (72
        # launches of their own cost ~1.4 ms of host time per reset)
        rows_of = [self.ring if (ly.sliding and self.ring) else self.smax for ly in weights.layers]
        per = [NKV * r * HD for r in rows_of]
        self._kv = z(2 * sum(per))
        self.kc, self.vc, off = [], [], 0
        for r, n in zip(rows_of, per):
            self.kc.append(self._kv[off:off + n].view(1, NKV, r, HD))
            self.vc.append(self._kv[off + n:off + 2 * n].view(1, NKV, r, HD))
            off += 2 * n
        inv, self.att_scale = yarn_inv_freq()
        self.inv_freq = inv.to(dev)
        self.scaling = HD ** -0.5
        self.seq = z(self.smax, dt=torch.int64)
        self.pred = z(self.smax, dt=torch.int64)
        self.pos = z(1, dt=torch.int64)
        self.n_forced = z(1, dt=torch.int64)
        self.tok = z(1, dt=torch.int64)
        self.mid, self.xbuf, self.hn, self.g = z(1, H), z(1, H), z(1, H), z(1, H)
        self.q, self.att = z(HQ), z(HQ)
        self.r_logits = z(NE, dt=torch.float32)
        self.r_counter = z(1, dt=torch.int32)
        self.ids = z(1, TOP_K, dt=torch.int64)
        self.wts = z(1, TOP_K)
        self.part = z(N.lib().na_core_lm_partials(weights.vocab), dt=torch.int64)
        self.logits = z(weights.vocab) if keep_logits else None
        # sampling tail (sample=True): temperature (<= 0: greedy) and seed live on the device, so a captured step
        # follows set_sampling() without a new capture; u: optional caller-refreshed uniforms [vocab] fp32
        self.sample = bool(sample)
        self.temp = z(1, dt=torch.float32)
        self.seed = z(1, dt=torch.int64)
        self.u = None
        ns_max = max(self.n_split, self.sliding_split)
        if not 1 <= self.n_split <= 64 or not 1 <= self.sliding_split <= 64:
            raise ValueError("n_split and sliding_split must be in [1, 64]")
        self.attn_work = z(max(N.lib().na_attn_workspace_floats(1, ns_max), 1), dt=torch.float32)
        self.attn_counters = z(NKV, dt=torch.int32)
        self.fused_attn = bool(fused_attn)
        self.sync = z(N.lib().na_core_attn_block_sync_words(), dt=torch.int32)   # fused block's handoff state
        self.sync_redos = 0                  # generate() calls redone with the multi-launch path (sync_error())
        self.graph = None

    def _check_weights(self):
        w = self.w
        shapes = dict(in_w=(H,), Wqkv=(QKV_ROWS, H), bqkv=(QKV_ROWS,), Wo=(H, HQ), bo=(H,), sinks=(NQ,), post_w=(H,),
                      Wr=(NE, H), br=(NE,))
        for li, ly in enumerate(w.layers):
            for nm, shp in shapes.items():
                t = getattr(ly, nm)
                if t.dtype is not torch.bfloat16 or tuple(t.shape) != shp or not t.is_contiguous() \
                        or t.device != self.dev:
                    raise ValueError(f"layer {li} {nm} must be contiguous bf16 {shp} on {self.dev}")
        for nm, shp in (("embed", (w.vocab, H)), ("lm_head", (w.vocab, H)), ("final_w", (H,))):
            t = getattr(w, nm)
            if t.dtype is not torch.bfloat16 or tuple(t.shape) != shp or not t.is_contiguous() or t.device != self.dev:
                raise ValueError(f"{nm} must be contiguous bf16 {shp} on {self.dev}")

    # ------------------------------------------------------------------------------------------------ host state
    def reset(self, tokens, n_forced: int | None = None, pos: int = 0) -> None:
        """Load a token sequence (its first ``n_forced`` tokens are kept, default all of them), zero the K/V caches
        and set the position.  Synchronous host -> device copies; not for use under capture."""
        t = torch.as_tensor(tokens, dtype=torch.int64).reshape(-1)
        if t.numel() > self.smax:
            raise ValueError(f"{t.numel()} tokens exceed smax {self.smax}")
        if t.numel() and (int(t.min()) < 0 or int(t.max()) >= self.w.vocab):
            raise ValueError("token ids outside the vocabulary")
        self.seq.zero_()
        self.seq[:t.numel()] = t.to(self.dev)
        self.pred.fill_(-1)
        self.n_forced.fill_(t.numel() if n_forced is None else int(n_forced))
        self.pos.fill_(int(pos))
        self._kv.zero_()                                   # every K / V cache

    # ------------------------------------------------------------------------------------------------ launches
    def layer(self, li: int, events: dict | None = None) -> None:
        """One layer's launches on the current stream (no host synchronisation, capturable).  events: None, or a dict
        with "attn" (2 timing events: the attention launch, or with fused_attn the whole attention block) and/or
        "experts" (the expert launches' events, ResidentExperts.launches(1)) for dispatch-timestamped timing of an
        eager call (measurement only)."""
        ly = self.w.layers[li]
        s = N.stream(self.dev)
        kc, vc = self.kc[li], self.vc[li]
        ring = self.ring if ly.sliding else 0
        rows = kc.shape[2]
        ns = self.sliding_split if ly.sliding else self.n_split
        if self.fused_attn:
            # with the single-launch expert body, the block stops at the router's logits and the expert body selects
            # the top 4 itself (no wait for every logit at the block's end); otherwise the block selects them
            select_here = not self.rx.one
            N.call("na_core_attn_block", self.mid.data_ptr(), self.g.data_ptr() if li else None, None,
                   self.xbuf.data_ptr(), ly.in_w.data_ptr(), ly.Wqkv.data_ptr(), ly.bqkv.data_ptr(),
                   self.pos.data_ptr(), self.inv_freq.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, ring,
                   self.q.data_ptr(), EPS, float(self.att_scale), ly.sinks.data_ptr(), float(self.scaling),
                   int(ly.sliding), ns, self.attn_work.data_ptr(), self.att.data_ptr(), ly.Wo.data_ptr(),
                   ly.bo.data_ptr(), ly.post_w.data_ptr(), ly.Wr.data_ptr(), ly.br.data_ptr(), self.hn.data_ptr(),
                   self.r_logits.data_ptr(), self.ids.data_ptr() if select_here else None,
                   self.wts.data_ptr() if select_here else None, self.sync.data_ptr(),
                   N.events_array(events.get("attn")) if events else None, s)
            if select_here:
                self.rx.forward_decode(li, self.hn, self.ids, self.wts, out=self.g,
                                       events=events.get("experts") if events else None)
            else:
                self.rx.forward_decode_logits(li, self.hn, self.r_logits, self.g, ids_out=self.ids,
                                              wts_out=self.wts, events=events.get("experts") if events else None)
            return
        N.call("na_core_qkv", self.mid.data_ptr(), self.g.data_ptr() if li else None, None, self.xbuf.data_ptr(),
               ly.in_w.data_ptr(), ly.Wqkv.data_ptr(), ly.bqkv.data_ptr(), self.pos.data_ptr(),
               self.inv_freq.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, ring, self.q.data_ptr(), EPS,
               float(self.att_scale), s)
        N.call("na_decode_attention", self.q.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, ly.sinks.data_ptr(),
               self.pos.data_ptr(), self.att.data_ptr(), 1, float(self.scaling), int(ly.sliding), ring, ns,
               self.attn_work.data_ptr(), self.attn_counters.data_ptr(),
               N.events_array(events.get("attn")) if events else None, s)
        N.call("na_core_oproj", self.att.data_ptr(), ly.Wo.data_ptr(), ly.bo.data_ptr(), self.xbuf.data_ptr(),
               self.mid.data_ptr(), s)
        N.call("na_core_router", self.mid.data_ptr(), ly.post_w.data_ptr(), EPS, ly.Wr.data_ptr(), ly.br.data_ptr(),
               self.hn.data_ptr(), self.r_logits.data_ptr(), self.r_counter.data_ptr(), self.ids.data_ptr(),
               self.wts.data_ptr(), s)
        self.rx.forward_decode(li, self.hn, self.ids, self.wts, out=self.g,
                               events=events.get("experts") if events else None)

    def embed(self) -> None:
        N.call("na_core_embed", self.w.embed.data_ptr(), self.w.vocab, self.seq.data_ptr(), self.smax,
               self.pos.data_ptr(), self.mid.data_ptr(), N.stream(self.dev))

    def tail(self, step_pos: bool = True) -> None:
        args = (self.mid.data_ptr(), self.g.data_ptr() if self.n_layers else None, None, self.w.final_w.data_ptr(),
                EPS, self.w.lm_head.data_ptr(), self.w.vocab, self.hn.data_ptr(), N.ptr(self.logits),
                self.part.data_ptr(), self.tok.data_ptr(), self.pos.data_ptr(), int(step_pos), self.seq.data_ptr(),
                self.n_forced.data_ptr(), self.pred.data_ptr(), self.smax)
        if self.sample:
            N.call("na_core_lm_tail_sample", *args, self.temp.data_ptr(), N.ptr(self.u), self.seed.data_ptr(),
                   N.stream(self.dev))
        else:
            N.call("na_core_lm_tail", *args, N.stream(self.dev))

    def set_sampling(self, temperature: float, seed: int = 0, u: torch.Tensor | None = None) -> None:
        """Sampling tail settings (needs sample=True): temperature > 0 draws from softmax(logits / temperature) by
        Gumbel-max (reference server.py:1576-1583), 0 is greedy; seed keys the on-device uniforms (one draw per
        position and vocabulary entry); u, if given, is a [vocab] fp32 tensor of uniforms the caller refreshes
        before each step instead (the reference's u_dev).  Device writes only: a captured graph picks them up, but
        switching between u and the seeded draws needs a new capture."""
        if not self.sample:
            raise RuntimeError("this DecodeModel was built without the sampling tail (sample=True)")
        if u is not None and (u.dtype is not torch.float32 or u.numel() != self.w.vocab or u.device != self.dev
                              or not u.is_contiguous()):
            raise ValueError(f"u must be contiguous fp32 [{self.w.vocab}] on {self.dev}")
        self.temp.fill_(float(temperature))
        self.seed.fill_(int(seed) & 0x7FFFFFFFFFFFFFFF)
        self.u = u

    def step(self, events=None) -> None:
        """One decode step (embed, every layer, tail) on the current stream.  events: None or one dict per layer (see
        layer())."""
        self.embed()
        for li in range(self.n_layers):
            self.layer(li, None if events is None else events[li])
        self.tail()

    def snapshot(self):
        """Copy of the decode state a later restore() returns to: position, sequence and every K/V cache (use it to
        rerun the same steps from the same context)."""
        return self.pos.clone(), self.seq.clone(), self.n_forced.clone(), self._kv.clone()

    def restore(self, snap) -> None:
        """In-place restore of a snapshot (buffer addresses unchanged, so captured graphs stay valid)."""
        pos, seq, nf, kv = snap
        self.pos.copy_(pos)
        self.seq.copy_(seq)
        self.n_forced.copy_(nf)
        self._kv.copy_(kv)                                 # every K / V cache

    # ------------------------------------------------------------------------------------------------ prompt
    def prefill(self, tokens, chunk: int = 4096, trace: list | None = None) -> None:
        """Prompt processing (reference server.py:2406-2418 _prefill_block, entry prefill :2446): load ``tokens``
        (as reset()), run them through every layer in blocks of ``chunk`` tokens (each block through all layers, its
        K/V written into the caches, so later blocks attend to earlier ones), then the tail of the last prompt token:
        its greedy successor goes to seq[T] (unless T < n_forced) and pos becomes T, where decode steps continue.

        Per layer and block: residual + input RMSNorm (na_rows_norm), Q|K|V = F.linear (a bf16 library GEMM, as the
        reference), RoPE + K/V store (na_rows_rope: straight into the linear cache, or into block buffers that
        na_ring_write copies into a rolling cache after the attention), prompt attention (na_prefill_attention),
        o_proj = F.linear, residual + post-attention RMSNorm, router logits = F.linear and top-4 (na_rows_topk), the
        experts (ResidentExperts.forward_prefill).  Host-driven launches on the current stream; not capturable (the
        block size sets the shapes).  trace: optional list that receives one dict of device tensors per (block,
        layer) with the stage inputs and outputs (for parity tests)."""
        t = torch.as_tensor(tokens, dtype=torch.int64).reshape(-1)
        T = t.numel()
        if T < 1 or T >= self.smax:
            raise ValueError(f"a prompt of 1 .. {self.smax - 1} tokens is needed (got {T})")
        if chunk < 1:
            raise ValueError("chunk must be positive")
        self.reset(t)
        x = m = None
        for a in range(0, T, chunk):
            x, m = self._prefill_block(a, min(chunk, T - a), trace)
        self.mid.copy_(x[-1:])
        self.g.copy_(m[-1:]) if m is not None else self.g.zero_()
        self.pos.fill_(T - 1)
        self.tail()

    def _prefill_block(self, p0: int, T: int, trace):
        import torch.nn.functional as F

        dev, s, bf = self.dev, N.stream(self.dev), torch.bfloat16
        x = torch.empty(T, H, dtype=bf, device=dev)
        hn = torch.empty(T, H, dtype=bf, device=dev)
        q = torch.empty(T, NQ, HD, dtype=bf, device=dev)
        ids = torch.empty(T, TOP_K, dtype=torch.int64, device=dev)
        wts = torch.empty(T, TOP_K, dtype=bf, device=dev)
        N.call("na_rows_embed", self.w.embed.data_ptr(), self.w.vocab, self.seq.data_ptr() + 8 * p0, T, x.data_ptr(),
               s)
        m = None
        for li, ly in enumerate(self.w.layers):
            rec = {"p0": p0, "layer": li, "x_in": x.clone(), "m_in": None if m is None else m} if trace is not None \
                else None
            N.call("na_rows_norm", x.data_ptr(), N.ptr(m), T, ly.in_w.data_ptr(), EPS, hn.data_ptr(), s)
            if rec is not None:
                rec.update(x=x.clone(), h=hn.clone())
            qkv = F.linear(hn, ly.Wqkv, ly.bqkv)
            kc, vc = self.kc[li], self.vc[li]
            rows = kc.shape[2]
            ring = self.ring if ly.sliding else 0
            if ring:
                kn = torch.empty(T, NKV, HD, dtype=bf, device=dev)
                vn = torch.empty(T, NKV, HD, dtype=bf, device=dev)
                N.call("na_rows_rope", qkv.data_ptr(), T, p0, self.inv_freq.data_ptr(), float(self.att_scale),
                       q.data_ptr(), kn.data_ptr(), NKV * HD, HD, vn.data_ptr(), NKV * HD, HD, s)
                o = prefill_attention(q, kc, vc, ly.sinks, p0, self.scaling, ly.sliding, self.smax, k_new=kn,
                                      v_new=vn, ring=ring)
                ring_write(kc, vc, kn, vn, p0, ring)
            else:
                kn = vn = None
                N.call("na_rows_rope", qkv.data_ptr(), T, p0, self.inv_freq.data_ptr(), float(self.att_scale),
                       q.data_ptr(), kc.data_ptr() + 2 * p0 * HD, HD, rows * HD, vc.data_ptr() + 2 * p0 * HD, HD,
                       rows * HD, s)
                o = prefill_attention(q, kc, vc, ly.sinks, p0, self.scaling, ly.sliding, rows)
            att = F.linear(o.view(T, HQ), ly.Wo, ly.bo)
            if rec is not None:
                rec.update(qkv=qkv, q=q.clone(), k_new=kn, v_new=vn, o=o, att=att)
            N.call("na_rows_norm", x.data_ptr(), att.data_ptr(), T, ly.post_w.data_ptr(), EPS, hn.data_ptr(), s)
            logits = F.linear(hn, ly.Wr, ly.br)
            N.call("na_rows_topk", logits.data_ptr(), T, ids.data_ptr(), wts.data_ptr(), s)
            m = self.rx.forward_prefill(li, hn, ids, wts)
            if rec is not None:
                rec.update(mid=x.clone(), hn=hn.clone(), logits=logits, ids=ids.clone(), wts=wts.clone(), m=m)
                if not ring:
                    rec.update(k_cache=kc[0, :, p0:p0 + T].clone(), v_cache=vc[0, :, p0:p0 + T].clone())
                trace.append(rec)
        return x, m

    # ------------------------------------------------------------------------------------------------ graphs
    def sync_error(self) -> bool:
        """Whether a fused attention block, a single-launch expert body or the tail gave up a wait since the last
        clear_sync_error() (the outputs of that step are then invalid).  Reads the device (synchronises).  The
        waits rely on every workgroup of a launch being resident together, which a kernel of another stream or
        process on the same GPU can break; a caller replaying captured steps (run(), capture()) polls this after
        its replays and redoes them with the multi-launch path on True, as generate() does."""
        return bool(int(self.sync[0].item())) or bool(int(self.part[0].item()) & 0xFFFFFFFF) \
            or self.rx.sync_error()

    def clear_sync_error(self) -> None:
        """Zero the error words (the kernels only ever set them)."""
        self.sync[:1].zero_()
        self.part[:1].zero_()
        self.rx.clear_sync_error()

    def capture(self) -> torch.cuda.CUDAGraph:
        """Capture one step as a hipGraph (replay = one greedy step at the device-side position).  The capture itself
        runs nothing; state is untouched."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g
        return g

    def run(self, n_steps: int, graph: bool = True) -> None:
        """n_steps decode steps from the current device state (graph replays when a graph was captured).  Nothing is
        checked here: the caller reads sync_error() afterwards (generate() does, and redoes the steps)."""
        if graph:
            if self.graph is None:
                self.capture()
            for _ in range(n_steps):
                self.graph.replay()
        else:
            for _ in range(n_steps):
                self.step()

    def generate(self, prompt, n_new: int, graph: bool = True):
        """Greedy decode: read the prompt token by token (its K/V written by decode steps), then ``n_new`` new
        tokens.  Returns the full sequence (prompt + new tokens) as a CPU int64 tensor."""
        p = torch.as_tensor(prompt, dtype=torch.int64).reshape(-1)
        if p.numel() < 1 or p.numel() + n_new > self.smax:
            raise ValueError("prompt must be non-empty and prompt + n_new must fit smax")
        n_steps = p.numel() - 1 + n_new
        self.reset(p)
        self.run(n_steps, graph)
        torch.cuda.synchronize(self.dev)
        if self.sync_error():
            # a bounded wait gave up somewhere, so some step used stale data: decode again from the prompt with the
            # multi-launch path (separate QKV / attention / o_proj / router launches and the two-launch expert
            # body: the same bits, and no wait between workgroups)
            self.sync_redos += 1
            self.clear_sync_error()
            fused, one = self.fused_attn, self.rx.one
            self.fused_attn, self.rx.one = False, False
            try:
                self.reset(p)
                self.run(n_steps, graph=False)
                torch.cuda.synchronize(self.dev)
            finally:
                self.fused_attn, self.rx.one = fused, one
            if self.sync_error():
                raise RuntimeError("the multi-launch decode path flagged its error word (it has no waits to give up)")
        return self.seq[:p.numel() + n_new].cpu()
