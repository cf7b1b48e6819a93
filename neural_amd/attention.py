"""GQA decode attention with learned sinks on MI355X: the call surface of the reference's fused_core.py attention
helpers (decode_attention, SplitAttn, ring_write, ring_reuse_ok; reference fused_core.py:63, 336-398, 787-820), backed
by the HIP kernel of neural_amd/csrc/attention.hip through the C ABI.

Shapes (reference fused_core.py:63): NQ = 64 query heads, NKV = 8 KV heads, HD = 64, REP = 8.  One decode query per
sequence: q [NQ*HD] bf16 (RoPE applied), K/V caches [1, NKV, S, HD] bf16 (S = smax, or the ring size on sliding
layers with a rolling cache), sinks [NQ] bf16, pos int64 on the device, out [NQ*HD] bf16.  The batched form takes
q [B, NQ*HD], caches [B, NKV, S, HD] and pos [B].

Arithmetic: scores s = bf16(bf16(q . k) * scaling) exactly as the reference (fp32 accumulation); the sink softmax
and P V are computed as flash decoding over key chunks (fp32 softmax, bf16 P into an fp32-accumulating MFMA),
combined in chunk order by the last workgroup of each (sequence, KV head): one launch per call.  Outputs match the
reference's within bf16 rounding; ring and linear caches give bit-identical outputs (only the addressing differs).
Everything runs on the current stream, allocates nothing per call, never synchronises and never reads pos on the
host, so a call can be captured in a hipGraph and replayed with pos changed on the device.
"""
from __future__ import annotations

import torch

from . import _native as N

H, HP, NQ, NKV, HD, NE, K = 2880, 4096, 64, 8, 64, 128, 4
REP = NQ // NKV
MAX_SPLIT = 64


def _check(q, kc, vc, sinks, pos_dev, out, B, ring, sliding):
    bf = torch.bfloat16
    for t, nm in ((q, "q"), (kc, "kc"), (vc, "vc"), (sinks, "sinks"), (out, "out")):
        if t.dtype is not bf:
            raise AssertionError(f"{nm} must be bf16")
        if not t.is_contiguous():
            raise AssertionError(f"{nm} must be contiguous")
        if t.device.type != "cuda" or t.device != q.device:
            raise AssertionError(f"{nm} must be on the query's CUDA device")
    if q.numel() != B * NQ * HD or out.numel() != B * NQ * HD:
        raise AssertionError(f"q and out must hold {B} x {NQ * HD} values")
    if kc.dim() != 4 or kc.shape[0] != B or kc.shape[1] != NKV or kc.shape[3] != HD or kc.shape != vc.shape:
        raise AssertionError(f"kc/vc must be [{B}, {NKV}, S, {HD}] and equal-shaped")
    if sinks.numel() != NQ:
        raise AssertionError(f"sinks must hold {NQ} values")
    if pos_dev.dtype is not torch.int64 or pos_dev.numel() != B or pos_dev.device != q.device:
        raise AssertionError(f"pos must be int64 [{B}] on the query's device")
    if ring:
        if not sliding or ring < int(sliding) or kc.shape[2] != ring:
            raise AssertionError(f"a ring cache needs a sliding layer, ring >= window and S == ring "
                                 f"(sliding={sliding}, ring={ring}, S={kc.shape[2]})")


def _launch(q, kc, vc, sinks, pos_dev, out, scaling, sliding, ring, ns, work, counters, B, events=None):
    N.call("na_decode_attention", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.shape[2], sinks.data_ptr(),
           pos_dev.data_ptr(), out.data_ptr(), B, float(scaling), int(sliding or 0), int(ring or 0), int(ns),
           N.ptr(work), N.ptr(counters), N.events_array(events), N.stream(q.device))


class SplitAttn:
    """Preallocated workspace + launcher for chunked decode attention (reference fused_core.py:336-382).

    ``ns`` chunks per (sequence, KV head), 1 <= ns <= 64; the key range of each chunk is computed on the device from
    pos with the reference's rule (64-key blocks, ceil(blocks / ns) per chunk).  One instance serves every layer of
    a model that runs on one stream (calls must not overlap: they share the workspace and the per-head counters,
    which every completed call leaves at zero).  ``bn``, ``cache_s`` and ``num_warps`` are accepted for interface
    compatibility and have no effect (the kernel keeps scores in registers and LDS)."""

    def __init__(self, ns, smax, dev, bn=64, cache_s=True, num_warps=4, batch=1):
        if not 1 <= int(ns) <= MAX_SPLIT:
            raise AssertionError(f"ns must be in [1, {MAX_SPLIT}]")
        self.ns, self.smax, self.bn, self.cache_s, self.num_warps = int(ns), int(smax), int(bn), bool(cache_s), num_warps
        self.batch = int(batch)
        nw = N.lib().na_attn_workspace_floats(self.batch, self.ns)
        self.work = torch.empty(max(nw, 1), dtype=torch.float32, device=dev)
        self.counters = torch.zeros(self.batch * NKV, dtype=torch.int32, device=dev)

    def launch(self, q, kc, vc, sinks, pos_dev, out, scaling, sliding=0, ring=0, events=None):
        B = kc.shape[0]
        if B > self.batch:
            raise AssertionError(f"this SplitAttn was sized for batch {self.batch}")
        if not ring and kc.shape[-2] != self.smax:
            raise AssertionError(f"cache rows {kc.shape[-2]} != smax {self.smax}")
        _check(q, kc, vc, sinks, pos_dev, out, B, ring, sliding)
        _launch(q, kc, vc, sinks, pos_dev, out, scaling, sliding, ring, self.ns, self.work, self.counters, B, events)


def decode_attention(q, kc, vc, sinks, pos_dev, out, scaling, sliding, smax, ring=0, bn=64, split=None):
    """Decode attention of one query (reference fused_core.py:385-398).  q [NQ*HD]; kc/vc [1, NKV, smax, HD] (or
    [1, NKV, ring, HD] with ring > 0, sliding layers only); pos_dev int64 [1]; out [NQ*HD].  split: a SplitAttn
    (chunked over the key range); None: one workgroup per KV head walks the whole range."""
    if split is not None:
        if sliding or ring:
            raise AssertionError("split-K is for full-attention layers")
        split.launch(q, kc, vc, sinks, pos_dev, out, scaling)
        return out
    if not ring and kc.shape[-2] != smax:
        raise AssertionError(f"cache rows {kc.shape[-2]} != smax {smax}")
    _check(q, kc, vc, sinks, pos_dev, out, 1, ring, sliding)
    _launch(q, kc, vc, sinks, pos_dev, out, scaling, sliding, ring, 1, None, None, 1)
    return out


def decode_attention_batched(q, kc, vc, sinks, pos_dev, out, scaling, sliding=0, ring=0, split=None, events=None):
    """B decode queries, one per sequence: q [B, NQ*HD], caches [B, NKV, S, HD], pos_dev int64 [B] (each sequence
    its own position), out [B, NQ*HD].  The reference serves one sequence per call; this is its batched form."""
    B = kc.shape[0]
    if split is not None:
        split.launch(q, kc, vc, sinks, pos_dev, out, scaling, sliding, ring, events)
        return out
    _check(q, kc, vc, sinks, pos_dev, out, B, ring, sliding)
    _launch(q, kc, vc, sinks, pos_dev, out, scaling, sliding, ring, 1, None, None, B, events)
    return out


def ring_write(kc, vc, k_new, v_new, p0, ring):
    """Store the last min(T, ring) positions of a block (positions p0 .. p0+T-1, K/V [T, NKV, HD]) into their ring
    slots (slot = position % ring), as reference fused_core.py:787-800: at most two contiguous slice copies on the
    device, no allocation, no host synchronisation."""
    T = k_new.shape[0]
    n = min(T, ring)
    a = T - n
    s0 = (p0 + a) % ring
    first = min(n, ring - s0)
    kc[0, :, s0:s0 + first] = k_new[a:a + first].transpose(0, 1)
    vc[0, :, s0:s0 + first] = v_new[a:a + first].transpose(0, 1)
    if first < n:
        kc[0, :, :n - first] = k_new[a + first:].transpose(0, 1)
        vc[0, :, :n - first] = v_new[a + first:].transpose(0, 1)


def ring_reuse_ok(n_written, c, ring, window=128):
    """Whether a rolling cache last written with positions 0 .. n_written-1 still holds the window a block starting
    at position c needs (reference fused_core.py:803-820): c <= n_written and (n_written <= ring or
    n_written - c <= ring - window + 1)."""
    if c > n_written:
        return False
    if n_written <= ring:
        return True
    return n_written - c <= ring - window + 1
