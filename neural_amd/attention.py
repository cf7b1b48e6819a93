"""GQA attention with learned sinks on MI355X: the call surface of the reference's fused_core.py attention helpers
(decode_attention, SplitAttn, prefill_attention, ring_write, ring_reuse_ok; reference fused_core.py:63, 336-398,
684-820), backed by the HIP kernels of neural_amd/csrc/attention.hip (decode) and neural_amd/csrc/prefill_attn.hip
(prompt attention, ring write) through the C ABI.

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
SUB_KEYS = 256                 # keys one chunk workgroup takes per pass (4 waves x 64)


def auto_split(smax: int) -> int:
    """Key chunks for full-attention layers over caches of ``smax`` positions: as few as keep every chunk within one
    256-key pass at the longest context.  Under the reference's chunk rule (64-key blocks, ceil(blocks / ns) per
    chunk) ns = ceil(ceil(smax / 64) / 4) gives chunks of at most 4 blocks; a chunk workgroup's time is that of its
    passes, so more chunks only add partials to combine, and fewer give some chunk a second pass."""
    blocks = -(-int(smax) // 64)
    return max(1, min(MAX_SPLIT, -(-blocks // (SUB_KEYS // 64))))


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


def _rows_ok(t):
    """[T, NKV, HD] bf16 on CUDA with a contiguous last dimension, 16-byte aligned rows and element strides that are
    multiples of 8 (what the kernels' 16-byte row loads need)."""
    return (t.dtype is torch.bfloat16 and t.dim() == 3 and t.shape[1:] == (NKV, HD) and t.stride(-1) == 1
            and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0)


def _as_rows(t):
    return t if _rows_ok(t) else t.contiguous()


def prefill_attention(q, kc, vc, sinks, p0, scaling, sliding, smax, BM=64, BN=64, k_new=None, v_new=None, ring=0,
                      out=None, events=None):
    """Prompt attention (reference fused_core.py:684-784): q [T, NQ, HD] bf16 (contiguous, RoPE applied) for positions
    p0 .. p0+T-1 -> o [T, NQ, HD] bf16.  Causal, sliding window when ``sliding`` > 0, learned sinks.

    ring = 0: kc / vc are the linear cache [1, NKV, smax, HD] ALREADY holding the block's K / V at p0 .. p0+T-1
              (k_new / v_new ignored).
    ring = R: sliding layers only; kc / vc are the rolling cache [1, NKV, R, HD] holding positions p0-R .. p0-1 (those
              that exist) and k_new / v_new [T, NKV, HD] (last dim contiguous) are the block's own K / V.  T may exceed
              R.  The ring is not updated here: call ring_write(kc, vc, k_new, v_new, p0, R) after the attention.
    Ring and linear mode give bit-identical outputs for the same key values.  ``BM`` / ``BN`` (the reference's Triton
    tiling) are accepted and have no effect: the kernel's tiling is fixed (32 queries x 8 heads per workgroup, 64-key
    tiles).  One launch on the current stream, no allocation beyond ``out`` (allocated when None), no host sync."""
    bf = torch.bfloat16
    T = q.shape[0]
    if q.dtype is not bf or q.dim() != 3 or q.shape[1:] != (NQ, HD) or not q.is_contiguous():
        raise AssertionError(f"q must be contiguous bf16 [T, {NQ}, {HD}]")
    for t, nm in ((kc, "kc"), (vc, "vc"), (sinks, "sinks")):
        if t.dtype is not bf or not t.is_contiguous() or t.device != q.device:
            raise AssertionError(f"{nm} must be contiguous bf16 on the query's device")
    if sinks.numel() != NQ:
        raise AssertionError(f"sinks must hold {NQ} values")
    rows = int(ring) if ring else int(smax)
    if kc.shape != (1, NKV, rows, HD) or vc.shape != kc.shape:
        raise AssertionError(f"kc/vc must be [1, {NKV}, {rows}, {HD}] (shape {tuple(kc.shape)})")
    p0 = int(p0)
    if ring:
        if not sliding or int(ring) < int(sliding):
            raise AssertionError(f"a ring cache needs a sliding layer and ring >= window ({sliding}, {ring})")
        if k_new is None or v_new is None or k_new.shape != (T, NKV, HD) or v_new.shape != (T, NKV, HD):
            raise AssertionError(f"k_new/v_new must be [{T}, {NKV}, {HD}]")
        if k_new.stride(-1) != 1 or v_new.stride(-1) != 1:
            raise AssertionError("k_new/v_new need a contiguous last dimension")
        kn, vn = _as_rows(k_new), _as_rows(v_new)
        st = (kn.stride(0), kn.stride(1), vn.stride(0), vn.stride(1))
        kp, vp = kn.data_ptr(), vn.data_ptr()
    else:
        if p0 + T > int(smax):
            raise AssertionError(f"positions up to {p0 + T} exceed the cache's {smax} rows")
        st, kp, vp = (0, 0, 0, 0), None, None
    if out is None:
        out = torch.empty_like(q)
    elif out.dtype is not bf or out.shape != q.shape or not out.is_contiguous():
        raise AssertionError("out must be contiguous bf16 shaped like q")
    N.call("na_prefill_attention", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows, kp, vp, *st, sinks.data_ptr(),
           out.data_ptr(), p0, T, float(scaling), int(sliding or 0), int(ring or 0), N.events_array(events),
           N.stream(q.device))
    return out


def ring_write(kc, vc, k_new, v_new, p0, ring):
    """Store the last min(T, ring) positions of a block (positions p0 .. p0+T-1, K/V [T, NKV, HD]) into their ring
    slots (slot = position % ring) of kc / vc [1, NKV, ring, HD], as reference fused_core.py:787-800.  One launch on
    the current stream, no host synchronisation; call it after the block's attention."""
    T = k_new.shape[0]
    if kc.shape != (1, NKV, int(ring), HD) or vc.shape != kc.shape or not kc.is_contiguous() or not vc.is_contiguous():
        raise AssertionError(f"kc/vc must be contiguous [1, {NKV}, {ring}, {HD}]")
    if kc.dtype is not torch.bfloat16 or vc.dtype is not torch.bfloat16:
        raise AssertionError("kc/vc must be bf16")
    if k_new.shape != (T, NKV, HD) or v_new.shape != (T, NKV, HD):
        raise AssertionError(f"k_new/v_new must be [{T}, {NKV}, {HD}]")
    kn, vn = _as_rows(k_new), _as_rows(v_new)
    N.call("na_ring_write", kc.data_ptr(), vc.data_ptr(), int(ring), kn.data_ptr(), vn.data_ptr(), kn.stride(0),
           kn.stride(1), vn.stride(0), vn.stride(1), int(p0), T, N.stream(kc.device))


def ring_reuse_ok(n_written, c, ring, window=128):
    """Whether a rolling cache last written with positions 0 .. n_written-1 still holds the window a block starting
    at position c needs (reference fused_core.py:803-820): c <= n_written and (n_written <= ring or
    n_written - c <= ring - window + 1)."""
    if c > n_written:
        return False
    if n_written <= ring:
        return True
    return n_written - c <= ring - window + 1
