"""MXFP4 expert products on MI355X: the Python call surface of the reference's ``neural/q80/mxfp4_kernels.py``,
dispatching to hand-written gfx950 HIP kernels (neural_amd/csrc) through the C-ABI library.

Kept from the reference (same names, argument meaning and error behaviour):
  * ``mxfp4_gemv`` / ``mxfp4_gemv_masked`` (reference :474-489, :542-569): decode GEMV over slots, out [E, N] bf16;
  * ``mxfp4_gemm`` / ``mxfp4_gemm_into`` (:202-231), ``GroupedGemmPlan`` (:318-382), ``mxfp4_gemm_grouped_into``
    (:385-419), ``_grouped_tile_rows`` (:298-315): prefill products;
  * ``_scale_layout`` (:72-84): the raw / PS4 scale layout is read off the scales view, an explicit ``packed=`` is
    checked against it and never trusted over it;
  * the module switches FAST_LAUNCH, PREFILL_BLOCK_M, PREFILL_GROUP, PREFILL_GROUPED_GEMM, PREFILL_GROUP_ROWS,
    PREFILL_GROUP_EXPERTS (:35-59), read from the same environment variables.
Triton tiling knobs (block_n, block_g, num_warps) are accepted; block_n maps to the rows a workgroup streams, the
others have no meaning for these kernels and are ignored.

Arithmetic: exact E2M1 x 2^(s-127) dequant in registers, fp32 accumulation, one bf16 rounding of each output
(the reference's contract, :1-7).  Deterministic: fixed grid, fixed reduction order, no atomics in the products;
every launch goes on torch's current stream and allocates nothing beyond the returned tensor, so calls are
hipGraph-capturable.
"""
from __future__ import annotations

import operator
import os

import numpy as np
import torch

from .. import _native as N

FAST_LAUNCH = os.environ.get("NEURAL_FAST_LAUNCH", "1") != "0"
PREFILL_BLOCK_M = int(os.environ.get("NEURAL_PREFILL_BM", "64"))
if PREFILL_BLOCK_M < 16 or PREFILL_BLOCK_M & (PREFILL_BLOCK_M - 1):
    raise ValueError(f"NEURAL_PREFILL_BM={PREFILL_BLOCK_M}: BLOCK_M must be a power of two >= 16")
PREFILL_GROUP = os.environ.get("NEURAL_PREFILL_GROUP", "0") != "0"
PREFILL_GROUPED_GEMM = os.environ.get("NEURAL_PREFILL_GROUPED_GEMM", "0") != "0"
PREFILL_GROUP_ROWS = int(os.environ.get("NEURAL_PREFILL_GROUP_ROWS", "16384"))
PREFILL_GROUP_EXPERTS = int(os.environ.get("NEURAL_PREFILL_GROUP_EXPERTS", "0"))
if PREFILL_GROUP_ROWS < 1 or PREFILL_GROUP_EXPERTS < 0:
    raise ValueError(f"NEURAL_PREFILL_GROUP_ROWS={PREFILL_GROUP_ROWS} (>= 1), NEURAL_PREFILL_GROUP_EXPERTS="
                     f"{PREFILL_GROUP_EXPERTS} (>= 0)")

GK_SUPPORTED = 90          # K = 2880: the GPT-OSS-120B geometry these kernels are built for


def _scale_layout(scales: torch.Tensor, GK: int, packed) -> bool:
    """Whether ``scales`` (..., N, w) holds PS4 rows (reference mxfp4_kernels.py:72-84).

    The row width decides: GK bytes is a raw E8M0 row, GK // 2 + 1 a PS4 row (a base byte and GK / 2 bytes of two
    4-bit deltas).  ``packed`` (None = infer) must agree with what the width says: a flag never overrides the
    view.  The rows must be dense (unit stride inside a row, rows back to back)."""
    row_kinds = {GK: False, GK // 2 + 1: True}
    width = int(scales.shape[-1])
    if width not in row_kinds:
        raise ValueError(f"scales view has row width {width}: want {GK} (raw E8M0) or {GK // 2 + 1} (packed 4-bit)")
    is_ps4 = row_kinds[width]
    if packed is not None and bool(packed) is not is_ps4:
        raise ValueError(f"packed={packed} but the scales view row width {width} says "
                         f"{'packed' if is_ps4 else 'raw'} (GK={GK})")
    if (scales.stride(-2), scales.stride(-1)) != (width, 1):
        raise ValueError(f"scales rows must be contiguous (strides {tuple(scales.stride())}, row width {width})")
    return is_ps4


def _check_pool_views(blocks: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, slots: torch.Tensor):
    if blocks.ndim != 4 or blocks.shape[-1] != 16 or blocks.dtype is not torch.uint8:
        raise ValueError("blocks must be a uint8 [cap, N, GK, 16] view")
    cap, n, gk, _ = blocks.shape
    if tuple(blocks.stride()[1:]) != (gk * 16, 16, 1):
        raise ValueError("blocks rows must be contiguous")
    if scales.dtype is not torch.uint8 or scales.ndim != 3 or tuple(scales.shape[:2]) != (cap, n):
        raise ValueError("scales must be a uint8 [cap, N, w] view matching blocks")
    if gk != GK_SUPPORTED:
        raise ValueError(f"GK={gk}: these kernels are built for K = {GK_SUPPORTED * 32} (GPT-OSS-120B)")
    if n % 2:
        raise ValueError(f"N={n}: rows are streamed in pairs, N must be even")
    for t, nm in ((blocks, "blocks"), (scales, "scales"), (slots, "slots")):
        if t.device != x.device or t.device.type != "cuda":
            raise ValueError(f"{nm} must be on the input's CUDA device")
    if slots.dtype is not torch.int64 or not slots.is_contiguous():
        raise ValueError("slots must be a contiguous int64 tensor")
    return cap, n, gk


def _gemv(x, blocks, scales, slots, active, per_expert_x, block_n, packed):
    E = slots.numel()
    cap, n, gk = _check_pool_views(blocks, scales, x, slots)
    pk = _scale_layout(scales, gk, packed)
    if (x.dtype is not torch.bfloat16 or not x.is_contiguous() or x.ndim != 2
            or tuple(x.shape) != ((E if per_expert_x else 1), gk * 32)):
        raise ValueError("GEMV requires contiguous bf16 x[1,K] or per-expert x[E,K]")
    out = torch.empty(E, n, dtype=torch.bfloat16, device=x.device)
    if E == 0:
        return out
    adt = 0
    if active is not None:
        adt = 1 if active.dtype is torch.bfloat16 else 2
    pairs = 2 if int(block_n) >= 32 else 1     # row pairs per wavefront (the Triton block_n has no direct analogue)
    N.call("na_mxfp4_gemv", x.data_ptr(), int(per_expert_x), blocks.data_ptr(), blocks.stride(0),
           scales.data_ptr(), scales.stride(0), int(pk), slots.data_ptr(), E, N.ptr(active), adt, out.data_ptr(),
           n, gk * 32, pairs, None, N.stream(x.device))
    return out


def mxfp4_gemv(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, slots: torch.Tensor, *,
               per_expert_x: bool = False, block_n: int = 64, block_g: int = 4, num_warps: int = 4,
               packed: bool | None = None) -> torch.Tensor:
    """Decode GEMV: x [1, K] shared, or [E, K] with per_expert_x=True.  Returns [E, N] bf16 with
    out[e, n] = bf16(sum_k x[k] * w_slot[e][n, k]) (reference mxfp4_kernels.py:474-489)."""
    return _gemv(x, blocks, scales, slots, None, per_expert_x, block_n, packed)


def mxfp4_gemv_masked(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, slots: torch.Tensor,
                      active_weights: torch.Tensor, *, per_expert_x=False, block_n=64, block_g=4, num_warps=4,
                      packed=None):
    """GEMV with zero-weight experts skipped: a slot whose active weight is +-0 writes +0 rows and reads none of its
    weights; NaN and nonzero weights take the stock arithmetic (reference mxfp4_kernels.py:492-569)."""
    E = slots.numel()
    if (active_weights.ndim != 1 or active_weights.numel() != E or not active_weights.is_contiguous()
            or active_weights.device != x.device or active_weights.dtype not in (torch.bfloat16, torch.float32)):
        raise ValueError("active_weights needs one contiguous bf16/fp32 scalar per slot on the input device")
    if (x.dtype is not torch.bfloat16 or not x.is_contiguous() or x.ndim != 2
            or x.shape[1] != blocks.shape[2] * 32 or x.shape[0] != (E if per_expert_x else 1)):
        raise ValueError("masked GEMV requires contiguous bf16 x[1,K] or per-expert x[E,K]")
    if slots.device != x.device or blocks.device != x.device or scales.device != x.device:
        raise ValueError("masked GEMV tensors must share a device")
    return _gemv(x, blocks, scales, slots, active_weights, per_expert_x, block_n, packed)


# ------------------------------------------------------------------------------------------ prefill planning
_I31 = 2 ** 31 - 1


def _tile_height(block_m) -> int:
    bm = operator.index(block_m)
    if bm < 16 or bm & (bm - 1):
        raise ValueError("block_m must be a power of two >= 16")
    return bm


def _descriptor_table(pair_descriptors) -> np.ndarray:
    """The (x address, y address, slot, M) descriptors as an int64 [P, 4] table, each entry an integer
    (operator.index), addresses and slots non-negative, 0 <= M <= 2^31 - 1."""
    table = []
    for desc in pair_descriptors:
        desc = tuple(desc)
        if len(desc) != 4:
            raise ValueError("pair descriptor must have four integers")
        table.append([operator.index(v) for v in desc])
    arr = np.array(table, dtype=object).reshape(-1, 4)
    if arr.size and ((arr[:, :3] < 0).any() or (arr[:, 3] < 0).any() or (arr[:, 3] > _I31).any()):
        raise ValueError("invalid pointer, slot or pair row count")
    return arr.astype(np.int64)


def _tile_table(descs: np.ndarray, bm: int) -> np.ndarray:
    """int64 [ntiles, 5]: pair by pair in the given order, one row (x, y, slot, M, pm) per block of bm rows of the
    pair, pm = 0 .. ceil(M / bm) - 1; a pair with M = 0 has no row."""
    per_pair = -(-descs[:, 3] // bm)
    first = np.cumsum(per_pair) - per_pair                 # index of each pair's first tile
    out = np.empty((int(per_pair.sum()), 5), dtype=np.int64)
    out[:, :4] = np.repeat(descs, per_pair, axis=0)
    out[:, 4] = np.arange(out.shape[0]) - np.repeat(first, per_pair)
    return out


def _grouped_tile_rows(pair_descriptors, block_m):
    """Tile rows of a ragged launch (reference mxfp4_kernels.py:298-315): for descriptors (x address, y address,
    slot, M), the tuples (x, y, slot, M, pm), pm = 0 .. ceil(M / block_m) - 1 per pair, pairs in the given order.
    Tiles never span two pairs; an empty pair has none.  ValueError for a block_m that is not a power of two >= 16
    and for a malformed descriptor."""
    bm = _tile_height(block_m)
    return [tuple(r) for r in _tile_table(_descriptor_table(pair_descriptors), bm).tolist()]


def _byte_spans(tensors) -> np.ndarray:
    """[n, 2] int64 half-open byte ranges [start, end) of contiguous tensors, sorted by start."""
    spans = np.array([(t.data_ptr(), t.data_ptr() + t.numel() * t.element_size()) for t in tensors],
                     dtype=np.int64).reshape(-1, 2)
    return spans[np.argsort(spans[:, 0], kind="stable")]


def _check_disjoint_outputs(xs, outs):
    """Outputs must not overlap one another, and no output may overlap any input (inputs may repeat)."""
    w = _byte_spans(outs)
    if (w[1:, 0] < w[:-1, 1]).any():
        raise ValueError("grouped output slices overlap")
    r = _byte_spans(xs)
    if len(w) and len(r):
        # w is sorted and disjoint, so its ends are sorted too: the first output ending after a read's start is the
        # only one that can reach into it from below; any later one starts after it.
        k = np.searchsorted(w[:, 1], r[:, 0], side="right")
        hit = k < len(w)
        if (w[np.minimum(k, len(w) - 1), 0][hit] < r[hit, 1]).any():
            raise ValueError("grouped outputs overlap an input slice")


def _aligned16(x, out) -> bool:
    return all(v % 16 == 0 for v in (x.data_ptr(), out.data_ptr(), x.shape[1] * x.element_size(),
                                     out.shape[1] * out.element_size()))


class GroupedGemmPlan:
    """Owned metadata of one ragged grouped GEMM launch (reference mxfp4_kernels.py:318-382).

    ``pairs``: iterable of (contiguous bf16 x[M, K], physical slot, contiguous bf16 out[M, N]).  Inputs may repeat;
    outputs must be disjoint and may not overlap any input.  Fields: ``pairs`` (the tuple, which keeps every pair
    tensor alive), ``metadata_host`` / ``metadata`` (the tile table [ntiles, 5] int64 of x address, out address,
    slot, M, pm: pinned host memory and its one asynchronous upload for a CUDA plan, the same CPU tensor otherwise),
    ``block_m``, ``K``, ``N``, ``device``, ``slots``, ``ntiles`` and ``aligned`` (every non-empty pair's addresses and
    row pitches are multiples of 16 bytes).  A CPU plan can be built for validation; launching needs a GPU."""
    __slots__ = ("pairs", "metadata_host", "metadata", "block_m", "K", "N",
                 "device", "slots", "ntiles", "aligned")

    def __init__(self, pairs, *, block_m=64):
        self.pairs = tuple(pairs)
        self.block_m = _tile_height(block_m)
        self.slots = tuple(operator.index(slot) for _, slot, _ in self.pairs)
        for x, _, out in self.pairs:
            self._check_pair(x, out)
        first = self.pairs[0] if self.pairs else None
        self.device = first[0].device if first else None
        self.K = first[0].shape[1] if first else None
        self.N = first[2].shape[1] if first else None
        for x, _, out in self.pairs:
            if (x.device != self.device or x.shape[1] != self.K or out.shape[1] != self.N
                    or self.K < 32 or self.K % 32 or self.N < 1):
                raise ValueError("grouped pairs need one device, common K (multiple of 32), and common N")
        live = [(x, out) for x, _, out in self.pairs if x.shape[0]]
        self.aligned = all(_aligned16(x, out) for x, out in live)
        _check_disjoint_outputs([x for x, _ in live], [out for _, out in live])
        descs = _descriptor_table((x.data_ptr(), out.data_ptr(), slot, x.shape[0]) for x, slot, out in self.pairs)
        table = torch.from_numpy(_tile_table(descs, self.block_m))
        self.ntiles = table.shape[0]
        cuda = self.device is not None and self.device.type == "cuda"
        self.metadata_host = table.pin_memory() if cuda else table
        self.metadata = self.metadata_host.to(self.device, non_blocking=True) if cuda else self.metadata_host

    @staticmethod
    def _check_pair(x, out):
        if x.ndim != 2 or out.ndim != 2 or x.shape[0] != out.shape[0]:
            raise ValueError("each grouped pair needs x[M,K] and out[M,N]")
        if x.dtype is not torch.bfloat16 or out.dtype is not torch.bfloat16:
            raise ValueError("grouped GEMM inputs and outputs must be bf16")
        if not (x.is_contiguous() and out.is_contiguous()):
            raise ValueError("grouped GEMM pair matrices must be contiguous")
        if x.device != out.device:
            raise ValueError("a grouped pair's input/output must share a device")


# ------------------------------------------------------------------------------------------ prefill products
def _gemm_views(x, blocks, scales, packed):
    if blocks.ndim != 4 or blocks.shape[-1] != 16 or blocks.dtype is not torch.uint8:
        raise ValueError("blocks must be a uint8 [cap, N, GK, 16] view")
    cap, n, gk, _ = blocks.shape
    if tuple(blocks.stride()[1:]) != (gk * 16, 16, 1):
        raise ValueError("blocks rows must be contiguous")
    if scales.dtype is not torch.uint8 or scales.ndim != 3 or tuple(scales.shape[:2]) != (cap, n):
        raise ValueError("scales must be a uint8 [cap, N, w] view matching blocks")
    if gk != GK_SUPPORTED:
        raise ValueError(f"GK={gk}: these kernels are built for K = {GK_SUPPORTED * 32} (GPT-OSS-120B)")
    if n % 192:
        raise ValueError(f"N={n}: the GEMM tiles 192 weight rows per workgroup")
    for t, nm in ((blocks, "blocks"), (scales, "scales")):
        if t.device != x.device or t.device.type != "cuda":
            raise ValueError(f"{nm} must be on the input's CUDA device")
    return cap, n, gk, _scale_layout(scales, gk, packed)


def _native_gemm(x, blocks, scales, slots, out, E, M, n, pk):
    N.call("na_mxfp4_gemm", x.data_ptr(), M, x.shape[1], blocks.data_ptr(), blocks.stride(0), scales.data_ptr(),
           scales.stride(0), int(pk), slots.data_ptr(), E, out.data_ptr(), n, N.stream(x.device))


def _gemm_args(x, blocks, scales, slots, packed):
    if x.dtype is not torch.bfloat16 or x.ndim != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous bf16 [M, K] tensor")
    cap, n, gk, pk = _gemm_views(x, blocks, scales, packed)
    M, K = x.shape
    if K != gk * 32:
        raise AssertionError(f"x has K={K}, the pool {gk * 32}")
    if slots.dtype is not torch.int64 or not slots.is_contiguous() or slots.device != x.device:
        raise ValueError("slots must be a contiguous int64 tensor on the input's device")
    return slots.numel(), M, n, pk


def mxfp4_gemm(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, slots: torch.Tensor, *,
               block_n: int = 128, block_m: int = 16, packed: bool | None = None) -> torch.Tensor:
    """x [M, K] bf16; blocks/scales = slot-pool u8 views; slots int64 [E].  Returns [E, M, N] bf16 with
    out[e, m, n] = bf16(sum_k x[m, k] w_slot[e][n, k]) (reference mxfp4_kernels.py:202-216; any E and M here).
    block_n / block_m are accepted for interface compatibility: the kernel tiles 64 tokens x 192 rows."""
    E, M, n, pk = _gemm_args(x, blocks, scales, slots, packed)
    out = torch.empty(E, M, n, dtype=torch.bfloat16, device=x.device)
    if E and M:
        _native_gemm(x, blocks, scales, slots, out, E, M, n, pk)
    return out


def mxfp4_gemm_into(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, slots: torch.Tensor,
                    out: torch.Tensor, *, block_n: int = 128, block_m: int = 16,
                    packed: bool | None = None) -> torch.Tensor:
    """mxfp4_gemm writing into a caller-provided contiguous bf16 ``out`` of E*M*N elements (reference
    mxfp4_kernels.py:218-231): same kernel and arithmetic; the caller owns the stream ordering of ``out``."""
    E, M, n, pk = _gemm_args(x, blocks, scales, slots, packed)
    if out.dtype is not torch.bfloat16 or out.numel() != E * M * n or not out.is_contiguous():
        raise AssertionError("out must be contiguous bf16 with E*M*N elements")
    if out.device != x.device:
        raise ValueError("out must be on the input's device")
    if E and M:
        _native_gemm(x, blocks, scales, slots, out, E, M, n, pk)
    return out


def _grouped_pool(plan, blocks, scales, packed):
    """Check the pool views against a plan; returns the PS4 flag.  The messages are the reference's
    (mxfp4_kernels.py:398-413), with this build's own limits (K = 2880, N a multiple of 192, aligned pairs)."""
    if blocks.ndim != 4 or blocks.shape[-1] != 16:
        raise ValueError("grouped blocks must have shape [capacity,N,GK,16]")
    cap, n, gk, _ = blocks.shape
    if (plan.K, plan.N) != (gk * 32, n) or max(plan.slots) >= cap:
        raise ValueError("grouped plan dimensions or slots do not match the pool")
    if blocks.device.type != "cuda" or {plan.device, scales.device} != {blocks.device}:
        raise ValueError("grouped launch needs plan, blocks and scales on the same CUDA device")
    if {blocks.dtype, scales.dtype} != {torch.uint8}:
        raise ValueError("grouped blocks and scales must be uint8")
    if blocks.stride()[1:] != (gk * 16, 16, 1) or tuple(scales.shape[:2]) != (cap, n):
        raise ValueError("grouped pool matrix rows must be contiguous and scales must match")
    if gk != GK_SUPPORTED or n % 192:
        raise ValueError(f"these kernels serve K = {GK_SUPPORTED * 32} and N a multiple of 192")
    if not plan.aligned:
        raise ValueError("pair rows must be 16-byte aligned (x and out addresses and row pitches)")
    return _scale_layout(scales, gk, packed)


def mxfp4_gemm_grouped_into(pairs_or_plan, blocks: torch.Tensor, scales: torch.Tensor, *, block_n=128, block_m=64,
                            packed=None):
    """One ragged GEMM launch writing each pair's own output slice (reference mxfp4_kernels.py:385-419).  Returns the
    GroupedGemmPlan (built here from pairs, or the one passed in, whose block_m must match) so a caller can reuse
    it.  Each output row gets exactly mxfp4_gemm's arithmetic.  block_n is validated as the reference does and
    otherwise unused (the kernel tiles 192 weight rows)."""
    if isinstance(pairs_or_plan, GroupedGemmPlan):
        plan = pairs_or_plan
        if plan.block_m != block_m:
            raise ValueError("plan block_m differs from the requested launch")
    else:
        plan = GroupedGemmPlan(pairs_or_plan, block_m=block_m)
    if plan.ntiles == 0:
        return plan
    bn = operator.index(block_n)
    if bn < 16 or bn & (bn - 1):
        raise ValueError("block_n must be a power of two >= 16")
    pk = _grouped_pool(plan, blocks, scales, packed)
    N.call("na_mxfp4_gemm_grouped", blocks.data_ptr(), blocks.stride(0), scales.data_ptr(), scales.stride(0), int(pk),
           plan.metadata.data_ptr(), plan.ntiles, plan.block_m, blocks.shape[1], blocks.shape[2] * 32,
           N.stream(blocks.device))
    return plan
