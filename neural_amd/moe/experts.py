"""All-resident GPT-OSS-120B experts on one MI355X: the ``experts.forward(hidden_states, router_indices,
routing_weights)`` seam the reference installs per layer (reference neural/moe/gptoss_adapter.py:267-284), backed by
one HBM slot pool [n_layers * n_experts, slot_bytes] that holds every expert (60.9 GB raw; nothing is offloaded).

Decode (T <= 8 tokens) runs the fused expert body of the reference's b_body (server.py:508-518) as HIP launches
(gate_up + bias + clamped SwiGLU; down + bias + routing weight; top-k combine, which the down kernel does itself for
T = 1 on the tile layout); routing is read on the device, so ``forward_decode`` never synchronises and can be
captured in a hipGraph.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .layout import GPTOSS_LAYOUT, TILE_REPR, ExpertLayout

MAX_DECODE_TOKENS = 8


class ResidentExperts:
    def __init__(self, pool: torch.Tensor, layout: ExpertLayout = GPTOSS_LAYOUT, bias_gu: torch.Tensor | None = None,
                 bias_dn: torch.Tensor | None = None, slot_tab: torch.Tensor | None = None,
                 max_batch: int = MAX_DECODE_TOKENS, gu_pairs_per_wave: int = 4, dn_pairs_per_wave: int = 2,
                 k_split: int = 0, combine_in_down: bool = True, one_launch: bool = True):
        """pool: uint8 [n, layout.slot_bytes] in the raw, PS4 or t950 (gfx950 tile) layout.  The t950 layout runs the
        block-scaled MFMA decode kernels (k_split waves per workgroup split K; 0 = automatic, 4); with
        combine_in_down, a single token takes two launches (the down kernel holds every expert of an output block
        and sums the top-k itself) instead of three, and with one_launch as well (and the automatic k_split) a single
        launch (na_moe_decode_t950_one: the same bits).  The store layouts run the VALU kernels (gu/dn_pairs_per_wave
        row pairs per wavefront)."""
        if layout.weight_repr not in ("mxfp4_g32", "mxfp4_g32_ps4", TILE_REPR):
            raise ValueError(f"ResidentExperts serves the raw, PS4 and t950 slot layouts, not {layout.weight_repr}")
        if k_split not in (0, 4, 8):
            raise ValueError("k_split must be 0 (automatic), 4 or 8")
        self.k_split = int(k_split)
        self.tiled = layout.weight_repr == TILE_REPR
        if pool.dtype is not torch.uint8 or pool.ndim != 2 or pool.shape[1] != layout.slot_bytes:
            raise ValueError(f"pool must be uint8 [n, {layout.slot_bytes}]")
        if not pool.is_contiguous() or pool.device.type != "cuda":
            raise ValueError("pool must be a contiguous CUDA tensor")
        n = layout.n_layers * layout.n_experts
        if slot_tab is None and pool.shape[0] < n:
            raise ValueError(f"pool holds {pool.shape[0]} slots; without a slot table it must hold all {n}")
        for b, w, nm in ((bias_gu, layout.gate_up_n, "bias_gu"), (bias_dn, layout.down_n, "bias_dn")):
            if b is not None and (b.dtype is not torch.bfloat16 or tuple(b.shape) != (n, w) or not b.is_contiguous()
                                  or b.device != pool.device):
                raise ValueError(f"{nm} must be contiguous bf16 [{n}, {w}] on the pool's device")
        if slot_tab is not None and (slot_tab.dtype is not torch.int64 or slot_tab.numel() != n
                                     or slot_tab.device != pool.device):
            raise ValueError(f"slot_tab must be int64 [{n}] on the pool's device")
        if not 1 <= max_batch <= MAX_DECODE_TOKENS:
            raise ValueError(f"max_batch must be in [1, {MAX_DECODE_TOKENS}]")
        self.pool, self.layout = pool, layout
        self.bias_gu, self.bias_dn, self.slot_tab = bias_gu, bias_dn, slot_tab
        self.max_batch = max_batch
        if gu_pairs_per_wave not in (1, 2, 4) or dn_pairs_per_wave not in (1, 2, 4):
            raise ValueError("row pairs per wave must be 1, 2 or 4")
        self.gu_pairs, self.dn_pairs = int(gu_pairs_per_wave), int(dn_pairs_per_wave)
        dev = pool.device
        self.down_mode = 0 if combine_in_down else 1
        self.h = torch.empty(max_batch * layout.top_k, layout.down_k, dtype=torch.bfloat16, device=dev)
        self.yw = torch.empty(max_batch * layout.top_k, layout.down_n, dtype=torch.bfloat16, device=dev)
        # the single-launch path's handoff words (zero before its first call; every call leaves them reusable)
        self.one = (self.tiled and combine_in_down and one_launch and self.k_split in (0, 4)
                    and bool(N.lib().na_moe_one_resident()))
        self.sync = (torch.zeros(N.lib().na_moe_one_sync_words(), dtype=torch.int32, device=dev) if self.one
                     else None)

    def sync_error(self) -> bool:
        """Whether a wait of the single-launch path ever gave up, so that some output since the last
        clear_sync_error() may be wrong (reads one device word: synchronises).  The waits can give up only if the
        launch's 720 workgroups are not all resident at once, e.g. under another process's kernels on the same
        GPU; callers that replay captured graphs poll this after their replays."""
        return bool(self.sync is not None and int(self.sync[0].item()) != 0)

    def clear_sync_error(self) -> None:
        """Zero the error word (the kernels only ever set it); stream-ordered, capturable."""
        if self.sync is not None:
            self.sync[:1].zero_()

    def forward_decode(self, layer: int, hidden: torch.Tensor, router_indices: torch.Tensor,
                       routing_weights: torch.Tensor, out: torch.Tensor | None = None, events=None) -> torch.Tensor:
        """hidden [B, 2880] bf16, router_indices [B, 4] int64 (expert ids within the layer), routing_weights [B, 4]
        bf16 -> [B, 2880] bf16 = bf16(sum_k bf16(bf16(expert_k(h) + b_dn) * w_k)) in top-k order.
        events: None, or recorded timing torch.cuda.Event objects timestamped by the dispatches themselves
        (measurement only; not for graph capture): start/stop of each launch, see launches().
        Calls that overlap on one device must use different ResidentExperts objects (they share scratch)."""
        L = self.layout
        B = hidden.shape[0]
        if hidden.dtype is not torch.bfloat16 or hidden.ndim != 2 or hidden.shape[1] != L.hidden \
                or not hidden.is_contiguous():
            raise ValueError("hidden must be contiguous bf16 [B, hidden]")
        if not 1 <= B <= self.max_batch:
            raise ValueError(f"decode batch {B} outside [1, {self.max_batch}]")
        if router_indices.dtype is not torch.int64 or tuple(router_indices.shape) != (B, L.top_k) \
                or not router_indices.is_contiguous():
            raise ValueError("router_indices must be contiguous int64 [B, top_k]")
        if routing_weights.dtype is not torch.bfloat16 or tuple(routing_weights.shape) != (B, L.top_k) \
                or not routing_weights.is_contiguous():
            raise ValueError("routing_weights must be contiguous bf16 [B, top_k]")
        if not 0 <= layer < L.n_layers:
            raise ValueError(f"layer {layer} outside [0, {L.n_layers})")
        if out is None:
            out = torch.empty(B, L.hidden, dtype=torch.bfloat16, device=hidden.device)
        elif out.dtype is not torch.bfloat16 or tuple(out.shape) != (B, L.hidden) or not out.is_contiguous():
            raise ValueError("out must be contiguous bf16 [B, hidden]")
        if self.one and B == 1:
            rc = N.call_status("na_moe_decode_t950_one", hidden.data_ptr(), router_indices.data_ptr(),
                               routing_weights.data_ptr(), self.pool.data_ptr(), L.slot_bytes, N.ptr(self.slot_tab),
                               layer * L.n_experts, N.ptr(self.bias_gu), N.ptr(self.bias_dn), self.h.data_ptr(),
                               self.yw.data_ptr(), out.data_ptr(), float(L.act_alpha), float(L.act_limit),
                               self.sync.data_ptr(), N.events_array(events), N.stream(hidden.device),
                               allow=(N.ERR_RESIDENT,))
            if rc == 0:
                return out
            # the device cannot hold all 720 workgroups at once (a smaller partition): nothing was launched; from
            # now on this object takes the two-launch form, which gives the same bits
            self.one = False
        if self.tiled:
            N.call("na_moe_decode_t950", hidden.data_ptr(), router_indices.data_ptr(), routing_weights.data_ptr(), B,
                   self.pool.data_ptr(), L.slot_bytes, N.ptr(self.slot_tab), layer * L.n_experts,
                   N.ptr(self.bias_gu), N.ptr(self.bias_dn), self.h.data_ptr(), self.yw.data_ptr(), out.data_ptr(),
                   float(L.act_alpha), float(L.act_limit), self.k_split, self.down_mode, N.events_array(events),
                   N.stream(hidden.device))
            return out
        N.call("na_moe_decode", hidden.data_ptr(), router_indices.data_ptr(), routing_weights.data_ptr(), B,
               self.pool.data_ptr(), L.slot_bytes, L.scale_layout_mode, N.ptr(self.slot_tab), layer * L.n_experts,
               N.ptr(self.bias_gu), N.ptr(self.bias_dn), self.h.data_ptr(), self.yw.data_ptr(), out.data_ptr(),
               float(L.act_alpha), float(L.act_limit), self.gu_pairs, self.dn_pairs, N.events_array(events),
               N.stream(hidden.device))
        return out


    def forward_decode_logits(self, layer: int, hidden: torch.Tensor, logits: torch.Tensor, out: torch.Tensor,
                              ids_out: torch.Tensor | None = None, wts_out: torch.Tensor | None = None,
                              events=None) -> torch.Tensor:
        """One token's expert body routed by the layer's 128 router logits (fp32, bf16 values): the top 4 and their
        softmax weights by the router's own rule (na_moe_decode_t950_one_logits selects them in the same launch),
        written to ids_out [1, 4] int64 / wts_out [1, 4] bf16 when given.  The same bits as forward_decode with the
        router's ids and weights.  Without the single-launch body (other layouts, or a device that cannot hold its
        720 workgroups) the selection runs as its own launch first."""
        L = self.layout
        if hidden.dtype is not torch.bfloat16 or tuple(hidden.shape) != (1, L.hidden) or not hidden.is_contiguous():
            raise ValueError("hidden must be contiguous bf16 [1, hidden]")
        if logits.dtype is not torch.float32 or logits.numel() != L.n_experts or not logits.is_contiguous():
            raise ValueError(f"logits must be contiguous fp32 [{L.n_experts}]")
        if out.dtype is not torch.bfloat16 or tuple(out.shape) != (1, L.hidden) or not out.is_contiguous():
            raise ValueError("out must be contiguous bf16 [1, hidden]")
        if (ids_out is None) != (wts_out is None):
            raise ValueError("ids_out and wts_out go together")
        for t, dt, nm in ((ids_out, torch.int64, "ids_out"), (wts_out, torch.bfloat16, "wts_out")):
            if t is not None and (t.dtype is not dt or t.numel() != L.top_k or not t.is_contiguous()):
                raise ValueError(f"{nm} must be contiguous {dt} [1, {L.top_k}]")
        if not 0 <= layer < L.n_layers:
            raise ValueError(f"layer {layer} outside [0, {L.n_layers})")
        if self.one:
            rc = N.call_status("na_moe_decode_t950_one_logits", hidden.data_ptr(), logits.data_ptr(),
                               N.ptr(ids_out), N.ptr(wts_out), self.pool.data_ptr(), L.slot_bytes,
                               N.ptr(self.slot_tab), layer * L.n_experts, N.ptr(self.bias_gu), N.ptr(self.bias_dn),
                               out.data_ptr(), float(L.act_alpha), float(L.act_limit), self.sync.data_ptr(),
                               N.events_array(events), N.stream(hidden.device), allow=(N.ERR_RESIDENT,))
            if rc == 0:
                return out
            self.one = False
        ids = ids_out if ids_out is not None else torch.empty(1, L.top_k, dtype=torch.int64, device=hidden.device)
        wts = wts_out if wts_out is not None else torch.empty(1, L.top_k, dtype=torch.bfloat16, device=hidden.device)
        lb = logits.to(torch.bfloat16)                   # exact: the router's logits are bf16 values
        N.call("na_rows_topk", lb.data_ptr(), 1, ids.data_ptr(), wts.data_ptr(), N.stream(hidden.device))
        return self.forward_decode(layer, hidden, ids.view(1, L.top_k), wts.view(1, L.top_k), out=out, events=events)

    def forward_prefill(self, layer: int, hidden: torch.Tensor, router_indices: torch.Tensor,
                        routing_weights: torch.Tensor, out: torch.Tensor | None = None, events=None) -> torch.Tensor:
        """Prompt tokens of one layer (the reference's moe_prefill, server.py:1837-1936, for an all-resident pool):
        hidden [T, 2880] bf16, router_indices [T, 4] int64, routing_weights [T, 4] bf16 -> [T, 2880] bf16 =
        per token bf16(sum_k bf16(bf16(expert_k(h) + b_dn) * w_k)) in top-k order, each expert product the
        reference's GEMM arithmetic.  Five launches on the current stream, no host synchronisation: pair counts per
        expert, a stable expert-major order of the pairs with its 64-token tiles, gate_up + bias + clamped SwiGLU
        (activation rows gathered through the order), down + bias + routing weight (scattered back to pair order),
        and the top-k sum.  The workspace (~ T x 53 KB) is allocated through torch's caching allocator.
        events: None or ten recorded timing events (start/stop of each launch; measurement only)."""
        L = self.layout
        T = hidden.shape[0]
        if hidden.dtype is not torch.bfloat16 or hidden.ndim != 2 or hidden.shape[1] != L.hidden \
                or not hidden.is_contiguous():
            raise ValueError("hidden must be contiguous bf16 [T, hidden]")
        if T < 1:
            raise ValueError("prefill needs at least one token")
        if router_indices.dtype is not torch.int64 or tuple(router_indices.shape) != (T, L.top_k) \
                or not router_indices.is_contiguous():
            raise ValueError("router_indices must be contiguous int64 [T, top_k]")
        if routing_weights.dtype is not torch.bfloat16 or tuple(routing_weights.shape) != (T, L.top_k) \
                or not routing_weights.is_contiguous():
            raise ValueError("routing_weights must be contiguous bf16 [T, top_k]")
        if not 0 <= layer < L.n_layers:
            raise ValueError(f"layer {layer} outside [0, {L.n_layers})")
        if out is None:
            out = torch.empty(T, L.hidden, dtype=torch.bfloat16, device=hidden.device)
        elif out.dtype is not torch.bfloat16 or tuple(out.shape) != (T, L.hidden) or not out.is_contiguous():
            raise ValueError("out must be contiguous bf16 [T, hidden]")
        nbytes = N.lib().na_moe_prefill_workspace_bytes(T)
        if nbytes < 0:
            raise ValueError(f"prefill of {T} tokens is beyond the kernel's limits")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=hidden.device)
        layout_code = 2 if self.tiled else L.scale_layout_mode
        N.call("na_moe_prefill", hidden.data_ptr(), router_indices.data_ptr(), routing_weights.data_ptr(), T,
               self.pool.data_ptr(), L.slot_bytes, layout_code, N.ptr(self.slot_tab), layer * L.n_experts,
               N.ptr(self.bias_gu), N.ptr(self.bias_dn), ws.data_ptr(), nbytes, out.data_ptr(), float(L.act_alpha),
               float(L.act_limit), N.events_array(events), N.stream(hidden.device))
        return out

    def launches(self, batch: int, with_out: bool = True) -> tuple:
        """Names of the kernels one forward_decode call launches, in order (two timing events per launch)."""
        if self.one and with_out and batch == 1:
            return ("experts",)
        if self.tiled and self.down_mode == 0 and with_out and batch == 1:
            return ("gate_up", "down_combine")
        return ("gate_up", "down", "combine") if with_out else ("gate_up", "down")


class Router:
    """Router GEMV + top-4 + softmax of one layer (reference fused_core.py:417-502 k_router / k_topk, without the
    offload bookkeeping): logits = bf16(xn . Wr^T + br); ids int64 [B, 4]; weights bf16 [B, 4]."""

    def __init__(self, device, max_batch: int = MAX_DECODE_TOKENS, n_experts: int = 128):
        self.n_experts = n_experts
        self.logits = torch.zeros(max_batch, n_experts, dtype=torch.float32, device=device)
        self.counter = torch.zeros(1, dtype=torch.int32, device=device)
        self.max_batch = max_batch

    def __call__(self, xn: torch.Tensor, w_router: torch.Tensor, b_router: torch.Tensor | None,
                 ids_out: torch.Tensor, w_out: torch.Tensor) -> None:
        B = xn.shape[0]
        if not 1 <= B <= self.max_batch or xn.dtype is not torch.bfloat16 or not xn.is_contiguous() \
                or xn.shape[1] != 2880:
            raise ValueError("xn must be contiguous bf16 [B <= max_batch, 2880]")
        if w_router.dtype is not torch.bfloat16 or tuple(w_router.shape) != (self.n_experts, 2880) \
                or not w_router.is_contiguous():
            raise ValueError("w_router must be contiguous bf16 [n_experts, 2880]")
        if b_router is not None and (b_router.dtype is not torch.bfloat16 or b_router.numel() != self.n_experts):
            raise ValueError("b_router must be bf16 [n_experts]")
        if ids_out.dtype is not torch.int64 or ids_out.numel() != 4 * B or w_out.dtype is not torch.bfloat16 \
                or w_out.numel() != 4 * B:
            raise ValueError("ids_out int64 [B, 4] and w_out bf16 [B, 4] required")
        N.call("na_router_topk", xn.data_ptr(), B, w_router.data_ptr(), N.ptr(b_router), self.n_experts,
               self.logits.data_ptr(), self.counter.data_ptr(), ids_out.data_ptr(), w_out.data_ptr(),
               N.stream(xn.device))
