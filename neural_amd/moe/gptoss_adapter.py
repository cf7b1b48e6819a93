"""GPT-OSS glue of the reference's neural/moe/gptoss_adapter.py, on MI355X: the store's layout, the exact MXFP4 dequant
and row de-interleave helpers, the per-layer ``experts.forward`` installer, and the loader that fills HBM with the
whole expert set from a prepacked store, repacking it into the gfx950 tile layout on the way.

Names and meanings follow the reference (gptoss_adapter.py:31-91, 267-284): GPTOSS_MODEL_ID, layout_for_store,
FP4_VALUES, mxfp4_dequant_nk, deinterleave_perm, install_gptoss_expert_runtime.  load_resident_store replaces the
reference's build_gptoss_neural (:287-320), whose host pool / LRU admission / PCIe streaming exist because a 24 GB
card cannot hold the 61 GB expert set; one MI355X holds it all, so the store is read once at start-up.
"""
from __future__ import annotations

import dataclasses
import time

from .layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_T950, ExpertLayout, gptoss_layout_for_repr

GPTOSS_MODEL_ID = "gpt-oss-120b-b5c939de"

# fp4 e2m1 value table: code c -> value (bit 3 the sign; code 8 is -0.0)
FP4_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def layout_for_store(pstore_root: str) -> ExpertLayout:
    """The ExpertLayout a gpt-oss prepacked store holds (GPTOSS_LAYOUT, raw scales, or GPTOSS_LAYOUT_PS4), read from its
    metadata.json (reference gptoss_adapter.py:34-52).  A missing, unknown or self-contradicting descriptor is a
    RuntimeError, never a guess."""
    from ..q80.prepacked_store import Q80PrepackedStore

    desc = Q80PrepackedStore.peek_layout(pstore_root)
    if desc is None:
        raise RuntimeError(f"{pstore_root}: no readable metadata.json (not a prepacked store, or an incomplete one)")
    try:
        lay = gptoss_layout_for_repr(desc.get("weight_repr"))
    except KeyError:
        raise RuntimeError(f"{pstore_root}: weight_repr {desc.get('weight_repr')!r} is not a gpt-oss store layout "
                           "(known: mxfp4_g32, mxfp4_g32_ps4)") from None
    if desc.get("slot_bytes") != lay.slot_bytes:
        raise RuntimeError(f"{pstore_root}: descriptor slot_bytes {desc.get('slot_bytes')} != {lay.slot_bytes} for "
                           f"weight_repr {lay.weight_repr}")
    return lay


def mxfp4_dequant_nk(blocks, scales, dtype=None):
    """[N, K/32, 16] u8 codes + [N, K/32] u8 E8M0 scales -> [N, K] float, exactly: byte j of a group holds element
    2j (low nibble) and 2j + 1 (high nibble); value = FP4_VALUES[code] * 2^(scale - 127) (reference
    gptoss_adapter.py:63-80).  fp32 by default.  Runs where the tensors are (a quality-gate helper, not a hot path)."""
    import torch

    dtype = dtype or torch.float32
    lut = torch.tensor(FP4_VALUES, dtype=dtype, device=blocks.device)
    n, g, b = blocks.shape
    codes = torch.stack(((blocks & 0x0F).long(), (blocks >> 4).long()), dim=-1).reshape(n, g, 2 * b)
    vals = lut[codes]
    exp = (scales.to(torch.int32) - 127).reshape(n, g, 1).expand(n, g, 2 * b)
    return torch.ldexp(vals, exp.to(dtype)).reshape(n, g * 2 * b)


def deinterleave_perm(n_rows: int):
    """The checkpoint's gate_up rows alternate gate / up; the permutation that orders them [gate | up]
    (reference gptoss_adapter.py:83-88): [0, 2, 4, ..., 1, 3, 5, ...]."""
    import torch

    return torch.cat([torch.arange(0, n_rows, 2), torch.arange(1, n_rows, 2)])


def install_gptoss_expert_runtime(runtime, model, n_layers: int | None = None) -> list:
    """Replace ``model.model.layers[li].mlp.experts.forward`` with the runtime's (reference gptoss_adapter.py:267-284):
    one token -> runtime.forward_decode, more -> runtime.forward_prefill, with the layer id bound.  Returns the
    (module, original forward) pairs, so a caller can restore them."""
    installed = []
    layers = model.model.layers
    n = len(layers) if n_layers is None else n_layers

    def make(layer_id: int):
        def forward(hidden_states, router_indices=None, routing_weights=None):
            if hidden_states.shape[0] == 1:
                return runtime.forward_decode(layer_id, hidden_states, router_indices, routing_weights)
            return runtime.forward_prefill(layer_id, hidden_states, router_indices, routing_weights)
        return forward

    for li in range(n):
        experts = layers[li].mlp.experts
        installed.append((experts, experts.forward))
        experts.forward = make(li)
    return installed


def load_resident_store(pstore_root: str, device, *, layout: ExpertLayout | None = None, tiles: bool = True,
                        expect_model_id: str | None = GPTOSS_MODEL_ID, verify: bool = False, chunk: int = 16,
                        **runtime_kw) -> dict:
    """Open a prepacked store strictly (Q80PrepackedStore.open) and fill HBM with every expert of every layer.

    layout: the store's ExpertLayout (default: layout_for_store, the full 36 x 128 model); tiles: repack into the
    gfx950 tile layout (t950) on the device while loading (raw and PS4 stores both give the same tiles), else keep
    the store's layout.  Rows stream layer by layer in chunks of ``chunk`` slots: memory-mapped file -> pinned host
    buffer -> HBM staging (a copy stream) -> repack kernel into the pool (the current stream), two buffers deep so
    the host copy of one chunk overlaps the transfer and repack of the previous one.  verify: re-hash every layer
    file against metadata.json first.  Biases from expert_biases.pt (torch.load weights_only=True).

    Returns {"runtime": ResidentExperts, "pool", "layout" (the pool's), "store_layout", "bias_gu", "bias_dn",
    "seconds", "gbps" (store bytes / load time)}."""
    import torch

    from .. import tiles as T
    from ..q80.prepacked_store import Q80PrepackedStore
    from .experts import ResidentExperts

    L = layout if layout is not None else layout_for_store(pstore_root)
    st = Q80PrepackedStore(pstore_root, L)
    res = st.open(expect_model_id=expect_model_id)
    if res["status"] != "ok":
        raise RuntimeError(f"{pstore_root}: {res}")
    if verify:
        bad = [li for li in range(L.n_layers) if not st.verify_layer(li)]
        if bad:
            raise RuntimeError(f"{pstore_root}: layers {bad} do not match their recorded SHA-256")
    dev = torch.device(device)
    dst_L = dataclasses.replace(GPTOSS_LAYOUT_T950, n_layers=L.n_layers, n_experts=L.n_experts) if tiles else L
    n = L.n_layers * L.n_experts
    pool = torch.empty(n, dst_L.slot_bytes, dtype=torch.uint8, device=dev)
    chunk = max(1, min(int(chunk), L.n_experts))
    pinned = [torch.empty(chunk, L.slot_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    stage = [torch.empty(chunk, L.slot_bytes, dtype=torch.uint8, device=dev) for _ in range(2)] if tiles else None
    copy_stream = torch.cuda.Stream(dev)
    compute = torch.cuda.current_stream(dev)
    copied = [torch.cuda.Event() for _ in range(2)]
    consumed = [torch.cuda.Event() for _ in range(2)]
    used = [False, False]
    ps4 = L.weight_repr == "mxfp4_g32_ps4"
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    i = 0
    for li in range(L.n_layers):
        rows = st.rows(li)
        for e0 in range(0, L.n_experts, chunk):
            cn = min(chunk, L.n_experts - e0)
            b = i & 1
            if used[b]:
                copied[b].synchronize()                  # the transfer out of pinned[b] has finished
            pinned[b][:cn].copy_(rows[e0:e0 + cn])
            s0 = li * L.n_experts + e0
            with torch.cuda.stream(copy_stream):
                if used[b]:
                    copy_stream.wait_event(consumed[b])  # the repack that read stage[b] has finished
                dst = stage[b][:cn] if tiles else pool[s0:s0 + cn]
                dst.copy_(pinned[b][:cn], non_blocking=True)
                copied[b].record(copy_stream)
            if tiles:
                compute.wait_event(copied[b])
                T.repack_to_t950(stage[b][:cn], pool[s0:s0 + cn], packed=ps4)
                consumed[b].record(compute)
            else:
                compute.wait_event(copied[b])
                consumed[b].record(compute)
            used[b] = True
            i += 1
    torch.cuda.synchronize(dev)
    secs = time.perf_counter() - t0
    bias = st.biases()
    bgu = bdn = None
    if bias is not None:
        bgu, bdn = (b_.to(torch.bfloat16).contiguous().to(dev) for b_ in bias)
    rx = ResidentExperts(pool, dst_L, bgu, bdn, **runtime_kw)
    return {"runtime": rx, "pool": pool, "layout": dst_L, "store_layout": L, "bias_gu": bgu, "bias_dn": bdn,
            "seconds": secs, "gbps": n * L.slot_bytes / secs / 1e9}


__all__ = ["GPTOSS_MODEL_ID", "FP4_VALUES", "layout_for_store", "mxfp4_dequant_nk", "deinterleave_perm",
           "install_gptoss_expert_runtime", "load_resident_store", "GPTOSS_LAYOUT"]
