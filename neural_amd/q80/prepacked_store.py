"""The reference's prepacked expert store, read (and, for tests and converters, written) on the MI355X host.

Format (reference neural/q80/prepacked_store.py:1-146, kept byte-compatible so an existing store opens unchanged):
    <root>/metadata.json       {"magic": "Q80-PREPACKED-SLOTS", "version": 1, "model_id", "layout": descriptor,
                                "sha256_per_layer": {"<li>": hex}, "built_unix", "build_seconds", ...}
    <root>/layer_<li>.slots    [n_experts, slot_bytes] uint8: each row one expert's slot bytes (raw or PS4 scales)
    <root>/expert_biases.pt    torch.save({"bias_gu": bf16 [n_layers * n_experts, 5760], "bias_dn": bf16 [.., 2880]})
The descriptor (neural_amd.moe.layout.prepacked_descriptor) is the store's identity: open() compares its structural
fields, kernel and weight_repr strictly (a raw store is never opened with the PS4 layout or the other way round); the
human-readable ``row`` label is informational.  Incompatible stores are rejected, never coerced.

Layer files are memory-mapped read-only (copy-on-write private mappings); rows are handed out as views, so a
retrieval is one contiguous copy.  No GPU work happens here: neural_amd.moe.gptoss_adapter.load_resident_store
streams the rows into HBM and repacks them into the gfx950 tile layout.
"""
from __future__ import annotations

import hashlib
import json
import time
from pathlib import Path
from typing import Any

from ..moe.layout import ExpertLayout, prepacked_descriptor

FORMAT_MAGIC = "Q80-PREPACKED-SLOTS"
FORMAT_VERSION = 1


class Q80PrepackedStore:
    """One store directory, opened against the ExpertLayout the runtime will use (reference prepacked_store.py:70)."""

    def __init__(self, root: Path | str, layout: ExpertLayout | None = None) -> None:
        if layout is None:
            raise ValueError("a gpt-oss store needs its ExpertLayout (peek_layout() / layout_for_store() name it)")
        self.root = Path(root)
        self.layout = layout
        self.meta: dict[str, Any] | None = None
        self._maps: dict[int, Any] = {}

    @property
    def slot_bytes(self) -> int:
        return self.layout.slot_bytes

    @property
    def weight_repr(self) -> str:
        return self.layout.weight_repr

    @staticmethod
    def peek_layout(root: Path | str) -> dict[str, Any] | None:
        """The layout descriptor recorded in <root>/metadata.json, or None without readable metadata (pure JSON)."""
        try:
            meta = json.loads((Path(root) / "metadata.json").read_text(encoding="utf-8"))
        except (OSError, ValueError):
            return None
        lay = meta.get("layout")
        return lay if isinstance(lay, dict) else None

    # ---- construction --------------------------------------------------------------------------------------------
    @staticmethod
    def build(root: Path | str, builder, *, model_id: str, layout: ExpertLayout, layers=None, progress=None,
              biases=None) -> dict[str, Any]:
        """Write a store from builder(layer, expert) -> slot bytes (a uint8 numpy array or torch tensor of
        layout.slot_bytes), streaming row by row (one row in memory), then metadata.json last, so an unfinished
        store has no metadata and cannot be opened.  biases: optional (bias_gu, bias_dn) bf16 tensors written to
        expert_biases.pt."""
        import numpy as np

        root = Path(root)
        root.mkdir(parents=True, exist_ok=True)
        layers = range(layout.n_layers) if layers is None else layers
        hashes: dict[str, str] = {}
        t0 = time.time()
        for li in layers:
            h = hashlib.sha256()
            with open(root / f"layer_{li}.slots", "wb") as f:
                for e in range(layout.n_experts):
                    buf = builder(li, e)
                    b = (buf.cpu().numpy() if hasattr(buf, "cpu") else np.asarray(buf)).astype(np.uint8, copy=False)
                    if b.size != layout.slot_bytes:
                        raise ValueError(f"builder row ({li}, {e}) holds {b.size} bytes, not {layout.slot_bytes}")
                    raw = b.tobytes()
                    f.write(raw)
                    h.update(raw)
            hashes[str(li)] = h.hexdigest()
            if progress:
                progress(li)
        if biases is not None:
            import torch
            torch.save({"bias_gu": biases[0], "bias_dn": biases[1]}, root / "expert_biases.pt")
        meta = {"magic": FORMAT_MAGIC, "version": FORMAT_VERSION, "model_id": model_id,
                "layout": prepacked_descriptor(layout), "sha256_per_layer": hashes, "built_unix": int(time.time()),
                "build_seconds": round(time.time() - t0, 1)}
        (root / "metadata.json").write_text(json.dumps(meta, indent=1), encoding="utf-8")
        return meta

    # ---- access --------------------------------------------------------------------------------------------------
    def open(self, *, expect_model_id: str | None = None, shared: bool = False) -> dict[str, Any]:
        """Validate and map the store (reference prepacked_store.py:149-207).  Returns {"status": "ok", "layers",
        "size_gib"[, "descriptor_note"]} or {"status": "fail", "reason", ...}: missing metadata, bad magic or
        version, a descriptor that differs in any structural field, kernel or weight_repr ("differs" names the
        fields; "store_weight_repr" / "runtime_weight_repr" when the representation differs), a different model
        id, a layer file missing or of the wrong size.  shared=False maps copy-on-write (the file is never written)."""
        import torch

        mp = self.root / "metadata.json"
        if not mp.is_file():
            return {"status": "fail", "reason": "no metadata.json"}
        try:
            meta = json.loads(mp.read_text(encoding="utf-8"))
        except ValueError:
            return {"status": "fail", "reason": "metadata.json is not JSON"}
        if meta.get("magic") != FORMAT_MAGIC:
            return {"status": "fail", "reason": "bad magic"}
        if meta.get("version") != FORMAT_VERSION:
            return {"status": "fail", "reason": f"version {meta.get('version')} != {FORMAT_VERSION}"}
        want = prepacked_descriptor(self.layout)
        have = meta.get("layout")
        if not isinstance(have, dict):
            return {"status": "fail", "reason": "layout descriptor mismatch (no descriptor)"}
        w = {k: v for k, v in want.items() if k != "row"}
        h = {k: v for k, v in have.items() if k != "row"}
        if w != h:
            out = {"status": "fail", "reason": "layout descriptor mismatch (kernel/layout change)",
                   "differs": sorted(k for k in set(w) | set(h) if w.get(k) != h.get(k))}
            if w.get("weight_repr") != h.get("weight_repr"):
                out["store_weight_repr"] = h.get("weight_repr")
                out["runtime_weight_repr"] = w.get("weight_repr")
            return out
        note = None
        if want.get("row") != have.get("row"):
            note = (f"row label differs (store {have.get('row')!r} vs current {want.get('row')!r}); structural "
                    "fields, kernel and weight_repr all match")
        if expect_model_id is not None and meta.get("model_id") != expect_model_id:
            return {"status": "fail", "reason": "model identity mismatch"}
        L = self.layout
        expected = L.n_experts * L.slot_bytes
        maps = {}
        for li in range(L.n_layers):
            p = self.root / f"layer_{li}.slots"
            if not p.is_file() or p.stat().st_size != expected:
                return {"status": "fail", "reason": f"layer {li} missing/size"}
            storage = torch.UntypedStorage.from_file(str(p), shared=shared, nbytes=expected)
            t = torch.empty(0, dtype=torch.uint8)
            t.set_(storage)
            maps[li] = t.view(L.n_experts, L.slot_bytes)
        self._maps = maps
        self.meta = meta
        out = {"status": "ok", "layers": L.n_layers, "size_gib": round(L.n_layers * expected / 1024 ** 3, 2)}
        if note:
            out["descriptor_note"] = note
        return out

    def _layer(self, layer: int):
        if layer not in self._maps:
            raise RuntimeError("store not opened (or layer out of range)")
        return self._maps[layer]

    def read_into(self, layer: int, expert: int, out_buf) -> None:
        """One contiguous copy of a slot row into out_buf (a uint8 tensor of slot_bytes)."""
        out_buf.copy_(self._layer(layer)[expert])

    def row(self, layer: int, expert: int):
        """The mapped row of (layer, expert) as a uint8 view [slot_bytes]."""
        return self._layer(layer)[expert]

    def rows(self, layer: int):
        """All rows of a layer as a uint8 view [n_experts, slot_bytes]."""
        return self._layer(layer)

    def verify_layer(self, layer: int) -> bool:
        """Re-hash a layer file against metadata.json's SHA-256 (corruption check)."""
        if self.meta is None:
            raise RuntimeError("store not opened")
        h = hashlib.sha256()
        with open(self.root / f"layer_{layer}.slots", "rb") as f:
            while True:
                chunk = f.read(1 << 24)
                if not chunk:
                    break
                h.update(chunk)
        return h.hexdigest() == self.meta.get("sha256_per_layer", {}).get(str(layer))

    def biases(self):
        """(bias_gu, bias_dn) from expert_biases.pt, loaded with torch.load(weights_only=True) (nothing in the file
        is executed), or None when the store has no bias file."""
        import torch

        p = self.root / "expert_biases.pt"
        if not p.is_file():
            return None
        d = torch.load(p, weights_only=True, map_location="cpu")
        return d["bias_gu"], d["bias_dn"]
