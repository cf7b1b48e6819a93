"""The reference's prepacked expert store, read (and, for tests and converters, written) on the MI355X host.

Format (reference neural/q80/prepacked_store.py:1-146, kept byte-compatible so an existing store opens unchanged):
    <root>/metadata.json       {"magic": "Q80-PREPACKED-SLOTS", "version": 1, "model_id", "layout": descriptor,
                                "sha256_per_layer": {"<li>": hex}, "built_unix", "build_seconds", ...}
    <root>/layer_<li>.slots    [n_experts, slot_bytes] uint8: each row one expert's slot bytes (raw or PS4 scales)
    <root>/expert_biases.pt    torch.save({"bias_gu": bf16 [n_layers * n_experts, 5760], "bias_dn": bf16 [.., 2880]})
The descriptor (neural_amd.moe.layout.prepacked_descriptor) is the store's identity: open() compares its structural
fields, kernel and weight_repr strictly (a raw store is never opened with the PS4 layout or the other way round); the
human-readable ``row`` label is informational.  Incompatible stores are rejected, never coerced.

Layer files are memory-mapped (numpy memmaps, copy-on-write private pages by default); rows are handed out as views,
so a retrieval is one contiguous copy.  No GPU work happens here: neural_amd.moe.gptoss_adapter.load_resident_store
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


def _fail(reason: str, **extra) -> dict[str, Any]:
    return {"status": "fail", "reason": reason, **extra}


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
    def _read_metadata(self):
        """(metadata dict, None) or (None, failure status)."""
        path = self.root / "metadata.json"
        if not path.is_file():
            return None, _fail("no metadata.json")
        try:
            meta = json.loads(path.read_text(encoding="utf-8"))
        except ValueError:
            return None, _fail("metadata.json is not JSON")
        if meta.get("magic") != FORMAT_MAGIC:
            return None, _fail("bad magic")
        if meta.get("version") != FORMAT_VERSION:
            return None, _fail(f"version {meta.get('version')} != {FORMAT_VERSION}")
        return meta, None

    def _compare_descriptor(self, recorded):
        """(note or None, None) when every field but the informational ``row`` label equals this runtime's layout
        descriptor, else (None, failure status naming the differing fields, and both representations when the
        weight_repr differs)."""
        current = prepacked_descriptor(self.layout)
        if not isinstance(recorded, dict):
            return None, _fail("layout descriptor mismatch (no descriptor)")
        structural = (set(current) | set(recorded)) - {"row"}
        differs = sorted(k for k in structural if current.get(k) != recorded.get(k))
        if differs:
            status = _fail("layout descriptor mismatch (kernel/layout change)", differs=differs)
            if "weight_repr" in differs:
                status.update(store_weight_repr=recorded.get("weight_repr"),
                              runtime_weight_repr=current.get("weight_repr"))
            return None, status
        if current.get("row") == recorded.get("row"):
            return None, None
        return (f"row label differs (store {recorded.get('row')!r} vs current {current.get('row')!r}); structural "
                "fields, kernel and weight_repr all match"), None

    def _map_layer(self, li: int, shared: bool):
        """Layer li's file as a uint8 tensor view [n_experts, slot_bytes] over a memory map, or None when the file
        is missing or not exactly n_experts * slot_bytes long."""
        import numpy as np
        import torch

        L = self.layout
        path = self.root / f"layer_{li}.slots"
        if not path.is_file() or path.stat().st_size != L.n_experts * L.slot_bytes:
            return None
        # "c": private copy-on-write pages (the file is never written); "r+": a shared writable mapping
        mm = np.memmap(path, dtype=np.uint8, mode="r+" if shared else "c", shape=(L.n_experts, L.slot_bytes))
        return torch.from_numpy(mm)

    def open(self, *, expect_model_id: str | None = None, shared: bool = False) -> dict[str, Any]:
        """Validate and map the store (reference prepacked_store.py:149-207).  Returns {"status": "ok", "layers",
        "size_gib"[, "descriptor_note"]} or {"status": "fail", "reason", ...}: missing metadata, bad magic or
        version, a descriptor that differs in any structural field, kernel or weight_repr ("differs" names the
        fields; "store_weight_repr" / "runtime_weight_repr" when the representation differs), a different model
        id, a layer file missing or of the wrong size.  shared=False maps copy-on-write (the file is never written).
        Nothing is mapped unless every check passes."""
        meta, failed = self._read_metadata()
        if failed:
            return failed
        note, failed = self._compare_descriptor(meta.get("layout"))
        if failed:
            return failed
        if expect_model_id is not None and meta.get("model_id") != expect_model_id:
            return _fail("model identity mismatch")
        maps = {}
        for li in range(self.layout.n_layers):
            view = self._map_layer(li, shared)
            if view is None:
                return _fail(f"layer {li} missing/size")
            maps[li] = view
        self._maps, self.meta = maps, meta
        L = self.layout
        status = {"status": "ok", "layers": L.n_layers,
                  "size_gib": round(L.n_layers * L.n_experts * L.slot_bytes / 2 ** 30, 2)}
        if note:
            status["descriptor_note"] = note
        return status

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
        """Re-read a layer file from disk and compare its SHA-256 with the one metadata.json records (a corruption
        check; False also when no hash is recorded for the layer)."""
        if self.meta is None:
            raise RuntimeError("store not opened")
        recorded = self.meta.get("sha256_per_layer", {}).get(str(layer))
        digest = hashlib.sha256()
        block = bytearray(16 << 20)
        view = memoryview(block)
        with open(self.root / f"layer_{layer}.slots", "rb", buffering=0) as f:
            while n := f.readinto(block):
                digest.update(view[:n])
        return digest.hexdigest() == recorded

    def biases(self):
        """(bias_gu, bias_dn) from expert_biases.pt, loaded with torch.load(weights_only=True) (nothing in the file
        is executed), or None when the store has no bias file."""
        import torch

        p = self.root / "expert_biases.pt"
        if not p.is_file():
            return None
        d = torch.load(p, weights_only=True, map_location="cpu")
        return d["bias_gu"], d["bias_dn"]
