"""Host codec of the PS4 scale rows (weight_repr "mxfp4_g32_ps4"), the packed form of an expert slot's E8M0 region.

Byte format (reference tools/scale_pack.py:6-12, read by kernels/gptoss_cpu_cap2.c:358-361 and the GPU kernels):
a slot keeps its 12,441,600 E2M1 code bytes unchanged and stores each of its 8,640 scale rows (5,760 gate_up rows,
then 2,880 down rows) of 90 E8M0 exponents in 46 bytes: the row's smallest exponent, then the 90 offsets from it as
4-bit fields, two per byte, the even group in the low nibble.  An exponent range above 15 within a row has no
encoding, so packing reports such rows (SpanError) instead of clipping them.

Public names follow the reference's codec (pack_scale_rows, unpack_scale_rows, pack_slot, unpack_slot, SpanError) so
its callers keep working; the geometry comes from neural_amd.moe.layout.
"""
from __future__ import annotations

import numpy as np

from .moe.layout import GPTOSS_LAYOUT as _RAW, GPTOSS_LAYOUT_PS4 as _PS4

HIDDEN = _RAW.down_n                                   # 2880
GATE_UP_ROWS = _RAW.gate_up_n                          # 5760
GROUPS = _RAW.gate_groups                              # 90 exponents per weight row
DOWN_CODES_AT = _RAW.gate_pack_bytes                   # 8,294,400: first byte of the down codes
SCALES_AT = _RAW.off_gate_scales                       # 12,441,600: the scale region (both layouts)
SCALE_ROWS = GATE_UP_ROWS + HIDDEN                     # 8,640
PS4_ROW_BYTES = 1 + GROUPS // 2                        # 46
RAW_SLOT_BYTES = _RAW.slot_bytes                       # 13,219,200
PS4_SLOT_BYTES = _PS4.slot_bytes                       # 12,839,040
if SCALES_AT + SCALE_ROWS * PS4_ROW_BYTES != PS4_SLOT_BYTES or SCALES_AT + SCALE_ROWS * GROUPS != RAW_SLOT_BYTES:
    raise ImportError("expert layout and PS4 geometry disagree")

_NIBBLE_WEIGHTS = np.array([1, 16], np.uint8)        # (even, odd) offset -> one byte


class SpanError(ValueError):
    """Raised by the packers for scale rows whose exponents differ by more than 15; ``rows`` holds their indices
    (within the rows given) and ``spans`` their max - min."""

    def __init__(self, rows, spans):
        self.rows = np.asarray(rows, np.int64)
        self.spans = np.asarray(spans, np.int64)
        shown = ", ".join(f"row {r}: range {s}" for r, s in zip(self.rows[:6].tolist(), self.spans[:6].tolist()))
        more = "" if self.rows.size <= 6 else f" (+{self.rows.size - 6} more)"
        super().__init__(f"PS4 stores 4-bit exponent offsets; {self.rows.size} scale row(s) exceed a range of 15: "
                         f"{shown}{more}")


def _as_matrix(a, width: int, what: str) -> np.ndarray:
    m = np.asarray(a)
    if m.dtype != np.uint8 or m.ndim != 2 or m.shape[1] != width:
        raise ValueError(f"{what}: expected a uint8 array of shape [rows, {width}], got {m.dtype} {m.shape}")
    return m


def pack_scale_rows(sc, want_span: bool = False):
    """E8M0 rows u8 [n, 90] -> PS4 rows u8 [n, 46].  want_span: also return each row's max - min (u8 [n])."""
    rows = _as_matrix(sc, GROUPS, "pack_scale_rows")
    lowest = rows.min(axis=1, initial=255)
    offsets = rows - lowest[:, None]                          # no wrap: every entry >= its row minimum
    widest = offsets.max(axis=1, initial=0)
    over = widest > 15
    if over.any():
        idx = np.nonzero(over)[0]
        raise SpanError(idx, widest[idx])
    pairs = offsets.reshape(rows.shape[0], GROUPS // 2, 2)
    body = (pairs * _NIBBLE_WEIGHTS).sum(axis=2, dtype=np.uint8)
    packed = np.concatenate([lowest[:, None], body], axis=1)
    return (packed, widest) if want_span else packed


def unpack_scale_rows(rows) -> np.ndarray:
    """PS4 rows u8 [n, 46] -> E8M0 rows u8 [n, 90]: the exact inverse of pack_scale_rows (u8 arithmetic wraps, as the
    kernels' byte reads do, for rows no packer produced)."""
    packed = _as_matrix(rows, PS4_ROW_BYTES, "unpack_scale_rows")
    body = packed[:, 1:]
    offsets = np.stack([body & 0x0F, body >> 4], axis=2).reshape(packed.shape[0], GROUPS)
    return (offsets + packed[:, :1]).astype(np.uint8)


def _split(slot, size: int, what: str):
    s = np.asarray(slot)
    if s.dtype != np.uint8 or s.shape != (size,):
        raise ValueError(f"{what}: expected uint8 [{size}], got {s.dtype} {s.shape}")
    return s[:SCALES_AT], s[SCALES_AT:]


def pack_slot(raw) -> np.ndarray:
    """Raw slot u8 [13,219,200] -> PS4 slot u8 [12,839,040] (codes copied, scale rows packed)."""
    codes, scales = _split(raw, RAW_SLOT_BYTES, "pack_slot")
    return np.concatenate([codes, pack_scale_rows(scales.reshape(SCALE_ROWS, GROUPS)).reshape(-1)])


def unpack_slot(packed) -> np.ndarray:
    """PS4 slot u8 [12,839,040] -> raw slot u8 [13,219,200] (exact inverse of pack_slot)."""
    codes, rows = _split(packed, PS4_SLOT_BYTES, "unpack_slot")
    return np.concatenate([codes, unpack_scale_rows(rows.reshape(SCALE_ROWS, PS4_ROW_BYTES)).reshape(-1)])
