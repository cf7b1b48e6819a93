"""PS4 scale codec of the GPT-OSS expert store (weight_repr "mxfp4_g32_ps4"), host side.

Same names and contract as the reference's tools/scale_pack.py:36-97 (``SpanError``, ``row_spans``,
``pack_scale_rows``, ``unpack_scale_rows``, ``pack_slot``, ``unpack_slot``):

    raw slot  (13,219,200 B) = 12,441,600 code bytes | 8,640 scale rows x 90 B (gate rows, then down rows)
    PS4 slot  (12,839,040 B) = the same code bytes   | 8,640 scale rows x 46 B
    PS4 row: byte 0 = base = min of the row's 90 scale bytes; byte 1 + k = d[2k] | d[2k+1] << 4 with d = s - base.

Lossless iff every row's span (max - min) <= 15; packing refuses wider rows (SpanError) and never clips.
"""
from __future__ import annotations

import numpy as np

H, GU, GK, RB = 2880, 5760, 90, 1440
OFF_DC = GU * RB
OFF_GS = OFF_DC + H * RB
OFF_DS = OFF_GS + GU * GK
SLOT_RAW = OFF_DS + H * GK
NROWS = GU + H
SR_P4 = 1 + GK // 2
SLOT_PACKED = OFF_GS + NROWS * SR_P4
assert SLOT_RAW == 13_219_200 and SLOT_PACKED == 12_839_040


class SpanError(ValueError):
    """Scale rows spanning more than 15 exponent steps cannot be stored as 4-bit deltas."""

    def __init__(self, rows, spans):
        self.rows, self.spans = np.asarray(rows), np.asarray(spans)
        super().__init__(f"{len(self.rows)} scale row(s) with span > 15 (rows {self.rows[:8].tolist()}..., "
                         f"spans {self.spans[:8].tolist()}...)")


def row_spans(raw) -> np.ndarray:
    """max - min of each scale row of a raw slot (or of a [..., 8640 * 90] scale region)."""
    sc = np.asarray(raw, np.uint8)[..., OFF_GS:].reshape(-1, NROWS, GK)
    return sc.max(axis=-1).astype(np.int16) - sc.min(axis=-1).astype(np.int16)


def pack_scale_rows(sc, want_span: bool = False):
    """raw u8 [n, 90] -> PS4 u8 [n, 46].  SpanError for any row with span > 15."""
    sc = np.asarray(sc, np.uint8)
    if sc.ndim != 2 or sc.shape[1] != GK:
        raise ValueError(f"scale rows must be [n, {GK}], got {sc.shape}")
    base = sc.min(axis=1)
    delta = sc - base[:, None]
    span = delta.max(axis=1) if sc.shape[0] else np.zeros(0, np.uint8)
    bad = np.flatnonzero(span > 15)
    if bad.size:
        raise SpanError(bad, span[bad].astype(np.int16))
    rows = np.empty((sc.shape[0], SR_P4), np.uint8)
    rows[:, 0] = base
    rows[:, 1:] = delta[:, 0::2] | (delta[:, 1::2] << 4)
    return (rows, span) if want_span else rows


def unpack_scale_rows(rows) -> np.ndarray:
    """PS4 u8 [n, 46] -> raw u8 [n, 90] (exact inverse of pack_scale_rows)."""
    rows = np.asarray(rows, np.uint8)
    if rows.ndim != 2 or rows.shape[1] != SR_P4:
        raise ValueError(f"packed rows must be [n, {SR_P4}], got {rows.shape}")
    base = rows[:, 0:1]
    sc = np.empty((rows.shape[0], GK), np.uint8)
    sc[:, 0::2] = base + (rows[:, 1:] & 15)
    sc[:, 1::2] = base + (rows[:, 1:] >> 4)
    return sc


def pack_slot(raw) -> np.ndarray:
    raw = np.asarray(raw, np.uint8)
    if raw.shape != (SLOT_RAW,):
        raise ValueError(f"raw slot must be [{SLOT_RAW}] bytes, got {raw.shape}")
    out = np.empty(SLOT_PACKED, np.uint8)
    out[:OFF_GS] = raw[:OFF_GS]
    out[OFF_GS:] = pack_scale_rows(raw[OFF_GS:].reshape(NROWS, GK)).ravel()
    return out


def unpack_slot(packed) -> np.ndarray:
    packed = np.asarray(packed, np.uint8)
    if packed.shape != (SLOT_PACKED,):
        raise ValueError(f"packed slot must be [{SLOT_PACKED}] bytes, got {packed.shape}")
    out = np.empty(SLOT_RAW, np.uint8)
    out[:OFF_GS] = packed[:OFF_GS]
    out[OFF_GS:] = unpack_scale_rows(packed[OFF_GS:].reshape(NROWS, SR_P4)).ravel()
    return out
