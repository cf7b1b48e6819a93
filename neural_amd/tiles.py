"""gfx950 tile layout ("t950", weight_repr "mxfp4_g32_t950") of the GPT-OSS-120B expert store: host codec and device
repack launchers.

A t950 slot (13,271,040 B) holds the same logical data as a raw store slot (13,219,200 B): 540 row blocks of 16 rows
(gate_up blocks 0..359, down blocks 360..539), each 24,576 B =
    codes  90 groups x 256 B, group-major: byte 256 g + 16 n + b = code byte b of (row n, group g), i.e. k-tile t
           (groups 4t..4t+3, the last one groups 88, 89 only) is the 1024 B at 1024 t and the 16 B at 1024 t + 16 l
           are the code bytes of (row n, group 4t + kb) for lane l = 16 kb + n;
    scales 16 rows x 96 B: byte 96 n + g = E8M0 of (row n, group g) for g < 90, 0 for g = 90..95.
One 128-bit load per lane of a k-tile is exactly the FP4 B operand of one v_mfma_scale_f32_16x16x128_f8f6f4 for the
block's 16 rows (lane 16 kb + n: B[32 kb .. 32 kb + 31][n]), and a lane's scales are one aligned row.  The repack
is a byte permutation (plus PS4 expansion and zero padding), so raw -> t950 -> raw and PS4 -> t950 -> PS4 (canonical
PS4, base = row minimum) are exact.
"""
from __future__ import annotations

import numpy as np

from . import scale_pack as sp

ROWS = 16
FULL_TILES = 22
CODE_BYTES = FULL_TILES * 1024 + 512          # 23,040 per row block
SCALE_PITCH = 96
BLOCK_BYTES = CODE_BYTES + ROWS * SCALE_PITCH  # 24,576
GATE_BLOCKS = sp.GATE_UP_ROWS // ROWS                   # 360
DOWN_BLOCKS = sp.HIDDEN // ROWS                    # 180
SLOT_T950 = (GATE_BLOCKS + DOWN_BLOCKS) * BLOCK_BYTES
assert SLOT_T950 == 13_271_040


# ------------------------------------------------------------------------------------------- host codec (numpy)
def _codes_to_blocks(codes: np.ndarray) -> np.ndarray:
    """codes u8 [N, 90, 16] -> [N / 16, 23040] tile bytes (per row block: [group][row][16 bytes])."""
    nrb = codes.shape[0] // ROWS
    return np.ascontiguousarray(codes.reshape(nrb, ROWS, sp.GROUPS, 16).transpose(0, 2, 1, 3)).reshape(nrb, CODE_BYTES)


def _blocks_to_codes(blk: np.ndarray) -> np.ndarray:
    nrb = blk.shape[0]
    c = blk.reshape(nrb, sp.GROUPS, ROWS, 16).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(c).reshape(nrb * ROWS, sp.GROUPS, 16)


def _scales_to_blocks(sc: np.ndarray) -> np.ndarray:
    """raw scale rows u8 [N, 90] -> [N / 16, 1536]."""
    nrb = sc.shape[0] // ROWS
    out = np.zeros((nrb, ROWS, SCALE_PITCH), np.uint8)
    out[:, :, :sp.GROUPS] = sc.reshape(nrb, ROWS, sp.GROUPS)
    return out.reshape(nrb, ROWS * SCALE_PITCH)


def slot_to_t950(slot: np.ndarray, packed: bool = False) -> np.ndarray:
    """A raw (or PS4) store slot -> t950 slot bytes."""
    slot = np.asarray(slot, np.uint8)
    raw = sp.unpack_slot(slot) if packed else slot
    if raw.shape != (sp.RAW_SLOT_BYTES,):
        raise ValueError(f"slot must be {sp.RAW_SLOT_BYTES} (raw) or {sp.PS4_SLOT_BYTES} (PS4) bytes")
    gc = raw[:sp.DOWN_CODES_AT].reshape(sp.GATE_UP_ROWS, sp.GROUPS, 16)
    dc = raw[sp.DOWN_CODES_AT:sp.SCALES_AT].reshape(sp.HIDDEN, sp.GROUPS, 16)
    sc = raw[sp.SCALES_AT:].reshape(sp.SCALE_ROWS, sp.GROUPS)
    out = np.empty((GATE_BLOCKS + DOWN_BLOCKS, BLOCK_BYTES), np.uint8)
    out[:GATE_BLOCKS, :CODE_BYTES] = _codes_to_blocks(gc)
    out[GATE_BLOCKS:, :CODE_BYTES] = _codes_to_blocks(dc)
    out[:GATE_BLOCKS, CODE_BYTES:] = _scales_to_blocks(sc[:sp.GATE_UP_ROWS])
    out[GATE_BLOCKS:, CODE_BYTES:] = _scales_to_blocks(sc[sp.GATE_UP_ROWS:])
    return out.reshape(-1)


def t950_to_slot(t: np.ndarray, packed: bool = False) -> np.ndarray:
    """t950 slot bytes -> raw (or canonical PS4) store slot."""
    t = np.asarray(t, np.uint8)
    if t.shape != (SLOT_T950,):
        raise ValueError(f"t950 slot must be {SLOT_T950} bytes")
    blk = t.reshape(GATE_BLOCKS + DOWN_BLOCKS, BLOCK_BYTES)
    raw = np.empty(sp.RAW_SLOT_BYTES, np.uint8)
    raw[:sp.DOWN_CODES_AT] = _blocks_to_codes(blk[:GATE_BLOCKS, :CODE_BYTES]).reshape(-1)
    raw[sp.DOWN_CODES_AT:sp.SCALES_AT] = _blocks_to_codes(blk[GATE_BLOCKS:, :CODE_BYTES]).reshape(-1)
    sc = blk[:, CODE_BYTES:].reshape(-1, ROWS, SCALE_PITCH)[:, :, :sp.GROUPS].reshape(sp.SCALE_ROWS, sp.GROUPS)
    raw[sp.SCALES_AT:] = sc.reshape(-1)
    return sp.pack_slot(raw) if packed else raw


# -------------------------------------------------------------------------------------------- device repack
def repack_to_t950(src, dst, packed: bool = False) -> None:
    """Device repack of a pool of store slots src [n, 13,219,200 | 12,839,040] u8 into dst [n, >= 13,271,040] u8."""
    import torch

    from . import _native as N

    if src.dtype is not torch.uint8 or dst.dtype is not torch.uint8 or src.ndim != 2 or dst.ndim != 2:
        raise ValueError("src and dst must be 2-D uint8 slot pools")
    if src.shape[0] != dst.shape[0] or src.device != dst.device or src.device.type != "cuda":
        raise ValueError("src and dst need the same slot count on one CUDA device")
    if src.stride(1) != 1 or dst.stride(1) != 1:
        raise ValueError("slot rows must be contiguous")
    want = sp.PS4_SLOT_BYTES if packed else sp.RAW_SLOT_BYTES
    if src.shape[1] != want or dst.shape[1] < SLOT_T950:
        raise ValueError(f"src rows must be {want} bytes, dst rows >= {SLOT_T950}")
    if src.shape[0]:
        N.call("na_repack_to_t950", src.data_ptr(), src.stride(0), int(packed), dst.data_ptr(), dst.stride(0),
               src.shape[0], N.stream(src.device))


def repack_from_t950(src, dst, packed: bool = False) -> None:
    """Device inverse of repack_to_t950 (PS4 output is canonical: base = row minimum)."""
    import torch

    from . import _native as N

    if src.dtype is not torch.uint8 or dst.dtype is not torch.uint8 or src.ndim != 2 or dst.ndim != 2:
        raise ValueError("src and dst must be 2-D uint8 slot pools")
    if src.shape[0] != dst.shape[0] or src.device != dst.device or src.device.type != "cuda":
        raise ValueError("src and dst need the same slot count on one CUDA device")
    if src.stride(1) != 1 or dst.stride(1) != 1:
        raise ValueError("slot rows must be contiguous")
    want = sp.PS4_SLOT_BYTES if packed else sp.RAW_SLOT_BYTES
    if dst.shape[1] != want or src.shape[1] < SLOT_T950:
        raise ValueError(f"dst rows must be {want} bytes, src rows >= {SLOT_T950}")
    if src.shape[0]:
        N.call("na_repack_from_t950", src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0), int(packed),
               src.shape[0], N.stream(src.device))
