"""Independent restatement of the gfx950 tile layout (test infrastructure; see oracle/__init__.py).

Written from the byte-position formula rather than reshapes: for every byte of a raw slot, where it lands in the t950
slot.  The product codec (neural_amd/tiles.py) is checked against this map, and the map itself is pinned by the
properties the tests check: it is a bijection onto the non-padding bytes, and dequantising through it reproduces
the raw slot's dequantised weights exactly.
"""
import numpy as np

from .mxfp4_oracle import GU, H, GK, OFF_DC, OFF_GS, SLOT_RAW

ROWS, FULL, CODE, PITCH = 16, 22, 22 * 1024 + 512, 96
BLOCK = CODE + ROWS * PITCH
SLOT_T950 = (GU // ROWS + H // ROWS) * BLOCK


def code_dest(mat: int, row: int, g: int, byte: int) -> int:
    """t950 offset of code byte `byte` of (row, group g) of matrix mat (0 = gate_up, 1 = down).  k-tile t holds groups
    4t .. 4t + 3 in 1024 bytes at 1024 t (the last, t = 22, only groups 88 and 89 in 512 bytes), in which the 16 bytes
    of MFMA lane l = 16 kb + n, at 16 l, are the code bytes 0..15 of (row n, group 4t + kb)."""
    blk = (0 if mat == 0 else GU // ROWS) + row // ROWS
    n = row % ROWS
    t, kb = g // 4, g % 4
    lane = 16 * kb + n
    return blk * BLOCK + t * 1024 + 16 * lane + byte


def scale_dest(mat: int, row: int, g: int) -> int:
    blk = (0 if mat == 0 else GU // ROWS) + row // ROWS
    return blk * BLOCK + CODE + (row % ROWS) * PITCH + g


def source_to_dest_map() -> np.ndarray:
    """int64 [13,219,200]: t950 offset of every raw-slot byte (vectorised evaluation of code_dest / scale_dest)."""
    out = np.empty(SLOT_RAW, np.int64)
    for mat, rows, off in ((0, GU, 0), (1, H, OFF_DC)):
        r, g, byte = np.meshgrid(np.arange(rows), np.arange(GK), np.arange(16), indexing="ij")
        blk = (0 if mat == 0 else GU // ROWS) + r // ROWS
        lane = 16 * (g % 4) + r % ROWS
        out[off:off + rows * GK * 16] = (blk * BLOCK + (g // 4) * 1024 + 16 * lane + byte).reshape(-1)
    rows = np.arange(GU + H)
    mat = (rows >= GU).astype(np.int64)
    r_in = np.where(mat == 0, rows, rows - GU)
    blk = np.where(mat == 0, 0, GU // ROWS) + r_in // ROWS
    base = blk * BLOCK + CODE + (r_in % ROWS) * PITCH
    out[OFF_GS:] = (base[:, None] + np.arange(GK)[None, :]).reshape(-1)
    return out


_MAP = None


def to_t950(raw: np.ndarray) -> np.ndarray:
    global _MAP
    if _MAP is None:
        _MAP = source_to_dest_map()
    out = np.zeros(SLOT_T950, np.uint8)
    out[_MAP] = np.asarray(raw, np.uint8)
    return out
