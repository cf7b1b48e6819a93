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
    """t950 offset of code byte `byte` of (row, group g) of matrix mat (0 = gate_up, 1 = down)."""
    blk = (0 if mat == 0 else GU // ROWS) + row // ROWS
    n = row % ROWS
    q, b = byte // 4, byte % 4
    lane = 16 * q + n
    if g < 88:
        t, j = g // 4, g % 4
        return blk * BLOCK + t * 1024 + 16 * lane + 4 * j + b
    return blk * BLOCK + FULL * 1024 + 8 * lane + 4 * (g - 88) + b


def scale_dest(mat: int, row: int, g: int) -> int:
    blk = (0 if mat == 0 else GU // ROWS) + row // ROWS
    return blk * BLOCK + CODE + (row % ROWS) * PITCH + g


def source_to_dest_map() -> np.ndarray:
    """int64 [13,219,200]: t950 offset of every raw-slot byte (vectorised evaluation of code_dest / scale_dest)."""
    out = np.empty(SLOT_RAW, np.int64)
    for mat, rows, off in ((0, GU, 0), (1, H, OFF_DC)):
        r, g, byte = np.meshgrid(np.arange(rows), np.arange(GK), np.arange(16), indexing="ij")
        blk = (0 if mat == 0 else GU // ROWS) + r // ROWS
        n, q, b = r % ROWS, byte // 4, byte % 4
        lane = 16 * q + n
        full = blk * BLOCK + (g // 4) * 1024 + 16 * lane + 4 * (g % 4) + b
        tail = blk * BLOCK + FULL * 1024 + 8 * lane + 4 * (g - 88) + b
        out[off:off + rows * GK * 16] = np.where(g < 88, full, tail).reshape(-1)
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
