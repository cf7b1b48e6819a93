"""Seeded synthetic inputs of the benchmark configurations (there is no checkpoint on this machine).

Distributions follow the configurations the path is measured on: E2M1 codes uniform over all 256 byte values (every
nibble), E8M0 exponents uniform in [119, 125], activations N(0, 1) bf16, router weights N(0, 0.02) bf16, biases zero
or N(0, 0.02) bf16.  Host generators use numpy's default_rng so the same seed gives the same bytes everywhere; the
device generators (torch) fill the 36 x 128 resident pool directly in HBM.
"""
from __future__ import annotations

import numpy as np

from .moe.layout import GPTOSS_LAYOUT as L

SCALE_LO, SCALE_HI = 119, 125
CODE_BYTES = L.gate_pack_bytes + L.down_pack_bytes          # 12,441,600
SCALE_BYTES = L.gate_saz_bytes + L.down_saz_bytes           # 777,600


def slot_raw(rng: np.random.Generator, lo: int = SCALE_LO, hi: int = SCALE_HI) -> np.ndarray:
    """One raw expert slot (13,219,200 B): uniform code bytes, scales uniform in [lo, hi]."""
    s = np.empty(L.slot_bytes, np.uint8)
    s[:CODE_BYTES] = rng.integers(0, 256, size=CODE_BYTES, dtype=np.uint8)
    s[CODE_BYTES:] = rng.integers(lo, hi + 1, size=SCALE_BYTES, dtype=np.uint8)
    return s


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0):
    """N(0, std) rounded to bf16; returned as a torch bf16 CPU tensor."""
    import torch

    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * np.float32(std)).to(torch.bfloat16)


def fill_pool_device(pool, seed: int, lo: int = SCALE_LO, hi: int = SCALE_HI) -> None:
    """Fill a device slot pool [n, slot_bytes] u8 in place: uniform codes, scales uniform in [lo, hi].  Uses torch's
    device generator (fast enough for 61 GB); the contents are a function of ``seed`` on a given torch build."""
    import torch

    g = torch.Generator(device=pool.device)
    g.manual_seed(seed)
    n = pool.shape[0]
    for i in range(n):
        row = pool[i]
        row[:CODE_BYTES].random_(0, 256, generator=g)
        row[CODE_BYTES:].random_(lo, hi + 1, generator=g)
