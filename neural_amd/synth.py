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


def zipf_routing(rng: np.random.Generator, T: int, n_exp: int = 128, s: float = 1.1, top_k: int = 4):
    """Prompt routing of configuration 2: per token ``top_k`` distinct experts drawn without replacement with
    probability proportional to Zipf(s) over a fixed random rank permutation of the experts, and softmax weights of
    random logits.  Returns (ids int64 [T, top_k], weights fp32 [T, top_k])."""
    ranks = rng.permutation(n_exp)
    p = 1.0 / np.arange(1, n_exp + 1) ** s
    p /= p.sum()
    ids = np.stack([ranks[rng.choice(n_exp, top_k, replace=False, p=p)] for _ in range(T)]).astype(np.int64)
    lg = rng.standard_normal((T, top_k)).astype(np.float32)
    e = np.exp(lg - lg.max(-1, keepdims=True))
    return ids, (e / e.sum(-1, keepdims=True)).astype(np.float32)


def t950_pool_device(n_slots: int, device, seed: int, chunk: int = 128):
    """A resident pool of ``n_slots`` experts in the gfx950 tile layout, built the way a store is loaded: raw store
    slots (uniform code bytes, E8M0 exponents uniform in [119, 125]) generated on the device ``chunk`` at a time and
    repacked into place.  Returns uint8 [n_slots, 13,271,040]; slot i is a function of (seed, i) on a given torch
    build.  All 36 x 128 experts take 61.2 GB."""
    import torch

    from . import tiles
    from .moe.layout import GPTOSS_LAYOUT_T950

    pool = torch.empty((n_slots, GPTOSS_LAYOUT_T950.slot_bytes), dtype=torch.uint8, device=device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    buf = torch.empty((min(chunk, n_slots), L.slot_bytes), dtype=torch.uint8, device=device)
    for c0 in range(0, n_slots, chunk):
        c = min(chunk, n_slots - c0)
        buf[:c, :CODE_BYTES].random_(0, 256, generator=g)
        buf[:c, CODE_BYTES:].random_(SCALE_LO, SCALE_HI + 1, generator=g)
        tiles.repack_to_t950(buf[:c], pool[c0:c0 + c])
    torch.cuda.synchronize(device)
    del buf
    return pool
