"""Activation rows whose elements sit 2^-16 .. 2^-20 below their 32-element block's largest magnitude, and the error
bounds the prefill GEMMs' E4M3 hi + lo activation rows are held to there (shared by the GPU parity test and the CPU
check that these bounds would catch a kernel that drops the lo row).

The block-scaled MFMA path quantises every 32-element block of an activation row into hi (scale 2^(e - 7) for the
block's largest magnitude m, 2^e <= m < 2^(e+1)) and lo (the remainder, scaled by its own block maximum).  An element
within 2^13 of m is reproduced exactly; one further below keeps 4 significant bits of its remainder on the lo grid, so
|x_q - x| <= 2^-21 m.  An output sum_k x_k w_k then deviates from the fp64 product of the exact operands by at most
2^-21 sum_k m_k |w_k| (quantisation) + 5,760 x 2^-24 sum_k |x_k w_k| (fp32 accumulation of the hi and lo products,
worst case) + 2^-8 |y| (one bf16 rounding).
"""
import numpy as np

from neural_amd import synth
from oracle import mxfp4_oracle as mo
from oracle.bf16 import rb

GU, H, GK = 5760, 2880, 90


def case(seed=1616, M=24):
    """(raw slot, x bf16-valued fp32 [M, 2880]).  Every block's largest element sits at column 32 g and is a power of
    two (2^-24 .. 2^24 over the rows); the slot's gate weight in those columns is +0, so each gate output is the sum
    over the far-below elements alone (each 2^-16 .. 2^-20 below its block maximum, random sign and bf16 mantissa)."""
    rng = np.random.default_rng(seed)
    slot = synth.slot_raw(rng)
    slot[:mo.OFF_DC].reshape(GU, GK, 16)[:, :, 0] &= 0xF0       # low nibble of byte 0 = element 32 g: code 0 (+0)
    a = rng.integers(-4, 5, (M, GK)) + rng.integers(-20, 21, (M, 1))
    m = np.exp2(a.astype(np.float64))
    x = np.where(rng.random((M, GK, 32)) < 0.5, -1.0, 1.0) * m[..., None] * np.exp2(-rng.uniform(16, 20, (M, GK, 32)))
    x[:, :, 0] = m * np.where(rng.random((M, GK)) < 0.5, -1.0, 1.0)
    return slot, rb(x.reshape(M, H).astype(np.float32))


def bounds(x, W):
    """(want, bound, rms): the fp64 product want [M, N] of x [M, K] and W [N, K], the per-output bound on |got - want|
    stated in the module docstring, and each row's rms of want [M, 1]."""
    x64 = np.asarray(x, np.float64)
    W64 = np.asarray(W, np.float64)
    want = x64 @ W64.T
    M = x64.shape[0]
    mblk = np.repeat(np.abs(x64).reshape(M, -1, 32).max(-1), 32, axis=1)
    quant = 2.0 ** -21 * (mblk @ np.abs(W64).T)
    accum = 5760 * 2.0 ** -24 * (np.abs(x64) @ np.abs(W64).T)
    bound = quant * (1 + 2.0 ** -8) + 2.0 ** -8 * np.abs(want) + accum
    rms = np.sqrt((want ** 2).mean(axis=1, keepdims=True))
    return want, bound, rms
