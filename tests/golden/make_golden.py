"""Write tests/golden/experts_ref.npz: golden vectors of the reference's own C expert kernel.

Inputs are regenerated from `seed` by neural_amd.synth.slot_raw (their SHA-256 is stored so a changed generator is
detected); x, biases and weights are stored verbatim; `out` is gptoss_experts() of the reference's
kernels/gptoss_cpu_portable.c (built from /root/reference by oracle/Makefile into oracle/_ref/), fp32.

    make -C oracle && python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from neural_amd import synth  # noqa: E402
from oracle.bf16 import rb  # noqa: E402
from oracle.refkernels import RefExperts  # noqa: E402

SEED, E = 424242, 4


def main():
    rng = np.random.default_rng(SEED)
    slots = [synth.slot_raw(rng) for _ in range(E)]
    digest = hashlib.sha256(b"".join(s.tobytes() for s in slots)).hexdigest()
    g = np.random.default_rng(SEED + 1)
    x = rb(g.standard_normal(2880).astype(np.float32))
    bgu = np.stack([rb(g.standard_normal(5760).astype(np.float32) * 0.02) for _ in range(E)])
    bdn = np.stack([rb(g.standard_normal(2880).astype(np.float32) * 0.02) for _ in range(E)])
    w = rb(np.array([0.37, 0.31, 0.2, 0.12], np.float32))
    out = RefExperts("portable").experts(slots, x, list(bgu), list(bdn), w, threads=4)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "experts_ref.npz")
    np.savez_compressed(path, seed=SEED, n_experts=E, slots_sha256=digest, x=x, bgu=bgu, bdn=bdn, w=w, out=out,
                        source="reference kernels/gptoss_cpu_portable.c gptoss_experts, -O3 -ffp-contract=off "
                               "-mavx2 -mfma, scale layout 0")
    print(f"wrote {path}: out max |.| {np.abs(out).max():.4g}")


if __name__ == "__main__":
    main()
