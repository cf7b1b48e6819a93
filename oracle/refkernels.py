"""ctypes binding of the reference's C expert kernels, compiled from /root/reference/kernels by oracle/Makefile into
oracle/_ref/ (test infrastructure and CPU baseline; see oracle/__init__.py).

The ABI is the reference's (kernels/gptoss_cpu_portable.c:296-305, 43-51; kernels/gptoss_cpu_multi.c:358, 484; the
Python side of the same binding is cpu_prefill.py:131-152):
    void gptoss_experts(int E, const uint8_t** slots, const float* x, const float** bgu, const float** bdn,
                        const float* w, float* out, float* scratch, int threads)
    int  gptoss_set_scale_layout(int mode)          0 raw, 1 PS4
scratch holds E*(GU+3H)+H(+64) floats (server.py:612).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")
H, GU = 2880, 5760
VP = ctypes.c_void_p


def cpu_has(flag: str) -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return flag in line.split()
    except OSError:
        pass
    return False


class RefExperts:
    """One loaded reference kernel library.  name: "portable" (AVX2+FMA) or "multi" (AVX-512, includes cap2)."""

    def __init__(self, name: str = "portable"):
        path = os.path.join(REF_DIR, f"libgptoss_{name}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path}: build it with `make -C oracle` (needs /root/reference)")
        if name == "multi" and not cpu_has("avx512f"):
            raise RuntimeError("libgptoss_multi.so needs AVX-512 on this host")
        self.name = name
        self.lib = ctypes.CDLL(path)
        self.lib.gptoss_experts.argtypes = [ctypes.c_int, VP, VP, VP, VP, VP, VP, VP, ctypes.c_int]
        self.lib.gptoss_experts.restype = None
        self.lib.gptoss_set_scale_layout.argtypes = [ctypes.c_int]
        self.lib.gptoss_set_scale_layout.restype = ctypes.c_int
        self.lib.gptoss_slot_bytes.argtypes = [ctypes.c_int]
        self.lib.gptoss_slot_bytes.restype = ctypes.c_longlong

    def set_scale_layout(self, mode: int) -> None:
        if self.lib.gptoss_set_scale_layout(int(mode)) != 0:
            raise ValueError(f"scale layout {mode} refused")

    def experts(self, slots, x, bgu, bdn, w, threads=1, packed=False, scratch=None):
        """out [2880] fp32 = sum_e w[e] * expert_e(x).  slots: list of contiguous u8 numpy arrays."""
        E = len(slots)
        self.set_scale_layout(1 if packed else 0)
        keep = [np.ascontiguousarray(s, dtype=np.uint8) for s in slots]
        bg = [np.ascontiguousarray(b, dtype=np.float32) for b in bgu]
        bd = [np.ascontiguousarray(b, dtype=np.float32) for b in bdn]
        sp = (VP * E)(*[s.ctypes.data for s in keep])
        gp = (VP * E)(*[b.ctypes.data for b in bg])
        dp = (VP * E)(*[b.ctypes.data for b in bd])
        xx = np.ascontiguousarray(x, dtype=np.float32).reshape(H)
        ww = np.ascontiguousarray(w, dtype=np.float32).reshape(E)
        out = np.zeros(H, np.float32)
        if scratch is None:
            scratch = np.zeros(E * (GU + 3 * H) + H + 64, np.float32)
        self.lib.gptoss_experts(E, ctypes.cast(sp, VP), xx.ctypes.data, ctypes.cast(gp, VP), ctypes.cast(dp, VP),
                                ww.ctypes.data, out.ctypes.data, scratch.ctypes.data, int(threads))
        return out
