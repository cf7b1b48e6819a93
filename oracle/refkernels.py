"""ctypes binding of the reference's C expert kernels, compiled from /root/reference/kernels by oracle/Makefile into
oracle/_ref/ (test infrastructure and CPU baseline; see oracle/__init__.py).

The ABI is the reference's (kernels/gptoss_cpu_portable.c:296-305, 43-51; kernels/gptoss_cpu_multi.c:345-360,
484-505; the Python side of the same binding is cpu_prefill.py:131-152):
    void gptoss_experts(int E, const uint8_t** slots, const float* x, const float** bgu, const float** bdn,
                        const float* w, float* out, float* scratch, int threads)
    int  gptoss_set_scale_layout(int mode)          0 raw, 1 PS4
    void gptoss_experts_multi(int E, const uint8_t** slots, const int* off, const float* X, const float** bgu,
                              const float** bdn, const float* W, float* Y, float* scratch, int threads)   (multi only)
    int  gptoss_multi_scratch_floats(int E, int P)
    void gptoss_combine_pairs(int N, int K, const int* idx, const float* w, const float* Yr, float* out, int threads)
scratch holds E*(GU+3H)+H(+64) floats for gptoss_experts (server.py:612), gptoss_multi_scratch_floats(E, P) for the
multi-token call.
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
        if name == "multi":
            self.lib.gptoss_experts_multi.argtypes = [ctypes.c_int, VP, VP, VP, VP, VP, VP, VP, VP, ctypes.c_int]
            self.lib.gptoss_experts_multi.restype = None
            self.lib.gptoss_multi_scratch_floats.argtypes = [ctypes.c_int, ctypes.c_int]
            self.lib.gptoss_multi_scratch_floats.restype = ctypes.c_int
            self.lib.gptoss_combine_pairs.argtypes = [ctypes.c_int, ctypes.c_int, VP, VP, VP, VP, ctypes.c_int]
            self.lib.gptoss_combine_pairs.restype = None

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

    def experts_multi(self, slots, off, X, W, bgu, bdn, threads=1, packed=False, scratch=None):
        """Pairs grouped by expert: rows [off[e], off[e+1]) of X (fp32 [P, 2880]) go through slots[e]; returns
        Y fp32 [P, 2880], Y[p] = W[p] * expert(X[p]) (reference gptoss_cpu_multi.c:350-360; W = 1 gives the raw
        outputs that combine_pairs expects).  slots: list of contiguous u8 numpy arrays (kept alive by the caller)."""
        E = len(slots)
        self.set_scale_layout(1 if packed else 0)
        off = np.ascontiguousarray(np.asarray(off, np.int32))
        P = int(off[-1])
        X = np.ascontiguousarray(X, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.float32)
        if off.shape != (E + 1,) or X.shape != (P, H) or W.shape != (P,):
            raise ValueError("off must be [E + 1], X [P, 2880] and W [P] with P = off[E]")
        need = int(self.lib.gptoss_multi_scratch_floats(E, P))
        if need < 0:
            raise ValueError(f"{P} pairs exceed one call of the multi-token kernel")
        if scratch is None or scratch.size < need:
            scratch = np.empty(need, np.float32)
        Y = np.zeros((P, H), np.float32)
        sp = (VP * E)(*[s.ctypes.data for s in slots])
        gp = (VP * E)(*[b.ctypes.data for b in bgu])
        dp = (VP * E)(*[b.ctypes.data for b in bdn])
        self.lib.gptoss_experts_multi(E, ctypes.cast(sp, VP), off.ctypes.data, X.ctypes.data, ctypes.cast(gp, VP),
                                      ctypes.cast(dp, VP), W.ctypes.data, Y.ctypes.data, scratch.ctypes.data,
                                      int(threads))
        return Y

    def combine_pairs(self, idx, w, Yr, threads=1):
        """out[t] = the reference CPU combine of the valid pairs idx[t, k] >= 0 of token t, in k order, over raw pair
        outputs Yr (gptoss_cpu_multi.c:472-505).  idx int32 [N, K], w fp32 [N, K]."""
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        Yr = np.ascontiguousarray(Yr, dtype=np.float32)
        N, K = idx.shape
        out = np.zeros((N, H), np.float32)
        self.lib.gptoss_combine_pairs(N, K, idx.ctypes.data, w.ctypes.data, Yr.ctypes.data, out.ctypes.data,
                                      int(threads))
        return out
