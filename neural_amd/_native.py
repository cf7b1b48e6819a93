"""ctypes binding of the C-ABI library neural_amd/_lib/libneural_amd.so (declared in include/neural_amd.h).

torch is imported first on purpose: its wheel carries its own libamdhip64.so.7, and loading our library afterwards
makes the dynamic linker resolve our DT_NEEDED libamdhip64.so.7 to that same runtime, so the hipStream_t values
torch hands out (torch.cuda.current_stream().cuda_stream) are valid streams for our launches.

There is no fallback: a missing library raises NativeLibraryMissing on first use.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

from .build import LIB_PATH

VP, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float

# name -> argtypes (every entry point returns int: 0 = launched, < 0 = error code)
SIGNATURES = {
    "na_version": [],
    "na_selftest_fp4": [VP, VP],
    "na_mxfp4_gemv": [VP, I32, VP, I64, VP, I64, I32, VP, I32, VP, I32, VP, I32, I32, I32, VP, VP],
    "na_moe_decode": [VP, VP, VP, I32, VP, I64, I32, VP, I64, VP, VP, VP, VP, VP, F32, F32, I32, I32, VP, VP],
    "na_router_topk": [VP, I32, VP, VP, I32, VP, VP, VP, VP, VP],
    "na_selftest_mfma": [VP, VP, VP, VP],
    "na_selftest_bf16": [VP, VP, VP, VP, I64, VP],
    "na_selftest_x8": [VP, I32, VP, VP, VP, VP],
    "na_selftest_mfma8": [VP, VP, VP, VP, VP, VP],
    "na_bench_mfma_rate": [I32, I32, I32, VP, VP, VP],
    "na_t950_slot_bytes": [],
    "na_repack_to_t950": [VP, I64, I32, VP, I64, I32, VP],
    "na_repack_from_t950": [VP, I64, VP, I64, I32, I32, VP],
    "na_moe_decode_t950": [VP, VP, VP, I32, VP, I64, VP, I64, VP, VP, VP, VP, VP, F32, F32, I32, I32, VP, VP],
    "na_moe_decode_t950_noalloc": [VP, VP, VP, I32, VP, I64, VP, I64, VP, VP, VP, F32, F32, I32, I32, VP],
    "na_moe_decode_t950_one": [VP, VP, VP, VP, I64, VP, I64, VP, VP, VP, VP, VP, F32, F32, VP, VP, VP],
    "na_moe_decode_t950_one_logits": [VP, VP, VP, VP, VP, I64, VP, I64, VP, VP, VP, F32, F32, VP, VP, VP],
    "na_moe_one_resident": [],
    "na_moe_one_sync_words": [],
    "na_attn_workspace_floats": [I32, I32],
    "na_moe_prefill_workspace_bytes": [I32],
    "na_moe_prefill_workspace_layout": [I32, VP],
    "na_moe_prefill": [VP, VP, VP, I32, VP, I64, I32, VP, I64, VP, VP, VP, I64, VP, F32, F32, VP, VP],
    "na_mxfp4_gemm": [VP, I32, I32, VP, I64, VP, I64, I32, VP, I32, VP, I32, VP],
    "na_mxfp4_gemm_grouped": [VP, I64, VP, I64, I32, VP, I32, I32, I32, I32, VP],
    "na_decode_attention": [VP, VP, VP, I64, VP, VP, VP, I32, F32, I32, I32, I32, VP, VP, VP, VP],
    "na_core_embed": [VP, I64, VP, I64, VP, VP, VP],
    "na_core_qkv": [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, I64, I32, VP, F32, F32, VP],
    "na_core_oproj": [VP, VP, VP, VP, VP, VP],
    "na_core_router": [VP, VP, F32, VP, VP, VP, VP, VP, VP, VP, VP],
    "na_core_lm_partials": [I32],
    "na_core_attn_block": [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, I64, I32, VP, F32, F32, VP, F32, I32, I32, VP,
                           VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP],
    "na_core_attn_block_sync_words": [],
    "na_core_route_pack": [VP, VP, VP, VP, VP, I64, VP, VP, I32, VP, VP, VP, VP],
    "na_core_lm_tail": [VP, VP, VP, VP, F32, VP, I32, VP, VP, VP, VP, VP, I32, VP, VP, VP, I64, VP],
    "na_prefill_attention": [VP, VP, VP, I64, VP, VP, I64, I64, I64, I64, VP, VP, I64, I32, F32, I32, I32, VP, VP],
    "na_ring_write": [VP, VP, I32, VP, VP, I64, I64, I64, I64, I64, I32, VP],
    "na_core_lm_tail_sample": [VP, VP, VP, VP, F32, VP, I32, VP, VP, VP, VP, VP, I32, VP, VP, VP, I64, VP, VP, VP,
                               VP],
    "na_rows_embed": [VP, I64, VP, I32, VP, VP],
    "na_rows_norm": [VP, VP, I32, VP, F32, VP, VP],
    "na_rows_rope": [VP, I32, I64, VP, F32, VP, VP, I64, I64, VP, I64, I64, VP],
    "na_rows_topk": [VP, I32, VP, VP, VP],
}
RESTYPES = {"na_t950_slot_bytes": I64, "na_attn_workspace_floats": I64, "na_moe_prefill_workspace_bytes": I64,
            "na_core_lm_partials": I64, "na_core_attn_block_sync_words": I64, "na_moe_one_sync_words": I64}

ERRORS = {-1: "invalid arguments", -2: "kernel launch failed", -3: "size beyond the kernel's limits",
          -4: "the device cannot hold every workgroup of the launch at once"}


class NativeLibraryMissing(RuntimeError):
    pass


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(f"{LIB_PATH} is missing: build it with `python -m neural_amd.build` "
                                       "(there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, I32)
        _LIB = handle
    return _LIB


ERR_RESIDENT = -4


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name}: {ERRORS.get(rc, 'error')} (status {rc})")


def call_status(name: str, *args, allow=()) -> int:
    """call() that returns the status instead of raising for the codes in ``allow``."""
    rc = getattr(lib(), name)(*args)
    if rc != 0 and rc not in allow:
        raise RuntimeError(f"{name}: {ERRORS.get(rc, 'error')} (status {rc})")
    return rc


def stream(device=None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def events_array(events):
    """ctypes array of raw hipEvent_t handles of recorded torch.cuda.Event objects (None -> NULL)."""
    if events is None:
        return None
    handles = [e.cuda_event for e in events]
    if not all(handles):
        raise ValueError("timing events must have been recorded once (torch creates them lazily)")
    return (VP * len(handles))(*handles)
