"""CPU oracle for the GPT-OSS MoE hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import anything under oracle/, and only as the
checker (or, for the baseline, as the thing timed on the CPU).  The product path (neural_amd) never imports it and
fails loudly when its HIP library is missing; nothing here is a fallback.

Modules (each function cites the reference file:line it restates):
  bf16            round-to-nearest-even fp32 -> bf16 emulation in numpy (the rounding points of the reference's torch
                  and Triton code).
  mxfp4_oracle    E2M1/E8M0 dequant, the PS4 scale codec, GEMV/GEMM in fp64, the clamped-SwiGLU expert forward at the
                  reference GPU path's bf16 rounding points, the CPU-kernel (fp32) variant, combine, router top-4.
  attention_oracle  sink attention: the fp64 closed form, and k_attn's bf16 rounding-point restatement (full, sliding,
                  ring addressing).
  refkernels      ctypes binding of the reference's own C expert kernels compiled from /root/reference by
                  oracle/Makefile into oracle/_ref/ (checker and CPU baseline).

How each function is pinned (the checks live in tests/test_oracle_*.py):
  dequant           two independent derivations of E2M1 (OCP MX bit formula vs the reference's 16-entry table) and the
                    reference C kernel's expert output;
  PS4 codec         the reference's known-answer edge rows and span-16 refusal, and the reference C kernel decoding
                    our packed slots bit-identically to raw ones;
  expert forward    the reference C kernel (fp32) on seeded full-size slots: fp32 variant to ~1e-5, bf16-rounding
                    variant to the north-star tolerance; committed golden vectors in tests/golden/;
  router            closed-form cases (ties -> lowest index, softmax of 4 equal logits = 1/4);
  attention         brute force on tiny cases, single-key closed form, uniform-score mean, sink -> -inf limit,
                    ring == linear invariance.
No function of this oracle is currently "parity unpinned".
"""
