"""Benchmark of the GPT-OSS-120B MoE decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--workload decode|experts|model|prefill|attention]

Default workload ("decode"): one resident pool of all 36 layers x 128 MXFP4 experts (gfx950 tile layout, 61.2 GB,
uniform E2M1 codes, E8M0 exponents uniform in [119, 125]) serves two measurements, printed as ONE JSON line:
  value         configuration 4: full 36-layer GPT-OSS-120B-shaped greedy decode, random-init weights (vocab 201,088),
                a 4096-token random context prefilled, then exactly K greedy tokens timed, one hipGraph replay per
                token (embed, 36 x [QKV + RoPE + cache write, attention, o_proj, router + top-4, experts], lm_head +
                argmax; the next step reads its token on the device).  value = tokens/s.
  config1       configuration 1: the expert body alone (gate_up GEMV + bias + clamped SwiGLU, down GEMV + bias +
                routing weight, top-k combine) of all 36 layers per step, random top-4 routing from 16 routing sets
                cycled so the 256 MB Infinity Cache never serves a repeated expert; batch 1 plus the batch 2 / 4 / 8
                sweep; whole-step HBM GB/s.
  roofline      the dominant expert kernel of configuration 1 at batch 1, the single-launch expert body
                k_moe_one_t950: algorithmic bytes per launch (4 experts x 13,219,200 B of E2M1 codes + E8M0 scales,
                gate_up and down) / its average launch duration, from events
                timestamped by the dispatches themselves on the launch stream (eager steps queued behind a spin
                kernel, so the launches run back to back as in the graph replays); peak 8 TB/s; traffic = HBM bytes
                per launch from the committed rocprofv3 --pmc table (null when the kernel sources changed since).
  cpu_baseline  the reference's own C expert kernel (kernels/gptoss_cpu_multi.c, AVX-512, or gptoss_cpu_portable.c,
                built from source into oracle/_ref/) on this host's cores: configuration 1's expert body, one
                gptoss_experts(E=4) call per layer per token, at all physical cores of one socket (capped at the CPUs
                this process may use) and at the reference's default of 8 threads.

Other workloads print one line each: experts (configuration 1 alone, any layout: t950 runs the MFMA kernels, raw and
ps4 the VALU na_moe_decode kernels), model (configuration 4 alone), prefill (configuration 2, with the reference CPU
kernel's multi-token call as its baseline and a per-expert GEMM sweep over M = 64 .. 2048 tokens per expert),
attention (configuration 3), gemv (the reference-named mxfp4_gemv at configuration 1's shapes on a raw or PS4 pool)
and mfma (the matrix cores' issue rate for the scaled FP8 x FP4 and the bf16 instructions).
"""
from __future__ import annotations

import os

# The reference server's OpenMP settings for its CPU expert kernels (server.py:25 sets GOMP_SPINCOUNT before torch
# loads libgomp); threads bound close to the master.  They must be in the environment before libgomp is loaded,
# i.e. before torch is imported, or they have no effect on the CPU baseline below.
os.environ.setdefault("GOMP_SPINCOUNT", "20000000")
os.environ.setdefault("OMP_PROC_BIND", "close")
# The CPUs this process may use, read before libgomp loads: with OMP_PROC_BIND set, libgomp binds the main thread to
# one CPU when it initialises, after which the main thread's affinity mask names only that CPU.
START_AFFINITY = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)

import argparse  # noqa: E402
import json  # noqa: E402
import statistics  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s GPT-OSS-120B shape; MXFP4 expert GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
GATE_UP_BYTES = 5760 * 1440 + 5760 * 90          # codes + E8M0 scales of one expert's gate_up rows
DOWN_BYTES = 2880 * 1440 + 2880 * 90
SLOT_ALGO_BYTES = GATE_UP_BYTES + DOWN_BYTES      # 13,219,200
N_LAYERS, N_EXPERTS, TOPK, H = 36, 128, 4, 2880


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
KERNEL_SOURCES = ("neural_amd/csrc/common.h", "neural_amd/csrc/t950.h", "neural_amd/csrc/handoff.h",
                  "neural_amd/csrc/topk.h", "neural_amd/csrc/tiles.hip", "neural_amd/csrc/moe_decode.hip")
# the attention block's sources (its traffic entries name them in "sources")
ATTN_BLOCK_SOURCES = ("neural_amd/csrc/common.h", "neural_amd/csrc/handoff.h", "neural_amd/csrc/attention_dev.h",
                      "neural_amd/csrc/core.hip")


def sources_sha256(files=KERNEL_SOURCES):
    import hashlib
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def measured_traffic(kernel, layout, batch, k_split):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by the factor a 1 GiB copy kernel calibrates), or None when no entry was measured on the
    current kernel sources for this workload."""
    try:
        with open(TRAFFIC_FILE) as fh:
            tab = json.load(fh)
    except (OSError, ValueError):
        return None, "no traffic table"
    e = traffic_entry(tab, kernel, layout, batch, k_split)
    if e is None:
        return None, "workload not in traffic table, or measured on other kernel sources"
    return int(e["hbm_bytes_per_launch"]), "ok"


def traffic_entry(tab, kernel, layout, batch, k_split):
    """The committed profile entry of a workload, if it was measured on the current kernel sources (the files the
    entry lists under "sources", else the expert kernels' KERNEL_SOURCES)."""
    for e in tab.get("entries", []):
        if (e["kernel"], e["layout"], e["batch"], e["k_split"]) == (kernel, layout, batch, k_split):
            files = tuple(e.get("sources", KERNEL_SOURCES))
            return e if e["sources_sha256"] == sources_sha256(files) else None
    return None


def attn_block_entry(kind):
    """The attention block's committed traffic entry for a sliding or full layer of configuration 4, or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            return traffic_entry(json.load(fh), "k_attn_block", kind, 1, 0)
    except (OSError, ValueError):
        return None


def rocprof_avg_us(kernel, layout, batch, k_split):
    """The kernel's average duration from the committed rocprofv3 --kernel-trace --stats run of the same workload on
    the current kernel sources (profiles/traffic.json, "rocprof_avg_us"), or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            e = traffic_entry(json.load(fh), kernel, layout, batch, k_split)
    except (OSError, ValueError):
        return None
    return e.get("rocprof_avg_us") if e else None


def effective_k_split(k_split, batch):
    """The k_split the library runs for a requested one (0 = automatic, as na_moe_decode_t950 picks it)."""
    return k_split if k_split > 0 else 4


def queue_behind_spin(torch, ms=4.0):
    """Hold the stream with a spin kernel of about `ms` so that the eager launches the host issues next queue up behind
    it and run back to back, as inside the timed graph replays (issued one by one from Python, each launch would
    otherwise start on an idle GPU and include its wake-up latency)."""
    torch.cuda._sleep(int(ms * 2.4e6))


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def routing_sets(rng, n_sets, B):
    """[n_sets, 36, B, 4] int64 ids and bf16-valued fp32 weights from random router logits (top-4, softmax)."""
    logits = rng.standard_normal((n_sets, N_LAYERS, B, N_EXPERTS)).astype(np.float32)
    ids = np.argsort(-logits, axis=-1, kind="stable")[..., :TOPK]
    top = np.take_along_axis(logits, ids, axis=-1)
    e = np.exp(top - top[..., :1])
    w = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int64), w


def cpu_info():
    """CPU model, sockets, physical cores of the first socket, and the CPUs this process may use (affinity, capped
    by a cgroup CPU quota when one is set)."""
    model, sockets, cores0, phys = None, set(), set(), None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                    sockets.add(v)
                elif k == "core id" and phys == min(sockets):
                    cores0.add(v)
    except OSError:
        pass
    usable = START_AFFINITY
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            q, per = fh.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) // int(per)))
    except (OSError, ValueError):
        pass
    return {"model": model, "model_name_line": f"model name\t: {model}" if model else None,
            "sockets": len(sockets) or None, "socket0_physical_cores": len(cores0) or None,
            "affinity_cpus": usable, "cgroup_cpus": quota, "usable_cpus": min(usable, quota or usable)}


def host_expert_slots(pool_dev, ids, n=160):
    """Store-layout host copies of ``n`` experts of the pool: the distinct (layer, expert) slots of one routing
    ids [36, B, 4], topped up with following slots (160 experts = 2.1 GB, so no CPU cache level holds them)."""
    import torch

    from neural_amd import tiles
    from neural_amd.moe.layout import GPTOSS_LAYOUT

    uniq = []
    for l in range(ids.shape[0]):
        for e in ids[l].reshape(-1).tolist():
            g = l * N_EXPERTS + int(e)
            if g not in uniq and len(uniq) < n:
                uniq.append(g)
    g = 0
    while len(uniq) < n:
        if g not in uniq:
            uniq.append(g)
        g += 1
    if pool_dev.shape[1] == SLOT_ALGO_BYTES:
        return [pool_dev[g].cpu().numpy() for g in uniq]
    buf = torch.empty(1, GPTOSS_LAYOUT.slot_bytes, dtype=torch.uint8, device=pool_dev.device)
    out = []
    for g in uniq:                                       # t950 pool: the reference kernel reads the store layout
        tiles.repack_from_t950(pool_dev[g:g + 1], buf)
        out.append(buf.cpu().numpy()[0].copy())
    return out


def cpu_baselines(pool_dev, ids, seconds):
    """The reference's C expert kernel on this host: configuration 1's expert body, gptoss_experts(4, ...) per token
    per layer (the reference has no batched CPU decode), over a 160-expert host copy (2.1 GB) rotated per call so
    that every call reads cold slots.  Timed as the reference's own A/B tool times kernels
    (tools/kernel_tuning_ab.py:130-158): every configuration once per round, rounds interleaved (the order reversed
    on odd rounds), 6 rounds of warm-up, then the median wall-clock time per call over at least 30 rounds (as many as
    fit ``seconds``).  Configurations: the AVX-512 build of gptoss_cpu_multi.c (the server's library) and the
    portable AVX2 build (gptoss_cpu_portable.c), each at all physical cores of the first socket (capped at the CPUs
    this process may use) and at 8 threads (the reference server's default, server.py:107).  OMP_PROC_BIND and
    GOMP_SPINCOUNT are set at the top of this file, before libgomp loads."""
    from oracle.refkernels import RefExperts, cpu_has

    info = cpu_info()
    host = host_expert_slots(pool_dev, ids)
    t_sock = min(info["socket0_physical_cores"] or info["usable_cpus"], info["usable_cpus"])
    libs = (["multi"] if cpu_has("avx512f") else []) + ["portable"]
    configs = [(lib, t) for lib in libs for t in ([t_sock] + ([8] if t_sock != 8 else []))]
    refs = {lib: RefExperts(lib) for lib in libs}
    rng = np.random.default_rng(5)
    x = rng.standard_normal(H).astype(np.float32)
    bgu = [np.zeros(5760, np.float32)] * 4
    bdn = [np.zeros(2880, np.float32)] * 4
    w = np.full(4, 0.25, np.float32)
    scratch = np.zeros(4 * (5760 + 3 * H) + H + 64, np.float32)
    times = {c: [] for c in configs}
    k, rounds, t_start, warm = 0, 0, time.perf_counter(), 6
    while True:
        for c in (configs if rounds % 2 == 0 else configs[::-1]):
            sel = [host[(k + j) % len(host)] for j in range(4)]
            k += 4
            t0 = time.perf_counter()
            refs[c[0]].experts(sel, x, bgu, bdn, w, threads=c[1], scratch=scratch)
            dt = time.perf_counter() - t0
            if rounds >= warm:
                times[c].append(dt)
        rounds += 1
        if rounds >= warm + 30 and time.perf_counter() - t_start >= seconds:
            break

    def summary(c):
        med = statistics.median(times[c])
        return {"value": round(1.0 / (N_LAYERS * med), 3), "cores": c[1], "ms_per_call": round(med * 1e3, 4),
                "mean_ms_per_call": round(statistics.fmean(times[c]) * 1e3, 4),
                "gbps": round(4 * SLOT_ALGO_BYTES / med / 1e9, 2), "calls": len(times[c])}

    main_c = configs[0]
    res = {**summary(main_c), "unit": "tok/s", "kind": "reference", "library": f"libgptoss_{main_c[0]}.so",
           "sample": (f"median of {len(times[main_c])} interleaved calls of gptoss_experts(E=4) ({main_c[1]} OpenMP "
                      f"threads) over a {len(host)}-expert host copy rotated per call, after {warm} warm-up rounds; "
                      "one call = the expert body of one layer for one token; tok/s = 1 / (36 x median ms/call) "
                      "(experts only: the reference has no CPU dense core)")}
    for c in configs[1:]:
        key = ("threads_8" if c[1] == 8 else "all_cores") if c[0] == main_c[0] else \
            (f"{c[0]}_threads_8" if c[1] == 8 else f"{c[0]}_all_cores")
        res[key] = {**summary(c), "library": f"libgptoss_{c[0]}.so"}
    res["cpu"] = info
    res["omp_env"] = {k: os.environ.get(k) for k in ("OMP_PROC_BIND", "GOMP_SPINCOUNT")}
    res["threads_rule"] = (f"min(physical cores of socket 0 = {info['socket0_physical_cores']}, CPUs this process "
                           f"may use = {info['usable_cpus']})")
    res["build"] = ("oracle/Makefile from the reference's kernels/*.c: gptoss_cpu_multi.c with gcc -O3 -fopenmp "
                    "-mavx2 -mfma -mavx512{f,bw,dq,vl} -Dsb_inited=1 (a declaration kernels/gptoss_cpu_cap2.c:113 "
                    "makes only on Win32); gptoss_cpu_portable.c with the reference's flags -O3 -ffp-contract=off "
                    "-fopenmp -mavx2 -mfma")
    return res


def cpu_prefill_baseline(pool_dev, ids, w, x, threads, seconds):
    """The reference CPU kernels' prompt path over one MoE layer (cpu_prefill.py:15-19, 118-315): the pairs grouped
    by expert (stable in the token index), gptoss_experts_multi with unit pair weights, then gptoss_combine_pairs in
    top-k order.  Timed: the two C calls, repeated until ``seconds`` have passed (at least once)."""
    import torch

    from neural_amd import tiles
    from neural_amd.moe.layout import GPTOSS_LAYOUT
    from oracle.refkernels import RefExperts

    ref = RefExperts("multi")
    T = ids.shape[0]
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    experts, counts = np.unique(flat, return_counts=True)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    buf = torch.empty(1, GPTOSS_LAYOUT.slot_bytes, dtype=torch.uint8, device=pool_dev.device)
    host = []
    for e in experts:
        tiles.repack_from_t950(pool_dev[int(e):int(e) + 1], buf)
        host.append(buf.cpu().numpy()[0].copy())
    X = np.ascontiguousarray(x[order // TOPK], np.float32)
    ones = np.ones(len(order), np.float32)
    idx = np.empty(T * TOPK, np.int32)
    idx[order] = np.arange(len(order), dtype=np.int32)
    idx = idx.reshape(T, TOPK)
    bgu = [np.zeros(5760, np.float32)] * len(experts)
    bdn = [np.zeros(2880, np.float32)] * len(experts)
    ref.experts_multi(host[:1], [0, 1], X[:1], ones[:1], bgu[:1], bdn[:1], threads=threads)    # thread pool start
    n, t0 = 0, time.perf_counter()
    while True:
        Y = ref.experts_multi(host, off, X, ones, bgu, bdn, threads=threads)
        ref.combine_pairs(idx, w, Y, threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    t_layer = el / n
    return {"value": round(T / t_layer, 2), "unit": "tok/s", "cores": threads, "kind": "reference",
            "library": "libgptoss_multi.so",
            "sample": f"the whole configuration-2 layer ({T} tokens, {len(order)} pairs over {len(experts)} experts), "
                      f"{n} run(s) of gptoss_experts_multi (unit pair weights) + gptoss_combine_pairs on {threads} "
                      f"OpenMP threads: {t_layer * 1e3:.1f} ms per layer",
            "ms_per_layer": round(t_layer * 1e3, 2), "cpu": cpu_info()}


def bench_prefill(A):
    """Configuration 2: one MoE layer over T = 2048 prompt tokens (hidden 2880, 128 experts, top-4, Zipf(1.1) expert
    popularity), weights MXFP4 as configuration 0 in the t950 pool, x bf16 N(0,1), zero biases.  One step = the fused
    prefill layer (five launches), captured in a hipGraph.  Reported: tokens/s, the layer's TFLOP/s on the bf16
    MFMA path, and the roofline fraction max(flop / 2.5 PF bf16, bytes / 8 TB/s) / measured time."""
    import torch

    from neural_amd import synth, tiles
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_T950

    dev = torch.device("cuda", 0)
    T = A.tokens
    L = GPTOSS_LAYOUT_T950
    pool = torch.empty(N_EXPERTS, L.slot_bytes, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    raw = torch.empty((N_EXPERTS, GPTOSS_LAYOUT.slot_bytes), dtype=torch.uint8, device=dev)
    cb = synth.CODE_BYTES
    raw[:, :cb].random_(0, 256, generator=g)
    raw[:, cb:].random_(synth.SCALE_LO, synth.SCALE_HI + 1, generator=g)
    tiles.repack_to_t950(raw, pool)
    del raw
    tab = torch.arange(N_LAYERS * N_EXPERTS, dtype=torch.int64, device=dev) % N_EXPERTS
    rx = ResidentExperts(pool, L, None, None, tab)
    rng = np.random.default_rng(2048)
    ids_np, w_np = synth.zipf_routing(rng, T)
    counts = np.bincount(ids_np.reshape(-1), minlength=N_EXPERTS)
    ids = torch.from_numpy(ids_np).to(dev)
    wts = torch.from_numpy(w_np).to(torch.bfloat16).to(dev)
    x = synth.bf16_normal(rng, (T, H)).to(dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    rx.forward_prefill(0, x, ids, wts, out=out)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        rx.forward_prefill(0, x, ids, wts, out=out)
    torch.cuda.current_stream().wait_stream(cs)
    with torch.cuda.graph(gr):
        rx.forward_prefill(0, x, ids, wts, out=out)
    for _ in range(max(A.warmup // 4, 3)):
        gr.replay()
    torch.cuda.synchronize()
    steps = max(A.steps // 10, 10)
    t0 = time.perf_counter()
    for _ in range(steps):
        gr.replay()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / steps
    # per-launch times (eager, dispatch-timestamped events)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(10)]
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    names = ("count", "order", "gate_up", "down", "combine")
    per = {nm: 0.0 for nm in names}
    R = 5
    for _ in range(R):
        queue_behind_spin(torch)
        rx.forward_prefill(0, x, ids, wts, out=out, events=ev)
        torch.cuda.synchronize()
        for i, nm in enumerate(names):
            per[nm] += ev[2 * i].elapsed_time(ev[2 * i + 1]) * 1e3 / R
    P = int(counts.sum())
    flop = 2.0 * P * (5760 * 2880 + 2880 * 2880)
    touched = int((counts > 0).sum())
    wbytes = touched * SLOT_ALGO_BYTES
    abytes = T * H * 2 + P * 2880 * 2 * 2 + P * H * 2 * 2 + T * H * 2
    t_roof = max(flop / 2.5e15, (wbytes + abytes) / (HBM_PEAK_GBS * 1e9))
    log(f"prefill T={T}: {el * 1e6:.1f} us/layer ({T / el:.0f} tok/s), {flop / el / 1e12:.1f} TFLOP/s; launches "
        + ", ".join(f"{nm} {v:.1f} us" for nm, v in per.items()))
    gu_flop = 2.0 * P * 5760 * 2880
    sweep = expert_gemm_sweep(rx, dev) if not A.no_batch_sweep else None
    cpu = None
    if not A.skip_cpu:
        try:
            info = cpu_info()
            threads = min(info["socket0_physical_cores"] or info["usable_cpus"], info["usable_cpus"])
            log(f"cpu baseline (reference multi-token kernel, {threads} threads) ...")
            cpu = cpu_prefill_baseline(pool, ids_np, wts.float().cpu().numpy(), x.float().cpu().numpy(), threads,
                                       A.cpu_seconds)
            log(f"cpu baseline: {cpu['value']} tok/s ({cpu['ms_per_layer']} ms per layer)")
        except Exception as e:      # the baseline is reported, not required
            log(f"cpu baseline unavailable: {e!r}")
            cpu = {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference", "sample": f"unavailable: {e}"}
    res = {"metric": "prefill MoE layer tokens/s (config 2)", "value": round(T / el, 1), "unit": "tok/s", "n_gpus": 1,
           "steps": steps, "ms_per_step": round(el * 1e3, 4), "higher_is_better": True, "dtype": "bf16",
           "data": "synthetic",
           "config": {"workload": f"config2: one MoE layer, {T} tokens, 128 experts top-4 Zipf(1.1), t950 pool, "
                                  "block-scaled FP8 x FP4 MFMA (activations as exact E4M3 hi + lo)", "tokens": T,
                      "pairs": P,
                      "experts_touched": touched, "max_expert_tokens": int(counts.max()),
                      "min_expert_tokens": int(counts[counts > 0].min()),
                      "launch_us": {k: round(v, 2) for k, v in per.items()},
                      "layer_tflops": round(flop / el / 1e12, 2),
                      "gate_up_tflops": round(gu_flop / (per["gate_up"] * 1e-6) / 1e12, 2),
                      "roofline_time_us": round(t_roof * 1e6, 1),
                      "roofline_fraction": round(t_roof / el, 4),
                      "expert_gemm_sweep": sweep},
           "roofline": {"bound": "hbm" if (wbytes + abytes) / (HBM_PEAK_GBS * 1e9) >= flop / 2.5e15 else "mfma",
                        "achieved": round((wbytes + abytes) / el / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round((wbytes + abytes) / el / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                        "kernel": "k_prefill_gate_up + k_prefill_down",
                        "mfma_frac_exact": round(flop / el / 2.5e15, 4),
                        "mfma_frac_fp4_peak": round(flop / el / 10.1e15, 4)},
           "cpu_baseline": cpu}
    print(json.dumps(res), flush=True)


def run_model(A, pool, dev):
    """Configuration 4 on a resident t950 pool: full 36-layer GPT-OSS-120B-shaped greedy decode on one GPU.
    Random-init weights (attention, router, embedding and lm_head bf16 N(0, 0.02), norms 1 + N(0, 0.02), sinks N(0, 1),
    vocab 201088), a context of 4096 random token ids prefilled (DecodeModel.prefill: the prompt through every layer
    at once, its K/V written into the caches and its greedy successor appended; or, with --context-mode decode, read
    token by token through the decode step), then greedy decode with one hipGraph per step (embed, 36 x [QKV + RoPE +
    cache write, attention, o_proj, router + top-4, experts], final norm + lm_head + argmax; the next step reads its
    token on the device).  Timed: exactly --steps greedy steps from the end of the context; the warm-up steps run
    from the same context snapshot and are rolled back; a second run from the snapshot must give the same tokens.
    Per-launch times come from dispatch-timestamped events over eager steps.  Returns a dict of the results."""
    import torch

    from neural_amd.model import DecodeModel, random_weights, use_tuned_prompt_gemms
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950

    ctx, n_new = A.context, A.steps
    rx = ResidentExperts(pool, GPTOSS_LAYOUT_T950, None, None, max_batch=1, k_split=A.k_split,
                         combine_in_down=A.down != "expert")
    log("model: random-init dense weights")
    w = random_weights(device=dev, seed=77)
    smax = ctx + max(n_new, A.warmup) + 2
    model = DecodeModel(w, rx, smax=smax, n_split=A.attn_split or None, sliding_split=A.sliding_split,
                        fused_attn=not A.unfused_attn)
    torch.cuda.synchronize()
    rng = np.random.default_rng(4096)
    prompt = rng.integers(0, w.vocab, ctx)
    # the prompt's library GEMMs: the committed hipBLASLt choices for these shapes (TunableOp, tuning off), or the
    # library's default heuristic
    tuned_read = use_tuned_prompt_gemms(A.prompt_gemms == "tuned")
    if A.prompt_gemms == "tuned":
        log(f"model: prompt GEMMs from the committed TunableOp results: {'read' if tuned_read else 'not read'}")
    if A.context_mode == "prefill":
        model.prefill(prompt, chunk=A.prefill_chunk)      # warm-up of the same shapes: library GEMM selection
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.prefill(prompt, chunk=A.prefill_chunk)      # K/V of positions 0..ctx-1, seq[ctx] = its greedy token
        torch.cuda.synchronize()
        t_ctx = time.perf_counter() - t0
        log(f"model: {ctx}-token context prefilled in {t_ctx * 1e3:.1f} ms ({ctx / t_ctx:.0f} tok/s)")
        model.capture()
    else:
        model.reset(prompt)
        model.capture()
        t0 = time.perf_counter()
        model.run(ctx - 1)                               # the context, token by token (graph replays)
        torch.cuda.synchronize()
        t_ctx = time.perf_counter() - t0
        log(f"model: context of {ctx} tokens read in {t_ctx:.2f} s ({(ctx - 1) / t_ctx:.0f} steps/s)")
        model.n_forced.fill_(ctx)
    snap = model.snapshot()
    model.run(A.warmup)
    torch.cuda.synchronize()
    model.restore(snap)
    torch.cuda.synchronize()
    # ------------------------------------------------------------------ timed region
    t0 = time.perf_counter()
    model.run(n_new)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    t_lo = int(model.pos.item()) - n_new                 # position of the first timed step's input token
    toks = model.seq[t_lo + 1:t_lo + 1 + n_new].cpu().numpy()
    tok_s = n_new / el
    log(f"model: {n_new} greedy tokens in {el * 1e3:.1f} ms: {el / n_new * 1e3:.3f} ms/token, {tok_s:.1f} tok/s")
    # determinism: the same steps again from the same snapshot give the same tokens
    model.restore(snap)
    model.run(n_new)
    torch.cuda.synchronize()
    same = bool(np.array_equal(model.seq[t_lo + 1:t_lo + 1 + n_new].cpu().numpy(), toks))
    # ------------------------------------------------------------------ per-kernel events (eager steps)
    model.restore(snap)
    names = rx.launches(1)
    ev = []
    for _ in range(N_LAYERS):
        d = {"attn": [torch.cuda.Event(enable_timing=True) for _ in range(2)],
             "experts": [torch.cuda.Event(enable_timing=True) for _ in range(2 * len(names))]}
        for e in d["attn"] + d["experts"]:
            e.record()
        ev.append(d)
    torch.cuda.synchronize()
    R = max(1, A.roofline_steps // 4)
    acc = {nm: 0.0 for nm in names}
    att_full = att_slide = 0.0
    for _ in range(R):
        queue_behind_spin(torch, 8.0)
        model.step(events=ev)
        torch.cuda.synchronize()
        for li in range(N_LAYERS):
            for k, nm in enumerate(names):
                acc[nm] += ev[li]["experts"][2 * k].elapsed_time(ev[li]["experts"][2 * k + 1]) * 1e3
            a = ev[li]["attn"][0].elapsed_time(ev[li]["attn"][1]) * 1e3
            if li % 2 == 0:
                att_slide += a
            else:
                att_full += a
    model.restore(snap)
    n_l = R * N_LAYERS
    avg = {nm: acc[nm] / n_l for nm in names}
    log("model: per launch " + ", ".join(f"{nm} {v:.2f} us" for nm, v in avg.items())
        + f", attention full {att_full / (n_l / 2):.2f} us, sliding {att_slide / (n_l / 2):.2f} us")
    attn_roof = None
    if not A.unfused_attn:
        # the attention block's algorithmic bytes: Q|K|V, o_proj and router weights with their biases, the two norm
        # weights and the sinks, plus the K and V cache rows its attention reads (128 ring rows on a sliding layer,
        # positions 0 .. p on a full layer, p averaged over the R timed steps)
        blk_w = 2 * (5120 * 2880 + 5120 + 2880 * 4096 + 2880 + 128 * 2880 + 128 + 2 * 2880 + 64)
        p_avg = ctx + (R - 1) / 2
        kinds = {"sliding": (att_slide / (n_l / 2), blk_w + 2 * 2 * 8 * 64 * 128),
                 "full": (att_full / (n_l / 2), blk_w + 2 * 2 * 8 * 64 * (p_avg + 1))}
        per = {k: {"avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": int(b),
                   "gbps": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
               for k, (us, b) in kinds.items()}
        # measured HBM bytes and rocprof durations per launch (profiles/traffic.json, current block sources)
        ents = {k: attn_block_entry(k) for k in kinds}
        for k, e in ents.items():
            if e is not None:
                per[k]["traffic"] = int(e["hbm_bytes_per_launch"])
                per[k]["rocprof_avg_launch_us"] = e["rocprof_avg_us"]
                per[k]["frac_rocprof"] = round(kinds[k][1] / e["rocprof_avg_us"] / 1e3 / HBM_PEAK_GBS, 4)
        pair_traffic = (sum(int(e["hbm_bytes_per_launch"]) for e in ents.values())
                        if all(e is not None for e in ents.values()) else None)
        log(f"model: attention block traffic per (sliding, full) launch pair: {pair_traffic}")
        tot_b, tot_us = sum(b for _, b in kinds.values()), sum(us for us, _ in kinds.values())
        attn_roof = {"kernel": "k_attn_block", "bound": "hbm", "achieved": round(tot_b / tot_us / 1e3, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4),
                     "traffic": pair_traffic, **per,
                     "workload": f"config4 decode step at context {ctx}: one sliding and one full layer's block "
                                 "(18 of each per token), dispatch-stamped events over eager steps; achieved, frac "
                                 "and traffic per pair of launches (one of each kind)"}
    dense = N_LAYERS * 2 * (5120 * 2880 + 2880 * 4096 + 128 * 2880) + 2 * 201088 * 2880
    experts = N_LAYERS * TOPK * SLOT_ALGO_BYTES
    kv = 2 * 2 * 8 * 64 * (18 * (ctx + n_new / 2) + 18 * 128)
    step_bytes = dense + experts + kv
    cfg = {"workload": f"config4: full 36-layer GPT-OSS-120B-shaped greedy decode, random-init weights, "
                       f"{ctx}-token context, {n_new} tokens, one hipGraph per step, experts t950 resident",
           "context": ctx, "tokens": n_new, "vocab": int(w.vocab), "attn_split_full": model.n_split,
           "attn_split_sliding": A.sliding_split, "deterministic_tokens": same,
           "attention_block": "four launches" if A.unfused_attn else "one launch per layer (na_core_attn_block)",
           "sync_error": model.sync_error(),
           "first_tokens": [int(t) for t in toks[:8]],
           "step_algorithmic_gb": round(step_bytes / 1e9, 3),
           "step_hbm_gbps": round(step_bytes / (el / n_new) / 1e9, 1),
           "launch_us": {**{nm: round(v, 2) for nm, v in avg.items()},
                         "attention_full": round(att_full / (n_l / 2), 2),
                         "attention_sliding": round(att_slide / (n_l / 2), 2)},
           "context_mode": A.context_mode,
           "prompt_gemms": ("hipBLASLt algorithms from neural_amd/tunableop_mi355x.csv (PyTorch TunableOp, tuning off)"
                            if tuned_read else "hipBLASLt default heuristic"),
           **({"context_prefill_ms": round(t_ctx * 1e3, 1), "prefill_tok_s": round(ctx / t_ctx, 1),
               "prefill_chunk": A.prefill_chunk} if A.context_mode == "prefill" else
              {"context_steps_per_s": round((ctx - 1) / t_ctx, 1)})}
    out = {"tok_s": tok_s, "ms_per_step": el / n_new * 1e3, "config": cfg, "gate_up_us": avg[names[0]],
           "expert_label": names[0], "attn_roofline": attn_roof}
    del model, w, rx
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


# bench kernel label -> (symbol, algorithmic bytes per distinct expert) of the batch-1 t950 expert launches
EXPERT_KERNELS = {"experts": ("k_moe_one_t950", GATE_UP_BYTES + DOWN_BYTES),
                  "gate_up": ("k_moe_gate_up_t950", GATE_UP_BYTES)}


def expert_roofline(label, avg_us, k_split):
    """The roofline object of the dominant batch-1 expert launch (4 distinct experts per launch): the single-launch
    expert body ("experts": gate_up, SwiGLU, down and the top-4 sum; 4 x 13,219,200 B) where the library runs it,
    else the gate_up kernel (4 x 8,812,800 B)."""
    kname, per_expert = EXPERT_KERNELS[label]
    nbytes = TOPK * per_expert
    gbps = nbytes / (avg_us * 1e-6) / 1e9
    traffic, why = measured_traffic(kname, "t950", 1, effective_k_split(k_split, 1))
    log(f"traffic: {traffic} ({why})")
    rp = rocprof_avg_us(kname, "t950", 1, effective_k_split(k_split, 1))
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kname,
            "avg_launch_us": round(avg_us, 3), "algorithmic_bytes_per_launch": nbytes,
            # the same bytes over rocprofv3's average duration of the kernel (includes its per-dispatch cost)
            "rocprof_avg_launch_us": rp, "frac_rocprof": round(nbytes / (rp * 1e3) / HBM_PEAK_GBS, 4) if rp else None}


def bench_model(A):
    """Configuration 4 alone (see run_model); roofline: the expert body inside the decode step."""
    import torch

    from neural_amd import synth

    dev = torch.device("cuda", 0)
    log(f"model: building the expert pool ({N_LAYERS * N_EXPERTS} slots, t950)")
    pool = synth.t950_pool_device(N_LAYERS * N_EXPERTS, dev, 4242)
    m = run_model(A, pool, dev)
    res = {"metric": METRIC, "value": round(m["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": A.steps,
           "warmup": A.warmup, "ms_per_step": round(m["ms_per_step"], 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic", "config": m["config"],
           "roofline": {**expert_roofline(m["expert_label"], m["gate_up_us"], A.k_split),
                        "workload": "config4 decode step"},
           "roofline_config4_attention": m["attn_roofline"], "cpu_baseline": None}
    print(json.dumps(res), flush=True)


def bench_attention(A):
    """Configuration 3: GQA decode attention (64 q / 8 KV heads, head_dim 64, bf16 K/V ~ N(0,1), sinks ~ N(0,1)),
    batch 1 and 4, contexts 1024 / 4096 / 8192, layers alternating full attention and a 128-token sliding window
    (rolling 128-row cache).  One step = 36 layers (18 full + 18 sliding) captured in one hipGraph; per layer one
    launch.  Reported per case: us per full and per sliding layer (graph replays; a graph of only full or only
    sliding layers), and the full layer's algorithmic HBM rate (K + V bytes = 2048 x ctx per sequence and layer)."""
    import torch

    from neural_amd import attention as AT

    dev = torch.device("cuda", 0)
    rng = torch.Generator(device=dev)
    rng.manual_seed(1234)
    NL = 18
    cases = []
    for B in (1, 4):
        for ctx in (1024, 4096, 8192):
            kf = [(torch.randn(B, AT.NKV, ctx, AT.HD, device=dev, generator=rng)).to(torch.bfloat16) for _ in range(2)]
            vf = [(torch.randn(B, AT.NKV, ctx, AT.HD, device=dev, generator=rng)).to(torch.bfloat16) for _ in range(2)]
            kr = (torch.randn(B, AT.NKV, 128, AT.HD, device=dev, generator=rng)).to(torch.bfloat16)
            vr = (torch.randn(B, AT.NKV, 128, AT.HD, device=dev, generator=rng)).to(torch.bfloat16)
            sinks = torch.randn(AT.NQ, device=dev, generator=rng).to(torch.bfloat16)
            q = torch.randn(B, AT.NQ * AT.HD, device=dev, generator=rng).to(torch.bfloat16)
            out = torch.empty_like(q)
            pos = torch.full((B,), ctx - 1, dtype=torch.int64, device=dev)
            def timed(fn):
                fn(0)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for l in range(NL):
                        fn(l)
                for _ in range(5):
                    g.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                R = 50
                e0.record()
                for _ in range(R):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) * 1e3 / (R * NL)

            res, sweep = {}, {}
            for ns in sorted({max(1, min(AT.MAX_SPLIT, ctx // c)) for c in (64, 128, 256, 512)}):
                split = AT.SplitAttn(ns, ctx, dev, batch=B)
                sweep[ns] = round(timed(lambda l, sp=split: AT.decode_attention_batched(
                    q, kf[l % 2], vf[l % 2], sinks, pos, out, 0.125, split=sp)), 3)
            ns = min(sweep, key=sweep.get)
            res["full"] = sweep[ns]
            res["sliding"] = timed(lambda l: AT.decode_attention_batched(q, kr, vr, sinks, pos, out, 0.125,
                                                                         sliding=128, ring=128))
            full_bytes = B * 2048 * ctx
            case = {"batch": B, "ctx": ctx, "n_split": ns, "n_split_sweep_us": sweep, "full_us": round(res["full"], 3),
                    "sliding_us": round(res["sliding"], 3),
                    "full_hbm_gbps": round(full_bytes / (res["full"] * 1e-6) / 1e9, 1),
                    "layer_pair_us": round(res["full"] + res["sliding"], 3)}
            log(f"attention B={B} ctx={ctx} ns={ns}: full {case['full_us']} us ({case['full_hbm_gbps']} GB/s), "
                f"sliding {case['sliding_us']} us")
            cases.append(case)
            del kf, vf, kr, vr
    worst = max(c["full_us"] for c in cases)
    res = {"metric": "decode attention us per full layer (config 3, worst case)", "value": worst, "unit": "us",
           "n_gpus": 1, "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "config3: GQA 64q/8kv hd64 decode attention with sinks, batch 1 and 4, ctx 1024/"
                                  "4096/8192, full layers chunked (SplitAttn), sliding layers on a 128-row ring",
                      "cases": cases},
           "roofline": {"bound": "hbm", "achieved": max(c["full_hbm_gbps"] for c in cases), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(max(c["full_hbm_gbps"] for c in cases) / HBM_PEAK_GBS, 4),
                        "traffic": None, "kernel": "k_decode_attn"},
           "cpu_baseline": None}
    print(json.dumps(res), flush=True)


def measure_experts(rx, dev, B, steps, warmup, n_sets, roofline_steps):
    """Configuration 1 on ResidentExperts ``rx``: graph-replayed 36-layer expert-body steps of batch B (n_sets
    routing sets cycled), then the per-kernel pass (eager steps with dispatch-timestamped events)."""
    import torch

    from neural_amd import synth

    launches = rx.launches(B)
    per_layer = len(launches)
    rng = np.random.default_rng(2026 + B)
    ids_np, w_np = routing_sets(rng, n_sets, B)
    distinct = np.array([[len(set(ids_np[s, l].reshape(-1).tolist())) for l in range(N_LAYERS)]
                         for s in range(n_sets)])
    ids = torch.from_numpy(ids_np).to(dev)
    wts = torch.from_numpy(w_np).to(torch.bfloat16).to(dev)
    x = synth.bf16_normal(rng, (N_LAYERS, B, H)).to(dev)
    out = torch.empty(N_LAYERS, B, H, dtype=torch.bfloat16, device=dev)

    def step(s, events=None):
        for l in range(N_LAYERS):
            rx.forward_decode(l, x[l], ids[s, l], wts[s, l], out=out[l], events=None if events is None else events[l])

    step(0)                                               # eager warm-up, then one graph per routing set
    torch.cuda.synchronize()
    graphs = []
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        step(0)
    torch.cuda.current_stream().wait_stream(cs)
    for s in range(n_sets):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            step(s)
        graphs.append(gr)
    torch.cuda.synchronize()
    log(f"config1 B={B}: captured {len(graphs)} graphs of {per_layer * N_LAYERS} kernels; warm-up {warmup} steps")
    for i in range(warmup):
        graphs[i % n_sets].replay()
    torch.cuda.synchronize()
    # ------------------------------------------------------------------ timed region
    t0 = time.perf_counter()
    for i in range(steps):
        graphs[i % n_sets].replay()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el / steps * 1e3
    tok_s = B * steps / el
    step_bytes = np.mean([distinct[i % n_sets].sum() for i in range(steps)]) * SLOT_ALGO_BYTES
    log(f"config1 B={B}: timed {steps} steps: {ms_step:.3f} ms/step, {tok_s:.1f} tok/s, "
        f"{step_bytes / (ms_step * 1e-3) / 1e9:.0f} GB/s whole-step")
    # ------------------------------------------------------------------ roofline pass (per-kernel events)
    per_kernel_bytes = {"gate_up": GATE_UP_BYTES, "down": DOWN_BYTES, "down_combine": DOWN_BYTES, "combine": 0,
                        "experts": GATE_UP_BYTES + DOWN_BYTES}
    kernels = tuple((nm, per_kernel_bytes[nm]) for nm in launches)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2 * len(kernels))] for _ in range(N_LAYERS)]
    for row in ev:
        for e in row:
            e.record()
    torch.cuda.synchronize()
    tot = {nm: [0.0, 0.0, 0] for nm, _ in kernels}
    for r in range(roofline_steps):
        s = r % n_sets
        queue_behind_spin(torch)
        step(s, events=ev)
        torch.cuda.synchronize()
        for l in range(N_LAYERS):
            d = int(distinct[s, l])
            for k, (nm, per) in enumerate(kernels):
                ms = ev[l][2 * k].elapsed_time(ev[l][2 * k + 1])
                tot[nm][0] += ms
                tot[nm][1] += d * per
                tot[nm][2] += 1
    kern = {nm: {"avg_us": v[0] / v[2] * 1e3, "gbps": (v[1] / (v[0] * 1e-3) / 1e9) if v[0] else 0.0}
            for nm, v in tot.items()}
    for nm, v in kern.items():
        log(f"config1 B={B}: kernel {nm}: avg {v['avg_us']:.2f} us/launch, {v['gbps']:.0f} GB/s algorithmic")
    dom = kernels[0][0]
    del graphs
    return {"tok_s": tok_s, "ms_step": ms_step, "step_bytes": step_bytes, "distinct": distinct, "kern": kern,
            "dom": dom, "per_launch": tot[dom][1] / tot[dom][2], "ids_np": ids_np}


def batch_sweep(rx, dev, A, skip):
    """Configuration 1's other batch sizes, shorter runs on the same resident pool."""
    sweep = {}
    for Bs in (1, 2, 4, 8):
        if Bs == skip:
            continue
        m = measure_experts(rx, dev, Bs, max(A.steps // 4, 20), 5, 8, max(A.roofline_steps // 4, 2))
        kd = m["kern"][m["dom"]]
        sweep[str(Bs)] = {"tok_s": round(m["tok_s"], 1), "ms_per_step": round(m["ms_step"], 4),
                          "distinct_experts_per_layer": round(float(m["distinct"].mean()), 3),
                          "step_hbm_gbps": round(m["step_bytes"] / (m["ms_step"] * 1e-3) / 1e9, 1),
                          "gate_up_avg_launch_us": round(kd["avg_us"], 3), "gate_up_gbps": round(kd["gbps"], 1),
                          "gate_up_frac": round(kd["gbps"] / HBM_PEAK_GBS, 4)}
    return sweep


def config1_summary(m, L, B):
    kern = m["kern"]
    out = {"workload": f"config1: decode expert body (gate_up+SwiGLU-clamp+down+combine), 36 layers x 128 experts "
                       f"resident ({L.weight_repr}), batch {B}, random top-4 routing",
           "batch": B, "tok_s": round(m["tok_s"], 2), "ms_per_step": round(m["ms_step"], 4),
           "distinct_experts_per_layer": round(float(m["distinct"].mean()), 3),
           "step_algorithmic_gb": round(m["step_bytes"] / 1e9, 4),
           "step_hbm_gbps": round(m["step_bytes"] / (m["ms_step"] * 1e-3) / 1e9, 1),
           "step_hbm_frac": round(m["step_bytes"] / (m["ms_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    for nm, v in kern.items():
        out[f"{nm}_avg_launch_us"] = round(v["avg_us"], 3)
        if v["gbps"]:
            out[f"{nm}_kernel_gbps"] = round(v["gbps"], 1)
    return out


NUMERICS = ("weights MXFP4 (E2M1 codes x E8M0 scales, consumed as stored by the block-scaled MFMA, exact); activations "
            "bf16 (x, and h between the expert products), fed to the MFMA as two E4M3 rows (hi + lo) per bf16 row "
            "with one E8M0 scale per 32-element block: exact for every element within 2^13 of its block's largest "
            "magnitude; fp32 accumulation, bf16 outputs at the reference's rounding points")


def bench_decode(A):
    """The default workload: configuration 4 (value) and configuration 1 (config1, roofline) on one resident pool,
    CPU baselines of the reference's expert kernel."""
    import torch

    from neural_amd import synth
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950

    dev = torch.device("cuda", 0)
    L = GPTOSS_LAYOUT_T950
    log(f"building the expert pool ({N_LAYERS * N_EXPERTS} slots, t950, "
        f"{N_LAYERS * N_EXPERTS * L.slot_bytes / 1e9:.1f} GB)")
    pool = synth.t950_pool_device(N_LAYERS * N_EXPERTS, dev, 4242)
    m4 = run_model(A, pool, dev)
    rx = ResidentExperts(pool, L, None, None, k_split=A.k_split, combine_in_down=A.down != "expert")
    m1 = measure_experts(rx, dev, 1, max(A.steps, 100), max(A.warmup, 5), A.sets, A.roofline_steps)
    c1 = config1_summary(m1, L, 1)
    if not A.no_batch_sweep:
        c1["batch_sweep"] = batch_sweep(rx, dev, A, 1)
    roof = expert_roofline(m1["dom"], m1["kern"][m1["dom"]]["avg_us"], A.k_split)
    roof.update(workload="config1 batch 1 (the expert GEMV stream the metric's GB/s half names)",
                config4_avg_launch_us=round(m4["gate_up_us"], 3))
    cpu = None
    if not A.skip_cpu:
        try:
            log("cpu baseline (reference C kernel) ...")
            cpu = cpu_baselines(pool, m1["ids_np"][0], A.cpu_seconds)
            log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads ({cpu['gbps']} GB/s), "
                f"8 threads: {cpu.get('threads_8', {}).get('value')}")
        except Exception as e:      # the baseline is reported, not required
            log(f"cpu baseline unavailable: {e!r}")
            cpu = {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference", "sample": f"unavailable: {e}"}
    cfg = dict(m4["config"])
    cfg["workload"] = (cfg["workload"] + "; config1 (expert GEMV stream, batch 1, 2, 4, 8) on the same pool under "
                       "config1")
    cfg["config1"] = c1
    res = {"metric": METRIC, "value": round(m4["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": A.steps,
           "warmup": A.warmup, "ms_per_step": round(m4["ms_per_step"], 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "numerics": NUMERICS, "data": "synthetic",
           "config": cfg, "roofline": roof, "roofline_config4_attention": m4["attn_roofline"],
           "cpu_baseline": cpu}
    print(json.dumps(res), flush=True)


def store_pool(dev, n_slots, layout, seed):
    """A device pool of n_slots expert slots in a store layout ("raw" E8M0 rows or "ps4" packed 4-bit scale rows):
    uniform E2M1 code bytes, E8M0 exponents uniform in [119, 125] (PS4: base 119, nibble deltas 0..6)."""
    import torch

    from neural_amd import synth
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4

    L = GPTOSS_LAYOUT_PS4 if layout == "ps4" else GPTOSS_LAYOUT
    pool = torch.empty((n_slots, L.slot_bytes), dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cb = GPTOSS_LAYOUT.gate_pack_bytes + GPTOSS_LAYOUT.down_pack_bytes
    pool[:, :cb].random_(0, 256, generator=g)
    if layout == "ps4":
        sc = pool[:, cb:].view(n_slots, -1, 46)
        sc[:, :, 0].fill_(synth.SCALE_LO)
        lo = torch.randint(0, 7, sc[:, :, 1:].shape, dtype=torch.uint8, device=dev, generator=g)
        hi = torch.randint(0, 7, sc[:, :, 1:].shape, dtype=torch.uint8, device=dev, generator=g)
        sc[:, :, 1:] = lo | (hi << 4)
        del lo, hi
    else:
        pool[:, cb:].random_(synth.SCALE_LO, synth.SCALE_HI + 1, generator=g)
    return pool


def bench_gemv(A):
    """The reference-named decode GEMV (q80.mxfp4_kernels.mxfp4_gemv, the VALU kernel k_mxfp4_gemv) at configuration
    1's shapes on a resident store-layout pool (raw E8M0 rows, or PS4 with --layout ps4): per layer, the 4 routed
    slots' gate_up rows [4 x 5760 x 2880] against one shared x row, then their down rows [4 x 2880 x 2880] against
    per-expert rows (per_expert_x=True), the reference's unfused decode call pattern (mxfp4_kernels.py:474-489).
    Timed: graph replays of 36 layers; per launch: events that the dispatches stamp themselves (eager steps queued
    behind a spin kernel)."""
    import torch

    from neural_amd import _native as N
    from neural_amd import synth
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, mxfp4_pool_views
    from neural_amd.q80.mxfp4_kernels import mxfp4_gemv

    dev = torch.device("cuda", 0)
    layout = "ps4" if A.layout == "ps4" else "raw"
    L = GPTOSS_LAYOUT_PS4 if layout == "ps4" else GPTOSS_LAYOUT
    n_slots = N_LAYERS * N_EXPERTS
    log(f"gemv: allocating {layout} pool {n_slots} x {L.slot_bytes} B = {n_slots * L.slot_bytes / 1e9:.1f} GB")
    pool = store_pool(dev, n_slots, layout, 77)
    gb, db, gs, ds = mxfp4_pool_views(pool, L)
    rng = np.random.default_rng(4747)
    n_sets = A.sets
    ids_np, _ = routing_sets(rng, n_sets, 1)
    slots = torch.from_numpy(ids_np[:, :, 0, :] + np.arange(N_LAYERS)[None, :, None] * N_EXPERTS).to(dev)
    x = synth.bf16_normal(rng, (N_LAYERS, 1, H)).to(dev)
    hh = synth.bf16_normal(rng, (N_LAYERS, TOPK, H)).to(dev)

    def step(s, ev=None):
        """One configuration-1 step through mxfp4_gemv; with ev, the same launches through the C ABI with dispatch-
        stamped events (ev[l] = 4 recorded events: gate_up start/end, down start/end)."""
        for l in range(N_LAYERS):
            if ev is None:
                mxfp4_gemv(x[l], gb, gs, slots[s, l])
                mxfp4_gemv(hh[l], db, ds, slots[s, l], per_expert_x=True)
                continue
            for k, (xx, bl, sc, n) in enumerate(((x[l], gb, gs, 5760), (hh[l], db, ds, 2880))):
                N.call("na_mxfp4_gemv", xx.data_ptr(), k, bl.data_ptr(), bl.stride(0), sc.data_ptr(), sc.stride(0),
                       int(layout == "ps4"), slots[s, l].data_ptr(), TOPK, None, 0, outs[k].data_ptr(), n, H, 2,
                       N.events_array(ev[l][2 * k:2 * k + 2]), N.stream(dev))

    outs = (torch.empty(TOPK, 5760, dtype=torch.bfloat16, device=dev),
            torch.empty(TOPK, 2880, dtype=torch.bfloat16, device=dev))
    step(0)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        step(0)
    torch.cuda.current_stream().wait_stream(cs)
    graphs = []
    for s in range(n_sets):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            step(s)
        graphs.append(gr)
    for i in range(A.warmup):
        graphs[i % n_sets].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(A.steps):
        graphs[i % n_sets].replay()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el / A.steps * 1e3
    step_bytes = N_LAYERS * TOPK * SLOT_ALGO_BYTES
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(N_LAYERS)]
    for row in ev:
        for e in row:
            e.record()
    torch.cuda.synchronize()
    gu_ms = dn_ms = 0.0
    R = max(A.roofline_steps, 1)
    for r in range(R):
        queue_behind_spin(torch)
        step(r % n_sets, ev)
        torch.cuda.synchronize()
        for l in range(N_LAYERS):
            gu_ms += ev[l][0].elapsed_time(ev[l][1])
            dn_ms += ev[l][2].elapsed_time(ev[l][3])
    n = R * N_LAYERS
    gu_us, dn_us = gu_ms / n * 1e3, dn_ms / n * 1e3
    gu_gbps = TOPK * GATE_UP_BYTES / (gu_us * 1e-6) / 1e9
    dn_gbps = TOPK * DOWN_BYTES / (dn_us * 1e-6) / 1e9
    log(f"gemv {layout}: {ms_step:.3f} ms/step ({step_bytes / (ms_step * 1e-3) / 1e9:.0f} GB/s whole step); "
        f"gate_up {gu_us:.2f} us ({gu_gbps:.0f} GB/s), down {dn_us:.2f} us ({dn_gbps:.0f} GB/s)")
    res = {"metric": "MXFP4 expert GEMV HBM GB/s (reference-named mxfp4_gemv, VALU kernel, decode shapes)",
           "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": A.steps,
           "warmup": A.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
           "config": {"workload": f"config1 shapes through mxfp4_gemv: 36 layers x (gate_up [4 x 5760 x 2880] + down "
                                  f"[4 x 2880 x 2880]) per step, {layout} store-layout pool (61 GB), random top-4 "
                                  f"routing from {n_sets} sets", "layout": layout,
                      "gate_up_avg_launch_us": round(gu_us, 3), "down_avg_launch_us": round(dn_us, 3),
                      "down_gbps": round(dn_gbps, 1), "down_frac": round(dn_gbps / HBM_PEAK_GBS, 4)},
           "roofline": {"bound": "hbm", "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gu_gbps / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_mxfp4_gemv (gate_up)",
                        "algorithmic_bytes_per_launch": TOPK * GATE_UP_BYTES},
           "cpu_baseline": None}
    print(json.dumps(res), flush=True)


def bench_mfma(A):
    """Matrix-core issue rate on this GPU: a grid of 256-thread workgroups each running chains of four independent
    MFMAs on register operands (na_bench_mfma_rate): kind 0 the scaled 16x16x128 FP8 x FP4 instruction the prefill
    and decode tile kernels use, kind 1 the bf16 16x16x32 one.  Timed with events the dispatch itself stamps."""
    import torch

    from neural_amd import _native as N

    dev = torch.device("cuda", 0)
    blocks = 256 * 8
    out = torch.empty(blocks * 4, dtype=torch.float32, device=dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    res = {}
    for kind, name, flop, peaks in ((0, "scaled_f8f6f4_16x16x128 (E4M3 x E2M1)", 2 * 16 * 16 * 128,
                                     {"fp8": 5.0e15, "fp4": 10.1e15}),
                                    (1, "bf16_16x16x32", 2 * 16 * 16 * 32, {"bf16": 2.5e15})):
        iters = 4096
        N.call("na_bench_mfma_rate", kind, blocks, iters, out.data_ptr(), None, N.stream(dev))
        torch.cuda.synchronize()
        best = None
        for _ in range(5):
            N.call("na_bench_mfma_rate", kind, blocks, 20000, out.data_ptr(), N.events_array(ev), N.stream(dev))
            torch.cuda.synchronize()
            ms = ev[0].elapsed_time(ev[1])
            best = ms if best is None else min(best, ms)
        total = blocks * 4 * 20000 * 4 * flop
        rate = total / (best * 1e-3)
        res[name] = {"ms": round(best, 4), "tflops": round(rate / 1e12, 1),
                     **{f"frac_{k}_peak": round(rate / v, 4) for k, v in peaks.items()}}
        log(f"mfma {name}: {rate / 1e12:.0f} TFLOP/s ({best:.3f} ms)")
    k0 = res["scaled_f8f6f4_16x16x128 (E4M3 x E2M1)"]["tflops"]
    print(json.dumps({"metric": "MFMA issue rate", "value": k0, "unit": "TFLOP/s", "n_gpus": 1, "steps": 5,
                      "higher_is_better": True, "dtype": "f8f6f4", "data": "synthetic",
                      "config": {"workload": f"{blocks} workgroups x 4 waves x 20000 rounds of 4 independent MFMAs",
                                 "kinds": res,
                                 "exact_product_rate_tflops": round(k0 / 2, 1),
                                 "note": "the prefill kernels issue two scaled MFMAs (E4M3 hi and lo) per exact "
                                         "bf16 x E2M1 product, so half kind 0's rate is their ceiling"}}),
          flush=True)


def expert_gemm_sweep(rx, dev, sizes=(64, 128, 330, 1024, 2048), reps=5):
    """Per-expert GEMM rates of the prefill kernels: every token routed to the same four experts (M pairs each), so
    each expert's gate_up and down products are M x 5760 x 2880 and M x 2880 x 2880; launch durations from
    dispatch-stamped events."""
    import torch

    from neural_amd import synth

    out = {}
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(10)]
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    rng = np.random.default_rng(330)
    for M in sizes:
        ids = torch.tensor([[5, 17, 64, 101]] * M, dtype=torch.int64, device=dev)
        wts = torch.full((M, TOPK), 0.25, dtype=torch.bfloat16, device=dev)
        x = synth.bf16_normal(rng, (M, H)).to(dev)
        y = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
        rx.forward_prefill(0, x, ids, wts, out=y)
        torch.cuda.synchronize()
        gu = dn = 0.0
        for _ in range(reps):
            queue_behind_spin(torch, 2.0)
            rx.forward_prefill(0, x, ids, wts, out=y, events=ev)
            torch.cuda.synchronize()
            gu += ev[4].elapsed_time(ev[5]) / reps
            dn += ev[6].elapsed_time(ev[7]) / reps
        gf = 2.0 * TOPK * M * 5760 * 2880
        df = 2.0 * TOPK * M * 2880 * 2880
        out[str(M)] = {"gate_up_us": round(gu * 1e3, 2), "down_us": round(dn * 1e3, 2),
                       "gate_up_tflops": round(gf / (gu * 1e-3) / 1e12, 1),
                       "down_tflops": round(df / (dn * 1e-3) / 1e12, 1),
                       "gate_up_frac_exact": round(gf / (gu * 1e-3) / 2.5e15, 4),
                       "down_frac_exact": round(df / (dn * 1e-3) / 2.5e15, 4)}
        log(f"expert GEMM M={M}: gate_up {gu * 1e3:.1f} us ({out[str(M)]['gate_up_tflops']} TFLOP/s), "
            f"down {dn * 1e3:.1f} us ({out[str(M)]['down_tflops']} TFLOP/s)")
    return out


def bench_experts(A):
    """Configuration 1 alone, on a pool of any layout (t950: MFMA kernels; raw / ps4: the VALU kernels)."""
    import torch

    from neural_amd import synth, tiles
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, GPTOSS_LAYOUT_T950

    dev = torch.device("cuda", 0)
    if A.calib_copy_mb:
        src = torch.empty(A.calib_copy_mb << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    L = {"t950": GPTOSS_LAYOUT_T950, "raw": GPTOSS_LAYOUT, "ps4": GPTOSS_LAYOUT_PS4}[A.layout]
    n_slots = N_LAYERS * N_EXPERTS
    log(f"allocating pool {n_slots} x {L.slot_bytes} B = {n_slots * L.slot_bytes / 1e9:.1f} GB ({L.weight_repr})")
    if A.layout == "t950":
        pool = synth.t950_pool_device(n_slots, dev, 4242)
    else:
        pool = store_pool(dev, n_slots, A.layout, 1234)
    torch.cuda.synchronize()
    log("pool filled")
    bias_gu = torch.zeros(n_slots, L.gate_up_n, dtype=torch.bfloat16, device=dev)
    bias_dn = torch.zeros(n_slots, L.down_n, dtype=torch.bfloat16, device=dev)
    rx = ResidentExperts(pool, L, bias_gu, bias_dn, gu_pairs_per_wave=A.gu_pairs, dn_pairs_per_wave=A.dn_pairs,
                         k_split=A.k_split, combine_in_down=A.down != "expert")
    B = A.batch
    m = measure_experts(rx, dev, B, A.steps, A.warmup, A.sets, A.roofline_steps)
    c1 = config1_summary(m, L, B)
    if not A.no_batch_sweep:
        c1["batch_sweep"] = batch_sweep(rx, dev, A, B)
    kname = ({"experts": "k_moe_one_t950", "gate_up": "k_moe_gate_up_t950"}[m["dom"]] if A.layout == "t950"
             else "k_moe_gate_up")
    traffic, why = measured_traffic(kname, A.layout, B, effective_k_split(A.k_split, B))
    log(f"traffic: {traffic} ({why})")
    top = m["kern"][m["dom"]]
    roofline = {"bound": "hbm", "achieved": round(top["gbps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(top["gbps"] / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kname,
                "avg_launch_us": round(top["avg_us"], 3), "algorithmic_bytes_per_launch": int(m["per_launch"])}
    cpu = None
    if not A.skip_cpu:
        try:
            cpu = cpu_baselines(pool, m["ids_np"][0], A.cpu_seconds)
        except Exception as e:
            cpu = {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference", "sample": f"unavailable: {e}"}
    res = {"metric": METRIC, "value": round(m["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": A.steps,
           "warmup": A.warmup, "ms_per_step": round(m["ms_step"], 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "numerics": NUMERICS, "data": "synthetic", "config": c1,
           "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (decode / model: greedy tokens, default 256; experts: 200)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1, help="experts workload: decode batch (1..8)")
    ap.add_argument("--layout", choices=("t950", "raw", "ps4"), default="t950",
                    help="experts workload: resident slot layout, gfx950 tiles (MFMA kernels) or the store layouts "
                         "(VALU kernels)")
    ap.add_argument("--k-split", type=int, default=0,
                    help="t950 gate_up: waves per workgroup splitting K (4, 8; 0 = automatic: 4)")
    ap.add_argument("--down", choices=("combine", "expert"), default="combine",
                    help="t950, batch 1: gate_up then down + combine (two launches, default), or expert-major down "
                         "+ a combine kernel (expert)")
    ap.add_argument("--sets", type=int, default=16, help="routing sets (graphs) cycled over the steps")
    ap.add_argument("--roofline-steps", type=int, default=20)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--no-batch-sweep", action="store_true",
                    help="skip the shorter runs of configuration 1's other batch sizes")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--gu-pairs", type=int, default=4, help="VALU gate_up row pairs per wavefront (1, 2, 4)")
    ap.add_argument("--dn-pairs", type=int, default=2, help="VALU down row pairs per wavefront (1, 2, 4)")
    ap.add_argument("--workload", choices=("decode", "experts", "attention", "prefill", "model", "gemv", "mfma"),
                    default="decode",
                    help="decode: configuration 4 (value) + configuration 1 on one pool (the default); experts: "
                         "configuration 1 alone; prefill: configuration 2; attention: configuration 3; model: "
                         "configuration 4 alone; gemv: the reference-named mxfp4_gemv at configuration 1's shapes; "
                         "mfma: matrix-core issue rate")
    ap.add_argument("--tokens", type=int, default=2048, help="prefill: prompt tokens")
    ap.add_argument("--context", type=int, default=4096, help="decode / model: context tokens before the timed decode")
    ap.add_argument("--context-mode", choices=("prefill", "decode"), default="prefill",
                    help="model: build the context by prompt processing (default) or token by token through the "
                         "decode step")
    ap.add_argument("--prefill-chunk", type=int, default=4096, help="model: prompt block size of the prefill")
    ap.add_argument("--prompt-gemms", choices=("tuned", "default"), default="tuned",
                    help="model: the context prefill's library GEMMs take the committed TunableOp choices (tuned) or "
                         "hipBLASLt's default heuristic")
    ap.add_argument("--attn-split", type=int, default=0,
                    help="model: key chunks of full-attention layers (0: attention.auto_split of the cache rows)")
    ap.add_argument("--sliding-split", type=int, default=1, help="model: key chunks of sliding-window layers")
    ap.add_argument("--unfused-attn", action="store_true",
                    help="model: QKV, attention, o_proj and router as four launches per layer instead of one")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="experts: run one device-to-device copy of this many MB first (a known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run)")
    A = ap.parse_args()
    if A.steps is None:
        A.steps = 256 if A.workload in ("decode", "model") else 200
    if A.gpus != 1:
        print(f"bench.py: this build runs on one GPU per process and measures one GPU; --gpus {A.gpus} is not "
              f"supported (sharding across GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if not 1 <= A.batch <= 8:
        sys.exit("--batch must be in [1, 8]")
    return {"attention": bench_attention, "prefill": bench_prefill, "model": bench_model, "experts": bench_experts,
            "decode": bench_decode, "gemv": bench_gemv, "mfma": bench_mfma}[A.workload](A)


if __name__ == "__main__":
    main()
