#!/usr/bin/env python
"""Abridged decode-attention benchmark on one MI355X.

Workload (the saturated serving decode stress): Qwen3-4B attention shape -- 36 layers in 6 KV-cache groups with the
per-layer code quotas 256/128/64 (6/18/12 layers), 32 query / 8 KV heads, head_dim 128, bf16, pages of 16 slots --
batch 256 with total content lengths T ~ U[2048, 32768] (32K cap) and prompts P ~ U[128, 1024]. Every request's
history (prefill chunks, code steps, block-boundary compactions) is replayed through the compaction planner to
build the page tables; K/V pages and queries are N(0,1) from the seed.

A step = one decode step of the attention path for all 36 layers: KV append of the query token's K/V at its slot,
then split-KV decode attention over the layer's group page table. Inputs are resident in HBM before timing.
Prints one JSON line (rank 0).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def profiled_traffic(name: str):
    """HBM bytes per launch of a kernel on this workload, from the committed rocprofv3 PMC summary
    profiles/<name> (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, calibrated on a plain 4 GiB copy); None if absent."""
    try:
        with open(os.path.join(PROFILES, name)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def profiled_mfma_util(name: str):
    """rocprofv3 MfmaUtil of a kernel on this workload (fraction of SIMD cycles the matrix cores are busy), from the
    committed PMC summary profiles/<name>; None if absent."""
    try:
        with open(os.path.join(PROFILES, name)) as f:
            for line in f:
                if line.startswith("mfma_util_rocprof:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 300 for serving, about 11 s of GPU work, so that a sampler of the "
                         "GPU's busy state running beside the bench sees the timed region; 10 otherwise)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=None, help="default: 64 for full_model, 256 otherwise")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--split-pages", type=int, default=None,
                    help="pages per decode split (default: ops.auto_split_pages per launch: 48, 40 or 32)")
    ap.add_argument("--workload", choices=["serving", "saturated", "full_model", "config1", "prefill", "prefill_bwd",
                                           "compaction", "packed", "code_step", "copy"],
                    default="serving")
    ap.add_argument("--code-requests", type=int, default=1,
                    help="code_step: requests coding in one launch (the serving stress averages ~0.5 per step)")
    ap.add_argument("--serial-code-step", action="store_true",
                    help="serving: run each layer's code step after its decode on one stream (for an A/B against "
                         "the default, the code step on a second stream)")
    ap.add_argument("--code-target-blocks", type=int, default=None,
                    help="serving: workgroups a code step's key splits aim at (default: a quarter of the compute units "
                         "with the code step on its own stream, every compute unit with --serial-code-step)")
    ap.add_argument("--retain-tail", type=int, default=0,
                    help="prefill / prefill_bwd: retained tail of T content rows per block (default 0)")
    ap.add_argument("--tail-policy", default="static", choices=("static", "rolling", "sticky"),
                    help="prefill / prefill_bwd: the retained tail's policy (default static)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seqs", type=int, default=8)
    args = ap.parse_args()
    if args.batch is None:
        args.batch = 64 if args.workload == "full_model" else 256
    if args.steps is None:
        args.steps = 300 if args.workload == "serving" else 10
    return args


def cpu_threads(torch) -> dict:
    """Give torch every host core this process may use and describe the host for the cpu_baseline record. The
    count is the CPU affinity set (on a shared GPU host that is this job's share, not the machine), capped by
    OMP_NUM_THREADS when the launcher sets it; nproc and the CPU model are recorded beside it."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    torch.set_num_threads(n)
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cores": torch.get_num_threads(), "nproc": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "omp_num_threads": omp or None, "cpu": model}


def copy_bandwidth(torch, gb=8.0):
    """Measured device copy bandwidth (read + write bytes / time) of a large torch copy."""
    n = int(gb * 1e9) // 2
    a = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    s.record()
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / reps
    del a, b
    torch.cuda.empty_cache()
    return 2 * n * 2 / t / 1e9


def cpu_baseline(torch, state, caches_gpu, qs, scale, n_seqs, target_s=12.0):
    """The reference's decode arithmetic (oracle.decode.decode_ref_torch) on the host cores, on a sample of the
    same workload: the first n_seqs requests, one layer of each group (every layer of a group has the same rows).
    Returns tokens/s for the full 36-layer step of those requests."""
    from oracle.decode import decode_ref_torch

    G = len(state.groups)
    layers = [state.groups[g][0] for g in range(G)]
    samples = []
    for l in layers:
        g = state.layer_group[l]
        tab = state.block_tables[g][:n_seqs]
        sl = state.seq_lens[g][:n_seqs]
        used = np.unique(np.concatenate([tab[b, : -(-int(sl[b]) // 16)] for b in range(n_seqs)]))
        remap = {int(p): i for i, p in enumerate(used)}
        cache = caches_gpu[state.layer_slot[l]][torch.from_numpy(used).cuda()].cpu()
        ctab = np.zeros_like(tab)
        for b in range(n_seqs):
            n = -(-int(sl[b]) // 16)
            ctab[b, :n] = [remap[int(p)] for p in tab[b, :n]]
        samples.append((qs[l][:n_seqs].cpu(), cache, torch.from_numpy(ctab), torch.from_numpy(sl.astype(np.int64))))
    for q, c, t, s in samples:                               # warm-up
        decode_ref_torch(q, c, t, s, scale)
    reps, t0 = 0, time.perf_counter()
    while True:
        for q, c, t, s in samples:
            decode_ref_torch(q, c, t, s, scale)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    per_step_6 = el / reps
    num_layers = state.num_layers
    step_time = per_step_6 * num_layers / G                  # each group holds num_layers / G identical layers
    return n_seqs / step_time, reps, el


# A single-launch workload reaches its steady rate only after ~15 launches (~20 ms) of sustained work on an idle GPU:
# measured on one box, ten launches after three warm-up launches averaged 1486 us, every later batch 1302-1323 us.
# The masked-prefill lines therefore warm up for at least this many launches before the timed ones.
MIN_PREFILL_WARMUP = 30


def bench_prefill(args, torch):
    """Teacher-forced prefill under the compression mask, B=4, N=16 blocks of [512 content | 128 codes]
    (S0 = 10240), 512-token raw prompt, 32 q / 8 kv heads, d128, bf16. FLOPs = 4 * D * visible pairs * heads * B."""
    from abridgekv_amd import ops
    from abridgekv_amd.workloads import visible_pairs_prompt_block

    B, C, K, N, plen, T = 4, 512, 128, 16, 512, args.retain_tail
    P = args.tail_policy if T else "static"
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    pl = torch.full((B,), plen, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    warmup = max(args.warmup, MIN_PREFILL_WARMUP)
    for _ in range(warmup):
        ops.prefill_masked_attention(q, k, v, C, K, N, prompt_len=pl, out=out, lse=lse, retain_tail=T,
                                     tail_policy=P)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        ops.prefill_masked_attention(q, k, v, C, K, N, prompt_len=pl, out=out, lse=lse, retain_tail=T,
                                     tail_policy=P)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / args.steps
    flops = 4.0 * 128 * visible_pairs_prompt_block(C, K, N, T, P) * 32 * B
    tflops = flops / t / 1e12
    cpu = None if args.no_cpu_baseline or T else prefill_cpu_baseline(torch, C, K, plen, flops, B, S0)
    return {
        **({"cpu_baseline": cpu} if cpu else {}),
        "metric": "masked teacher-forced prefill TFLOP/s (visible QK+PV flops); % of bf16 dense MFMA peak",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": warmup,
        "ms_per_step": t * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) q/k/v from the seed",
        "config": {"workload": f"masked prefill B={B}, N={N} blocks of [{C} content | {K} codes], S0={S0}, "
                               f"raw prompt {plen}, 32q/8kv heads, d128"
                               + (f", {P} retained tail {T}" if T else ""), "global_batch": B, "seq_len": S0},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": tflops / 2500.0,
                     "traffic": profiled_traffic("prefill_masked_b4_s10240_pmc_traffic.md"),
                     "traffic_source": "profiles/prefill_masked_b4_s10240_pmc_traffic.md", "kernel": "prefill_masked_kernel",
                     "alg_flops_per_launch": flops, "avg_launch_us": t * 1e6,
                     "mfma_util_rocprof": profiled_mfma_util("prefill_masked_b4_s10240_pmc_mfma.md"),
                     "mfma_util_source": "profiles/prefill_masked_b4_s10240_pmc_mfma.md (MfmaUtil)"},
    }


def prefill_cpu_baseline(torch, C, K, plen, flops_full, B_full, S0_full, N_cpu=4, target_s=10.0):
    """The reference's dense masked attention (oracle.prefill.dense_masked_attention_ref_torch: bf16 scores with an
    additive mask, fp32 softmax, gen_compress.py:1176-1179) on the host cores, on one sequence of N_cpu blocks of the
    same geometry. The dense path costs S0^2 per sequence and head whatever the mask, so the full workload's time is
    the sample's x B x (S0_full / S0_cpu)^2; value = the full workload's visible-pair FLOPs / that time."""
    from oracle import prefill as op

    host = cpu_threads(torch)
    S = N_cpu * (C + K)
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 32, S, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 8, S, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 8, S, 128), generator=g).to(torch.bfloat16)
    mask = torch.from_numpy(op.arith_mask(C, K, N_cpu, [plen])[0])
    op.dense_masked_attention_ref_torch(q, k, v, mask, 128 ** -0.5)          # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        op.dense_masked_attention_ref_torch(q, k, v, mask, 128 ** -0.5)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    t_full = el / reps * B_full * (S0_full / S) ** 2
    return {"value": flops_full / t_full / 1e12, "unit": "TFLOP/s", "kind": "port", **host,
            "sample": f"one sequence of {N_cpu} blocks [{C} | {K}] (S0={S}, raw prompt {plen}), {reps} reps in "
                      f"{el:.1f} s ({el / reps * 1e3:.0f} ms each), scaled to B={B_full}, S0={S0_full} by the dense "
                      f"path's B x S0^2 cost; torch CPU bf16 restatement of gen_compress.py:1176-1179"}


def bench_prefill_bwd(args, torch):
    """Backward of the B=4, S0=10240 masked prefill (gradients of q, k, v through the compression mask; what
    training CompressLM runs per layer after the forward). FLOPs = 10 * D * visible pairs * heads * B: the five products of the attention backward
    (S recomputed, dP, dV, dK, dQ) over the visible pairs, 2.5x the forward's; the kernels execute seven (the dQ and
    the dK/dV kernels each recompute S and dP)."""
    from abridgekv_amd import ops
    from abridgekv_amd.workloads import visible_pairs_prompt_block

    B, C, K, N, plen, T = 4, 512, 128, 16, 512, args.retain_tail
    P = args.tail_policy if T else "static"
    S0 = N * (C + K)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, S0, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    dout = torch.randn((B, S0, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    pl = torch.full((B,), plen, dtype=torch.int32, device=dev)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(q, k, v, C, K, N, prompt_len=pl, lse=lse, retain_tail=T, tail_policy=P)
    warmup = max(args.warmup, MIN_PREFILL_WARMUP)
    for _ in range(warmup):
        ops.prefill_masked_attention_backward(q, k, v, out, lse, dout, C, K, N, prompt_len=pl, retain_tail=T,
                                              tail_policy=P)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        ops.prefill_masked_attention_backward(q, k, v, out, lse, dout, C, K, N, prompt_len=pl, retain_tail=T,
                                              tail_policy=P)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / args.steps
    flops = 10.0 * 128 * visible_pairs_prompt_block(C, K, N, T, P) * 32 * B
    tflops = flops / t / 1e12
    return {
        "metric": "masked teacher-forced attention backward TFLOP/s (visible-pair flops, 2.5x forward); % of bf16 "
                  "dense MFMA peak",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": warmup,
        "ms_per_step": t * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) q/k/v/dout from the seed",
        "config": {"workload": f"masked prefill backward B={B}, N={N} blocks of [{C} content | {K} codes], "
                               f"S0={S0}, raw prompt {plen}, 32q/8kv heads, d128"
                               + (f", {P} retained tail {T}" if T else ""), "global_batch": B, "seq_len": S0},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s", "frac": tflops / 2500.0,
                     "traffic": profiled_traffic("prefill_masked_bwd_b4_s10240_pmc_traffic.md"),
                     "traffic_source": "profiles/prefill_masked_bwd_b4_s10240_pmc_traffic.md (the three kernels)",
                     "kernel": "prefill_bwd_prep_kernel + prefill_bwd_dq_kernel + prefill_bwd_dkv_kernel",
                     "alg_flops_per_launch": flops,
                     "avg_launch_us": t * 1e6},
    }


def bench_compaction(args, torch):
    """Compaction: 64 sequences each close one 512-token block (256 code rows computed) in one step; Qwen3-4B shape,
    36 layers in 6 quota groups, page 16, seeded fragmented free list. Timed: the planner step (the span removals with
    the reference's bookkeeping -- spans, page lists, truncations, free queue -- without the reference-format op
    rows the fused path does not execute), the move-list preparation (the planner writes per-run descriptors into
    pinned memory, one copy to the device, and abkv_moves_expand writes the move lists there) and the fused device
    moves; algorithmic bytes = 2 x (kept code rows x 4096 B) summed over layers. The host-written move lists of the
    same step (abkv_planner_take_moves_packed + upload) are timed beside it."""
    from abridgekv_amd import ops, worker, workloads

    B = 64
    st = workloads.build_compaction_state(B, seed=args.seed, op_rows=False)      # the fused path needs no op rows
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    n_tensors = max(len(g) for g in st.groups)
    caches = []
    for _ in range(n_tensors):
        c = torch.empty(ops.kv_cache_shape(st.num_pages), dtype=torch.bfloat16, device=dev)
        c.normal_(generator=gen)
        caches.append(c)
    by_group = [[caches[i] for i in range(len(layers))] for layers in st.groups]
    st.planner.reserve_outputs(0, 0, B)
    st_host = workloads.build_compaction_state(B, seed=args.seed, op_rows=False)   # the same step, host-packed lists
    st_host.planner.reserve_outputs(0, 0, B)
    uploader = worker.MoveUploader(dev, capacity=8 << 20)     # pinned staging, sized once (8 Mi int32)
    run_uploader = worker.MoveRunUploader(dev, capacity=1 << 20, out_capacity=8 << 20)
    for up in (uploader, run_uploader):                        # first use pays one-off runtime setup
        warm = workloads.build_compaction_state(B, seed=args.seed + 1, op_rows=False)
        warm.planner.apply_events(warm.pending)
        up.take(warm.planner)
    torch.cuda.synchronize()
    del warm
    t0 = time.perf_counter()
    st.planner.apply_events(st.pending)                        # the planner step (host C++), reference semantics
    plan_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    _, prepared = run_uploader.take(st.planner)                # run descriptors uploaded, move lists written on device
    torch.cuda.synchronize()
    prep_s = time.perf_counter() - t0
    st_host.planner.apply_events(st_host.pending)
    t0 = time.perf_counter()
    _, prepared_host = uploader.take(st_host.planner)          # move lists written into pinned memory, one upload
    torch.cuda.synchronize()
    prep_host_s = time.perf_counter() - t0
    for (ga, oa, sa, fa), (gb, ob, sb, fb) in zip(prepared, prepared_host):   # the two paths give the same lists
        if ga != gb or not (torch.equal(oa, ob) and torch.equal(sa, sb) and torch.equal(fa, fb)):
            raise RuntimeError("device-expanded move lists differ from the host-written ones")
    n_fused = sum(int(o.shape[0]) + int(f.shape[0]) for _, o, _, f in prepared)
    st_ref = workloads.build_compaction_state(B, seed=args.seed)
    outs = st_ref.compact()                                    # same step, reference-format op dict for comparison
    ref_rows = sum(len(b) for v in outs.kv_copy_operations.values() for g in v for b in g)
    layers_per_group = len(st.groups[0])
    alg_bytes = 2 * n_fused * layers_per_group * 4096
    for _ in range(args.warmup):
        worker.launch_moves(prepared, by_group)
    torch.cuda.synchronize()
    events = []
    for _ in range(args.steps):
        worker.launch_moves(prepared, by_group, events)
    torch.cuda.synchronize()
    n_launch = len(events)
    t = sum(s_.elapsed_time(e_) for s_, e_ in events) / 1e3 / args.steps
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        worker.execute_kv_copy_operations(outs.kv_copy_operations, by_group, check=False)
    e.record()
    torch.cuda.synchronize()
    t_ref = s.elapsed_time(e) / 1e3 / args.steps
    gbps = alg_bytes / t / 1e9
    # the copy ceiling for these bytes: plain device copies of one launch's moved bytes (read + write each once),
    # each from the next of 16 slices of a buffer far larger than the 256 MB last-level cache, as the mover's pages are
    n_copy = int(alg_bytes / (n_launch / args.steps)) // 2
    n_el = n_copy // 2
    src_buf = torch.ones(16 * n_el, dtype=torch.bfloat16, device=dev)
    dst_buf = torch.empty_like(src_buf)
    for i in range(max(args.warmup, 1)):
        dst_buf[i * n_el:(i + 1) * n_el].copy_(src_buf[i * n_el:(i + 1) * n_el])
    torch.cuda.synchronize()
    reps = 16 * max(1, args.steps // 4)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(reps):
        sl = slice((i % 16) * n_el, (i % 16 + 1) * n_el)
        dst_buf[sl].copy_(src_buf[sl])
    e.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * n_copy / (s.elapsed_time(e) / 1e3 / reps) / 1e9
    del src_buf, dst_buf
    probe = same_pattern_probe(torch, prepared, by_group, st.num_pages, args)
    probe["mover_frac_of_probe"] = gbps / probe["gbps"]
    cpu = None if args.no_cpu_baseline else compaction_cpu_baseline(torch, B, args.seed, layers_per_group)
    return {
        **({"cpu_baseline": cpu} if cpu else {}),
        "metric": "block-boundary compaction: sequences compacted per second (64 seqs x 36 layers)",
        "value": B / (t + plan_s + prep_s), "unit": "sequences/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": (t + plan_s + prep_s) * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 (row copies)", "data": "synthetic histories replayed through the planner",
        "config": {"workload": "compaction: 64 sequences close a 512-token block (256 code rows), Qwen3-4B 36 layers "
                               "/ 6 quota groups, page 16, seeded free list", "global_batch": B},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / HBM_PEAK_GBPS,
                     "traffic": profiled_traffic("kv_move_compaction_64seq_pmc_traffic.md"),
                     "traffic_source": "profiles/kv_move_compaction_64seq_pmc_traffic.md",
                     "kernel": "kv_move_kernel (fused moves)",
                     "alg_bytes_per_launch": alg_bytes / (n_launch / args.steps),
                     "avg_launch_us": t / (n_launch / args.steps) * 1e6},
        "copy_ceiling": {"gbps": copy_gbps, "bytes_read": n_copy, "bytes_written": n_copy,
                         "what": "torch device copies of one move launch's bytes, contiguous, cycling through 16 "
                                 "slices of a buffer larger than the last-level cache",
                         "mover_frac_of_copy": gbps / copy_gbps},
        "same_pattern_probe": probe,
        "planner_ms": plan_s * 1e3, "move_list_prep_ms": prep_s * 1e3, "host_packed_upload_ms": prep_host_s * 1e3,
        "device_moves_ms": t * 1e3,
        "reference_format_moves_ms": t_ref * 1e3, "reference_format_rows": ref_rows, "fused_rows": n_fused,
    }


def same_pattern_probe(torch, prepared, by_group, num_pages, args):
    """Ceiling of the mover's access pattern: abkv_probe_row_copy (libabridgekv_probes.so) copies the same rows of the
    same layers -- every (src page, slot) -> (dst page, slot) of each group launch, 4 KiB each -- into a second set of
    caches, all ops in parallel (no segment order to keep). Swept over 4, 8 and 16 rows per workgroup; the best is
    the ceiling. Returns its GB/s (read + write bytes / time of the same launches) and the sweep."""
    import ctypes as C
    from pathlib import Path

    from abridgekv_amd import ops

    path = Path(__file__).resolve().parent / "abridgekv_amd" / "libabridgekv_probes.so"
    lib = C.CDLL(str(path))
    fn = lib.abkv_probe_row_copy
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_long, C.c_long, C.c_int, C.c_int,
                   C.c_int, C.c_int, C.c_void_p]
    n_tensors = max(len(c) for c in by_group)
    dst = [torch.empty_like(by_group[0][0]) for _ in range(n_tensors)]
    launches, total_bytes = [], 0
    for gid, ord_d, _, free_d in prepared:
        ops_d = torch.cat([ord_d, free_d])
        caches = by_group[gid]
        for lo in range(0, len(caches), 16):
            src_l = caches[lo: lo + 16]
            srcs = (C.c_void_p * len(src_l))(*[c.data_ptr() for c in src_l])
            dsts = (C.c_void_p * len(src_l))(*[d.data_ptr() for d in dst[:len(src_l)]])
            launches.append((srcs, dsts, len(src_l), ops_d))
            total_bytes += 2 * ops_d.shape[0] * len(src_l) * 2 * ops.SLOT_BYTES
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(rows, events=None):
        for srcs, dsts, n_l, ops_d in launches:
            if events is not None:
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
            rc = fn(srcs, dsts, n_l, C.c_void_p(ops_d.data_ptr()), int(ops_d.shape[0]), ops.PAGE_BYTES,
                    ops.HALF_BYTES, ops.SLOT_BYTES, num_pages, ops.PAGE, rows, stream)
            if rc != 0:
                raise RuntimeError(f"abkv_probe_row_copy failed: {rc}")
            if events is not None:
                e.record()
                events.append((s, e))

    sweep = {}
    for rows in (4, 8, 16):                                    # events around every launch, as for the mover
        for _ in range(max(args.warmup, 1)):
            run(rows)
        torch.cuda.synchronize()
        events = []
        for _ in range(args.steps):
            run(rows, events)
        torch.cuda.synchronize()
        t = sum(s_.elapsed_time(e_) for s_, e_ in events) / 1e3 / args.steps
        sweep[rows] = total_bytes / t / 1e9
    del dst
    best = max(sweep, key=sweep.get)
    return {"gbps": sweep[best], "rows_per_workgroup": best, "sweep_gbps": sweep, "bytes_per_step": total_bytes,
            "what": "the same (layer, src slot, dst slot) rows copied into a second cache set, every op in parallel "
                    "(abkv_probe_row_copy)"}


def compaction_cpu_baseline(torch, B, seed, layers_per_group):
    """The reference's compaction path on the host: the sequential planner restatement (oracle.compaction.Planner:
    scheduler.py:2060-2204 with the KV manager and block pool) plans the step, then the worker's gather-then-scatter
    (oracle.compaction.execute_kv_copy_operations, gpu_model_runner.py:1194-1224) runs its op batches over 36 layer
    caches (2-byte rows of the bf16 layout) holding the pages the ops touch. Both are single-threaded, as the
    reference's scheduler is."""
    from abridgekv_amd import workloads
    from oracle import compaction as oc

    st = workloads.build_compaction_state(B, seed=seed)
    G = len(st.groups)
    oracle = oc.Planner(st.num_pages, G, 16, free_order=st.free_order)
    oracle.apply_events(st.history)
    oracle.take_step_outputs()
    t0 = time.perf_counter()
    oracle.apply_events(st.pending)
    kv_ops, _ = oracle.take_step_outputs()
    plan_s = time.perf_counter() - t0
    # compact host caches per group: only the pages the ops name, renumbered
    remapped, caches = {}, []
    for g in range(G):
        pages = sorted({p for per in kv_ops.values() for b in per[g] for op_ in b for p in (op_[0], op_[2])})
        idx = {p: i for i, p in enumerate(pages)}
        caches.append([np.full((max(1, len(pages)), 2, 16, 8, 128), g + 1, dtype=np.uint16)])
        for rid, per in kv_ops.items():
            remapped.setdefault(rid, [[] for _ in range(G)])[g] = [
                [(idx[a], o1, idx[c], o2) for a, o1, c, o2 in b] for b in per[g]]
    oc.execute_kv_copy_operations(remapped, caches)            # warm-up (first touch of the gather buffers)
    t0 = time.perf_counter()
    oc.execute_kv_copy_operations(remapped, caches)            # one layer per group; every layer moves the same rows
    move_s = (time.perf_counter() - t0) * layers_per_group
    rows = sum(len(b) for per in kv_ops.values() for g in per for b in g)
    return {"value": B / (plan_s + move_s), "unit": "sequences/s", "kind": "port", "cores": 1,
            "cpu": cpu_threads(torch)["cpu"],
            "sample": f"the whole step: {B} sequences, planner {plan_s * 1e3:.0f} ms + gather-then-scatter of "
                      f"{rows} reference-format ops per layer, timed on one layer per group and scaled x"
                      f"{layers_per_group} to {layers_per_group * G} layers: {move_s * 1e3:.0f} ms (numpy fancy "
                      f"indexing, one thread)"}


def bench_code_step(args, torch):
    """The code step of the saturated serving stress: a request whose 512-token block just filled attends its K=256
    code rows (32 q heads) to every row it holds before them (raw prompt, earlier blocks' codes), the block's 512
    content rows and the first q of its own code rows (non-causal, key limit code_start + q per group), one launch per
    layer over the 36 layers (6 groups, quotas 256/64/64/128/128/128), keys split over workgroups and merged
    (ops.paged_split_plan). Requests: the first R of the saturated workload's (T, P) draws, each at its last closed
    block b = T // 512 - 1. value = visible QK+PV FLOPs (4 * D * 256 * limit * 32 heads per request and layer) over the
    launches' event time (kernel + merge)."""
    import ctypes as C_

    from abridgekv_amd import ops, workloads
    from abridgekv_amd._lib import check, lib

    R, C, K = args.code_requests, workloads.BLOCK_C, workloads.CODES_K_MAX
    T, P = workloads.saturated_decode_lengths(256, seed=args.seed)
    T, P = [int(t) for t in T[:R]], [int(p) for p in P[:R]]
    groups, gq = workloads.quota_groups(workloads.QWEN3_4B_LAYER_QUOTAS)
    layer_quota = {l: gq[g] for g, ls in enumerate(groups) for l in ls}
    L = len(workloads.QWEN3_4B_LAYER_QUOTAS)
    blocks = [t // C - 1 for t in T]
    # physical rows before block b's code rows = the group's rows once the block's last content token is computed
    starts = [[workloads.rows_per_group((b + 1) * C, p, layer_quota[l], C) for b, p in zip(blocks, P)] for l in range(L)]
    limits = [[s + min(layer_quota[l], K) for s in starts[l]] for l in range(L)]
    need = [[-(-(s + K) // 16) for s in starts[l]] for l in range(L)]
    n_pages = sum(sum(x) for x in need) + 1
    W = max(max(x) for x in need)
    rng = np.random.default_rng(args.seed)
    perm = rng.permutation(np.arange(1, n_pages)).astype(np.int32)
    tables, at = [], 0
    for l in range(L):
        tab = np.zeros((R, W), np.int32)
        for r in range(R):
            tab[r, : need[l][r]] = perm[at: at + need[l][r]]
            at += need[l][r]
        tables.append(tab)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    cache = torch.empty(ops.kv_cache_shape(n_pages), dtype=torch.bfloat16, device=dev).normal_(generator=gen)
    q = torch.randn((R * K, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    tiles = np.array([(r, q0) for r in range(R) for q0 in range(0, K, 64)], np.int32)
    n_tiles = tiles.shape[0]
    tl = torch.from_numpy(np.ascontiguousarray(tiles.T)).to(dev)
    q_start = torch.from_numpy(np.arange(R + 1, dtype=np.int32) * K).to(dev)
    meta = [(torch.from_numpy(tables[l]).to(dev), torch.tensor(starts[l], dtype=torch.int32, device=dev),
             torch.tensor(limits[l], dtype=torch.int32, device=dev), ops.paged_split_plan(n_tiles, max(limits[l])))
            for l in range(L)]
    ws_bytes = max((lib().abkv_paged_prefill_workspace_size(R * K, m[3][0]) for m in meta if m[3][0] > 1), default=0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    scale = ops.default_scale()
    stream = C_.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: C_.c_void_p(t.data_ptr())

    def launch(l):
        bt, ks, kl, (n_sp, sp_tiles) = meta[l]
        check(lib().abkv_paged_prefill_attn(ptr(q), q.stride(0), q.stride(1), ptr(cache), n_pages, ptr(bt), W, W,
                                            ptr(q_start), ptr(ks), ptr(kl), None, ptr(tl[0]), ptr(tl[1]), n_tiles, None, 0,
                                            C_.c_float(scale), ptr(out), out.stride(0), out.stride(1), None, R * K,
                                            n_sp, sp_tiles, ptr(ws) if n_sp > 1 else None,
                                            C_.c_size_t(ws_bytes if n_sp > 1 else 0), stream),
              "abkv_paged_prefill_attn")

    for _ in range(args.warmup):
        for l in range(L):
            launch(l)
    torch.cuda.synchronize()
    evs = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for l in range(L):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch(l)
            e1.record()
            evs.append((e0, e1))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_launch = sum(a.elapsed_time(b) for a, b in evs) / 1e3 / len(evs)
    flops_step = sum(4.0 * 128 * K * sum(limits[l]) * 32 for l in range(L))
    flops_launch = flops_step / L
    kv_bytes_launch = sum(4096.0 * sum(limits[l]) for l in range(L)) / L
    tflops = flops_launch / t_launch / 1e12
    res = {
        "metric": "serving code-step attention TFLOP/s (visible QK+PV flops); % of bf16 dense MFMA peak",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic N(0,1) K/V pages and code-row queries from the seed",
        "config": {"workload": f"code step of the saturated serving stress: {R} request(s) (T={T}, P={P}) attend "
                               f"their {K} code rows to the rows before them + the block's {C} content rows + the "
                               f"first q own code rows, 36 layers (quotas 256/64/64/128/128/128), 32q/8kv, d128, "
                               f"page 16", "global_batch": R, "layers": L,
                   "key_limits_per_group": [limits[groups[g][0]] for g in range(len(groups))],
                   "splits_per_group": [meta[groups[g][0]][3][0] for g in range(len(groups))]},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s", "frac": tflops / 2500.0,
                     "traffic": None, "kernel": "paged_prefill_kernel (+ paged_merge_kernel), per layer launch",
                     "alg_flops_per_launch": flops_launch, "avg_launch_us": t_launch * 1e6,
                     "kv_bytes_per_launch": kv_bytes_launch,
                     "kv_stream_gbps": kv_bytes_launch / t_launch / 1e9},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = code_step_cpu_baseline(torch, cache, q, tables, starts, limits, groups, K, scale)
    return res


def code_step_cpu_baseline(torch, cache, q, tables, starts, limits, groups, K, scale, target_s=10.0):
    """The reference's per-request multi-query arithmetic (oracle.decode.request_ref_torch, restating
    compresslm_packed_kv.py:648-745: bf16 scores, fp32 softmax, bf16 weights) on the host cores, over the same code
    steps: every request, one layer per group (the other layers of a group have the same key counts). value = the
    sample's visible FLOPs over its time."""
    from oracle.decode import request_ref_torch

    host = cpu_threads(torch)
    samples, flops = [], 0.0
    for g in range(len(groups)):
        l = groups[g][0]
        for r in range(len(starts[l])):
            n = starts[l][r] + K
            rows = torch.arange(n)
            pages = torch.from_numpy(tables[l][r].astype(np.int64)).cuda()[rows.cuda() // 16]
            kv = cache[pages, :, (rows % 16).cuda()].cpu()                     # [n, 2, 8, 128]
            key = kv[:, 0].permute(1, 0, 2).contiguous()
            value = kv[:, 1].permute(1, 0, 2).contiguous()
            samples.append((q[r * K: (r + 1) * K].cpu(), key, value, limits[l][r]))
            flops += 4.0 * 128 * K * limits[l][r] * 32
    for qq, k, v, lim in samples:                                            # warm-up
        request_ref_torch(qq, k, v, scale, lim)
    reps, t0 = 0, time.perf_counter()
    while True:
        for qq, k, v, lim in samples:
            request_ref_torch(qq, k, v, scale, lim)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    return {"value": flops * reps / el / 1e12, "unit": "TFLOP/s", "kind": "port", **host,
            "sample": f"the same code steps, one layer per KV group ({len(samples)} request-layers), {reps} reps in "
                      f"{el:.1f} s; torch CPU restatement of compresslm_packed_kv.py:648-745"}


def bench_config1(args, torch):
    """Single-layer abridged decode attention, B=1, quota K=128: 256 prompt rows at positions 0..255, 4 closed
    blocks of C=512 starting at 256 compressed to 128 code rows at in-block bitrev positions, an open block of 300 rows
    at 2304..2603 -> 1068 resident rows (812 without the prompt rows, the count the workload text gives; the reference
    never evicts prompt rows, so both are run). K/V/Q N(0,1) from the seed; the fused RoPE + append kernel rotates
    them at the stated positions (theta 1e6) while writing the rows to random pages. GPU: decode latency per launch;
    CPU: the reference decode arithmetic (oracle.decode.decode_ref_torch) over the same rows."""
    from abridgekv_amd import ops
    from abridgekv_amd.config import bitrev_offsets
    from oracle.decode import decode_ref_torch

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    scale = ops.default_scale()
    cos_sin = ops.rope_cos_sin_cache(2604, device=dev)
    variants, host = {}, None
    for name, with_prompt in (("rows_1068", True), ("rows_812", False)):
        pos = list(range(256)) if with_prompt else []
        for b in range(4):
            pos += (256 + 512 * b + bitrev_offsets(128, 512)).tolist()
        pos += list(range(2304, 2604))
        n = len(pos)
        need = -(-n // 16)
        num_pages = 256
        cache = torch.empty(ops.kv_cache_shape(num_pages), dtype=torch.bfloat16, device=dev).normal_(generator=gen)
        table = torch.from_numpy(rng.permutation(np.arange(1, num_pages))[:need].astype(np.int32)).view(1, -1).to(dev)
        k = torch.randn((n, 8, 128), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((n, 8, 128), generator=gen, device=dev).to(torch.bfloat16)
        qk = torch.empty((n, 32, 128), dtype=torch.bfloat16, device=dev)
        slots = ops.slot_mapping(torch.zeros(n, dtype=torch.int32, device=dev), torch.arange(n, device=dev), table)
        ops.rope_kv_append(qk, k, v, torch.tensor(pos, device=dev), cos_sin, slot_mapping=slots, kv_cache=cache,
                           max_position=2603)
        q = torch.randn((1, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
        ops.rope_kv_append(q, torch.zeros((1, 8, 128), dtype=torch.bfloat16, device=dev), v[:1],
                           torch.tensor([2603], device=dev), cos_sin, max_position=2603)
        sl = torch.tensor([n], dtype=torch.int32, device=dev)
        out = torch.empty((1, 32, 128), dtype=torch.bfloat16, device=dev)
        per_split = {}
        for sp in (4, 8, 16, 32):
            ws = ops.decode_workspace(1, need, sp, device=dev)
            for _ in range(args.warmup + 20):
                ops.decode_attention(q, cache, table, sl, scale, out=out, split_pages=sp, workspace=ws)
            torch.cuda.synchronize()
            reps = 200 * max(1, args.steps // 10)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                ops.decode_attention(q, cache, table, sl, scale, out=out, split_pages=sp, workspace=ws)
            e1.record()
            torch.cuda.synchronize()
            per_split[sp] = e0.elapsed_time(e1) * 1e3 / reps
        sp_best = min(per_split, key=per_split.get)
        entry = {"rows": n, "us_per_launch": per_split[sp_best], "split_pages": sp_best,
                 "us_per_launch_by_split_pages": per_split, "gbps": (n * 4096 + 16384) / per_split[sp_best] / 1e3}
        if not args.no_cpu_baseline:
            host = host or cpu_threads(torch)
            used = table[0].long()
            cpu_cache = cache[used].cpu()
            cpu_tab = torch.arange(need, dtype=torch.int32).view(1, -1)
            cpu_q, cpu_sl = q.cpu(), torch.tensor([n])
            decode_ref_torch(cpu_q, cpu_cache, cpu_tab, cpu_sl, scale)
            creps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 4.0:
                decode_ref_torch(cpu_q, cpu_cache, cpu_tab, cpu_sl, scale)
                creps += 1
            entry["cpu_us_per_call"] = (time.perf_counter() - t0) / creps * 1e6
            entry["cpu_reps"] = creps
        variants[name] = entry
    main = variants["rows_1068"]
    us = main["us_per_launch"]
    res = {
        "metric": "single-layer abridged decode attention, B=1: tokens/s (1 / launch latency)",
        "value": 1e6 / us, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": us / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/Q from the seed, RoPE theta 1e6 at the layout's positions",
        "config": {"workload": "single-layer decode: one layer, B=1, quota 128, prompt 256 + 4 closed blocks x 128 code rows + "
                               "open block 300 (1068 rows; the 812-row variant without prompt rows alongside)",
                   "global_batch": 1},
        "roofline": {"bound": "hbm (latency-bound at B=1: 4.4 MB per launch)", "achieved": main["gbps"],
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": main["gbps"] / HBM_PEAK_GBPS, "traffic": None,
                     "kernel": "decode_attn_kernel + decode_merge_kernel", "alg_bytes_per_launch": 1068 * 4096 + 16384,
                     "avg_launch_us": us},
        "variants": variants,
    }
    if "cpu_us_per_call" in main:
        res["cpu_baseline"] = {"value": 1e6 / main["cpu_us_per_call"], "unit": "tokens/s", "kind": "port", **host,
                               "sample": f"the same 1068 rows, {main['cpu_reps']} calls in 4 s (812 rows: "
                                         f"{variants['rows_812']['cpu_us_per_call']:.0f} us per call); torch CPU "
                                         f"restatement of the reference decode arithmetic"}
    return res


def bench_serving(args, torch):
    """The saturated serving stress with compaction interleaved: every request decodes one token per step; a request
    whose open block fills runs its 256 code rows in the next step (code-step attention with per-group key limits)
    and is then compacted (planner removals + fused row moves). value = decode tokens per second of wall time."""
    from abridgekv_amd import ops
    from abridgekv_amd.serving import ServingStress

    T, P = workloads_lengths(args)
    copy_bw = copy_bandwidth(torch)                            # before the 212 GB of caches are allocated
    t0 = time.perf_counter()
    s = ServingStress(T, P, seed=args.seed, split_pages=args.split_pages,
                      growth_tokens=args.steps + args.warmup + 16, concurrent_code_step=not args.serial_code_step,
                      code_target_blocks=args.code_target_blocks)
    build_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        s.step()
    torch.cuda.synchronize()
    before = dict(s.stats)
    # the decode launches of every stride-th timed step carry a pair of timing events (each event costs ~10 us of
    # host time, 2 % of a step when every launch is timed, so timing all of them would slow the loop it measures)
    stride = max(1, args.steps // 30)
    events = []
    alg = 0
    t1 = time.perf_counter()
    for i in range(args.steps):
        s.decode_events = events if i % stride == 0 else None
        m = s.step()
        if i % stride == 0:
            alg += s.decode_bytes(m)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t1
    dec_s = sum(a.elapsed_time(b) for a, b in events) / 1e3
    n_launch = len(events)
    s.decode_events = None
    stats = {k: s.stats[k] - before[k] for k in s.stats}
    achieved = alg / dec_s / 1e9
    B = len(T)
    res = {
        "metric": "abridged decode-attn tokens/s per GPU (B=256, 32K ctx); % HBM peak BW",
        "value": stats["decode_tokens"] / wall, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall / args.steps * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (N(0,1) K/V pages, queries and new rows from the seed; histories replayed through the "
                "compaction planner)",
        "config": {"workload": f"saturated serving stress with compaction, Qwen3-4B attention (36 layers, 6 quota "
                               f"groups 256/128/64, 32q/8kv, d128, bf16, page 16), B={B}, T~U[2048,32768], "
                               f"P~U[128,1024]; a request closing a 512-token block runs its 256 code rows next step "
                               f"and is compacted", "global_batch": B, "layers": s.L, "kv_groups": s.G,
                   "split_pages": args.split_pages or ("auto" if args.serial_code_step else "auto, at most 40"),
                   "seed": args.seed, "parallelism": "none (1 GPU)",
                   "code_step_stream": "main (serial)" if args.serial_code_step else "second stream (concurrent)",
                   "code_target_blocks": args.code_target_blocks or ("compute units" if args.serial_code_step else "compute units / 4")},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": profiled_traffic("decode_attn_serving_b256_pmc_traffic.md"),
                     "traffic_source": "profiles/decode_attn_serving_b256_pmc_traffic.md (decode_attn_kernel)",
                     "kernel": "decode_attn_kernel (+ decode_merge_kernel), per layer launch",
                     "alg_bytes_per_launch": alg / n_launch, "avg_launch_us": dec_s / n_launch * 1e6,
                     "timed_launches": n_launch,
                     "timed_sample": f"the 36 decode launches of every {stride}th timed step"},
        "decode_attn_ms_per_step": dec_s / n_launch * s.L * 1e3,
        "code_steps": stats["code_steps"], "compacted_rows_moved": stats["moved_rows"],
        "state_build_s": build_s, "copy_bw_gbps_measured": copy_bw,
    }
    if not args.no_cpu_baseline:
        host = cpu_threads(torch)
        n = min(args.cpu_seqs, B)
        view = _CpuView(s)
        tps, reps, el = cpu_baseline(torch, view, s.caches, [s.q_pool[:B]] * s.L, ops.default_scale(), n)
        res["cpu_baseline"] = {"value": tps, "unit": "tokens/s", "kind": "port", **host,
                               "sample": f"first {n} requests of the batch at the end of the run, one layer per KV "
                                         f"group (6 of 36, scaled x6), {reps} reps in {el:.1f} s; torch CPU "
                                         f"restatement of the reference arithmetic (bf16 scores, fp32 softmax, bf16 "
                                         f"probs)"}
    return res


class _CpuView:
    """The attributes cpu_baseline reads, from a serving loop's current page tables and lengths."""

    def __init__(self, s):
        self.groups = s.st.groups
        self.layer_group = s.st.layer_group
        self.layer_slot = s.st.layer_slot
        self.block_tables = list(s.tables)
        self.seq_lens = [sl.astype(np.int32) for sl in s.seq_lens]
        self.num_layers = s.L


def workloads_lengths(args):
    from abridgekv_amd import workloads
    return workloads.saturated_decode_lengths(args.batch, seed=args.seed)


PACKED_HEAD_QUOTAS = (32, 64, 96, 128, 128, 160, 192, 224)    # a per-head schedule with mean 128 of K = 256


def bench_packed(args, torch):
    """Decode with per-head packed code pages, one layer: B=256 sequences of 32K logical context (42 closed blocks of
    512 content + 256 codes archived as packed pages with the per-head quotas above, 1024 rows per page), paged rows =
    512-token raw prompt + open block U[1, 511]. Algorithmic bytes = paged rows x 4096 B + packed rows x 512 B (K+V of
    one head) + q/out. Times abkv_decode_attn_packed (paged splits + side splits + merge)."""
    import numpy as np

    from abridgekv_amd import ops

    B, blocks, prompt = args.batch, 42, 512
    rng = np.random.default_rng(args.seed)
    rows_paged = prompt + rng.integers(1, 512, size=B)
    pages_per = -(-rows_paged // 16)
    W = int(pages_per.max())
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    cache = torch.empty(ops.kv_cache_shape(B * W), dtype=torch.bfloat16, device=dev)
    cache.normal_(generator=gen)
    bt = torch.from_numpy(np.arange(B * W, dtype=np.int32).reshape(B, W)).to(dev)
    seq_lens = torch.from_numpy(rows_paged.astype(np.int32)).to(dev)
    rows = sum(PACKED_HEAD_QUOTAS)
    pool = torch.empty((B * blocks, 2, rows, 128), dtype=torch.bfloat16, device=dev)
    pool.normal_(generator=gen)
    ptab = torch.from_numpy(rng.permutation(B * blocks).astype(np.int32).reshape(B, blocks)).to(dev)
    pcount = torch.full((B,), blocks, dtype=torch.int32, device=dev)
    q = torch.randn((B, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    lse = torch.empty((B, 32), dtype=torch.float32, device=dev)
    scale = ops.default_scale()
    sr = ops.lib().abkv_decode_side_split_rows(min(PACKED_HEAD_QUOTAS))
    sp = args.split_pages or ops.DEFAULT_SPLIT_PAGES
    need = ops.lib().abkv_decode_packed_workspace_size(B, W, sp, blocks, max(PACKED_HEAD_QUOTAS), sr)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)

    def launch():
        ops.decode_attention_packed(q, cache, bt, seq_lens, pool, PACKED_HEAD_QUOTAS, ptab, pcount, scale,
                                    max_pages=W, max_packed=blocks, out=out, lse=lse, split_pages=sp,
                                    workspace=ws)

    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        launch()
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / args.steps
    alg = int(rows_paged.sum()) * 4096 + B * blocks * rows * 512 + B * 2 * 32 * 128 * 2
    gbps = alg / t / 1e9
    return {
        "metric": "packed per-head decode GB/s (one layer launch, B=256, 32K ctx); % HBM peak BW",
        "value": gbps, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": t * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) paged rows, packed pages and queries from the seed",
        "config": {"workload": f"packed per-head decode, B={B}, {blocks} packed pages per sequence, head quotas "
                               f"{list(PACKED_HEAD_QUOTAS)} ({rows} rows per page), paged rows 512 + U[1,511]",
                   "global_batch": B},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / HBM_PEAK_GBPS, "traffic": None,
                     "kernel": "decode_side_kernel + decode_attn_kernel + decode_merge_kernel",
                     "alg_bytes_per_launch": alg, "avg_launch_us": t * 1e6},
        "tokens_per_s_one_layer": B / t,
    }


def bench_copy(args, torch):
    """Calibration kernel for the traffic counters: a plain device copy of 4 GiB (reads 4 GiB, writes 4 GiB)."""
    n = 4 << 30
    a = torch.ones(n // 2, dtype=torch.bfloat16, device="cuda")
    b = torch.empty_like(a)
    for _ in range(args.warmup):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / args.steps
    return {"metric": "device copy bandwidth (read + write)", "value": 2 * n / t / 1e9, "unit": "GB/s",
            "bytes_read_per_launch": n, "bytes_written_per_launch": n, "ms_per_step": t * 1e3, "steps": args.steps}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); the path shards by sequence or KV "
              f"head with no exchange, so whole-job throughput at N GPUs is N x the one-GPU figure.", file=sys.stderr)
        return 2
    import torch

    if args.workload in ("serving", "config1", "prefill", "prefill_bwd", "compaction", "packed", "code_step", "copy"):
        res = {"serving": bench_serving, "config1": bench_config1, "prefill": bench_prefill,
               "prefill_bwd": bench_prefill_bwd, "compaction": bench_compaction, "packed": bench_packed,
               "code_step": bench_code_step, "copy": bench_copy}[args.workload](args, torch)
        print(json.dumps(res), flush=True)
        return 0

    from abridgekv_amd import ops, workloads

    torch.manual_seed(args.seed)
    if args.workload == "saturated":
        T, P = workloads.saturated_decode_lengths(args.batch, seed=args.seed)
        wl = (f"saturated serving decode, Qwen3-4B attention (36 layers, 6 quota groups 256/128/64, 32q/8kv, d128, "
              f"bf16, page 16), B={args.batch}, T~U[2048,32768], P~U[128,1024]")
    else:
        T, P = workloads.full_model_decode_lengths(args.batch, seed=args.seed)
        wl = (f"full-model decode, Qwen3-4B attention (36 layers, 6 quota groups), B={args.batch}, P=512, "
              f"32 closed generated blocks, open block U[1,511]")
    t0 = time.perf_counter()
    st = workloads.build_decode_state(T, P, seed=args.seed)
    build_s = time.perf_counter() - t0
    B, L, G = len(T), st.num_layers, len(st.groups)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    n_tensors = max(len(g) for g in st.groups)
    caches = []
    for _ in range(n_tensors):
        c = torch.empty(ops.kv_cache_shape(st.num_pages), dtype=torch.bfloat16, device=dev)
        c.normal_(generator=gen)
        caches.append(c)
    qs = [torch.randn((B, 32, 128), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
          for _ in range(L)]
    knew = [torch.randn((B, 8, 128), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
            for _ in range(L)]
    vnew = [torch.randn((B, 8, 128), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
            for _ in range(L)]
    outs = [torch.empty((B, 32, 128), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    lses = [torch.empty((B, 32), dtype=torch.float32, device=dev) for _ in range(L)]
    bts = [torch.from_numpy(t).to(dev) for t in st.block_tables]
    sls = [torch.from_numpy(s).to(dev) for s in st.seq_lens]
    slots = [torch.from_numpy(s).to(dev) for s in st.slots]
    W = st.block_tables[0].shape[1]
    # per-group page bound (what a metadata builder passes: the batch's longest sequence in that group)
    gmax = [max(1, int(-(-int(sl.max()) // 16))) for sl in st.seq_lens]
    ws = ops.decode_workspace(B, W, min(args.split_pages or ops.DEFAULT_SPLIT_PAGES, ops.DEFAULT_SPLIT_PAGES),
                              device=dev)
    gsplit = [args.split_pages or ops.auto_split_pages(sl) for sl in st.seq_lens]
    scale = ops.default_scale()
    # one event pair per layer launch of every timed step, read after the last step: the host enqueues the steps
    # back to back without waiting, so it stays ahead of the GPU and no pair measures the host's own launch latency
    # (with a synchronisation after every step the GPU idled at each step's first layer while the host issued it)
    starts = [[torch.cuda.Event(enable_timing=True) for _ in range(L)] for _ in range(args.steps)]
    ends = [[torch.cuda.Event(enable_timing=True) for _ in range(L)] for _ in range(args.steps)]

    def step(k=None):
        for l in range(L):
            g, i = st.layer_group[l], st.layer_slot[l]
            ops.kv_append(knew[l], vnew[l], slots[g], caches[i])
            if k is not None:
                starts[k][l].record()
            ops.decode_attention(qs[l], caches[i], bts[g], sls[g], scale, max_pages=gmax[g], out=outs[l], lse=lses[l],
                                 split_pages=gsplit[g], workspace=ws)
            if k is not None:
                ends[k][l].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    step()                                                   # untimed: puts the host ahead of the GPU
    t_begin = time.perf_counter()
    for k in range(args.steps):
        step(k)
    torch.cuda.synchronize()
    total_s = time.perf_counter() - t_begin
    attn_ms = sum(starts[k][l].elapsed_time(ends[k][l]) for k in range(args.steps) for l in range(L))
    # a separate, event-free pass for the wall-clock step time
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t1) / args.steps

    traffic_profile = ("decode_attn_saturated_b256_pmc_traffic.md" if args.workload == "saturated"
                       else "decode_attn_full_model_b64_pmc_traffic.md")
    kv_bytes = st.kv_bytes_per_step()
    qo_bytes = L * B * (32 * 128 * 2) * 2
    alg_bytes = kv_bytes + qo_bytes
    attn_s_per_step = attn_ms / 1e3 / args.steps
    achieved = alg_bytes / attn_s_per_step / 1e9
    res = {
        "metric": ("abridged decode-attn tokens/s per GPU (B=256, 32K ctx); % HBM peak BW" if args.workload ==
                   "saturated" else "abridged full-model decode-attn tokens/s per GPU (B=64, 17K ctx); % HBM peak BW"),
        "value": B / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) K/V pages and queries from the seed; page tables from the compaction planner)",
        "config": {"workload": wl, "global_batch": B, "layers": L, "kv_groups": G,
                   "split_pages": args.split_pages or "auto", "seed": args.seed, "parallelism": "none (1 GPU)",
                   "code_step_stream": "main (serial)" if args.serial_code_step else "second stream (concurrent)",
                   "code_target_blocks": args.code_target_blocks or ("compute units" if args.serial_code_step else "compute units / 4")},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": (profiled_traffic(traffic_profile) if args.seed == 0 and
                                 args.batch == (256 if args.workload == "saturated" else 64) else None),
                     "traffic_source": f"profiles/{traffic_profile} (decode_attn_kernel)",
                     "kernel": "decode_attn_kernel (+ decode_merge_kernel), per layer launch",
                     "alg_bytes_per_launch": alg_bytes / L, "avg_launch_us": attn_s_per_step / L * 1e6},
        "attn_tokens_per_s": B / attn_s_per_step,
        "attn_ms_per_step": attn_s_per_step * 1e3,
        "kv_gb_per_step": kv_bytes / 1e9,
        "state_build_s": build_s,
    }
    try:
        res["copy_bw_gbps_measured"] = copy_bandwidth(torch)
    except RuntimeError as exc:                               # out of memory next to a 200 GB cache
        res["copy_bw_gbps_measured"] = f"skipped: {exc.__class__.__name__}"
    if not args.no_cpu_baseline:
        host = cpu_threads(torch)
        n = min(args.cpu_seqs, B)
        tps, reps, el = cpu_baseline(torch, st, caches, qs, scale, n)
        res["cpu_baseline"] = {"value": tps, "unit": "tokens/s", "kind": "port", **host,
                               "sample": f"first {n} requests of the same batch, one layer per KV group (6 of 36, "
                                         f"scaled x6), {reps} reps in {el:.1f} s; torch CPU restatement of the "
                                         f"reference arithmetic (bf16 scores, fp32 softmax, bf16 probs)"}
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
