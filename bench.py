#!/usr/bin/env python
"""AWQ W4A16 GEMM throughput on one MI355X.

Workload (decode regime, HBM-bound): one Qwen3-4B decoder layer's four AWQ
linears -- qkv 2560->6144, o_proj 4096->2560, gate_up 2560->19456,
down 9728->2560 -- int4 with group-128 zero points and fp16 scales (nibbles
uniform 0..15, scales uniform [0.002, 0.02]), fp16 activations ~N(0,1) at
M = 1, 8 and 32.  One step runs the four linears at each of the three M
values (12 GEMMs) on one of 36 distinct weight copies (1.9 GB in total, far
past the 256 MB Infinity Cache), rotating copies from step to step; each step
is one HIP-graph replay, as decode steps are replayed in SGLite, timed between
its own pair of HIP events.

value = algorithmic bytes of one step / the median step time (GB/s), where one
linear moves K*N/2 (int4) + (K/128)*N/2 (zeros) + (K/128)*N*2 (scales)
+ 2*M*K (x) + 2*M*N (y) bytes (config.value_from_mean gives the mean-based
figure).  Every other duration is also a median of >= 50 samples.

Also reported on the same line:
  roofline      the dominant decode kernel of the step (the one that moves the
                most of its algorithmic bytes; ops.plan_info names the kernel
                of each shape): algorithmic
                bytes of its launches / their durations, measured with HIP events
                around graphs of back-to-back launches on the launch stream,
                against 8 TB/s HBM; `traffic` is its HBM bytes per launch from
                the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE,
                calibrated on a copy of known size; --pmc-workload/--pmc-summary);
                `attainable_GB/s` / `frac_of_attainable` set it against the
                streaming probe (awq_stream_probe) run with the same grid, block
                and bytes: what a launch of that shape reaches with no arithmetic.
  decode_kernels, per_m   the same per kernel and per batch size, with each
                linear's probe ceiling (and the best ceiling over a few grids).
  llama3_8b     Llama-3-8B's four linears at M = 1, 16, 256, 2048, 8192
                (GB/s and fraction of HBM at decode sizes, TFLOP/s and fraction of
                the 2.5 PFLOP/s dense fp16 MFMA peak from M = 256);
  prefill       its M = 2048 aggregate (and M = 8192).
  mlp           the Qwen3-4B gated MLP with the activation fused vs unfused.
  moe           the Qwen3-30B-A3B-shaped grouped MoE forward.
  stack70b      the Llama-3.1-70B-shaped 80-layer stack (35.6 GB) at
                M = 64 (GB/s, one graph per pass) and M = 4096 (TFLOP/s).
  bounds        the MFMA-rate probe (awq_mfma_probe) at one and two waves per
                SIMD: the compute bound the prefill TFLOP/s are read against.
  cpu_baseline  the CPU oracle on the host cores for every workload above
                (dequantisation and matmul timed separately, 2 warm-ups, median
                of 5); value is the Qwen3-4B layer at M = 1, 8, 32 in GB/s.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]

Profiles (summaries committed under profiles/):
  rocprofv3 --kernel-trace --stats -f csv -d <dir> -o bench -- python3 bench.py --steps 300 \
      --no-cpu-baseline --no-prefill --no-moe --no-stack --no-mlp;  python3 bench.py --rocprof-summary decode <dir>
  rocprofv3 --kernel-trace --stats -f csv -d <dir> -o bench -- python3 bench.py --profile-workload NAME;
      python3 bench.py --rocprof-summary NAME <dir>   (NAME: prefill-2048, prefill-8192, moe, stack70b-64,
      stack70b-4096, mlp, probes)
  rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) ... -- python3 bench.py --pmc-workload;
      python3 bench.py --pmc-summary <fetch_dir> <write_dir>
  rocprofv3 --marker-trace --kernel-trace -f csv -d <dir> -o bench -- python3 bench.py --profile-workload NAME;
      python3 bench.py --marker-summary <dir>   (the C ABI's per-call roctx ranges)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "AWQ W4A16 GEMM GB/s (M≤32) & TFLOP/s (M≥2048) vs roofline, 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
G = 128
LAYER = [("qkv_proj", 2560, 6144), ("o_proj", 4096, 2560), ("gate_up_proj", 2560, 19456), ("down_proj", 9728, 2560)]
PREFILL = [("qkv_proj", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up_proj", 4096, 28672), ("down_proj", 14336, 4096)]
M_SET = (1, 8, 32)
PREFILL_M = 2048
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def gemm_bytes(M: int, N: int, K: int) -> int:
    return K * N // 2 + (K // G) * N // 2 + (K // G) * N * 2 + 2 * M * K + 2 * M * N


def pack_awq_gpu(q: torch.Tensor) -> torch.Tensor:
    """Logical 4-bit [R, C] -> AWQ int32 [R, C/8] (nibble p holds column 8j + AWQ_ORDER[p])."""
    q = q.view(q.shape[0], -1, 8)
    w = torch.zeros(q.shape[:2], dtype=torch.int32, device=q.device)
    for p, col in enumerate(AWQ_ORDER):
        w |= q[:, :, col] << (4 * p)
    return w


def make_repacked(ops, K: int, N: int, gen: torch.Generator, dev: torch.device, dtype=torch.float16):
    q = torch.randint(0, 16, (K, N), generator=gen, device=dev, dtype=torch.int32)
    z = torch.randint(0, 16, (K // G, N), generator=gen, device=dev, dtype=torch.int32)
    s = (torch.rand((K // G, N), generator=gen, device=dev) * 0.018 + 0.002).to(dtype)
    r = ops.repack(pack_awq_gpu(q), pack_awq_gpu(z), s)
    del q, z, s
    return r


STACK70B = [("qkv_proj", 8192, 10240), ("o_proj", 8192, 8192), ("gate_up_proj", 8192, 57344),
            ("down_proj", 28672, 8192)]
STACK70B_LAYERS = 80


def random_repacked(ops, K: int, N: int, gen: torch.Generator, dev: torch.device):
    """A linear's repacked tensors filled directly with random nibbles, zero
    points and U[0.002, 0.02] fp16 scales (the CDNA4 layout of random AWQ
    tensors is random in the same way), without the AWQ round trip."""
    wb, sb, zb = ops.repacked_sizes(K, N, G)
    w = torch.randint(-2**31, 2**31, (wb // 4,), generator=gen, device=dev, dtype=torch.int32)
    z = torch.randint(-2**31, 2**31, (zb // 4,), generator=gen, device=dev, dtype=torch.int32).view(torch.int64)
    s = (torch.rand((sb // 2,), generator=gen, device=dev) * 0.018 + 0.002).to(torch.float16)
    NT, NG = (N + 15) // 16, K // G
    return ops.Repacked(w, s.view(NT, NG, 16), z.view(NT, NG))


def stack70b_bench(ops, dev: torch.device, gen: torch.Generator, only_m: int = 0) -> dict:
    """Llama-3.1-70B-shaped AWQ stack on one GPU: 80 layers x {qkv 8192->10240,
    o 8192->8192, gate_up 8192->57344, down 28672->8192}, int4 group 128
    (35.6 GB of int4 weights, zeros and scales), run layer after layer at
    M = 64 (a batched decode step: whole-stack weight-stream GB/s) and
    M = 4096 (a prefill chunk: TFLOP/s).  Each linear reads a fixed random
    activation of its input width (values are not carried from layer to
    layer: without the model's norms they would overflow); launches are
    back to back on one stream, as in the model."""
    layers = [{name: random_repacked(ops, K, N, gen, dev) for name, K, N in STACK70B}
              for _ in range(STACK70B_LAYERS)]
    cnts = {name: ops.make_counters(N, dev) for name, K, N in STACK70B}
    res = {}
    for M, passes in ((64, 20), (4096, 3)):
        if only_m and M != only_m:
            continue
        xs = {K: torch.randn((M, K), generator=gen, device=dev).to(torch.float16) for _, K, _ in STACK70B}
        outs = {name: torch.empty((M, N), dtype=torch.float16, device=dev) for name, _, N in STACK70B}

        def stack():
            for lay in layers:
                for name, K, N in STACK70B:
                    ops.gemm(xs[K], lay[name], K, N, G, counters=cnts[name], out=outs[name])

        if M <= 256:
            # a batched decode step is replayed as one graph (cuda_graph.py:153-157)
            g = graph_of(stack)
            time_replays([g], 2)
            ms = median(replay_samples([g], passes))
            del g
        else:
            stack()
            ms = median(call_samples(stack, passes))
        byt = STACK70B_LAYERS * sum(gemm_bytes(M, N, K) for _, K, N in STACK70B)
        fl = STACK70B_LAYERS * sum(2 * M * N * K for _, K, N in STACK70B)
        res[str(M)] = {"ms_per_pass": round(ms, 2), "passes": passes, "GB/s": round(byt / ms / 1e6, 1),
                       "frac_hbm": round(byt / ms / 1e6 / HBM_PEAK_GBS, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
                       "frac_mfma": round(fl / ms / 1e9 / MFMA_FP16_PEAK_TFLOPS, 4),
                       "launch": "one HIP graph per pass" if M <= 256 else "eager, back to back"}
        del xs, outs
    del layers
    torch.cuda.synchronize()
    return {"workload": "Llama-3.1-70B-shaped AWQ stack, 80 x {qkv 8192x10240, o 8192x8192, gate_up 8192x57344, "
                        "down 28672x8192}, int4 group 128 with zeros, fp16; layer-by-layer launches; median over "
                        "the passes",
            "weight_bytes": STACK70B_LAYERS * sum(gemm_bytes(0, N, K) for _, K, N in STACK70B), "per_m": res}


def graph_of(fn) -> torch.cuda.CUDAGraph:
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_replays(graphs, n: int) -> float:
    """ms for n back-to-back replays cycling through graphs, HIP events on the current stream."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for i in range(n):
        graphs[i % len(graphs)].replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


def replay_samples(graphs, n: int) -> list:
    """ms of each of n replays (cycling through graphs), each between its own pair of HIP events on
    the launch stream; the replays still run back to back."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    evs[0].record()
    for i in range(n):
        graphs[i % len(graphs)].replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(n)]


def call_samples(fn, n: int) -> list:
    """ms of each of n eager calls of fn, between HIP events on the current stream."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    evs[0].record()
    for i in range(n):
        fn()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(n)]


def median(v) -> float:
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


MEDIAN_SAMPLES = 60  # samples behind every median (>= 50)


def mlp_bench(ops, dev: torch.device, gen: torch.Generator, copies: int = 12, reps: int = MEDIAN_SAMPLES) -> dict:
    """Qwen3-4B gated MLP block (gate_up 2560x19456 -> silu(gate) * up -> down 9728x2560)
    at M = 1, 8, 32: the activation fused into the gate_up GEMM's epilogue, against
    the same GEMMs with the activation as separate torch ops (the reference's
    GatedMLP.forward: gate_up_proj, silu_and_mul, down_proj).  HIP-graph replay
    over rotating weight copies."""
    H, I = 2560, 9728
    gu = [make_repacked(ops, H, 2 * I, gen, dev) for _ in range(copies)]
    dn = [make_repacked(ops, I, H, gen, dev) for _ in range(copies)]
    cg, cd, cm = ops.make_counters(2 * I, dev), ops.make_counters(H, dev), ops.make_mlp_counters(dev)
    res = {}
    for M in M_SET:
        x = torch.randn((M, H), generator=gen, device=dev).to(torch.float16)
        y = torch.empty((M, 2 * I), dtype=torch.float16, device=dev)
        h = torch.empty((M, I), dtype=torch.float16, device=dev)
        o = torch.empty((M, H), dtype=torch.float16, device=dev)

        def unfused(c):
            ops.gemm(x, gu[c], H, 2 * I, G, counters=cg, out=y)
            torch.mul(torch.nn.functional.silu(y[:, :I]), y[:, I:], out=h)
            ops.gemm(h, dn[c], I, H, G, counters=cd, out=o)

        def fused(c):
            ops.gemm(x, gu[c], H, 2 * I, G, counters=cg, out=h, activation="silu")
            ops.gemm(h, dn[c], I, H, G, counters=cd, out=o)

        def one_launch(c):
            ops.gated_mlp(x, gu[c], dn[c], H, I, G, cm, "silu", out=o)

        plan = ops.gated_mlp_plan(M, H, I, G)
        forms = [("unfused", unfused), ("fused", fused)] + ([("one_launch", one_launch)] if plan else [])
        t = {}
        for name, fn in forms:
            g = graph_of(lambda: [fn(c) for c in range(copies)])
            time_replays([g], 3)
            t[name] = median(replay_samples([g], reps)) * 1e3 / copies
        r = {"fused_us": round(t["fused"], 2), "unfused_us": round(t["unfused"], 2),
             "speedup": round(t["unfused"] / t["fused"], 3)}
        if plan:
            ops.mlp_check(cm)  # no workgroup gave up waiting in any of the timed calls
            r.update({"one_launch_us": round(t["one_launch"], 2), "one_launch_workgroups": plan.workgroups,
                      "one_launch_vs_fused": round(t["fused"] / t["one_launch"], 3)})
        res[str(M)] = r
    return {"workload": "Qwen3-4B gated MLP block: gate_up 2560x19456 + silu(gate)*up + down 9728x2560, int4 group "
                        "128, fp16; fused = activation in the gate_up GEMM epilogue, unfused = torch silu and mul "
                        "between the GEMMs, one_launch = the whole block as one kernel (awq_gated_mlp, M <= 16)",
            "per_m": res}


def moe_bench(ops, dev: torch.device, gen: torch.Generator, copies: int = 3, reps: int = MEDIAN_SAMPLES) -> dict:
    """Qwen3-30B-A3B-shaped experts: E=128, H=2048, I=768, top-8 of softmax(N(0,1) logits), T=512.

    One forward = routing, alignment, grouped gate_up GEMM with silu_and_mul,
    grouped down GEMM with the routed weight, top-k combine; replayed as one
    HIP graph over `copies` distinct expert stacks (314 MB each, past the
    Infinity Cache).  Algorithmic bytes: all experts' int4 weights, zeros and
    fp16 scales, plus 2 bytes per element of each routed row's activation
    traffic (x row, gate_up output, activation output, down output)."""
    from sglite_amd.moe import fused_experts_impl, fused_topk, process_awq_moe_weights

    E, H, I, k, T = 128, 2048, 768, 8, 512

    def stack(K, N):
        q = torch.randint(0, 16, (E, K, N), generator=gen, device=dev, dtype=torch.int32)
        qw = pack_awq_gpu(q.view(E * K, N)).view(E, K, N // 8)
        del q
        z = torch.randint(0, 16, (E * (K // G), N), generator=gen, device=dev, dtype=torch.int32)
        qz = pack_awq_gpu(z).view(E, K // G, N // 8)
        s = (torch.rand((E, K // G, N), generator=gen, device=dev) * 0.018 + 0.002).to(torch.float16)
        w = process_awq_moe_weights(qw, qz, s)
        del qw, qz, s
        return w

    stacks = [(stack(H, 2 * I), stack(I, H)) for _ in range(copies)]
    xg = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((T, H), generator=xg, device=dev).to(torch.float16)
    logits = torch.randn((T, E), generator=xg, device=dev)
    buf = x.clone()

    def forward(c):
        w1, w2 = stacks[c]

        def f():
            tw, ids = fused_topk(buf, logits, k, True)
            fused_experts_impl(buf, w1, w2, tw, ids, "silu")
        return f

    graphs = [graph_of(forward(c)) for c in range(copies)]
    time_replays(graphs, 10)
    us = median(replay_samples(graphs, reps)) * 1e3

    # Per-kernel durations: graphs of `copies` back-to-back launches of one stage.
    tw, ids = fused_topk(x, logits, k, True)
    align = ops.moe_align_block_size(ids, 16, E)
    h = ops.moe_gemm(x, stacks[0][0].experts, H, 2 * I, G, align, tw, T * k, k, "silu", False)
    y = ops.moe_gemm(h, stacks[0][1].experts, I, H, G, align, tw, T * k, 1, None, True)
    stages = {
        "topk_softmax": lambda c: ops.moe_topk_softmax(logits, k, True),
        "align": lambda c: ops.moe_align_block_size(ids, 16, E),
        "gate_up_silu": lambda c: ops.moe_gemm(x, stacks[c][0].experts, H, 2 * I, G, align, tw, T * k, k, "silu",
                                               False, out=h),
        "down_routed": lambda c: ops.moe_gemm(h, stacks[c][1].experts, I, H, G, align, tw, T * k, 1, None, True,
                                              out=y),
        "sum_reduce": lambda c: ops.moe_sum_reduce(y.view(T, k, H), buf),
    }
    kern = {}
    for name, fn in stages.items():
        # The GEMMs rotate over the weight copies; the small routing and
        # combine kernels repeat 20 times so that the graph's own launch cost
        # is spread thin.
        n = copies if name in ("gate_up_silu", "down_routed") else 20
        g = graph_of(lambda fn=fn, n=n: [fn(c % copies) for c in range(n)])
        time_replays([g], 3)
        kern[name] = round(median(replay_samples([g], MEDIAN_SAMPLES)) * 1e3 / n, 2)
        del g

    def wbytes(K, N):
        return E * (K * N // 2 + (K // G) * N // 2 + (K // G) * N * 2)

    weights = wbytes(H, 2 * I) + wbytes(I, H)
    act = T * k * (H + 2 * I + I + H) * 2
    flops = 2 * T * k * (H * 2 * I + I * H)
    gemm_us = kern["gate_up_silu"] + kern["down_routed"]
    return {"workload": "Qwen3-30B-A3B-shaped MoE experts: E=128, H=2048, I=768, top-8, T=512, int4 group 128 "
                        "with zero points, fp16; routing from softmax(N(0,1) logits)",
            "us": round(us, 2), "GB/s": round((weights + act) / us / 1e3, 1),
            "frac": round((weights + act) / us / 1e3 / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(flops / us / 1e6, 1), "algorithmic_bytes": weights + act, "flops": flops,
            "gemm_GB/s": round((weights + act) / gemm_us / 1e3, 1), "kernels_us": kern,
            "kernel": "moe_gemm_kernel (grouped W4A16)", "copies": copies}


def _host_cores() -> int:
    """Cores this process may use: the affinity set, capped by OMP_NUM_THREADS when the host sets it
    (a GPU box allots each GPU a share of its cores), never more than os.cpu_count()."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_baseline(warmup: int = 2, runs: int = 5) -> dict:
    """The CPU oracle on the host cores: the oracle's torch dequantisation
    (unpack in AWQ nibble order, (q - z) * s rounded once; pinned bit for bit against the numpy
    oracle) and fp32 matmul + cast, timed separately; `warmup` untimed runs, then the median of
    `runs`.  The Qwen3-4B qkv at M = 16, the Qwen3-4B layer and Llama-3-8B's linears in full except
    Llama-3-8B's M = 2048 and 8192, which time the o_proj (4096x4096) alone; the Llama-3.1-70B
    stack times one 70B-shaped o_proj (8192x8192) and scales it by the layer's weight and flop
    counts (the full stack would need ~137 GB of fp16 weights); the Qwen3-30B-A3B MoE runs the
    expert loop over 16 of the 128 experts and scales by 8.  value = the headline workload (the
    Qwen3-4B layer at M = 1, 8, 32) in the metric's GB/s."""
    from oracle import awq_oracle as oracle

    threads = _host_cores()
    torch.set_num_threads(threads)
    t_start = time.perf_counter()

    def med(fn):
        for _ in range(warmup):
            fn()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return median(ts)

    def linear_times(K, N, Ms, seed):
        t = oracle.make_awq_linear(K, N, G, seed=seed)
        box = {}
        td = med(lambda: box.__setitem__("W", oracle.dequantize_torch(t["qweight"], t["qzeros"], t["scales"], G)))
        Wf = box["W"].float()
        tm = {}
        for M in Ms:
            x = oracle.make_activation(M, K, seed=100 + M).float()
            tm[M] = med(lambda: (x @ Wf).to(torch.float16))
        return td, tm

    res = {}
    # Qwen3-4B qkv at M = 16
    td, tm = linear_times(2560, 6144, (16,), 0)
    res["qwen3_4b_qkv_m16"] = {"dequant_s": round(td, 4), "matmul_s": round(tm[16], 4),
                              "GB/s": round(gemm_bytes(16, 6144, 2560) / (td + tm[16]) / 1e9, 3)}
    # the Qwen3-4B layer at M = 1, 8, 32 (the headline workload)
    step_b, step_t, deq_t, mm_t = 0, 0.0, 0.0, 0.0
    for i, (_, K, N) in enumerate(LAYER):
        td, tm = linear_times(K, N, M_SET, i)
        for M in M_SET:
            step_b += gemm_bytes(M, N, K)
            step_t += td + tm[M]
            mm_t += tm[M]
        deq_t += td
    res["qwen3_4b_layer"] = {"dequant_s_per_layer": round(deq_t, 4), "matmul_s_per_step": round(mm_t, 4),
                             "GB/s": round(step_b / step_t / 1e9, 3)}
    value = step_b / step_t / 1e9
    # Llama-3-8B layer at M = 1, 16, 256 in full; 2048 and 8192 on the o_proj
    per_m = {M: [0, 0, 0.0] for M in LLAMA_M}
    for i, (name, K, N) in enumerate(PREFILL):
        Ms = [M for M in LLAMA_M if M <= 256 or name == "o_proj"]
        td, tm = linear_times(K, N, Ms, 10 + i)
        for M in Ms:
            per_m[M][0] += gemm_bytes(M, N, K)
            per_m[M][1] += 2 * M * N * K
            per_m[M][2] += td + tm[M]
    res["llama3_8b"] = {str(M): {"GB/s": round(b / t / 1e9, 3), "TFLOP/s": round(f / t / 1e12, 4)}
                        for M, (b, f, t) in per_m.items()}
    # one 70B-shaped o_proj, scaled to the 80-layer stack
    K3, N3 = 8192, 8192
    td, tm = linear_times(K3, N3, (64, 4096), 20)
    w_layer = sum(K * N for _, K, N in STACK70B)
    c3 = {}
    for M in (64, 4096):
        t_stack = 80 * (td + tm[M]) * w_layer / (K3 * N3)
        c3[str(M)] = {"s_per_stack_estimate": round(t_stack, 2),
                      "GB/s": round(80 * sum(gemm_bytes(M, N, K) for _, K, N in STACK70B) / t_stack / 1e9, 3),
                      "TFLOP/s": round(80 * sum(2 * M * N * K for _, K, N in STACK70B) / t_stack / 1e12, 4)}
    res["llama31_70b_stack"] = c3
    # Qwen3-30B-A3B expert loop (gate_up 2048->1536 + silu_and_mul + down 768->2048), 16 of 128 experts
    E, Es, H, I, T, k = 128, 16, 2048, 768, 512, 8
    ex = [(oracle.make_awq_linear(H, 2 * I, G, seed=30 + e), oracle.make_awq_linear(I, H, G, seed=300 + e))
          for e in range(Es)]
    rows = T * k // E  # routed rows per expert on average
    xe = oracle.make_activation(rows, H, seed=5).float()

    def experts():
        for w1, w2 in ex:
            W1 = oracle.dequantize_torch(w1["qweight"], w1["qzeros"], w1["scales"], G).float()
            W2 = oracle.dequantize_torch(w2["qweight"], w2["qzeros"], w2["scales"], G).float()
            h = (xe @ W1).to(torch.float16).float()
            a = (h[:, :I] / (1.0 + torch.exp(-h[:, :I])) * h[:, I:]).to(torch.float16).float()
            (a @ W2).to(torch.float16)
    t4 = med(experts) * E / Es
    wb = E * (gemm_bytes(0, 2 * I, H) + gemm_bytes(0, H, I))
    res["qwen3_30b_a3b_moe"] = {"s_estimate": round(t4, 3), "GB/s": round((wb + T * k * (H + 2 * I + I + H) * 2) / t4 / 1e9, 3)}
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(value, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle (torch dequantise, pinned bit-exact to the numpy oracle, + fp32 matmul + fp16 "
                      f"cast), {warmup} warm-ups then the median of {runs}; value = the Qwen3-4B layer at M = 1, 8, "
                      f"32; the other workloads in per_workload ({time.perf_counter() - t_start:.1f} s in all); "
                      f"host {model}, os.cpu_count() = {os.cpu_count()}",
            "per_workload": res}


PMC_COPY_BYTES = 256 << 20
PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_kernels_qwen3_4b_layer_hbm_traffic.md")


def pmc_workload(ops, dev: torch.device, gen: torch.Generator) -> int:
    """The step's decode GEMMs, each 4 times over 4 weight copies (one
    dispatch per call, eagerly), then a 256 MiB device copy 3 times: the
    calibration of the FETCH_SIZE / WRITE_SIZE counters."""
    reps = [{name: make_repacked(ops, K, N, gen, dev) for name, K, N in LAYER} for _ in range(4)]
    cnts = {name: ops.make_counters(N, dev) for name, K, N in LAYER}
    xg = torch.Generator(device=dev).manual_seed(1)
    torch.cuda.synchronize()
    for M in M_SET:
        for name, K, N in LAYER:
            x = torch.randn((M, K), generator=xg, device=dev).to(torch.float16)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            for c in range(4):
                ops.gemm(x, reps[c][name], K, N, G, counters=cnts[name], out=out)
    src = torch.empty(PMC_COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc workload done", flush=True)
    return 0


def _pmc_rows(d: str):
    import csv
    import glob

    path = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))[0]
    return list(csv.DictReader(open(path)))


def pmc_summary(fetch_dir: str, write_dir: str) -> str:
    """Markdown summary of FETCH_SIZE / WRITE_SIZE (KiB per dispatch) for the
    decode kernels of --pmc-workload, each scaled by the counter's reading for
    a device copy of known size (the copy reads and writes PMC_COPY_BYTES)."""
    from collections import defaultdict

    def per_kernel(d: str, counter: str):
        vals = defaultdict(list)
        for r in _pmc_rows(d):
            if r["Counter_Name"] != counter:
                continue
            name = r["Kernel_Name"]
            key = next((k for k in DECODE_KERNELS if k + "<" in name), None)
            if key is None and "copyBuffer" in name:  # torch's device-to-device copy is a runtime blit
                key = "copy"
            if key is not None:
                vals[key].append(float(r["Counter_Value"]) * 1024.0)  # KiB -> bytes
        return {k: sum(v) / len(v) for k, v in vals.items()}, {k: len(v) for k, v in vals.items()}

    fetch, nf = per_kernel(fetch_dir, "FETCH_SIZE")
    write, nw = per_kernel(write_dir, "WRITE_SIZE")
    cf = PMC_COPY_BYTES / fetch["copy"]
    cw = PMC_COPY_BYTES / write["copy"]
    from sglite_amd import ops

    algo = defaultdict(list)
    for M in M_SET:
        for _, K, N in LAYER:
            algo[ops.plan_info(M, N, K, G).function].append(gemm_bytes(M, N, K))
    lines = [
        "# HBM traffic of the decode kernels (Qwen3-4B layer, M = 1, 8, 32), rocprofv3 PMC",
        "",
        "Commands (from the repository root, TMPDIR=/tmp), one counter per run:",
        "`rocprofv3 --pmc FETCH_SIZE -f csv -d <fetch_dir> -o pmc -- python3 bench.py --pmc-workload`,",
        "`rocprofv3 --pmc WRITE_SIZE -f csv -d <write_dir> -o pmc -- python3 bench.py --pmc-workload`,",
        "`python3 bench.py --pmc-summary <fetch_dir> <write_dir>`.",
        "",
        f"Calibration: a {PMC_COPY_BYTES >> 20} MiB device copy reads FETCH_SIZE {fetch['copy'] / 1e6:.2f} MB and "
        f"WRITE_SIZE {write['copy'] / 1e6:.2f} MB per dispatch, so the factors are {cf:.4f} (fetch) and "
        f"{cw:.4f} (write).",
        "",
        "| kernel | dispatches | FETCH_SIZE (MB) | WRITE_SIZE (MB) | calibrated traffic (MB) | algorithmic (MB) |",
        "|---|---|---|---|---|---|",
    ]
    for k in DECODE_KERNELS:
        if k not in fetch or k not in write:
            continue
        t = fetch[k] * cf + write[k] * cw
        a = sum(algo[k]) / len(algo[k]) if algo[k] else float("nan")
        lines.append(f"| `{k}` | {nf[k]} | {fetch[k] / 1e6:.3f} | {write[k] / 1e6:.3f} | {t / 1e6:.3f} | {a / 1e6:.3f} |")
    lines.append("")
    for k in DECODE_KERNELS:
        if k in fetch and k in write:
            lines.append(f"traffic_bytes_per_launch {k} {int(fetch[k] * cf + write[k] * cw)}")
    return "\n".join(lines) + "\n"


def committed_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None."""
    try:
        for line in open(PMC_SUMMARY):
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                return int(parts[2])
    except OSError:
        pass
    return None


# The HIP kernels a decode GEMM launch can run (ops.PlanInfo.function); the
# tiled kind runs tiled_kernel (16x16x32 MFMAs) or mfma32_kernel (32x32x16).
DECODE_KERNELS = ("skinny_kernel", "gemv_kernel", "tiled_kernel", "mfma32_kernel", "kslice_kernel")
TRACE_KERNELS = ("skinny_kernel", "gemv_kernel", "tiled_kernel", "mfma32_kernel", "splitk_reduce_kernel", "moe_",
                 "topk_softmax_kernel", "align_kernel", "kslice_kernel", "mlp_kernel")


def _trace_rows(trace_dir: str):
    """(short name, workgroups, grid y, block, start ns, duration us) of the engine's GEMM/MoE dispatches, in
    time order (probe and torch kernels are left out)."""
    import csv
    import glob

    path = sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True))[0]
    rows = []
    for r in csv.DictReader(open(path)):
        name = r["Kernel_Name"]
        if not any(k in name for k in TRACE_KERNELS):
            continue
        short = name.replace("(anonymous namespace)::", "").replace("sgl_awq::", "").replace("void ", "")
        short = short[:short.index("(")] if "(" in short else short
        bx = int(r["Workgroup_Size_X"])
        start, end = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        rows.append((short, int(r["Grid_Size_X"]) // bx, int(r["Grid_Size_Y"]), bx, start, (end - start) / 1e3))
    rows.sort(key=lambda r: r[4])
    return rows


def _trace_groups(trace_dir: str):
    """Kernel-trace durations (us) grouped by (short name, grid, block)."""
    from collections import defaultdict

    groups = defaultdict(list)
    for short, gx, gy, bx, _, d in _trace_rows(trace_dir):
        groups[(short, gx, gy, bx)].append(d)
    return groups


def _trace_table(groups) -> list:
    lines = ["| kernel | grid (x, y) | block | dispatches | mean us | min us | max us |",
             "|---|---|---|---|---|---|---|"]
    for (name, gx, gy, bx), ds in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {gx}, {gy} | {bx} | {len(ds)} | {sum(ds) / len(ds):.2f} | "
                     f"{min(ds):.2f} | {max(ds):.2f} |")
    return lines


PROFILE_REPS = 10  # timed calls per shape in the --profile-workload runs (after 2 warm-ups)

PROBE_ITERS = 4000  # rounds of eight 32x32x16 MFMAs per wave in one MFMA-probe launch
PROBE_FLOP_PER_WAVE_ITER = 8 * 2 * 32 * 32 * 16


def probe_grids(ops) -> dict:
    """MFMA-probe grids: 256-thread workgroups, one and two per CU (one and two waves per SIMD)."""
    cus = ops.device_cu_count()
    return {"1_wave_per_simd": cus, "2_waves_per_simd": 2 * cus}


def bounds_bench(ops, dev: torch.device, reps: int = 7) -> dict:
    """Compute bounds the prefill kernels are read against: the MFMA probe (awq_mfma_probe: eight
    independent 32x32x16 fp16 MFMAs per wave, operands in registers, no memory traffic) at one and
    two waves per SIMD, median of `reps` launches each; TFLOP/s and fraction of the 2.5 PFLOP/s
    dense peak.  A W4A16 GEMM also spends vector-ALU time dequantising every weight between its MFMAs,
    so its attainable rate lies below the probe's."""
    sink = torch.empty(4 * 2 * ops.device_cu_count(), dtype=torch.float32, device=dev)
    out = {"probe": "awq_mfma_probe, eight independent v_mfma_f32_32x32x16_f16 per wave, "
                    f"{PROBE_ITERS} rounds per launch, 256-thread workgroups"}
    for label, grid in probe_grids(ops).items():
        ops.mfma_probe(PROBE_ITERS, grid, 256, sink)
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            ops.mfma_probe(PROBE_ITERS, grid, 256, sink)
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e-3)
        t = median(ts)
        tf = grid * 4 * PROBE_ITERS * PROBE_FLOP_PER_WAVE_ITER / t / 1e12
        out[label] = {"workgroups": grid, "us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
                      "frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4)}
    return out


def _launches_per_call(ops, M: int, N: int, K: int, activation=None) -> int:
    info = ops.plan_info(M, N, K, G, activation)
    return 2 if info.kernel == "tiled_kernel" and info.k_slices > 1 and not info.fixup else 1


SQ_CASES = ([(f"Llama-3-8B {n} M=2048", 2048, K, N) for n, K, N in PREFILL]
            + [("Llama-3-8B gate_up_proj M=8192", 8192, 4096, 28672)]
            + [(f"Qwen3-4B {n} M={M}", M, K, N) for M in M_SET for n, K, N in LAYER]
            + [(f"Llama-3-8B {n} M={M}", M, K, N) for M in (64, 256) for n, K, N in PREFILL])
SQ_PASSES = (
    "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_VALU_MFMA_COEXEC_CYCLES SQ_WAIT_ANY "
    "SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY GRBM_GUI_ACTIVE",
    "SQ_WAVES SQ_WAVE_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_SCA "
    "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE",
    "SQ_WAVES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_INSTS_VMEM SQ_INSTS_SALU SQ_INSTS_SMEM SQ_WAIT_INST_LDS",
)
SQ_DENSE = [("hipBLASLt dense fp16 gate_up_proj M=2048", 2048, 4096, 28672),
            ("hipBLASLt dense fp16 gate_up_proj M=8192", 8192, 4096, 28672)]
SQ_REPS = 3  # counted calls per case (after one warm-up)
SQ_MIN_CLOCK_US = 50.0  # shorter dispatches: GRBM_GUI_ACTIVE also counts the dispatch's set-up and drain
MFMA_PEAK_GHZ = 2.4  # engine clock of the 2.5 PFLOP/s dense fp16 figure


def sq_workload(ops, dev: torch.device, gen: torch.Generator) -> None:
    """Launch sequence for the SQ-counter passes: the MFMA probe at one and two waves per SIMD, every
    SQ_CASES GEMM, then the SQ_DENSE dense fp16 GEMMs (1 warm-up + SQ_REPS calls each, eager, in order)."""
    sink = torch.empty(4 * 2 * ops.device_cu_count(), dtype=torch.float32, device=dev)
    for grid in probe_grids(ops).values():
        for _ in range(1 + SQ_REPS):
            ops.mfma_probe(PROBE_ITERS, grid, 256, sink)
    torch.cuda.synchronize()
    for _, M, K, N in SQ_CASES:
        r = make_repacked(ops, K, N, gen, dev)
        cnt = ops.make_counters(N, dev)
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.float16)
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        for _ in range(1 + SQ_REPS):
            ops.gemm(x, r, K, N, G, counters=cnt, out=out)
        torch.cuda.synchronize()
        del r, x, out
    for _, M, K, N in SQ_DENSE:  # the vendor library's dense GEMM on fp16 weights of the same shape
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.float16)
        w = (torch.randn((K, N), generator=gen, device=dev) * 0.02).to(torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        torch.cuda.synchronize()
        for _ in range(1 + SQ_REPS):
            torch.matmul(x, w, out=y)
        torch.cuda.synchronize()
        del x, w, y


def sq_summary(dirs: list) -> str:
    """Markdown summary of the SQ-counter passes (one rocprofv3 --pmc run of `--profile-workload sq` per
    SQ_PASSES entry).  Counters are summed over the device by rocprofv3; each case's row is the mean over
    its counted calls (the warm-up call is dropped), matched by kernel function, grid and block from
    ops.plan_info.  Wave-time fractions divide SQ_WAIT_* / SQ_ACTIVE_INST_* by SQ_WAVE_CYCLES (all in
    quad-cycles, summed over waves); MFMA and VALU busy divide the per-SIMD busy cycles by the SIMD count
    times the kernel's cycles (GRBM_GUI_ACTIVE, counted per XCD, over the XCD count); the MFMA probe,
    which issues nothing but independent MFMAs, calibrates the MFMA figure."""
    from collections import defaultdict
    from sglite_amd import ops

    cus = ops.device_cu_count()
    simds, xcds = 4 * cus, max(1, cus // 32)
    # The workload's engine dispatches in order: (function, workgroups, block) per case, 1 + SQ_REPS each.
    plan = [(f"MFMA probe, {label.replace('_', ' ')}", "mfma_probe_kernel", grid, 256)
            for label, grid in probe_grids(ops).items()]
    for label, M, K, N in SQ_CASES:
        info = ops.plan_info(M, N, K, G)
        plan.append((label, info.function, info.workgroups, info.threads))
    plan += [(label, "Cijk_", 0, 0) for label, *_ in SQ_DENSE]  # hipBLASLt kernels: matched by name prefix
    counted = [defaultdict(list) for _ in plan]  # per case: counter -> values of its counted calls
    kernels = [""] * len(plan)
    for d in dirs:
        disp = {}
        for r in _pmc_rows(d):
            name = r["Kernel_Name"]
            short = name.replace("(anonymous namespace)::", "").replace("sgl_awq::", "").replace("void ", "")
            short = short[:short.index("(")] if "(" in short else short
            bx = int(r["Workgroup_Size"])  # counter-collection rows give total sizes (work-items)
            e = disp.setdefault(int(r["Dispatch_Id"]), [(short, int(r["Grid_Size"]) // bx, bx), {}])
            e[1][r["Counter_Name"]] = float(r["Counter_Value"])
            e[1]["duration_ns"] = float(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        seq = [disp[i] for i in sorted(disp)]
        pos = 0
        for ci, (_, fn, wgs, block) in enumerate(plan):
            got = 0
            while pos < len(seq) and got < 1 + SQ_REPS:
                (short, w, b), cs = seq[pos]
                pos += 1
                if fn == "Cijk_":
                    hit = short.startswith(fn)
                else:
                    hit = (short == fn or short.startswith(fn + "<")) and w == wgs and b == block
                if hit:
                    if got > 0:  # the first call is the warm-up
                        for c, v in cs.items():
                            counted[ci][c].append(v)
                    kernels[ci] = short
                    got += 1

    def div(a: float, b: float) -> float:
        return a / b if b else float("nan")

    def metrics(cs: dict) -> dict:
        g = lambda n: sum(cs[n]) / len(cs[n]) if cs.get(n) else float("nan")
        cyc = g("GRBM_GUI_ACTIVE") / xcds
        wc = g("SQ_WAVE_CYCLES")
        waves = g("SQ_WAVES")
        us = g("duration_ns") / 1e3
        ghz = cyc / (us * 1e3) if us >= SQ_MIN_CLOCK_US else float("nan")
        mfma = div(g("SQ_VALU_MFMA_BUSY_CYCLES"), simds * cyc)
        return {
            "us": us, "ghz": ghz, "rate": mfma * ghz / MFMA_PEAK_GHZ,
            "mfma": mfma,
            "valu": div(4 * g("SQ_ACTIVE_INST_VALU"), simds * cyc),
            "coexec": div(g("SQ_VALU_MFMA_COEXEC_CYCLES"), g("SQ_VALU_MFMA_BUSY_CYCLES")),
            "w_issue": div(g("SQ_WAIT_INST_ANY"), wc), "w_any": div(g("SQ_WAIT_ANY"), wc),
            "a_any": div(g("SQ_ACTIVE_INST_ANY"), wc), "a_valu": div(g("SQ_ACTIVE_INST_VALU"), wc),
            "a_lds": div(g("SQ_ACTIVE_INST_LDS"), wc), "a_vmem": div(g("SQ_ACTIVE_INST_VMEM"), wc),
            "a_sca": div(g("SQ_ACTIVE_INST_SCA"), wc),
            "conflict": div(g("SQ_LDS_BANK_CONFLICT"), g("SQ_LDS_IDX_ACTIVE")),
            "i_valu": div(g("SQ_INSTS_VALU"), waves), "i_mfma": div(g("SQ_INSTS_MFMA"), waves),
            "i_lds": div(g("SQ_INSTS_LDS"), waves), "i_vmem": div(g("SQ_INSTS_VMEM"), waves),
            "i_salu": div(g("SQ_INSTS_SALU") + g("SQ_INSTS_SMEM"), waves),
        }

    cases = [(plan[i][0], kernels[i] if plan[i][1] != "Cijk_" else kernels[i][:40] + "...", metrics(counted[i]))
             for i in range(len(plan)) if kernels[i]]
    f = lambda v, d=2: "n/a" if v != v else f"{v:.{d}f}"
    lines = [
        "# SQ counters of the prefill, mid-size and decode kernels (rocprofv3 --pmc), with the MFMA probe", "",
        "Commands (from the repository root, TMPDIR=/tmp), one counter set per run:", ""]
    for i, p in enumerate(SQ_PASSES):
        lines.append(f"    rocprofv3 --pmc {p} -f csv -d <dir{i + 1}> -o pmc -- python3 bench.py --profile-workload sq")
    lines += [f"    python3 bench.py --sq-summary <dir1> <dir2> <dir3>", "",
              "Workload: the MFMA probe (eight independent 32x32x16 fp16 MFMAs per wave, no memory traffic) at one",
              "and two waves per SIMD, the Llama-3-8B linears at M = 2048, its gate_up at M = 8192, and the",
              f"Qwen3-4B decode linears at M = 1, 8, 32, the Llama-3-8B linears at M = 64 and 256; fp16, int4 group "
              "128; then the vendor library's dense fp16 "
              "GEMM (torch.matmul, hipBLASLt) on fp16 weights of the Llama-3-8B gate_up shape at M = 2048 and 8192.",
              f"Each case 1 warm-up + {SQ_REPS} counted calls (dispatches are serialised under counter collection).",
              "",
              "* us: mean dispatch duration under counter collection.  Clock: kernel cycles (GRBM_GUI_ACTIVE / XCDs)",
              f"  over that duration, shown for dispatches of at least {SQ_MIN_CLOCK_US:.0f} us (shorter ones are "
              "dominated by set-up and drain).",
              "* MFMA busy: SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x kernel cycles) "
              f"({simds} SIMDs, {xcds} XCDs); times clock / 2.4 GHz it estimates the",
              "  fraction of the 2.5 PFLOP/s dense fp16 peak (the probe's estimate matches its timed rate).",
              "  VALU busy: 4 x SQ_ACTIVE_INST_VALU over the same.",
              "* co-exec: SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES (MFMA-busy cycles in which a VALU",
              "  instruction also issued).",
              "* wait issue / wait any / active: SQ_WAIT_INST_ANY, SQ_WAIT_ANY and SQ_ACTIVE_INST_{ANY,VALU,LDS,VMEM,SCA}",
              "  over SQ_WAVE_CYCLES (fractions of the waves' resident time; categories overlap).",
              "* LDS conflict: SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.  Instructions per wave: SQ_INSTS_* / SQ_WAVES",
              "  (SALU includes SMEM).",
              "",
              "| case | kernel | us | clock GHz | MFMA busy | MFMA busy x clock / 2.4 GHz | VALU busy | co-exec | "
              "wait issue | wait any | active any | active VALU | active LDS | active VMEM | active SALU | "
              "LDS conflict | VALU / MFMA / LDS / VMEM / SALU instructions per wave |",
              "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for label, kern, m in cases:
        lines.append(
            f"| {label} | `{kern}` | {f(m['us'], 1)} | {f(m['ghz'])} | {f(m['mfma'])} | {f(m['rate'])} | "
            f"{f(m['valu'])} | {f(m['coexec'])} | {f(m['w_issue'])} | "
            f"{f(m['w_any'])} | {f(m['a_any'])} | {f(m['a_valu'])} | {f(m['a_lds'])} | {f(m['a_vmem'])} | "
            f"{f(m['a_sca'])} | {f(m['conflict'], 3)} | {f(m['i_valu'], 0)} / {f(m['i_mfma'], 0)} / "
            f"{f(m['i_lds'], 0)} / {f(m['i_vmem'], 0)} / {f(m['i_salu'], 0)} |")
    return "\n".join(lines) + "\n"


def profile_workload(name: str, ops, dev: torch.device, gen: torch.Generator) -> None:
    """A fixed launch sequence for `rocprofv3 --kernel-trace` (one section of the benchmark, eager calls
    in a known order), read back by --rocprof-summary NAME; `sq` is the SQ-counter workload
    (--sq-summary)."""
    if name == "sq":
        sq_workload(ops, dev, gen)
    elif name.startswith("prefill"):
        M = int(name.split("-")[1])
        x = {K: torch.randn((M, K), generator=gen, device=dev).to(torch.float16) for K in {k for _, k, _ in PREFILL}}
        for lname, K, N in PREFILL:
            r = make_repacked(ops, K, N, gen, dev)
            cnt = ops.make_counters(N, dev)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            for _ in range(2 + PROFILE_REPS):
                ops.gemm(x[K], r, K, N, G, counters=cnt, out=out)
            torch.cuda.synchronize()
            del r
    elif name == "moe":
        moe_bench(ops, dev, gen, reps=20)
    elif name.startswith("stack70b"):
        stack70b_bench(ops, dev, gen, only_m=int(name.split("-")[1]))
    elif name == "mlp":
        mlp_bench(ops, dev, gen, reps=20)
    elif name == "probes":
        sink = torch.empty(4 * 2 * ops.device_cu_count(), dtype=torch.float32, device=dev)
        for grid in probe_grids(ops).values():
            for _ in range(2 + PROFILE_REPS):
                ops.mfma_probe(PROBE_ITERS, grid, 256, sink)
            torch.cuda.synchronize()
    else:
        raise ValueError(f"unknown profile workload {name!r}")
    torch.cuda.synchronize()
    print(f"profile workload {name} done", flush=True)


def marker_summary(trace_dir: str, command: str) -> str:
    """Markdown summary of a rocprofv3 --marker-trace --kernel-trace run: the roctx ranges the C ABI
    opens around each compute entry point (host-side span of the call, which encloses its kernel
    launches), and the kernels dispatched in the same run."""
    import csv
    import glob

    def rows(pattern):
        path = sorted(glob.glob(os.path.join(trace_dir, "**", pattern), recursive=True))[0]
        with open(path) as f:
            return list(csv.DictReader(f))
    ranges: dict = {}
    for r in rows("*marker_api_trace.csv"):
        ranges.setdefault(r["Function"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    kernels: dict = {}
    for r in rows("*kernel_trace.csv"):
        if "sgl_awq" not in r["Kernel_Name"]:
            continue  # the workload's own set-up (torch kernels)
        name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0].replace("void sgl_awq::", "")
        kernels.setdefault(name, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = ["# roctx ranges of the C ABI, rocprofv3 marker trace", "",
           f"Command (from the repository root, TMPDIR=/tmp): `{command}`", "",
           "Every compute entry point of the C ABI (`awq_repack_cdna4`, `awq_w4a16_gemm[_act|_noalloc]`, the",
           "MoE stages, the dequantisation probes) opens a roctx range named after itself for the duration",
           "of the call, so a trace attributes each kernel launch to the operation that issued it.  A range",
           "spans the host-side call (argument checks, planning, launches); the kernels run asynchronously.",
           "", "| range | calls | median host us | max host us |", "|---|---|---|---|"]
    for name, v in sorted(ranges.items()):
        out.append(f"| `{name}` | {len(v)} | {median(v):.2f} | {max(v):.2f} |")
    out += ["", "Kernels of the engine in the same run:", "", "| kernel | dispatches | median us |", "|---|---|---|"]
    for name, v in sorted(kernels.items(), key=lambda kv: -len(kv[1])):
        out.append(f"| `{name}` | {len(v)} | {median(v):.2f} |")
    return "\n".join(out) + "\n"


def _probe_summary(trace_dir: str, command: str, ops) -> str:
    import csv
    import glob

    path = sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True))[0]
    runs: dict = {}
    for r in csv.DictReader(open(path)):
        if "mfma_probe_kernel" not in r["Kernel_Name"]:
            continue
        wgs = int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"])
        runs.setdefault(wgs, []).append((int(r["Start_Timestamp"]),
                                         (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    runs = {wgs: [d for _, d in sorted(v)] for wgs, v in runs.items()}  # launch order
    lines = ["# MFMA-rate probe (the compute bound of the prefill kernels), rocprofv3 kernel trace", "",
             f"Command (from the repository root, TMPDIR=/tmp): `{command}`", "",
             "`mfma_probe_kernel`: eight independent `v_mfma_f32_32x32x16_f16` per wave, operands in registers,",
             f"no memory traffic, {PROBE_ITERS} rounds per launch, 256-thread workgroups; one workgroup per CU is one",
             "wave per SIMD, two are two.  Per grid 2 warm-ups then the timed launches, back to back (mean of",
             "those; the first and last timed launch show any clock change under the sustained load).  The",
             "benchmark's `bounds` section times isolated launches (a synchronisation between them) instead.",
             "The prefill kernels dequantise every weight on the vector ALU between their MFMAs, so they are",
             "read against this rate, not against the 2.5 PFLOP/s peak alone.", "",
             "| workgroups | waves per SIMD | launches | mean us | first us | last us | TFLOP/s | fraction of 2.5 PFLOP/s |",
             "|---|---|---|---|---|---|---|---|"]
    cus = ops.device_cu_count()
    for wgs, ds in sorted(runs.items()):
        timed = ds[2:] if len(ds) > 2 else ds
        us = sum(timed) / len(timed)
        tf = wgs * 4 * PROBE_ITERS * PROBE_FLOP_PER_WAVE_ITER / (us * 1e-6) / 1e12
        lines.append(f"| {wgs} | {wgs // cus} | {len(timed)} | {us:.1f} | {timed[0]:.1f} | {timed[-1]:.1f} | {tf:.1f} | "
                     f"{tf / MFMA_FP16_PEAK_TFLOPS:.4f} |")
    return "\n".join(lines) + "\n"


def rocprof_summary(trace_dir: str, command: str, section: str) -> str:
    """Markdown summary of a rocprofv3 --kernel-trace run of this benchmark.

    decode: the decode step; every (M, linear) is launched equally often, so a
    kernel's mean algorithmic bytes per launch is the mean over the (M, linear)
    pairs it serves (ops.plan_info names the kernel of each shape); a split-K
    GEMM on the tiled kernels also runs splitk_reduce_kernel, listed apart.
    prefill-M (--profile-workload prefill-M): the four Llama-3-8B linears at M,
    each launched 2 + PROFILE_REPS times in order; per linear the mean of the
    timed calls (GEMM plus any reduction) and TFLOP/s.
    moe, stack70b-M, mlp: the section's kernels with their durations.
    probes: the MFMA probe at one and two waves per SIMD (mean of the timed launches).
    """
    from sglite_amd import ops

    if section == "probes":
        return _probe_summary(trace_dir, command, ops)

    groups = _trace_groups(trace_dir)
    head = [f"Command (from the repository root, TMPDIR=/tmp): `{command}`", ""]
    if section == "decode":
        lines = ["# Decode kernels on the Qwen3-4B layer workload (M = 1, 8, 32), rocprofv3 kernel trace", ""] + head + [
            "Every (M, linear) of the step is launched equally often, so a kernel's mean algorithmic bytes per",
            "launch is the mean over the (M, linear) pairs it serves.  Split-K GEMMs on the tiled kernels also",
            "launch `splitk_reduce_kernel` (listed in the table, not in the kernel's duration).",
            "",
        ]
        for kern in DECODE_KERNELS:
            pairs = [(M, N, K) for M in M_SET for _, K, N in LAYER if ops.plan_info(M, N, K, G).function == kern]
            ds = [d for (k, *_), v in groups.items() if k.startswith(kern + "<") for d in v]
            if not pairs or not ds:
                continue
            mean_b = sum(gemm_bytes(*p) for p in pairs) / len(pairs)
            mean_us = sum(ds) / len(ds)
            lines.append(f"* `{kern}`: {len(pairs)} of the step's {len(M_SET) * len(LAYER)} launches; "
                         f"{len(ds)} dispatches, mean duration {mean_us:.3f} us; mean algorithmic bytes "
                         f"{mean_b / 1e6:.3f} MB; achieved {mean_b / mean_us / 1e3:.1f} GB/s = "
                         f"{mean_b / mean_us / 1e3 / HBM_PEAK_GBS:.4f} of 8 TB/s.")
    elif section.startswith("prefill"):
        M = int(section.split("-")[1])
        rows = _trace_rows(trace_dir)
        lines = [f"# Prefill kernels on the Llama-3-8B linears at M = {M}, rocprofv3 kernel trace", ""] + head + [
            f"Each linear is launched {2 + PROFILE_REPS} times in order (2 warm-ups, {PROFILE_REPS} timed), fp16, "
            "int4 group 128; a call's duration is its GEMM kernel plus its split-K reduction, if any.",
            "",
            "| linear | kernel | calls | mean us per call | TFLOP/s | fraction of 2.5 PFLOP/s |",
            "|---|---|---|---|---|---|"]
        i, tot_f, tot_t = 0, 0, 0.0
        for lname, K, N in PREFILL:
            per = _launches_per_call(ops, M, N, K)
            calls = []
            for c in range(2 + PROFILE_REPS):
                seg = rows[i:i + per]
                i += per
                calls.append((seg[0][0], sum(r[5] for r in seg)))
            timed = [d for _, d in calls[2:]]
            us = sum(timed) / len(timed)
            fl = 2 * M * N * K
            tot_f += fl * len(timed)
            tot_t += sum(timed)
            lines.append(f"| {lname} {K}x{N} | `{calls[-1][0]}` | {len(timed)} | {us:.1f} | {fl / us / 1e6:.1f} | "
                         f"{fl / us / 1e6 / MFMA_FP16_PEAK_TFLOPS:.4f} |")
        tf = tot_f / tot_t / 1e6
        lines += ["", f"* All four linears: {tf:.1f} TFLOP/s = {tf / MFMA_FP16_PEAK_TFLOPS:.4f} of the 2.5 PFLOP/s "
                  "dense fp16 MFMA peak (FLOPs of the timed calls over their summed kernel durations)."]
    elif section == "moe":
        E, H, I, k, T = 128, 2048, 768, 8, 512
        lines = ["# Grouped MoE kernels, Qwen3-30B-A3B-shaped experts (E=128, H=2048, I=768, top-8, T=512), "
                 "rocprofv3 kernel trace", ""] + head + [
            "The forward (top-k softmax, alignment, grouped gate_up GEMM with silu_and_mul, grouped down GEMM",
            "with the routed weight, top-k sum) replayed as HIP graphs over three expert stacks, then each stage",
            "on its own; int4 group 128 with zeros, fp16.  Algorithmic bytes of a GEMM: all experts' int4",
            "weights, zeros and scales plus 2 bytes per element of the routed rows it reads and writes.", ""]
        stage_b = {"<1, 1,": E * gemm_bytes(0, 2 * I, H) + T * k * (H + I) * 2,
                   "<1, 0,": E * gemm_bytes(0, H, I) + T * k * (I + H) * 2}
        tot = 0.0
        for (n, gx, gy, bx), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            mean = sum(v) / len(v)
            tot += mean
            b = next((bb for key, bb in stage_b.items() if n.startswith("moe_gemm_kernel" + key)), None)
            if b is not None:
                lines.append(f"* `{n}` (grid {gx} x {gy}): {len(v)} dispatches, mean {mean:.2f} us, "
                             f"{b / 1e6:.1f} MB -> {b / mean / 1e3:.1f} GB/s = {b / mean / 1e3 / HBM_PEAK_GBS:.4f} "
                             "of 8 TB/s.")
        allb = E * (gemm_bytes(0, 2 * I, H) + gemm_bytes(0, H, I)) + T * k * (H + 2 * I + I + H) * 2
        lines.append(f"* Sum of the stages' mean durations: {tot:.1f} us -> {allb / tot / 1e3:.1f} GB/s = "
                     f"{allb / tot / 1e3 / HBM_PEAK_GBS:.4f} of 8 TB/s for the forward's {allb / 1e6:.1f} MB.")
    elif section.startswith("stack70b"):
        M = int(section.split("-")[1])
        total = sum(d for v in groups.values() for d in v)
        n = sum(len(v) for v in groups.values())
        passes = 22 if M <= 256 else 4  # 2 + 20 graph replays, or 1 + 3 eager passes
        ms = total / passes / 1e3
        byt = STACK70B_LAYERS * sum(gemm_bytes(M, N, K) for _, K, N in STACK70B)
        fl = STACK70B_LAYERS * sum(2 * M * N * K for _, K, N in STACK70B)
        lines = [f"# Llama-3.1-70B-shaped 80-layer AWQ stack at M = {M}, rocprofv3 kernel trace", ""] + head + [
            f"* {n} dispatches over {passes} passes (the warm-up included): {ms:.2f} ms of kernel time per pass "
            f"= {byt / ms / 1e6:.1f} GB/s ({byt / ms / 1e6 / HBM_PEAK_GBS:.4f} of 8 TB/s) and "
            f"{fl / ms / 1e9:.1f} TFLOP/s ({fl / ms / 1e9 / MFMA_FP16_PEAK_TFLOPS:.4f} of 2.5 PFLOP/s)."]
    elif section == "mlp":
        lines = ["# Qwen3-4B gated MLP block (gate_up 2560x19456, silu, down 9728x2560) at M = 1, 8, 32, "
                 "rocprofv3 kernel trace", ""] + head + [
            "The bench's mlp section: each form replayed as HIP graphs over 12 weight copies -- the GEMMs with",
            "the activation as torch ops, the activation in the gate_up GEMM's epilogue (two launches), and at",
            "M <= 16 the whole block in one launch (`mlp_kernel`, 256 workgroups); int4 group 128, fp16."]
    else:
        lines = [f"# {section}, rocprofv3 kernel trace", ""] + head
    lines += [""] + _trace_table(groups)
    return "\n".join(lines) + "\n"


PROBE_GRIDS = ((256, 256), (256, 1024), (512, 256), (1024, 256), (2048, 256))


class Prober:
    """The streaming probe (awq_stream_probe) over C distinct regions of one device buffer: per
    launch shape and byte count, the median duration of one launch, from graphs of C back-to-back
    launches (each region read once per graph, so nothing is served from the Infinity Cache)."""

    def __init__(self, ops, dev, C: int, region_bytes: int):
        self.ops, self.C, self.region = ops, C, (region_bytes + 4095) // 4096 * 4096
        self.buf = torch.empty(C * self.region, dtype=torch.uint8, device=dev)
        self.buf.fill_(7)
        self.sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
        self.cache = {}

    def us(self, nbytes: int, grid: int, block: int) -> float:
        nbytes = nbytes // 16 * 16
        key = (nbytes, grid, block)
        if key not in self.cache:
            def f():
                for c in range(self.C):
                    self.ops.stream_probe(self.buf[c * self.region:], nbytes, grid, block, self.sink)
            g = graph_of(f)
            time_replays([g], 2)
            self.cache[key] = median(replay_samples([g], MEDIAN_SAMPLES)) * 1e3 / self.C
            del g
        return self.cache[key]

    def best(self, nbytes: int) -> tuple:
        return min((self.us(nbytes, g, b), g, b) for g, b in PROBE_GRIDS)


def decode_bench(ops, args, C, linear, step_fn, step_bytes, prober):
    """The decode step: `args.steps` timed graph replays over the C weight copies (each between its
    own HIP events; value from the median), then the median per-launch duration of every
    (M, linear), its attainable ceiling from the streaming probe at the same grid, block and bytes,
    and the dominant kernel's roofline figures."""
    steps = [graph_of(step_fn(c)) for c in range(C)]
    time_replays(steps, args.warmup)
    samples = replay_samples(steps, args.steps)
    ms_med, ms_mean = median(samples), sum(samples) / len(samples)
    del steps

    # Per-launch durations: graphs of C back-to-back launches of one (M, linear)
    # over the C weight copies, MEDIAN_SAMPLES replays.
    per_m, per_kernel = {}, {}
    for M in M_SET:
        mb, mt, mp, lin = 0, 0.0, 0.0, {}
        for name, K, N in LAYER:
            def f(M=M, name=name, K=K, N=N):
                for c in range(C):
                    linear(c, M, name, K, N)
            g = graph_of(f)
            time_replays([g], 2)
            us = median(replay_samples([g], MEDIAN_SAMPLES)) * 1e3 / C
            del g
            b = gemm_bytes(M, N, K)
            info = ops.plan_info(M, N, K, G)
            probe = prober.us(b, info.workgroups, info.threads)
            best_us, best_g, best_b = prober.best(b)
            kern = info.function
            lin[name] = {"us": round(us, 3), "GB/s": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                         "kernel": kern, "grid": info.workgroups, "block": info.threads, "k_slices": info.k_slices,
                         "ceiling_us": round(probe, 3), "frac_of_ceiling": round(probe / us, 4),
                         "best_grid_ceiling_us": round(best_us, 3), "best_grid": [best_g, best_b]}
            acc = per_kernel.setdefault(kern, {"launches": 0, "bytes": 0, "us": 0.0, "probe_us": 0.0})
            acc["launches"] += 1
            acc["bytes"] += b
            acc["us"] += us
            acc["probe_us"] += probe
            mb += b
            mt += us
            mp += probe
        per_m[str(M)] = {"GB/s": round(mb / mt / 1e3, 1), "frac_hbm": round(mb / mt / 1e3 / HBM_PEAK_GBS, 4),
                         "us_per_layer": round(mt, 3), "ceiling_us_per_layer": round(mp, 3),
                         "frac_of_ceiling": round(mp / mt, 4), "linears": lin}
    # The dominant kernel is the one that moves the most of the step's
    # algorithmic bytes.  (Not the most event-timed time: a split-K GEMM on
    # the tiled kernels also runs splitk_reduce_kernel, whose time the events
    # around the GEMM include, so its kernel would be charged for both.)
    dom = max(per_kernel, key=lambda k: per_kernel[k]["bytes"])
    d = per_kernel[dom]
    achieved = d["bytes"] / d["us"] / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(dom),
                "kernel": dom, "launches_per_step": d["launches"],
                "bytes_per_launch_avg": d["bytes"] // d["launches"],
                "us_per_launch_avg": round(d["us"] / d["launches"], 3),
                "attainable_GB/s": round(d["bytes"] / d["probe_us"] / 1e3, 1),
                "frac_of_attainable": round(d["probe_us"] / d["us"], 4)}
    kernels = {k: {"launches_per_step": v["launches"], "GB/s": round(v["bytes"] / v["us"] / 1e3, 1),
                   "us_per_step": round(v["us"], 3), "frac_of_ceiling": round(v["probe_us"] / v["us"], 4)}
               for k, v in per_kernel.items()}
    return {"value": step_bytes / (ms_med * 1e-3) / 1e9, "value_mean": step_bytes / (ms_mean * 1e-3) / 1e9,
            "ms_per_step": ms_med, "ms_per_step_mean": ms_mean, "roofline": roofline, "kernels": kernels,
            "per_m": per_m}


# Llama-3-8B's batches, the reference's graph-captured decode batches below 16
# (cuda_graph.py:76: [1, 2, 4] + multiples of 8), and the decode batches
# 64..160 that graph capture covers.
LLAMA_M = (1, 2, 4, 8, 16, 64, 128, 160, 256, 2048, 8192)

# One GPU's share of tensor-parallel shards (column-parallel layers split N,
# row-parallel ones K: weight_loader.py:40-69, linear.py:127-194): the
# Llama-3.1-70B stack at TP8 and Llama-3-8B at TP2 and TP4.
TP_SHARDS = {
    "70b_tp8": [("qkv_proj", 8192, 1280), ("o_proj", 1024, 8192), ("gate_up_proj", 8192, 7168),
                ("down_proj", 3584, 8192)],
    "llama3_8b_tp2": [("qkv_proj", 4096, 3072), ("o_proj", 2048, 4096), ("gate_up_proj", 4096, 14336),
                      ("down_proj", 7168, 4096)],
    "llama3_8b_tp4": [("qkv_proj", 4096, 1536), ("o_proj", 1024, 4096), ("gate_up_proj", 4096, 7168),
                      ("down_proj", 3584, 4096)],
}
TP_M = (1, 8, 32, 2048)


def linears_bench(ops, dev, prober, shapes, Ms, dtype=torch.float16, copies: int = 10, seed: int = 3,
                  ceilings: bool = True) -> dict:
    """A set of linears at several M: M <= 256 as graphs of back-to-back launches over `copies`
    weight copies, larger M as eager calls; median over MEDIAN_SAMPLES samples.  GB/s against the
    HBM peak (and the streaming probe's ceiling at M <= 32) and TFLOP/s against the dense MFMA peak;
    `bound` is the roofline the layer's arithmetic intensity (flop per algorithmic byte) puts it
    under; `kernel` names the HIP kernel the GEMM launch runs."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    reps = [{name: make_repacked(ops, K, N, gen, dev, dtype) for name, K, N in shapes} for _ in range(copies)]
    cnts = {name: ops.make_counters(N, dev) for name, K, N in shapes}
    xg = torch.Generator(device=dev).manual_seed(seed + 1)
    res = {}
    for M in Ms:
        xs = {K: torch.randn((M, K), generator=xg, device=dev).to(dtype) for K in {k for _, k, _ in shapes}}
        outs = {name: torch.empty((M, N), dtype=dtype, device=dev) for name, _, N in shapes}
        lin, tb, tf, tt = {}, 0, 0, 0.0
        for name, K, N in shapes:
            def call(c, name=name, K=K, N=N):
                ops.gemm(xs[K], reps[c][name], K, N, G, counters=cnts[name], out=outs[name])
            if M <= 256:
                g = graph_of(lambda: [call(c) for c in range(copies)])
                time_replays([g], 2)
                us = median(replay_samples([g], MEDIAN_SAMPLES)) * 1e3 / copies
                del g
            else:
                for _ in range(3):
                    call(0)
                it = iter(range(10 ** 9))
                us = median(call_samples(lambda: call(next(it) % copies), MEDIAN_SAMPLES)) * 1e3
            b, fl = gemm_bytes(M, N, K), 2 * M * N * K
            info = ops.plan_info(M, N, K, G)
            e = {"us": round(us, 2), "GB/s": round(b / us / 1e3, 1), "TFLOP/s": round(fl / us / 1e6, 1),
                 "kernel": info.function, "grid": info.workgroups, "k_slices": info.k_slices}
            e.update({"frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                      "frac_mfma": round(fl / us / 1e6 / MFMA_FP16_PEAK_TFLOPS, 4)})
            if M <= 32 and ceilings:
                probe = prober.us(b, info.workgroups, info.threads)
                e.update({"ceiling_us": round(probe, 3), "frac_of_ceiling": round(probe / us, 4)})
            lin[name] = e
            tb, tf, tt = tb + b, tf + fl, tt + us
        res[str(M)] = {"us_per_layer": round(tt, 2), "GB/s": round(tb / tt / 1e3, 1),
                       "frac_hbm": round(tb / tt / 1e3 / HBM_PEAK_GBS, 4), "TFLOP/s": round(tf / tt / 1e6, 1),
                       "frac_mfma": round(tf / tt / 1e6 / MFMA_FP16_PEAK_TFLOPS, 4),
                       "bound": "hbm" if tf / tb < MFMA_FP16_PEAK_TFLOPS * 1e3 / HBM_PEAK_GBS else "mfma",
                       "linears": lin}
        del xs, outs
    del reps
    torch.cuda.synchronize()
    return res


def llama_bench(ops, dev, gen, prober, copies: int = 10) -> dict:
    """Llama-3-8B's four linears at every M the workload names (1, 16, 256, 2048, 8192), at the
    graph-captured decode batches 2, 4, 8 and 64, 128, 160; int4 group 128, fp16."""
    res = linears_bench(ops, dev, prober, PREFILL, LLAMA_M, copies=copies)
    return {"workload": "Llama-3-8B AWQ linears (qkv 4096x6144, o 4096x4096, gate_up 4096x28672, down 14336x4096), "
                        f"int4 group 128 with zeros, fp16, M in {list(LLAMA_M)}; {copies} weight copies; median of "
                        f"{MEDIAN_SAMPLES}", "per_m": res}


def _compact(res: dict) -> dict:
    """Per-M summary plus each linear's time, rate and kernel (a shorter record)."""
    out = {}
    for M, v in res.items():
        out[M] = {k: v[k] for k in ("us_per_layer", "GB/s", "frac_hbm", "TFLOP/s", "frac_mfma", "bound")}
        out[M]["linears"] = {n: {k: e[k] for k in ("us", "kernel", "k_slices", "frac_of_ceiling") if k in e}
                             for n, e in v["linears"].items()}
    return out


def tp_bench(ops, dev, prober) -> dict:
    """One GPU's share of the tensor-parallel shards (TP_SHARDS) at M = 1, 8, 32 and 2048, fp16."""
    out = {"workload": "one GPU's shard of column-parallel (N / tp) and row-parallel (K / tp) AWQ linears, "
                       "int4 group 128 with zeros, fp16; Llama-3.1-70B at TP8 (qkv 8192x1280, o 1024x8192, "
                       "gate_up 8192x7168, down 3584x8192), Llama-3-8B at TP2 and TP4; the all-reduce of the "
                       "row-parallel partials is not timed (one GPU)"}
    for name, shapes in TP_SHARDS.items():
        out[name] = _compact(linears_bench(ops, dev, prober, shapes, TP_M, copies=10, seed=11))
    return out


def bf16_bench(ops, dev, prober) -> dict:
    """bf16 activations and scales (the reference engine's default dtype, llm/llm.py:34, with
    scales cast to it, engine.py:171): the Qwen3-4B decode layer at M = 1, 8, 32 and the
    Llama-3-8B linears at M = 2048."""
    dec = linears_bench(ops, dev, prober, LAYER, M_SET, dtype=torch.bfloat16, copies=12, seed=21)
    pf = linears_bench(ops, dev, prober, PREFILL, (PREFILL_M,), dtype=torch.bfloat16, copies=3, seed=23)
    return {"workload": "bf16 activations and scales: Qwen3-4B decode layer (M = 1, 8, 32) and Llama-3-8B linears "
                        f"at M = {PREFILL_M}, int4 group 128 with zeros",
            "decode": _compact(dec), "prefill": _compact(pf)}


def hipblaslt_bench(ops, dev, reps: int = 15) -> dict:
    """The vendor library's dense fp16 GEMM (torch.matmul, hipBLASLt on ROCm) on the Llama-3-8B
    linears at M = 2048 and 8192 with fp16 weights of the same shapes: the dense-GEMM rate the
    W4A16 kernels (which also dequantise every weight) are compared with."""
    gen = torch.Generator(device=dev).manual_seed(31)
    out = {"library": "torch.matmul (hipBLASLt), fp16 dense weights [K, N], fp32 accumulation"}
    for M in (PREFILL_M, 8192):
        tt, tf, lin = 0.0, 0, {}
        for name, K, N in PREFILL:
            x = torch.randn((M, K), generator=gen, device=dev).to(torch.float16)
            w = (torch.randn((K, N), generator=gen, device=dev) * 0.02).to(torch.float16)
            y = torch.empty((M, N), dtype=torch.float16, device=dev)
            for _ in range(3):
                torch.matmul(x, w, out=y)
            us = median(call_samples(lambda: torch.matmul(x, w, out=y), reps)) * 1e3
            fl = 2 * M * N * K
            lin[name] = {"us": round(us, 2), "TFLOP/s": round(fl / us / 1e6, 1)}
            tt, tf = tt + us, tf + fl
            del x, w, y
        out[str(M)] = {"TFLOP/s": round(tf / tt / 1e6, 1), "frac": round(tf / tt / 1e6 / MFMA_FP16_PEAK_TFLOPS, 4),
                       "linears": lin}
    torch.cuda.synchronize()
    return out


# Planner check on shapes it was not tuned on: one GPU's share of tensor-
# parallel linears, beside the Qwen3-4B and Llama-3-8B configuration shapes.
# Every other built kernel form is forced through the planner overrides and
# timed the same way (graph replay over rotating weight copies, best of two
# rounds); a case passes when the planner's plan is within 5% of the fastest.
SWEEP_GROUPS = {"qwen3_4b": LAYER, "llama3_8b": PREFILL, "llama31_70b": STACK70B, **TP_SHARDS}
_FORCE_TILED = 99999


def _sweep_forms(M: int) -> list:
    if M > 32:
        return [{"tiled_min_m": 1, "tiled_bm": c} for c in (64, 128, 1064, 1128, 2064, 2128, 8064, 8128, 9064, 9128)]
    forms = [{"tiled_min_m": _FORCE_TILED, "gemv_max_m": 32, "gemv_variant": v}
             for v in (11083, 11084, 11086, 11088, 11165, 11168, 12083, 12084, 15037, 21083, 23054)]
    forms += [{"tiled_min_m": _FORCE_TILED, "gemv_max_m": 0, "skinny_variant": v}
              for v in (10104, 10108, 10116, 10202, 10401, 10404, 20202, 20401, 20204)]
    forms += [{"kslice_variant": v} for v in (142, 141, 222, 412)]
    forms += [{"tiled_min_m": 1, "tiled_bm": c} for c in (32, 4032, 64, 1064)]
    return forms


def planner_sweep(ops, dev, groups, Ms) -> None:
    gen = torch.Generator(device=dev).manual_seed(0)
    print("| shapes | layer | K x N | M | planner's plan | us | fastest form | us | ratio |", flush=True)
    print("|---|---|---|---|---|---|---|---|---|", flush=True)
    for grp in groups:
        for name, K, N in SWEEP_GROUPS[grp]:
            for M in Ms:
                C = 3 if M >= 1024 else 8
                reps = [make_repacked(ops, K, N, gen, dev) for _ in range(C)]
                cnt = ops.make_counters(N, dev)
                x = torch.randn((M, K), generator=gen, device=dev).to(torch.float16)
                out = torch.empty((M, N), dtype=torch.float16, device=dev)

                def timed():
                    f = lambda: [ops.gemm(x, r, K, N, G, counters=cnt, out=out) for r in reps]  # noqa: E731
                    for _ in range(2):
                        f()
                    g = graph_of(f)
                    time_replays([g], 2)
                    return median(replay_samples([g], 15 if M >= 1024 else 30)) * 1e3 / C

                best = {}
                default = None
                for _ in range(2):
                    for ov in [None] + _sweep_forms(M):
                        ops.clear_plan_overrides()
                        for k, v in (ov or {}).items():
                            ops.set_plan_override(k, v)
                        i = ops.plan_info(M, N, K, G)
                        key = f"{i.function} {i.variant} ks{i.k_slices} {i.workgroups}x{i.threads}"
                        if ov is None:
                            default = key
                        best[key] = min(best.get(key, float("inf")), timed())
                ops.clear_plan_overrides()
                fk = min(best, key=best.get)
                print(f"| {grp} | {name} | {K} x {N} | {M} | {default} | {best[default]:.2f} | {fk} | "
                      f"{best[fk]:.2f} | {best[default] / best[fk]:.3f} |", flush=True)
                del reps
                torch.cuda.empty_cache()


def headline_summary(dec, prefill, moe, llama, stack, mlp, bounds) -> dict:
    """The sections' key figures in a few hundred characters, printed last on the JSON line so that a
    log that keeps only the end of the line still holds them: per decode batch [us per layer, fraction
    of the streaming ceiling, GB/s]; per Llama-3-8B batch [us per layer, fraction of the roofline its
    arithmetic intensity puts it under]; prefill, MoE, 70B-stack, gated-MLP and bound fractions."""
    out: dict = {}
    if dec is not None:
        out["decode_per_m"] = {M: [v["us_per_layer"], v["frac_of_ceiling"], v["GB/s"]] for M, v in dec["per_m"].items()}
    if prefill is not None:
        out["prefill_frac"] = {"2048": prefill["frac"], "8192": prefill["m8192"]["frac"]}
    if moe is not None:
        out["moe"] = [moe["us"], moe["frac"]]
    if llama is not None:
        out["llama3_8b"] = {M: [v["us_per_layer"], v["frac_hbm"] if v["bound"] == "hbm" else v["frac_mfma"]]
                            for M, v in llama["per_m"].items()}
    if stack is not None:
        out["stack70b"] = {M: v["frac_hbm"] if M == "64" else v["frac_mfma"] for M, v in stack["per_m"].items()}
    if mlp is not None:
        out["gated_mlp_fused_us"] = {M: v["fused_us"] for M, v in mlp["per_m"].items()}
    if bounds is not None:
        out["mfma_probe_frac"] = [bounds[k]["frac"] for k in ("1_wave_per_simd", "2_waves_per_simd") if k in bounds]
        hb = bounds.get("hipblaslt_dense_fp16")
        if hb:
            out["hipblaslt_frac"] = {M: hb[M]["frac"] for M in ("2048", "8192") if M in hb}
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--copies", type=int, default=36, help="distinct weight copies rotated through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-mlp", action="store_true", help="skip the fused/unfused gated MLP block comparison")
    ap.add_argument("--no-stack", action="store_true", help="skip the 70B-shaped stack (35.6 GB of weights)")
    ap.add_argument("--planner-sweep", nargs=2, metavar=("GROUPS", "MS"),
                    help="time the planner's plan against every other built form on shape groups (comma list of "
                         + ", ".join(SWEEP_GROUPS) + ") at batch sizes MS (comma list); print a markdown table")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the tensor-parallel shard, bf16 and hipBLASLt comparison sections")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the decode step (profiling runs of the other sections; no value is reported)")
    ap.add_argument("--rocprof-summary", nargs=2, metavar=("SECTION", "TRACE_DIR"),
                    help="print a markdown summary (decode or a --profile-workload NAME) of a rocprofv3 --kernel-trace run "
                         "of this script and exit")
    ap.add_argument("--rocprof-command", default="rocprofv3 --kernel-trace --stats -f csv -d <dir> -o bench -- "
                                                  "python3 bench.py <args>",
                    help="the profiled command, quoted in the summary's header")
    ap.add_argument("--profile-workload", metavar="NAME",
                    help="run one section's launch sequence for rocprofv3 --kernel-trace and exit: prefill-2048, "
                         "prefill-8192, moe, stack70b-64, stack70b-4096, mlp, probes, or sq (the SQ-counter workload)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run each decode GEMM of the step a few times eagerly plus a 256 MiB copy, for rocprofv3 --pmc")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print a markdown summary of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of --pmc-workload")
    ap.add_argument("--sq-summary", nargs="+", metavar="PMC_DIR",
                    help="print a markdown summary of the SQ-counter passes (rocprofv3 --pmc of --profile-workload sq, "
                         "one directory per counter set) and exit")
    ap.add_argument("--marker-summary", metavar="TRACE_DIR",
                    help="print a markdown summary of a rocprofv3 --marker-trace --kernel-trace run (the C ABI's "
                         "roctx ranges) and exit")
    args = ap.parse_args()
    if args.marker_summary:
        print(marker_summary(args.marker_summary, args.rocprof_command), end="")
        return 0
    if args.rocprof_summary:
        section, trace_dir = args.rocprof_summary
        print(rocprof_summary(trace_dir, args.rocprof_command, section), end="")
        return 0
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary), end="")
        return 0
    if args.sq_summary:
        print(sq_summary(args.sq_summary), end="")
        return 0
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the engine's multi-GPU sharding is a "
              "design, not a measured path", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        return 2

    from sglite_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    if args.pmc_workload:
        return pmc_workload(ops, dev, gen)
    if args.planner_sweep:
        planner_sweep(ops, dev, args.planner_sweep[0].split(","), [int(m) for m in args.planner_sweep[1].split(",")])
        return 0
    if args.profile_workload:
        profile_workload(args.profile_workload, ops, dev, gen)
        return 0
    C = args.copies
    if args.no_decode:
        C = 0
    reps = [{name: make_repacked(ops, K, N, gen, dev) for name, K, N in LAYER} for _ in range(C)]
    cnts = [{name: ops.make_counters(N, dev) for name, K, N in LAYER} for _ in range(C)]
    xg = torch.Generator(device=dev).manual_seed(1)
    xs = {(M, K): torch.randn((M, K), generator=xg, device=dev).to(torch.float16)
          for M in M_SET for K in {k for _, k, _ in LAYER}}
    outs = {(M, name): torch.empty((M, N), dtype=torch.float16, device=dev) for M in M_SET for name, _, N in LAYER}
    torch.cuda.synchronize()

    def linear(c, M, name, K, N):
        ops.gemm(xs[(M, K)], reps[c][name], K, N, G, counters=cnts[c][name], out=outs[(M, name)])

    def step_fn(c):
        def f():
            for M in M_SET:
                for name, K, N in LAYER:
                    linear(c, M, name, K, N)
        return f

    step_bytes = sum(gemm_bytes(M, N, K) for M in M_SET for _, K, N in LAYER)
    # Region per probe launch: the largest decode linear's bytes (Qwen3-4B gate_up / Llama-3-8B gate_up).
    prober = Prober(ops, dev, max(C, 10), max(gemm_bytes(32, N, K) for _, K, N in LAYER + PREFILL))
    dec = None
    if C > 0:
        progress("decode step")
        dec = decode_bench(ops, args, C, linear, step_fn, step_bytes, prober)
    del reps
    torch.cuda.synchronize()

    llama = tp = bf16 = None
    if not args.no_prefill:
        progress("llama3-8b sweep")
        llama = llama_bench(ops, dev, gen, prober)
    if not args.no_extra:
        progress("tensor-parallel shards")
        tp = tp_bench(ops, dev, prober)
        progress("bf16")
        bf16 = bf16_bench(ops, dev, prober)
    del prober
    torch.cuda.synchronize()
    prefill = None
    if llama is not None:
        pm = llama["per_m"][str(PREFILL_M)]
        prefill = {"workload": "Llama-3-8B AWQ linears (qkv 4096x6144, o 4096x4096, gate_up 4096x28672, "
                               f"down 14336x4096) at M={PREFILL_M}, fp16", "TFLOP/s": pm["TFLOP/s"],
                   "peak": MFMA_FP16_PEAK_TFLOPS, "frac": pm["frac_mfma"],
                   "linears": {k: {"us": v["us"], "TFLOP/s": v["TFLOP/s"], "kernel": v["kernel"]}
                               for k, v in pm["linears"].items()},
                   "m8192": {"TFLOP/s": llama["per_m"]["8192"]["TFLOP/s"],
                             "frac": llama["per_m"]["8192"]["frac_mfma"]}}

    mlp = moe = stack = None
    if not args.no_mlp:
        progress("gated mlp")
        mlp = mlp_bench(ops, dev, gen)
    if not args.no_moe:
        progress("moe")
        moe = moe_bench(ops, dev, gen)
    if not args.no_stack:
        progress("70b stack")
        stack = stack70b_bench(ops, dev, gen)

    bounds = None
    if not args.no_prefill:
        progress("mfma probe")
        bounds = bounds_bench(ops, dev)
        if not args.no_extra:
            progress("hipblaslt")
            bounds["hipblaslt_dense_fp16"] = hipblaslt_bench(ops, dev)

    cpu = None
    if not args.no_cpu_baseline:
        progress("cpu baseline")
        cpu = cpu_baseline()

    line = {
        "metric": METRIC,
        "value": None if dec is None else round(dec["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None if dec is None else round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "Qwen3-4B decoder layer AWQ linears (qkv 2560x6144, o_proj 4096x2560, "
                               "gate_up 2560x19456, down 9728x2560), int4 group 128 with zero points, fp16 "
                               "scales/activations, M in {1, 8, 32} per step, HIP-graph replay; value and "
                               "ms_per_step from the median of the timed steps",
                   "weight_copies": C, "weight_bytes_rotated": C * sum(gemm_bytes(0, N, K) for _, K, N in LAYER),
                   "step_bytes": step_bytes,
                   "value_from_mean": None if dec is None else round(dec["value_mean"], 1),
                   "ms_per_step_mean": None if dec is None else round(dec["ms_per_step_mean"], 5)},
        "roofline": None if dec is None else dec["roofline"],
        "cpu_baseline": cpu,
        # The long sections first, the decode summary last: the end of the
        # line is what a truncated log keeps.
        "llama3_8b": llama,
        "tp_shards": tp,
        "bf16": bf16,
        "stack70b": stack,
        "bounds": bounds,
        "moe": moe,
        "mlp": mlp,
        "prefill": prefill,
        "decode_kernels": None if dec is None else dec["kernels"],
        "per_m": None if dec is None else dec["per_m"],
        "summary": headline_summary(dec, prefill, moe, llama, stack, mlp, bounds),
    }
    print(json.dumps(line))
    return 0


def progress(what: str) -> None:
    print(f"[bench] {what} ({time.strftime('%H:%M:%S')})", file=sys.stderr, flush=True)


if __name__ == "__main__":
    sys.exit(main())
