"""Benchmark of the quantized dequant-GEMV hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: Q4_K GEMV, W 14336 x 4096 in GGUF Q4_K
superblocks, f32 x ~ N(0,1), batch 1.  A step is one hip_gemv_async call over
one of ROT weight copies (>= 768 MB in total, so the 256 MB MALL cannot serve
repeats); weights and x are resident in HBM before the timed region.  The W
warm-up steps and the K timed steps go out back to back on one stream, with a
device timestamp on each side of the K.
Prints ONE JSON line.  `value` = algorithmic bytes (weights + x + y) per step x K
/ GPU time of the K steps (device wall-clock stamps around them).
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
Q4K = 12


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # ~15 ms of back-to-back launches before the timed region: the timed steps then
    # run at the clocks of a sustained stream (20 warm-up steps measured ~1% slower)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--lead-ms", type=float, default=0.0,
                    help="spin ahead of the headline's launches (0: sized for the launch count)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-decode", action="store_true", help="skip the 8B-shape decode-step leg")
    ap.add_argument("--decode-reps", type=int, default=20)
    ap.add_argument("--only-moe", action="store_true",
                    help="only the configs[4] MoE leg (grouped, per-expert and routed), one JSON line")
    ap.add_argument("--only-forward", action="store_true",
                    help="only run the end-to-end decode-step leg (for profiling its kernels)")
    ap.add_argument("--forward-n", type=str, default="1,4,16,32",
                    help="token batches of the end-to-end decode-step leg (comma separated)")
    ap.add_argument("--batched-suite", action="store_true",
                    help="only time hip_gemm at the batched shapes of configs[3]/[4] (16 tokens; for profiling "
                         "the matrix-core GEMM kernels)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 device copies of 256 MiB (torch copy kernel), to calibrate the "
                         "FETCH_SIZE / WRITE_SIZE counters against known bytes")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus N>1 is not supported "
                                   "(across GPUs the GEMV would shard by output rows, each GPU holding its rows' blocks)"}))
        sys.exit(2)
    import torch

    if args.copy_calibration:
        src = torch.empty(256 * 2**20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel(), "copies": 5}))
        return

    if args.batched_suite:
        print(json.dumps({"batched": batched_suite(torch)}), flush=True)
        return

    if args.only_moe:
        print(json.dumps({"moe": moe_leg(torch, args.decode_reps)}), flush=True)
        return

    if args.only_forward:
        from saient_quartz_amd.decode import ModelConfig
        wbytes = ModelConfig().weight_bytes()
        ns = [int(v) for v in args.forward_n.split(",")]
        print(json.dumps({"forward": forward_leg(torch, args.decode_reps, wbytes, ns)}), flush=True)
        return

    from saient_quartz_amd import lib, synth_device, type_size
    from saient_quartz_amd.api import check

    L = lib()
    out_dim, in_dim = 14336, 4096
    wbytes = type_size(Q4K, out_dim * in_dim)
    alg_bytes = wbytes + 4 * in_dim + 4 * out_dim
    rot = max(3, -(-768 * 2**20 // wbytes))
    Ws = [synth_device.q4k(out_dim, in_dim, seed=20261201 + 1 + i) for i in range(rot)]
    x = torch.randn(in_dim, device="cuda", generator=torch.Generator(device="cuda").manual_seed(7))
    y = torch.empty(out_dim, device="cuda")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def step(i):
        check("hip_gemv_async", L.hip_gemv_async(Q4K, Ws[i % rot].data_ptr(), x.data_ptr(), y.data_ptr(),
                                                 in_dim, out_dim, sp))

    stamps = torch.zeros(2, dtype=torch.int64, device="cuda")
    khz = L.hip_wallclock_khz()
    if khz <= 0:
        raise SystemExit("hip_wallclock_khz failed")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    y_ref = y.clone()
    step(args.warmup + args.steps - 1)  # the timed region's last step, on its own
    torch.cuda.synchronize()
    y_ref.copy_(y)

    # Timed region: the launches go out eagerly on one stream behind a spin
    # kernel that keeps the GPU busy while the host enqueues them (a HIP graph
    # replay of the same launches measured 0.27 us slower per launch on this
    # image).  W warm-up steps, a device timestamp, the K timed steps and a
    # second timestamp; each stamp is a one-thread kernel writing
    # s_memrealtime once the step before it has completed, so the stamps
    # bracket exactly the K steps.  Step i uses weight copy i % rot.
    # host enqueue time (about 6 us per launch), with margin
    lead_ms = args.lead_ms if args.lead_ms > 0 else 1.0 + 0.006 * (args.warmup + args.steps)
    torch.cuda._sleep(int(lead_ms * 2.0e6))
    for i in range(args.warmup):
        step(i)
    check("hip_timestamp_async", L.hip_timestamp_async(stamps.data_ptr(), sp))
    h0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    h1 = time.perf_counter()
    check("hip_timestamp_async", L.hip_timestamp_async(stamps.data_ptr() + 8, sp))
    torch.cuda.synchronize()
    if not torch.equal(y, y_ref):
        raise SystemExit("the timed region's last result differs from the same step launched on its own")
    t0, t1 = (int(v) for v in stamps.tolist())
    total_ms = (t1 - t0) / khz
    ms_per_step = total_ms / args.steps
    if (h1 - h0) * 1e3 > total_ms + lead_ms:
        print(f"warning: host enqueue ({(h1 - h0) * 1e3:.2f} ms) may have trailed the GPU", file=sys.stderr)

    # Kernel duration: the K kernels run back to back, so the per-step average
    # is the interval between consecutive completions.  The rocprofv3
    # kernel-trace average of the same command's timed launches is committed
    # beside it (rocprof_kernel_us).
    kern_ms = ms_per_step
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9

    traffic = measured_traffic(ROOT / "profiles" / "mmv16_q4k_14336x4096_traffic.md")
    del Ws
    decode = None if args.no_decode else decode_leg(torch, args.decode_reps)
    moe = None if args.no_decode else moe_leg(torch, args.decode_reps)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(out_dim, in_dim, args.cpu_seconds)

    rec = {
        "metric": "Q4_K GEMV effective HBM GB/s (% of peak); 8B-shape decode tok/s at 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 activations/accumulate",
        "data": f"synthetic seeded GGUF Q4_K blocks, {rot} rotated copies ({rot * wbytes / 2**20:.0f} MiB)",
        "config": {"workload": "Q4_K dequant-GEMV 14336x4096 (Llama-3-8B ffn_up), batch 1",
                   "out_dim": out_dim, "in_dim": in_dim, "batch": 1, "bytes_per_step": alg_bytes},
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "qh_mmv16<M16Q4K, 16, 1, true, false, false, 1>",
                     "kernel_us": round(kern_ms * 1e3, 3),
                     "kernel_us_source": "device wall-clock stamps around the K back-to-back launches of the timed "
                                         "region, per launch (the time between consecutive completions)",
                     "rocprof_kernel_us": profiled_kernel_us(ROOT / "profiles" / "mmv16_q4k_14336x4096_kernel_stats.md")},
        "cpu_baseline": cpu,
        "decode": decode,
        "moe": moe,
    }
    print(json.dumps(rec), flush=True)


def batched_suite(torch, reps=50):
    """hip_gemm with 16 tokens (4 for the 4-sequence step's big matrices, 32 for
    the 17-32-token tile) at
    the batched shapes of BASELINE.json configs[3] (Q4_K gate/up, Q6_K down)
    and configs[4] (IQ3_S / IQ2_XXS expert gate/up and down): each shape's
    `reps` calls over rotated weights captured in one HIP graph, events around
    a replay.  Reports us per call and weight GB/s."""
    from saient_quartz_amd import lib, synth_device, type_size
    from saient_quartz_amd.api import check

    L = lib()
    out = {}
    for t, o, i, n in ((12, 14336, 4096, 16), (14, 4096, 14336, 16), (12, 14336, 4096, 4), (14, 4096, 14336, 4),
                       (21, 14336, 4096, 16), (21, 4096, 14336, 16), (16, 14336, 4096, 16), (16, 4096, 14336, 16),
                       (12, 14336, 4096, 32), (14, 4096, 14336, 32), (21, 14336, 4096, 32), (16, 14336, 4096, 32)):
        wb = type_size(t, o * i)
        rot = max(3, -(-768 * 2**20 // wb))
        Ws = [synth_device.weights(t, o, i, seed=40 + k) for k in range(rot)]
        x = torch.randn(n, i, device="cuda")
        y = torch.empty(n, o, device="cuda")
        sp = torch.cuda.current_stream().cuda_stream
        for k in range(3):
            check("hip_gemm_async", L.hip_gemm_async(t, Ws[k % rot].data_ptr(), x.data_ptr(), y.data_ptr(), i, o, n, sp))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = torch.cuda.current_stream().cuda_stream
            for k in range(reps):
                check("hip_gemm_async", L.hip_gemm_async(t, Ws[k % rot].data_ptr(), x.data_ptr(), y.data_ptr(), i, o,
                                                         n, cs))
        g.replay()
        torch.cuda.synchronize()
        us = timed_replay(torch, g) / reps * 1e3
        out[f"type{t}_{o}x{i}_n{n}"] = {"us": round(us, 2), "weight_GB_s": round(wb / us / 1e3, 1)}
        del Ws, g
        torch.cuda.empty_cache()
    return out


def decode_leg(torch, reps):
    """Llama-3-8B-shaped Q4_K_M decode step: the 225
    weight GEMVs of one step (32 layers x 7 + head) captured in one HIP graph,
    timed over `reps` replays, for N = 1, 4, 16 tokens.  At N = 1 the q+k and
    gate+up projections go out as one hip_gemv_multi launch each ("n1"; "n1_unfused"
    is one launch per matrix).  Weight streaming only; the end-to-end steps with
    the glue are forward_leg's n*_full_* entries."""
    from saient_quartz_amd.decode import DecodeStep, Shape

    shape = Shape()
    wbytes = shape.weight_bytes()
    step = DecodeStep(shape, n_max=16)
    out = {"workload": "Llama-3-8B-shaped Q4_K_M decode step, random-init weights: n*_full_* end to end (embedding "
                       "to logits, N sequences in lockstep), n1/n4/n16 the weight GEMVs/GEMMs alone",
           "weight_bytes": wbytes, "roofline_tok_s_n1": round(HBM_PEAK_GBS * 1e9 / wbytes, 1)}
    full = forward_leg(torch, reps, wbytes)
    out.update(full)
    for n, fuse in ((1, False), (1, True), (4, True), (16, True)):
        g = torch.cuda.CUDAGraph()
        step.issue(n, fuse=fuse)  # eager warm-up (first-call device queries happen outside capture)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            step.issue(n, fuse=fuse)
        g.replay()
        torch.cuda.synchronize()
        ms = timed_replay(torch, g, reps) / reps
        out[f"n{n}" + ("" if fuse or n > 1 else "_unfused")] = {"ms_per_step": round(ms, 4), "tok_s": round(n * 1e3 / ms, 1),
                        "weight_GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                        "frac_of_weight_roofline": round(wbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)}
        del g
    del step
    torch.cuda.empty_cache()
    return out


def forward_leg(torch, reps, wbytes, ns=(1, 4, 16, 32)):
    """End-to-end Llama-3-8B-shaped decode steps generating tokens, with the
    tokens and the position in device memory (issue(dev=True, greedy=True):
    each step ends with the greedy pick, which writes the next tokens and
    advances the position), `reps` consecutive steps from KV position 0 and
    from 511, i.e. positions p0 .. p0 + reps - 1, each step feeding the next:
      n*_full_pos*: the steps issued eagerly on one stream (no host sync, no
             host read between steps; events around them, a spin kernel ahead
             so the host's enqueue is not timed; issue_ms_per_step is the
             host's own time to enqueue a step);
      n*_graph_pos*: the same step captured once in a HIP graph and replayed.
      N = 1: ForwardStep (embedding lookup, 32 x [fused norm + q/k/v, RoPE + KV
             append + attention, o + residual, fused norm + gate/up + SwiGLU,
             down + residual], fused final norm + head, greedy pick; 5
             launches per layer);
      N = 4, 16, 32: BatchStep, N sequences in lockstep with their own K/V
             caches (batched matrix-core GEMMs, one weight pass per 16 tokens,
             or per 32 on two image halves, and batched glue).
    n1_eager_hostargs_pos0: N = 1 with host token and position arguments (the
    reference's calling convention), issued eagerly."""
    from saient_quartz_amd.decode import BatchStep, ForwardStep, ModelConfig

    cfg = ModelConfig(max_seq=1024)
    weights = ForwardStep.random_weights(cfg)
    out = {}

    def rec_of(ms, n, pos):
        return {"ms_per_step": round(ms, 4), "tok_s": round(n * 1e3 / ms, 1),
                "weight_GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                "frac_of_weight_roofline": round(wbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
                "positions": [pos, pos + reps - 1]}

    for n in ns:
        step = ForwardStep(cfg, weights) if n == 1 else BatchStep(cfg, weights, n)
        tokens = [(7 * i + 3) % 1000 for i in range(n)]
        set_state = (lambda pos: step.set_state(tokens[0], pos)) if n == 1 else (lambda pos: step.set_state(tokens, pos))
        set_state(0)
        step.issue(dev=True, greedy=True)  # warm-up (first-call device queries happen outside capture)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step.issue(dev=True, greedy=True)
        for pos in (0, 511):
            # eager
            set_state(pos)
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(int(2.0e6 * (1.0 + 3.0 * reps)))  # ~3 ms of lead per step
            t0.record()
            h0 = time.perf_counter()
            for _ in range(reps):
                step.issue(dev=True, greedy=True)
            h1 = time.perf_counter()
            t1.record()
            torch.cuda.synchronize()
            ms = t0.elapsed_time(t1) / reps
            st = step.state.cpu().tolist()
            if st[-1] != pos + reps:
                raise SystemExit(f"decode state did not advance: {st[-1]} != {pos + reps}")
            if not torch.isfinite(step.logits).all():
                raise SystemExit("decode step produced non-finite logits")
            r = rec_of(ms, n, pos)
            r["issue_ms_per_step"] = round((h1 - h0) * 1e3 / reps, 4)
            if n == 1:
                r["launches"] = 1 + 5 * cfg.layers + 2
            out[f"n{n}_full_pos{pos}"] = r
            # graph
            set_state(pos)
            g.replay()
            set_state(pos)
            torch.cuda.synchronize()
            ms = timed_replay(torch, g, reps) / reps
            if step.state.cpu().tolist()[-1] != pos + reps:
                raise SystemExit("decode state did not advance in the graph replays")
            out[f"n{n}_graph_pos{pos}"] = rec_of(ms, n, pos)
        del g
        if n == 1:
            out["n1_eager_hostargs_pos0"] = eager_steps(torch, step, reps)
        del step
        torch.cuda.empty_cache()
    del weights
    torch.cuda.empty_cache()
    return out


def eager_steps(torch, step, reps):
    """`reps` ForwardStep steps at positions 0 .. reps-1 issued eagerly with
    host arguments: GPU time between events, and the host's issue time."""
    for pos in range(3):
        step.issue(11, pos)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1_000_000)
    t0.record()
    h0 = time.perf_counter()
    for pos in range(reps):
        step.issue(11 + pos, pos)
    h1 = time.perf_counter()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    return {"ms_per_step": round(ms, 4), "tok_s": round(1e3 / ms, 1),
            "issue_ms_per_step": round((h1 - h0) * 1e3 / reps, 4), "positions": [0, reps - 1]}


def moe_leg(torch, reps):
    """Mixtral-shaped MoE expert layer: 8 experts x
    (gate, up, down) with 16 gathered tokens each, IQ3_S and IQ2_XXS, one HIP
    graph per layer step, timed over `reps` replays: grouped (gate+up of all
    experts in one hip_gemm_grouped call, down in one hip_gemm_moe call) and
    per expert (24 hip_gemm calls, "<type>_per_expert")."""
    from saient_quartz_amd.decode import MoeLayer

    out = {"workload": "Mixtral-8x7B-shaped MoE expert layer: 8 experts, gate/up 14336x4096 + down 4096x14336, "
                       "16 tokens gathered per expert (top-2 of 64 tokens), random-init weights"}
    for name, t, grouped in (("iq3_s", 21, True), ("iq3_s_per_expert", 21, False), ("iq2_xxs", 16, True),
                             ("iq2_xxs_per_expert", 16, False)):
        layer = MoeLayer(t)
        wbytes = layer.weight_bytes()
        layer.issue(grouped=grouped)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            layer.issue(grouped=grouped)
        g.replay()
        torch.cuda.synchronize()
        ms = timed_replay(torch, g, reps) / reps
        out[name] = {"ms_per_layer": round(ms, 4), "weight_bytes": wbytes,
                     "weight_GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_of_weight_roofline": round(wbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
                     "tokens_per_s": round(64 / (ms * 1e-3), 1)}
        if grouped:
            out[name + "_routed"] = routed_moe(torch, layer, t, reps)
        del g, layer
        torch.cuda.empty_cache()
    return out


def routed_moe(torch, layer, t, reps):
    """The whole MoE FFN for 64 tokens with top-2 routing on the device
    (MoeStep: F32 router GEMM, hip_moe_route / plan, gather, expert GEMMs with
    the token ranges read on the device, SwiGLU folded into the down GEMM,
    weighted combine), on the same expert weights, one HIP graph per layer
    step; and "host_ranges": the same step with tok_off copied back to build
    the expert launches on the host (not capturable: events around `reps`
    eager calls, the round trip included)."""
    from saient_quartz_amd.decode import MoeStep

    E, k, n, d, f = layer.E, 2, 64, layer.h, layer.f
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20261207)
    rw = torch.randn(E, d, device="cuda", generator=gen) / d ** 0.5
    x = torch.randn(n, d, device="cuda", generator=gen)
    y = torch.empty(n, d, device="cuda")
    step = MoeStep((t, t, t), layer.wg, layer.wu, layer.wd, rw, E, k, d, f, n_max=n)
    assert step.device_driven
    step.issue(x, y, n)
    torch.cuda.synchronize()
    off = step.tok_off.cpu().tolist()
    counts = [b - a for a, b in zip(off[:-1], off[1:])]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step.issue(x, y, n)
    g.replay()
    torch.cuda.synchronize()
    ms = timed_replay(torch, g, reps) / reps
    del g
    step.device_driven = False
    step.issue(x, y, n)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        step.issue(x, y, n)
    t1.record()
    torch.cuda.synchronize()
    ms_host = t0.elapsed_time(t1) / reps
    wbytes = sum(3 * layer.slice for c in counts if c)
    return {"ms_per_layer": round(ms, 4), "tokens_per_s": round(n / (ms * 1e-3), 1), "tokens_per_expert": counts,
            "weight_bytes_touched": wbytes, "weight_GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "host_ranges_ms_per_layer": round(ms_host, 4)}


def timed_replay(torch, graph, reps=1):
    """GPU time (ms) of `reps` replays of `graph` on the current stream, HIP
    events around them, with a ~0.4 ms spin kernel queued ahead so the
    replays' submission overlaps it instead of being timed."""
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1_000_000)
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def profiled_kernel_us(path):
    """The kernel-trace average (us) from the committed rocprofv3 summary; None if absent."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("kernel_avg_us"):
                return float(line.split("=")[1])
    except (OSError, ValueError):
        pass
    return None


def measured_traffic(path):
    """HBM bytes per launch of the GEMV kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-kernel calibrated); None if absent."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def host_llc_bytes():
    """Total last-level (L3) cache of the host: the sizes of the distinct L3
    instances sysfs lists (0 if unknown)."""
    seen, total = set(), 0
    base = Path("/sys/devices/system/cpu")
    for idx in base.glob("cpu[0-9]*/cache/index[0-9]*"):
        try:
            if (idx / "level").read_text().strip() != "3":
                continue
            key = (idx / "shared_cpu_list").read_text().strip()
            if key in seen:
                continue
            seen.add(key)
            size = (idx / "size").read_text().strip()
            mult = {"K": 2**10, "M": 2**20, "G": 2**30}.get(size[-1], 1)
            total += int(size.rstrip("KMG")) * mult
        except (OSError, ValueError):
            continue
    return total


def cpu_threads():
    """Threads for the CPU baseline: the host's CPUs available to this process,
    capped at the GPU box's CPU share for one GPU (16; OMP_NUM_THREADS is set to
    it there), so the baseline's worker pool stays within the box's limits."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(avail, 16)), avail


def _time_calls(fn, seconds):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while reps < 2 or time.perf_counter() - t0 < seconds:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_baseline(out_dim, in_dim, seconds):
    """Quartz's CPU path restated in C (oracle/quartz_oracle.c), timed on this
    host's cores over bounded samples (about `seconds` of CPU work in all):
      value: Q4_K 14336x4096 GEMV (fused q4k_row, OpenMP over rows = rayon), the
             GPU headline's workload, on `cores` threads;
      legs:  the same on 1 core; Q8_0 4096x4096 through the `_` arm as the
             reference runs it (whole-matrix dequant + matmul,
             src/dequant.rs:26-29, src/main.rs:710-718); the batched gemm at
             N = 16 (src/dequant.rs:143-200); and the 8B decode step's GEMV set
             (one layer's 7 matrices x 32 + the Q6_K head) as tok/s."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import Oracle
    from saient_quartz_amd import synth
    from saient_quartz_amd.decode import ModelConfig

    o = Oracle.load()
    cores, avail = cpu_threads()
    share = seconds / 5.0
    o.set_threads(cores)
    data = synth.weights(Q4K, out_dim, in_dim, seed=20261202)
    # Copies of the weights at distinct addresses, rotated call by call, twice
    # the host's last-level cache in all, so no call reads weights the cache
    # kept from an earlier one.
    llc = host_llc_bytes()
    n_copies = max(2, -(-2 * max(llc, 1) // data.nbytes))
    copies = [data] + [data.copy() for _ in range(n_copies - 1)]
    x = synth.activations(1, in_dim, seed=3)[0]
    alg = data.nbytes + 4 * in_dim + 4 * out_dim
    rot = [0]

    def gemv_rot():
        o.gemv(Q4K, x, copies[rot[0] % n_copies], in_dim, out_dim)
        rot[0] += 1

    dt, reps = _time_calls(gemv_rot, share)
    rec = {"value": round(alg / dt / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
           "sample": f"{reps} x Q4_K 14336x4096 GEMV (C restatement of q4k_row, OpenMP over rows), "
                     f"{dt * 1e3:.2f} ms each, weights rotated over {n_copies} copies "
                     f"({n_copies * data.nbytes / 2**20:.0f} MiB, 2x the host LLC)",
           "host_cpus": os.cpu_count(), "cpus_available": avail, "host_llc_bytes": llc}
    legs = {}
    o.set_threads(1)
    dt1, reps = _time_calls(gemv_rot, share)
    legs["q4_k_14336x4096_1core"] = {"GB_s": round(alg / dt1 / 1e9, 2), "ms": round(dt1 * 1e3, 2), "cores": 1,
                                     "reps": reps}
    o.set_threads(cores)
    # Q8_0 configs[0] through the dequant + matmul arm (a 64 MB f32 W per call, as the reference)
    q8 = synth.weights(8, 4096, 4096, seed=20261201)
    x8 = synth.activations(1, 4096, seed=4)[0]
    wbuf = np.empty(4096 * 4096, dtype=np.float32)
    dt8, reps = _time_calls(lambda: o.gemv_dequant_matmul(8, x8, q8, 4096, 4096, wbuf), share)
    a8 = q8.nbytes + 4 * 4096 * 2
    legs["q8_0_4096x4096_dequant_matmul"] = {"GB_s": round(a8 / dt8 / 1e9, 2), "ms": round(dt8 * 1e3, 2),
                                             "cores": cores, "reps": reps}
    # batched gemm, 16 tokens, Q4_K 14336x4096 (rotated copies as above)
    x16 = synth.activations(16, in_dim, seed=6)

    def gemm_rot():
        o.gemm(Q4K, x16, copies[rot[0] % n_copies], in_dim, out_dim, 16)
        rot[0] += 1

    dtg, reps = _time_calls(gemm_rot, share)
    legs["q4_k_14336x4096_gemm_n16"] = {"GB_s": round(data.nbytes / dtg / 1e9, 2), "ms": round(dtg * 1e3, 2),
                                        "tokens_per_s": round(16 / dtg, 1), "cores": cores, "reps": reps}
    del x16, wbuf, copies
    # the 8B decode step's GEMVs: one layer's 7 matrices (x 32 layers) + the
    # head; layers alternate between weight sets covering twice the LLC
    cfg = ModelConfig()
    mats = [(cfg.type_of(n), oo, ii, synth.weights(cfg.type_of(n), oo, ii, seed=20261300 + k))
            for k, (n, oo, ii) in enumerate(cfg.mats())]
    layer_bytes = sum(d.nbytes for _, _, _, d in mats)
    n_sets = max(2, -(-2 * max(llc, 1) // layer_bytes))
    sets = [mats] + [[(t, oo, ii, d.copy()) for t, oo, ii, d in mats] for _ in range(n_sets - 1)]
    xs = {ii: synth.activations(1, ii, seed=ii)[0] for _, _, ii, _ in mats}

    def layer():
        for t, oo, ii, d in sets[rot[0] % n_sets]:
            o.gemv(t, xs[ii], d, ii, oo)
        rot[0] += 1

    dtl, reps = _time_calls(layer, share * 0.6)
    head = synth.weights(cfg.type_of("head"), cfg.vocab, cfg.hidden, seed=20261399)
    dth, reps_h = _time_calls(lambda: o.gemv(cfg.type_of("head"), xs[cfg.hidden], head, cfg.hidden, cfg.vocab),
                              share * 0.4)
    step = cfg.layers * dtl + dth
    legs["llama8b_q4km_step_gemvs"] = {"tok_s": round(1.0 / step, 2), "ms_per_step": round(step * 1e3, 2),
                                       "weight_GB_s": round(cfg.weight_bytes() / step / 1e9, 2), "cores": cores,
                                       "layer_ms": round(dtl * 1e3, 3), "head_ms": round(dth * 1e3, 3),
                                       "reps": [reps, reps_h]}
    rec["legs"] = legs
    return rec


if __name__ == "__main__":
    main()
