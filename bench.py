"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

Headline (``value``): Qwen3-0.6B decode GEMV set: all 28
layers x 7 projections (Q4_K, v_proj Q6_K), M=1, run back to back as one fused
launch per step (a GemvPlan over 196 descriptors), the K steps replayed from a
HIP graph (also reported: the same steps launched one by one from the host).
Algorithmic bytes per step =
sum(weight bytes + 4K + 4N) = 255.4 MB. Weight copies rotate so the working set
(3 x 255 MB) exceeds the 256 MB Infinity Cache twice over.

Also reported: the same set as dependent per-layer launches (qkv / o / gate+up /
down), the M=512 int8-MMQ prefill GEMM at 0.6B shapes (config 3) and one 8B
layer (config 4), the roofline of the dominant kernel (HIP-event timed, on the
stream it runs on) and the CPU baseline (dequant restatement + f32 matmul on the
host cores, bounded sample).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV GB/s & M=512 prefill TOPS (% of MI355X peak), Qwen3-0.6B shapes"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X published
F16_PEAK_TOPS = 2500.0   # dense f16 MFMA, MI355X published (the prefill kernels' arithmetic)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    # ~100 ms of warm-up: the first ~20 ms of sustained load on a fresh process
    # run ~15% slower (measured: 54 us per step, then 46 us)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="skip prefill, 8B and CPU legs")
    ap.add_argument("--legs", default=None,
                    help="comma list of the legs to run after the headline (decode_8b, prefill, q8_0, moe); "
                         "no CPU leg")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-only", action="store_true",
                    help="only the CPU baseline leg, as one JSON line (no GPU; run by the full bench in a child "
                         "process with the caller's OpenMP settings)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only replay the fused GEMV plan and a calibration copy (for rocprofv3 --pmc runs)")
    ap.add_argument("--prefill-probe", nargs="?", const="gate8b", choices=("gate8b", "set06b"),
                    help="only run the 8B gate GEMM (14336x4096 Q4_K, M=512; gate8b, the default) or the "
                         "Qwen3-0.6B M=512 set's GEMM plan (set06b) a few times (for rocprofv3 --pmc runs)")
    ap.add_argument("--moe-probe", action="store_true",
                    help="only run config 5's device-routed MoE prefill (512 tokens) ten times (for rocprofv3 --pmc runs)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, WRITE_SIZE) of a "
                         "--traffic-probe run into profiles/gemv_decode06b_traffic.json")
    args = ap.parse_args()
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        return 2
    if args.cpu_only:
        import numpy as np

        from reflex_amd import synth

        layer, L = synth.QWEN3_06B_LAYER, synth.QWEN3_06B_LAYERS
        host_w = {(li, pi): synth.weights(ty, n, k, synth.seed_for(2, li, pi))
                  for li in range(L) for pi, (_, ty, n, k) in enumerate(layer)}
        print(json.dumps(cpu_leg(host_w, layer, L, np)), flush=True)
        return 0
    # the caller's environment, for the CPU baseline's child process
    child_env = dict(os.environ)

    # The host-routed MoE call routes its tokens on OpenMP threads. With the
    # default (active) wait policy, idle OpenMP workers spin and take cores
    # from the host work that follows them. That made the call host-bound:
    # 359-406 us against 196-204 us. Passive waiting is set before any
    # OpenMP runtime starts, unless the caller set a policy.
    os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")
    import numpy as np
    import torch

    import reflex_amd as rq
    from reflex_amd import synth

    dev = "cuda:0"
    torch.cuda.set_device(0)
    rq.init(0)
    stream = torch.cuda.current_stream()

    if args.prefill_probe == "set06b":
        # the GEMM launches of bench's config 3 step (activation buffers written once)
        gen = torch.Generator(device=dev)
        gen.manual_seed(4242)
        _, q_items, keep = prefill_set(rq, synth, torch, dev, synth.QWEN3_06B_LAYER, synth.QWEN3_06B_LAYERS, 3, gen)
        qplan = rq.GemmPlan(q_items, 512, quantized=True)
        for _ in range(10):
            qplan.run()
        torch.cuda.synchronize()
        return 0
    if args.moe_probe:
        cfg = synth.MOE
        E, H, F, K, tokens = cfg["experts"], cfg["hidden"], cfg["ffn"], cfg["top_k"], cfg["tokens"]
        gate, up, down = (rq.Weight.from_blocks(cfg["ty"], synth.weights(cfg["ty"], E * o, i, synth.seed_for(5, 0, p)),
                                                i, o, expert_count=E, device=dev)
                          for p, i, o in ((0, H, F), (1, H, F), (2, F, H)))
        x = torch.from_numpy(synth.activations(tokens * H, synth.seed_for(5, 0, 3))).to(dev)
        lg = torch.from_numpy(synth.normals(synth.seed_for(5, 0, 4), tokens * E).reshape(tokens, E)).to(dev)
        y = torch.empty(tokens * H, device=dev)
        for _ in range(10):
            rq.moe_ffn_grouped_device(x, tokens, H, lg, E, K, True, 1.0, gate, up, down, y)
        torch.cuda.synchronize()
        return 0
    if args.prefill_probe:
        name, ty, n, k = synth.QWEN3_8B_LAYER[4]
        w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(4, 0, 4)), k, n, device=dev)
        x = torch.from_numpy(synth.activations(512 * k, synth.seed_for(4, 0, 99))).to(dev)
        y = torch.empty(512 * n, device=dev)
        ws = torch.empty(rq.gemm_workspace_size(w, 512), dtype=torch.uint8, device=dev)
        for _ in range(5):
            rq.gemm(x, w, 512, workspace=ws, out=y)
        torch.cuda.synchronize()
        return 0

    # ------------------------------------------------------------ data (config 2)
    t0 = time.time()
    layer = synth.QWEN3_06B_LAYER
    L = synth.QWEN3_06B_LAYERS
    host_w = {}
    for li in range(L):
        for pi, (name, ty, n, k) in enumerate(layer):
            host_w[(li, pi)] = synth.weights(ty, n, k, synth.seed_for(2, li, pi))
    copies = []
    for c in range(args.copies):
        ws = {}
        for (li, pi), a in host_w.items():
            name, ty, n, k = layer[pi]
            ws[(li, pi)] = rq.Weight.from_blocks(ty, a, k, n, device=dev)
        copies.append(ws)
    xs = {k: torch.from_numpy(synth.activations(k, synth.seed_for(2, 99, k % 97))).to(dev)
          for k in {k for _, _, _, k in layer}}
    ys = {(li, pi): torch.empty(layer[pi][2], device=dev) for li in range(L) for pi in range(len(layer))}
    step_bytes = sum(synth.weight_bytes(ty, n, k) + 4 * k + 4 * n for _, ty, n, k in layer) * L
    log(f"data ready in {time.time() - t0:.1f}s; step bytes {step_bytes / 1e6:.1f} MB")

    plans = []
    for c in range(args.copies):
        items = [(xs[layer[pi][3]], copies[c][(li, pi)], ys[(li, pi)]) for li in range(L) for pi in range(len(layer))]
        plans.append(rq.GemvPlan(items))

    def timed(fn, steps, warmup):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps  # ms per step

    if args.traffic_probe:
        # 5 launches of each plan copy, then a plain copy of COPY_BYTES (the
        # counters' calibration: its algorithmic bytes are known exactly)
        for i in range(5 * args.copies):
            plans[i % args.copies].run()
        src = torch.empty(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1.0, out=dst)  # an elementwise kernel: reads and writes COPY_BYTES
        torch.cuda.synchronize()
        return 0

    # headline: one fused launch per step, the steps replayed from a HIP graph
    # (as a serving loop replays its decode step: no host launch work between
    # steps); W warm-up steps in a graph of their own, then exactly K steps
    def step_graph(n):
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for i in range(n):
                    plans[i % args.copies].run()
        return g
    g_warm, g_steps = step_graph(max(args.warmup, 1)), step_graph(args.steps)
    torch.cuda.synchronize()
    g_warm.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g_steps.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps  # ms per step
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"decode GEMV set (fused launch, graph-replayed steps): {ms * 1e3:.1f} us/step  {gbs:.0f} GB/s")
    # the same steps launched one by one from the host
    ms_e = timed(lambda i: plans[i % args.copies].run(), args.steps, args.warmup)
    gbs_e = step_bytes / (ms_e * 1e-3) / 1e9
    log(f"decode GEMV set (fused launch, host-launched steps): {ms_e * 1e3:.1f} us/step  {gbs_e:.0f} GB/s")

    # dependent per-layer launches: q/k/v fused, o, gate+up fused, down
    def layered(i):
        ws = copies[i % args.copies]
        for li in range(L):
            rq.gemv_batch([(xs[layer[p][3]], ws[(li, p)], ys[(li, p)]) for p in (0, 1, 2)])
            rq.gemv_to(xs[layer[3][3]], ws[(li, 3)], ys[(li, 3)])
            rq.gemv_batch([(xs[layer[p][3]], ws[(li, p)], ys[(li, p)]) for p in (4, 5)])
            rq.gemv_to(xs[layer[6][3]], ws[(li, 6)], ys[(li, 6)])

    ms_l = timed(layered, 10, 2)
    gbs_l = step_bytes / (ms_l * 1e-3) / 1e9
    log(f"decode GEMV set (112 dependent launches): {ms_l * 1e3:.1f} us/step  {gbs_l:.0f} GB/s")

    # the same 112 launches per step from GEMV plans captured in a HIP graph
    # (how an engine replays its decode step: no per-launch host work)
    groups = [(0, 1, 2), (3,), (4, 5), (6,)]
    graphs = []
    for c in range(args.copies):
        ws = copies[c]
        gplans = [rq.GemvPlan([(xs[layer[p][3]], ws[(li, p)], ys[(li, p)]) for p in g])
                  for li in range(L) for g in groups]
        for p in gplans:
            p.run()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for p in gplans:
                    p.run()
        graphs.append((graph, gplans))
    torch.cuda.synchronize()
    ms_g = timed(lambda i: graphs[i % args.copies][0].replay(), 50, 5)
    gbs_g = step_bytes / (ms_g * 1e-3) / 1e9
    log(f"decode GEMV set (112 dependent launches, HIP graph): {ms_g * 1e3:.1f} us/step  {gbs_g:.0f} GB/s")

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-0.6b decode GEMV set: 28 layers x (q,k,o,gate,up,down Q4_K + v Q6_K), M=1, "
                        "one fused launch per step",
            "global_batch": 1,
            "weights_mb_per_step": round(step_bytes / 1e6, 1),
            "weight_copies_rotated": args.copies,
        },
        "roofline": {
            "kernel": "rfxq_gemv",
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "host_launched_steps": {"gbs": round(gbs_e, 1), "ms_per_step": round(ms_e, 4)},
        "layered_launches": {"gbs": round(gbs_l, 1), "ms_per_step": round(ms_l, 4), "launches_per_step": 112},
        "layered_graph": {"gbs": round(gbs_g, 1), "ms_per_step": round(ms_g, 4), "launches_per_step": 112},
    }
    traffic_file = os.path.join(ROOT, "profiles", "gemv_decode06b_traffic.json")
    if os.path.exists(traffic_file):
        result["roofline"]["traffic"] = json.load(open(traffic_file)).get("bytes_per_launch")

    del plans, copies
    legs = {"decode_8b", "prefill", "q8_0", "moe"} if args.legs is None else set(args.legs.split(","))
    if args.quick:
        legs = set()
    if "decode_8b" in legs:
        result["decode_8b"] = decode_8b_leg(rq, synth, torch, np, dev, timed)
    if "prefill" in legs:
        result["prefill"] = prefill_leg(rq, synth, torch, np, dev, timed)
        # the metric's second half as top-level keys (the config 3 set)
        pf = result["prefill"]["qwen3_06b_m512"]
        result["prefill_tops"] = pf["tops"]
        result["prefill_frac_int8_peak"] = pf["frac_int8_peak"]
        result["prefill_frac_f16_peak"] = pf["frac_f16_peak"]
        result["prefill_ms_per_step"] = pf["ms_per_step"]
        result["prefill_tops_with_act_pass"] = pf["tops_with_act_pass"]
        result["prefill_kernel"] = "rfxq_mmqh_q4k (+ rfxq_mmqh_q6k for v_proj)"
    if "q8_0" in legs:
        result["q8_0"] = q8_0_leg(rq, synth, torch, np, dev, timed)
    if "moe" in legs:
        result["moe"] = moe_leg(rq, synth, torch, np, dev, timed)
    torch.cuda.empty_cache()
    if not args.quick and not args.no_cpu and args.legs is None:
        # in a child process with the caller's OpenMP settings: the passive
        # waiting set above slows the baseline's many short parallel regions
        import subprocess

        out = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-only"], env=child_env,
                             capture_output=True, text=True, timeout=300, check=True).stdout
        result["cpu_baseline"] = json.loads(out.strip().splitlines()[-1])
    print(json.dumps(result), flush=True)
    return 0


COPY_BYTES = 256 << 20


def traffic_summary(fetch_csv: str, write_csv: str) -> int:
    """HBM bytes per rfxq_gemv launch from FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch), each scaled by the factor that makes the calibration copy's
    counter equal its known bytes (COPY_BYTES read, COPY_BYTES written)."""
    import csv
    import statistics

    def per_kernel(path):
        vals = {}
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            key = "gemv" if name == "rfxq_gemv" else ("copy" if "elementwise" in name.lower() else None)
            if key:
                vals.setdefault(key, []).append(float(r["Counter_Value"]) * 1024.0)
        return {k: statistics.median(v) for k, v in vals.items()}

    f, w = per_kernel(fetch_csv), per_kernel(write_csv)
    f_scale, w_scale = COPY_BYTES / f["copy"], COPY_BYTES / w["copy"]
    out = {
        "kernel": "rfxq_gemv", "workload": "qwen3-0.6b decode GEMV set, one fused launch",
        "fetch_bytes_raw": f["gemv"], "write_bytes_raw": w["gemv"],
        "fetch_scale": f_scale, "write_scale": w_scale,
        "bytes_per_launch": f["gemv"] * f_scale + w["gemv"] * w_scale,
        "algorithmic_bytes_per_launch": None,
    }
    from reflex_amd import synth
    layer = synth.QWEN3_06B_LAYER
    out["algorithmic_bytes_per_launch"] = sum(synth.weight_bytes(ty, n, k) + 4 * k + 4 * n
                                              for _, ty, n, k in layer) * synth.QWEN3_06B_LAYERS
    path = os.path.join(ROOT, "profiles", "gemv_decode06b_traffic.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out))
    return 0


def decode_8b_leg(rq, synth, torch, np, dev, timed):
    """Config 4 at M=1: one Qwen3-8B layer's seven GEMVs as one fused launch
    (q/o 4096x4096, k 1024x4096, gate/up 14336x4096 Q4_K; v 1024x4096 and down
    4096x14336 Q6_K; 138 MB), and the tied LM head 151936x1024 Q6_K (128 MB),
    each with three rotated weight copies (beyond the 256 MB Infinity Cache)."""
    out = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(synth.seed_for(4, 0, 98))
    for tag, layer in (("layer", synth.QWEN3_8B_LAYER), ("lm_head", [synth.LM_HEAD])):
        xs = {k: torch.randn(k, device=dev, generator=gen) for k in sorted({k for *_, k in layer})}
        plans, keep = [], []
        for c in range(3):
            items = []
            for pi, (_, ty, n, k) in enumerate(layer):
                w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(4, c, pi)), k, n, device=dev)
                keep.append(w)
                items.append((xs[k], w, torch.empty(n, device=dev)))
            plans.append(rq.GemvPlan(items))
        nbytes = sum(synth.weight_bytes(ty, n, k) + 4 * (n + k) for _, ty, n, k in layer)
        # warm-up past the slower first ~20 ms of sustained load, as for the headline
        ms = timed(lambda i: plans[i % 3].run(), 300, 2000)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[tag] = {"us_per_step": round(ms * 1e3, 1), "mb_per_step": round(nbytes / 1e6, 1), "gbs": round(gbs, 1),
                    "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        print(f"decode 8B {tag}: {ms * 1e3:.1f} us/step  {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM)",
              file=sys.stderr, flush=True)
        del plans, keep
    return out


def q8_0_leg(rq, synth, torch, np, dev, timed):
    """Q8_0 weights: BASELINE config 1's 1024 x 1024 matrix at M=1 (one GEMV;
    1.1 MB, so the figure is launch latency, not bandwidth: 64 rotated copies
    keep it out of the L2) and at M=512, and one Qwen3-8B layer with every
    projection in Q8_0 at M=512 (a Q8_0 model's prefill)."""
    out = {}
    n = k = 1024
    copies = [rq.Weight.from_blocks(synth.Q8_0, synth.weights(synth.Q8_0, n, k, synth.seed_for(1, c, 0)), k, n,
                                    device=dev) for c in range(64)]
    x = torch.from_numpy(synth.activations(k, synth.seed_for(1, 0, 1))).to(dev)
    y = torch.empty(n, device=dev)
    ms = timed(lambda i: rq.gemv_to(x, copies[i % 64], y), 2000, 500)
    nbytes = synth.weight_bytes(synth.Q8_0, n, k) + 4 * (n + k)
    out["config1_gemv_m1"] = {"us_per_call": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                              "mb_per_call": round(nbytes / 1e6, 3)}
    print(f"Q8_0 config 1 GEMV M=1: {ms * 1e3:.2f} us/call", file=sys.stderr, flush=True)
    xs = torch.randn(512 * k, device=dev)
    ys = torch.empty(512 * n, device=dev)
    plan = rq.GemmPlan([(xs, copies[0], ys)], 512)
    ms = timed(lambda i: plan.run(), 200, 50)
    tops = 2 * 512 * n * k / (ms * 1e-3) / 1e12
    out["config1_gemm_m512"] = {"us_per_call": round(ms * 1e3, 1), "tops": round(tops, 1)}
    print(f"Q8_0 config 1 GEMM M=512: {ms * 1e3:.1f} us  {tops:.0f} TOPS", file=sys.stderr, flush=True)
    del plan, copies
    group = {"q_proj": "qkv", "k_proj": "qkv", "v_proj": "qkv", "o_proj": "o",
             "gate_proj": "gu", "up_proj": "gu", "down_proj": "down"}
    gen = torch.Generator(device=dev)
    gen.manual_seed(4343)
    xs, items, keep = {}, [], []
    for pi, (name, _, n, k) in enumerate(synth.QWEN3_8B_LAYER):
        g = group[name]
        if g not in xs:
            xs[g] = torch.randn(512 * k, device=dev, generator=gen)
        w = rq.Weight.from_blocks(synth.Q8_0, synth.weights(synth.Q8_0, n, k, synth.seed_for(4, 7, pi)), k, n,
                                  device=dev)
        keep.append(w)
        items.append((xs[g], w, torch.empty(512 * n, device=dev)))
    plan = rq.GemmPlan(items, 512)
    ms = timed(lambda i: plan.run(), 40, 80)
    ops = sum(2 * 512 * n * k for _, _, n, k in synth.QWEN3_8B_LAYER)
    tops = ops / (ms * 1e-3) / 1e12
    out["qwen3_8b_m512_1layer_q8_0"] = {"ms_per_step": round(ms, 3), "tops": round(tops, 1),
                                        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                        "frac_f16_peak": round(tops / F16_PEAK_TOPS, 4)}
    print(f"Q8_0 8B layer M=512: {ms:.3f} ms  {tops:.0f} TOPS", file=sys.stderr, flush=True)
    del plan, items, keep
    return out


def moe_leg(rq, synth, torch, np, dev, timed):
    """Qwen3-MoE-style grouped expert FFN (config 5): 128 experts, hidden 2048,
    FFN 768, Q4_K gate/up/down, routed top-8 (softmax, renormalised) by seeded
    N(0,1) logits. Prefill: 512 tokens (4096 routed pairs); decode: 1 token.
    A step is one moe_ffn_grouped call (host routing from host logits, one
    table upload, quantize / grouped GEMMs / SiLU*up / combine launches, no
    host synchronisation). HBM-bound: GB/s counts the weight bytes of the
    experts the step routes to."""
    cfg = synth.MOE
    E, H, F, K = cfg["experts"], cfg["hidden"], cfg["ffn"], cfg["top_k"]
    W = lambda p, i, o: rq.Weight.from_blocks(cfg["ty"], synth.weights(cfg["ty"], E * o, i, synth.seed_for(5, 0, p)),  # noqa: E731
                                              i, o, expert_count=E, device=dev)
    gate, up, down = W(0, H, F), W(1, H, F), W(2, F, H)
    per_expert = 3 * F * H * 144 // 256
    out = {}
    for tag, tokens in (("prefill_512", cfg["tokens"]), ("decode_1", 1)):
        x = torch.from_numpy(synth.activations(tokens * H, synth.seed_for(5, 0, 3))).to(dev)
        logits = synth.normals(synth.seed_for(5, 0, 4), tokens * E).reshape(tokens, E)
        y = torch.empty(tokens * H, device=dev)
        used = len({e for t in range(tokens) for e, _ in rq.route_top_k(logits[t], K)})
        # warm-up of ~20 ms or more: the first few dozen prefill calls of a
        # process issue up to twice as slowly on the host (measured: 394 us per
        # call in the second batch of 30, then 196 us from the third on)
        steps, warm = (30, 150) if tokens > 1 else (100, 500)
        ms = timed(lambda i: rq.moe_ffn_grouped(x, tokens, H, logits, E, K, True, 1.0, gate, up, down, y), steps, warm)
        wbytes = used * per_expert
        ops = tokens * K * 2 * 3 * F * H
        gbs = wbytes / (ms * 1e-3) / 1e9
        out[tag] = {"ms_per_step": round(ms, 4), "experts_used": used, "weight_mb": round(wbytes / 1e6, 1),
                    "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                    "tops": round(ops / (ms * 1e-3) / 1e12, 2)}
        print(f"moe {tag}: {ms * 1e3:.1f} us/step  {gbs:.0f} GB/s of routed expert weights "
              f"({gbs / HBM_PEAK_GBS:.1%} of HBM), {used} experts", file=sys.stderr, flush=True)
        # the same step with routing on the device (logits in device memory)
        lg = torch.from_numpy(logits).to(dev)
        ms_d = timed(lambda i: rq.moe_ffn_grouped_device(x, tokens, H, lg, E, K, True, 1.0, gate, up, down, y),
                     steps, warm)
        gbs_d = wbytes / (ms_d * 1e-3) / 1e9
        out[tag + "_device_routing"] = {"ms_per_step": round(ms_d, 4), "gbs": round(gbs_d, 1),
                                        "frac_hbm_peak": round(gbs_d / HBM_PEAK_GBS, 4)}
        print(f"moe {tag} (device routing): {ms_d * 1e3:.1f} us/step  {gbs_d:.0f} GB/s", file=sys.stderr,
              flush=True)
    del gate, up, down
    return out


def prefill_set(rq, synth, torch, dev, layer, nl, cfg, gen):
    """nl layers of M=512 GEMMs, each layer with its own four activations (q/k/v
    share one, as do gate/up; o and down have their own): (f32 items, items
    over activation buffers written once by rfxq_quantize_act_q8_1, weights)."""
    group = {"q_proj": "qkv", "k_proj": "qkv", "v_proj": "qkv", "o_proj": "o",
             "gate_proj": "gu", "up_proj": "gu", "down_proj": "down"}
    items, q_items, keep = [], [], []
    for li in range(nl):
        xs, acts = {}, {}
        for pi, (name, ty, n, k) in enumerate(layer):
            g = group[name]
            if g not in xs:
                xs[g] = torch.randn(512 * k, device=dev, generator=gen)
                acts[g] = rq.quantize_act_q8_1(xs[g], 512, k)
            w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(cfg, li, pi)), k, n, device=dev)
            y = torch.empty(512 * n, device=dev)
            keep.append(w)
            items.append((xs[g], w, y))
            q_items.append((acts[g], w, y))
    return items, q_items, keep


def prefill_leg(rq, synth, torch, np, dev, timed):
    """M=512 MMQ GEMMs: the 0.6B layer set (config 3) and one 8B layer (config 4).

    Each layer has its own four activations (q/k/v share one, as do gate/up;
    o and down have their own), and a step runs all of the set's GEMMs as one
    grouped plan: one launch quantizes every activation, then one MMQ launch
    per weight type (Q4_K, Q6_K)."""
    out = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(4242)
    for tag, layer, nl in (("qwen3_06b_m512", synth.QWEN3_06B_LAYER, synth.QWEN3_06B_LAYERS),
                           ("qwen3_8b_m512_1layer", synth.QWEN3_8B_LAYER, 1)):
        items, q_items, keep = prefill_set(rq, synth, torch, dev, layer, nl, 3 if nl > 1 else 4, gen)
        ops = sum(2 * 512 * n * k for _, _, n, k in layer) * nl
        # warm-up long enough for the clocks to settle (~30 ms of load)
        steps, warm = (20, 40) if nl > 1 else (40, 80)
        # the GEMM kernels alone, from activation buffers a producer wrote
        # (the reference times its MMA kernel the same way,
        # quantized-mma-prefill.md:518-528; the activation pass is below)
        qplan = rq.GemmPlan(q_items, 512, quantized=True)
        ms = timed(lambda i: qplan.run(), steps, warm)
        del qplan
        # the same GEMMs from f32 activations: one f16 activation pass first
        plan = rq.GemmPlan(items, 512)
        ms_a = timed(lambda i: plan.run(), steps, warm)
        tops, tops_a = ops / (ms * 1e-3) / 1e12, ops / (ms_a * 1e-3) / 1e12
        out[tag] = {"tops": round(tops, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                    "frac_f16_peak": round(tops / F16_PEAK_TOPS, 4),
                    "ms_per_step": round(ms, 3), "gop_per_step": round(ops / 1e9, 1),
                    "dtype": "f16 MFMA, f32 accumulate" if rq.get_options()["mmq_f16"] else "int8 MFMA (Q8_1)",
                    "gemms_per_step": len(items),
                    "tops_with_act_pass": round(tops_a, 1), "ms_per_step_with_act_pass": round(ms_a, 3)}
        print(f"prefill {tag}: GEMMs {ms:.3f} ms/step  {tops:.0f} TOPS ({tops / INT8_PEAK_TOPS:.1%} of int8 peak); "
              f"with the activation pass {ms_a:.3f} ms  {tops_a:.0f} TOPS", file=sys.stderr, flush=True)
        del plan, items, q_items, keep
    # config 4's tied LM head at M=512 (one GEMM, 151936 x 1024 Q6_K) and the
    # few-row GEMMs of short prompts (the reference's fused-path measurements:
    # 12 and 29 rows) over one Qwen3-0.6B layer set, weights read once per step
    name, ty, n, k = synth.LM_HEAD
    w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(4, 0, 50)), k, n, device=dev)
    x = torch.randn(512 * k, device=dev, generator=gen)
    y = torch.empty(512 * n, device=dev)
    plan = rq.GemmPlan([(x, w, y)], 512)
    ms = timed(lambda i: plan.run(), 20, 60)
    ops = 2 * 512 * n * k
    tops = ops / (ms * 1e-3) / 1e12
    out["qwen3_8b_lm_head_m512"] = {"tops": round(tops, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                    "frac_f16_peak": round(tops / F16_PEAK_TOPS, 4), "ms_per_step": round(ms, 3)}
    print(f"prefill lm_head M=512: {ms:.3f} ms  {tops:.0f} TOPS", file=sys.stderr, flush=True)
    del plan, w, x, y
    # reference point: the 8B gate GEMM (512 x 4096 x 14336) as a plain f16
    # GEMM on pre-dequantized weights (torch.matmul: hipBLASLt), against the
    # Q4_K kernel on the same shape (the reference compares its MMA kernel
    # with f16 cuBLAS the same way, quantized-mma-prefill.md:518-528)
    name, ty, n, k = synth.QWEN3_8B_LAYER[4]
    a16 = torch.randn(512, k, device=dev, dtype=torch.float16, generator=gen)
    b16 = torch.randn(k, n, device=dev, dtype=torch.float16, generator=gen)
    ms_f16 = timed(lambda i: torch.matmul(a16, b16), 40, 20)
    w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(4, 0, 4)), k, n, device=dev)
    act = rq.quantize_act_q8_1(torch.randn(512 * k, device=dev, generator=gen), 512, k)
    y = torch.empty(512 * n, device=dev)
    qplan = rq.GemmPlan([(act, w, y)], 512, quantized=True)
    ms_q = timed(lambda i: qplan.run(), 40, 20)
    ops = 2 * 512 * n * k
    out["gate_8b_m512_vs_f16_gemm"] = {"q4k_kernel_us": round(ms_q * 1e3, 1),
                                       "q4k_kernel_tops": round(ops / (ms_q * 1e-3) / 1e12, 1),
                                       "f16_hipblaslt_us": round(ms_f16 * 1e3, 1),
                                       "f16_hipblaslt_tops": round(ops / (ms_f16 * 1e-3) / 1e12, 1)}
    print(f"8B gate 512x4096x14336: Q4_K kernel {ms_q * 1e3:.1f} us, f16 hipBLASLt on dequantized weights "
          f"{ms_f16 * 1e3:.1f} us", file=sys.stderr, flush=True)
    del qplan, w, act, y, a16, b16
    layer = synth.QWEN3_06B_LAYER
    ws = [rq.Weight.from_blocks(ty, synth.weights(ty, n, k, synth.seed_for(3, 0, pi)), k, n, device=dev)
          for pi, (_, ty, n, k) in enumerate(layer)]
    wbytes = sum(synth.weight_bytes(ty, n, k) for _, ty, n, k in layer)
    for rows in (12, 29):
        items = [(torch.randn(rows * k, device=dev, generator=gen), w, torch.empty(rows * n, device=dev))
                 for w, (_, ty, n, k) in zip(ws, layer)]
        plan = rq.GemmPlan(items, rows)
        ms = timed(lambda i: plan.run(), 50, 10)
        out[f"qwen3_06b_layer_rows{rows}"] = {"us_per_step": round(ms * 1e3, 1),
                                             "weight_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1)}
        print(f"prefill 0.6B layer, {rows} rows: {ms * 1e3:.1f} us  ({wbytes / (ms * 1e-3) / 1e9:.0f} GB/s of weights)",
              file=sys.stderr, flush=True)
        del plan, items
    del ws
    # fused activation producers at the 8B shapes (rmsnorm before q/k/v and
    # gate/up, SiLU·up before down): one launch writes the quantized layouts
    rows, hid, ffn = 512, 4096, 14336
    x = torch.randn(rows * hid, device=dev, generator=gen)
    g = torch.ones(hid, device=dev)
    gate = torch.randn(rows * ffn, device=dev, generator=gen)
    up = torch.randn(rows * ffn, device=dev, generator=gen)
    act_h = torch.empty(rq.act_q8_1_size(rows, hid), dtype=torch.uint8, device=dev)
    act_f = torch.empty(rq.act_q8_1_size(rows, ffn), dtype=torch.uint8, device=dev)
    lib, st = rq.lib(), lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ms_rms = timed(lambda i: lib.rfxq_rmsnorm_q8_1(x.data_ptr(), g.data_ptr(), rows, hid, 1e-6,
                                                    act_h.data_ptr(), None, st()), 50, 5)
    ms_silu = timed(lambda i: lib.rfxq_silu_and_mul_q8_1(gate.data_ptr(), up.data_ptr(), rows, ffn,
                                                         act_f.data_ptr(), None, st()), 50, 5)
    tmp = torch.empty(rows * ffn, device=dev)
    ms_unfused = timed(lambda i: (lib.rfxq_silu_and_mul(gate.data_ptr(), up.data_ptr(), tmp.data_ptr(),
                                                        rows * ffn, st()),
                                  lib.rfxq_quantize_act_q8_1(tmp.data_ptr(), rows, ffn, act_f.data_ptr(), st())), 50, 5)
    act_bytes = lambda k: rows * k * 3 + rows * (k // 32) * 4 + rows * (k // 256) * 64
    out["producers_8b_m512"] = {
        "rmsnorm_q8_1_us": round(ms_rms * 1e3, 1),
        "rmsnorm_q8_1_gbs": round((rows * hid * 4 + act_bytes(hid)) / (ms_rms * 1e-3) / 1e9, 1),
        "silu_and_mul_q8_1_us": round(ms_silu * 1e3, 1),
        "silu_and_mul_q8_1_gbs": round((rows * ffn * 8 + act_bytes(ffn)) / (ms_silu * 1e-3) / 1e9, 1),
        "silu_and_mul_then_quantize_us": round(ms_unfused * 1e3, 1)}
    print(f"producers 8B M=512: rmsnorm_q8_1 {ms_rms * 1e3:.1f} us, silu_and_mul_q8_1 {ms_silu * 1e3:.1f} us "
          f"(unfused {ms_unfused * 1e3:.1f} us)", file=sys.stderr, flush=True)
    del x, gate, up, tmp
    # an 8B FFN's gate + up + SiLU·up at M=512 from the rmsnorm's buffer, up to
    # the down GEMM's activation buffer: two GEMMs and the fused SiLU·up
    # producer, against rfxq_gemm_gate_up_silu_q8_1 (gate/up pair tiles)
    wg = rq.Weight.from_blocks(synth.Q4K, synth.weights(synth.Q4K, ffn, hid, synth.seed_for(4, 0, 4)), hid, ffn,
                               device=dev)
    wu = rq.Weight.from_blocks(synth.Q4K, synth.weights(synth.Q4K, ffn, hid, synth.seed_for(4, 0, 5)), hid, ffn,
                               device=dev)
    g_out = torch.empty(rows * ffn, device=dev)
    u_out = torch.empty(rows * ffn, device=dev)
    y_s = torch.empty(rows * ffn, device=dev)

    def separate(i):
        rq.gemm_q8_1(act_h, wg, rows, out=g_out)
        rq.gemm_q8_1(act_h, wu, rows, out=u_out)
        lib.rfxq_silu_and_mul_q8_1(g_out.data_ptr(), u_out.data_ptr(), rows, ffn, act_f.data_ptr(), None, st())

    def fused(i):
        lib.rfxq_gemm_gate_up_silu_q8_1(act_h.data_ptr(), rows, wg.cref(), wu.cref(), act_f.data_ptr(),
                                        y_s.data_ptr(), None, 0, st())

    ms_sep = timed(separate, 40, 20)
    ms_fus = timed(fused, 40, 20)
    ops = 2 * 2 * rows * ffn * hid
    out["gate_up_silu_8b_m512"] = {"separate_us": round(ms_sep * 1e3, 1), "fused_us": round(ms_fus * 1e3, 1),
                                   "fused_tops": round(ops / (ms_fus * 1e-3) / 1e12, 1)}
    print(f"8B gate + up + SiLU·up M=512: separate {ms_sep * 1e3:.1f} us, fused {ms_fus * 1e3:.1f} us "
          f"({ops / (ms_fus * 1e-3) / 1e12:.0f} TOPS)", file=sys.stderr, flush=True)
    return out


def cpu_leg(host_w, layer, L, np):
    """Dequant restatement (oracle/, src/dequant.rs semantics) + f32 matmul over the
    same decode set, on the host cores: ~10 s bounded sample of whole layers."""
    import oracle
    from reflex_amd import synth

    threads = os.cpu_count() or 1
    xs = {k: synth.activations(k, synth.seed_for(2, 99, k % 97)) for k in {k for *_, k in layer}}

    def run(nthreads, budget_s):
        done_bytes, t0, li = 0, time.time(), 0
        while time.time() - t0 < budget_s:
            for pi, (_, ty, n, k) in enumerate(layer):
                oracle.cpu_dequant_matmul(ty, host_w[(li % L, pi)], n, k, xs[k], nthreads)
                done_bytes += synth.weight_bytes(ty, n, k) + 4 * k + 4 * n
            li += 1
        dt = time.time() - t0
        return done_bytes / dt / 1e9, li

    gbs_all, layers_all = run(threads, 10.0)
    gbs_one, layers_one = run(1, 5.0)
    return {"value": round(gbs_all, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{layers_all} Qwen3-0.6B layers (7 GEMVs each, M=1) in ~10 s, "
                      "restatement of src/dequant.rs + f32 matmul, OpenMP",
            "single_thread_value": round(gbs_one, 3)}


if __name__ == "__main__":
    sys.exit(main())
