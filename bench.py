"""MoE decode benchmark on one MI355X.

Workload (the north-star config): a
Qwen3.5-397B-A17B-shaped MoE stack, 60 layers, hidden 4096, 512 routed experts
in grouped int3 (g128, uniform random codes, |N(0,0.01)| scales), top-10
softmax router (fp32 ~N(0,0.02)), one int8 shared expert (intermediate 1024);
all 157 GB of expert weights resident in HBM; batch-1 decode with seeded
N(0,1) activations per (step, layer).  `--workload s35` runs configs[1]
(35B-A3B shape, 40 layers, int4) instead.

A step is one decoded token through every layer of the stack, layer l+1
starting after layer l's output is written (strict decode order).  `value` is
tokens/s with all inputs already in HBM.  The roofline object reports the
dominant kernel of the step: algorithmic bytes per launch over its average
duration, measured with HIP events on the context stream.  cpu_baseline times
the reference's own CPU MoE code (c/qwen.c moe_forward, compiled in place into
oracle/_ref) on the host cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "MoE decode tok/s at 35B/397B shapes; achieved HBM GB/s vs MI355X peak"

WORKLOADS = {
    # name: (H, E, K, I, I_sh, fmt, layers, seed, description)
    "s397": (4096, 512, 10, 1024, 1024, 3, 60, 397,
             "config2: Qwen3.5-397B-A17B-shaped MoE stack, 60 layers, int3-g128 routed experts "
             "(512, top-10) + int8 shared expert, 157 GB HBM-resident, batch-1 decode"),
    "s35": (2048, 256, 8, 512, 512, 4, 40, 35,
            "config1: Qwen3.5-35B-A3B-shaped MoE stack, 40 layers, int4-g128 routed experts "
            "(256, top-8) + int8 shared expert, 17 GB HBM-resident, batch-1 decode"),
}

KERNELS = ["route", "experts", "down"]


def row_bytes(fmt, cols, gs=128):
    ng = (cols + gs - 1) // gs
    return ng * gs // 2 if fmt == 4 else ng * gs * 3 // 8


def kernel_bytes(H, E, K, I, Ish, fmt):
    """Algorithmic HBM bytes per layer step of each decode kernel: the weights
    and scales it must stream (activations, < 0.1%, omitted).
      route:   router f32 [E x H] + shared gate row [H] + shared gate/up int8 [2 Ish x H]
      experts: K routed gate/up (codes + group scales)
      down:    K routed down (codes + group scales) + shared down int8 [H x Ish]
               + shared row scales (gate, up, down)"""
    ngh, ngi = (H + 127) // 128, (I + 127) // 128
    gate = I * row_bytes(fmt, H) + I * ngh * 4
    down = H * row_bytes(fmt, I) + H * ngi * 4
    return [E * H * 4 + H * 4 + 2 * Ish * H,
            K * 2 * gate,
            K * down + H * Ish + 2 * Ish * 4 + H * 4]


def cpu_baseline(cfg, budget_s: float):
    """The reference CPU path on a bounded sample: two layers of the stack
    materialised on the host (identical bytes), decode tokens until the time
    budget is spent; tok/s scaled to the full stack."""
    H, E, K, I, Ish, fmt, layers, seed, _ = cfg
    from oracle import pyoracle as po
    o = po.Oracle()
    kind = "port"
    runner = None
    try:
        ref = po.Reference()
        kind = "reference"
    except Exception:
        ref = None
    threads = os.cpu_count() or 1
    sample_layers = 2
    hls = [o.host_layer(seed, l, H, E, K, I, Ish, fmt) for l in range(sample_layers)]
    if ref is not None:
        ref.set_threads(threads)
        rls = [ref.layer(hl) for hl in hls]
        runner = lambda l, x: rls[l].forward(x)  # noqa: E731
    else:
        o.set_threads(threads)
        runner = lambda l, x: o.moe_forward(hls[l], x)  # noqa: E731
    # warm the caches once per layer
    for l in range(sample_layers):
        runner(l, o.synth_x(seed, l, 0, H))
    n, t0 = 0, time.perf_counter()
    step = 1
    while time.perf_counter() - t0 < budget_s and n < 4096:
        for l in range(sample_layers):
            runner(l, o.synth_x(seed, l, step, H))
            n += 1
        step += 1
    dt = time.perf_counter() - t0
    per_token_layer = dt / n
    value = 1.0 / (per_token_layer * layers)
    return {"value": round(value, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{n} token-layers over layers 0..{sample_layers - 1} of the same synthetic stack "
                      f"({dt:.1f} s, {per_token_layer * 1e3:.3f} ms per token-layer), scaled to {layers} layers",
            "lib": os.path.basename(ref.path) if ref is not None else "liboracle.so"}


def copy_probe(mib: int):
    """A plain copy of known size through coli_cuda_copy (HIP's own blit
    kernel): the reference point that scales the HBM byte counters."""
    from shiftwing_amd import Backend
    be = Backend(0)
    n = mib << 20
    src, dst = be.alloc(n), be.alloc(n)
    be.check(be.lib.coli_cuda_memset(be.ctx, src.p, 1, C.c_size_t(n)))
    reps = 4
    be.check(be.lib.coli_cuda_copy(be.ctx, dst.p, src.p, C.c_size_t(n)))
    be.sync()
    be.check(be.lib.coli_cuda_timer_start(be.ctx))
    for _ in range(reps):
        be.check(be.lib.coli_cuda_copy(be.ctx, dst.p, src.p, C.c_size_t(n)))
    ms = C.c_float()
    be.check(be.lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)))
    sec = ms.value / 1e3 / reps
    print(json.dumps({"copy_bytes": n, "read_bytes": n, "write_bytes": n, "ms": round(sec * 1e3, 4),
                      "gbs_read_plus_write": round(2 * n / sec / 1e9, 1), "launches": reps + 1}), flush=True)


def measured_traffic(workload: str, kernel: str, layers_per_launch: int):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/hbm_traffic_<workload>.txt: FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by what the counter reads for a copy of known
    size), scaled to this launch's layer count.  None when no summary covers
    the kernel."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 4 and parts[0] == "traffic" and parts[1] == kernel:
                return int(round(int(parts[2]) * layers_per_launch / int(parts[3])))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--workload", default="s397", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (testing)")
    ap.add_argument("--decode-kernels", type=int, default=1, choices=[1, 2],
                    help="1: the persistent decode kernel, one launch per stack step (default); "
                         "2: the three per-layer decode kernels")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="time a plain device-to-device copy of MIB MiB (the counter calibration kernel) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return

    from shiftwing_amd import Backend, MoeLayer
    H, E, K, I, Ish, fmt, layers, seed, desc = WORKLOADS[args.workload]
    if args.layers:
        layers = args.layers
    be = Backend(0)
    be.set_decode_kernels(args.decode_kernels)
    lib = be.lib
    t0 = time.perf_counter()
    stack = []
    for l in range(layers):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, l)
        stack.append(L)
    be.sync()
    gen_s = time.perf_counter() - t0
    resident = sum(L.nbytes() for L in stack)
    total_steps = args.warmup + args.steps
    xs = be.alloc(layers * total_steps * H * 4)
    for l in range(layers):
        be.check(lib.coli_cuda_synth_activations(
            be.ctx, C.c_void_p(xs.ptr + l * total_steps * H * 4), total_steps, H, C.c_ulonglong(seed), l, 0))
    ys = be.alloc(layers * H * 4)
    arr = (C.c_void_p * layers)(*[L.h.value for L in stack])

    def run(step):
        be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, layers, ys.p, C.c_void_p(xs.ptr + step * H * 4),
                                                  1, total_steps * H, H), "forward_layers")

    for s in range(args.warmup):
        run(s)
    be.sync()
    be.check(lib.coli_cuda_timer_start(be.ctx))
    for s in range(args.warmup, total_steps):
        run(s)
    ms = C.c_float()
    be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)))
    total_ms = ms.value
    ms_per_step = total_ms / args.steps
    tok_s = args.steps / (total_ms / 1e3)

    kb = kernel_bytes(H, E, K, I, Ish, fmt)
    step_bytes = sum(kb)
    if args.decode_kernels == 1:
        # one persistent kernel per step: HIP events on the context stream
        # right before and after single launches give its duration
        durs = []
        for s in range(args.warmup, args.warmup + min(args.steps, 16)):
            be.check(lib.coli_cuda_timer_start(be.ctx))
            run(s)
            m1 = C.c_float()
            be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(m1)))
            durs.append(m1.value)
        launch_ms = sum(durs) / len(durs)
        kname, launch_bytes, layers_per_launch = "k_stack", layers * step_bytes, layers
        kernel_us = {"k_stack": round(launch_ms * 1e3, 3), "per_layer": round(launch_ms * 1e3 / layers, 3)}
        kernel_gbs = {"k_stack": round(launch_bytes / (launch_ms * 1e-3) / 1e9, 1)}
    else:
        # per-kernel timing pass: HIP events on the context stream around each
        # of the three decode kernels (the kernels' own stream)
        be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 1))
        nst = min(args.steps, 8)
        for s in range(args.warmup, args.warmup + nst):
            run(s)
        be.sync()
        kms = (C.c_double * 3)()
        calls = C.c_ulonglong()
        be.check(lib.coli_cuda_moe_decode_times(be.ctx, kms, C.byref(calls)))
        be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 0))
        per_call = [kms[i] / max(calls.value, 1) for i in range(3)]
        dom = max(range(3), key=lambda i: per_call[i])
        kname, launch_bytes, layers_per_launch = KERNELS[dom], kb[dom], 1
        launch_ms = per_call[dom]
        kernel_us = {KERNELS[i]: round(per_call[i] * 1e3, 3) for i in range(3)}
        kernel_gbs = {KERNELS[i]: round(kb[i] / (per_call[i] * 1e-3) / 1e9, 1) for i in range(3)}
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    stats = [L.route_stats_full() for L in stack]
    tokens_routed = sum(t for t, _, _ in stats)
    fallbacks = sum(f for _, f, _ in stats)
    full = sum(u for _, _, u in stats)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": desc,
            "hidden": H, "experts": E, "topk": K, "intermediate": I, "shared_intermediate": Ish,
            "expert_format": f"int{fmt}-g128", "layers": layers, "batch": 1, "seed": seed,
            "resident_gb": round(resident / 1e9, 2),
            "arithmetic": "int3/int4 codes x two int8 activation digits on MFMA, fp32 group scaling; "
                          "int8 IDOT shared expert; fp64-certified exact fp32 router",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kname,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.workload, kname, layers_per_launch),
            "bytes_per_launch": launch_bytes,
            "avg_launch_us": round(launch_ms * 1e3, 3),
        },
        "step": {
            "algorithmic_bytes_per_layer": step_bytes,
            "effective_gbs": round(step_bytes * layers / (ms_per_step * 1e-3) / 1e9, 1),
            "frac_of_peak": round(step_bytes * layers / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel_us": kernel_us,
            "kernel_gbs": kernel_gbs,
            "router_not_certified": f"{fallbacks}/{tokens_routed} token-layers ({full} needed every chain)",
            "weight_generation_s": round(gen_s, 1),
        },
    }
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(WORKLOADS[args.workload], args.cpu_seconds)
        except Exception as e:  # the CPU leg never hides the GPU number
            result["cpu_baseline"] = {"value": None, "error": str(e)}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
