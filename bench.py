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
            "(256, top-8) + int8 shared expert, 17 GB HBM-resident, batch-1 decode, Zipf(1.1) routing"),
}
# batch-1 workloads whose router carries the Zipf(1.1) feature
ZIPF_DECODE = {"s35"}

# many-token workloads: (shape workload, layers, tokens per step or None for
# --batch, Zipf routing, description)
MANY = {
    "s397-batch": ("s397", 60, None, True,
                   "config3: continuous-batch decode on the config-2 stack (60 layers, int3, 157 GB "
                   "HBM-resident), B concurrent tokens per step, Zipf(1.1) routing"),
    "prefill-s35": ("s35", 4, 512, False,
                    "config4: prefill chunk of 512 tokens through one S35-shaped int4 layer "
                    "(4 resident copies used in turn), bf16-valued N(0,1) activations"),
    "prefill-s397": ("s397", 4, 512, False,
                     "config4: prefill chunk of 512 tokens through one S397-shaped int3 layer "
                     "(4 resident copies used in turn), bf16-valued N(0,1) activations"),
}
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0

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


def set_constant_feature(be, buf, rows: int, H: int):
    """x[r, H-1] = 1 for every activation row of a device buffer (the Zipf
    routing feature)."""
    x = np.empty((rows, H), np.float32)
    be.check(be.lib.coli_cuda_download(be.ctx, x.ctypes.data_as(C.c_void_p), buf.p, x.nbytes), "download")
    be.sync()
    x[:, H - 1] = 1.0
    be.check(be.lib.coli_cuda_upload(be.ctx, buf.p, x.ctypes.data_as(C.c_void_p), x.nbytes), "upload")
    be.sync()


def apply_zipf(be, stack, cfg):
    """Zipf(1.1) router columns for every layer of `stack`; returns the
    calibration record for the bench line."""
    from shiftwing_amd import zipf
    H, E, K, I, Ish, fmt, layers, seed, _ = cfg
    beta, fit = zipf.calibrate_beta(H, E, K)
    for l, L in enumerate(stack):
        zipf.apply_to_layer(be, L, beta, seed, l)
    return {"s": 1.1, "beta": round(beta, 4), "fitted_exponent": round(fit, 4),
            "feature": "x[H-1]=1, router[:, H-1] = beta*log p(rank)"}


def stage_model(H, E, K, I, Ish, fmt, T, U):
    """Algorithmic HBM bytes and flops of each stage of the many-token step
    (coli_cuda_moe_stage_times order) for T tokens whose routes touch U
    distinct experts.  Bytes are the weights each stage must stream plus the
    step's f32 input (route) and output (combine); their sum is
    U*expert + shared + router + gate row + T*H*8.  Flops count 2 per
    multiply-add of the layer's own arithmetic (router, shared, routed)."""
    ngh, ngi = (H + 127) // 128, (I + 127) // 128
    gate = I * row_bytes(fmt, H) + I * ngh * 4
    down = H * row_bytes(fmt, I) + H * ngi * 4
    R = T * K
    names = ["route", "bucket", "shared_gateup", "routed_gateup", "hidden_prep", "down", "combine"]
    nbytes = [E * H * 4 + H * 4 + T * H * 4, 0, 2 * Ish * H + 2 * Ish * 4, U * 2 * gate, 0,
              U * down + H * Ish + H * 4, T * H * 4]
    flops = [2 * T * E * H, 0, 2 * 2 * T * Ish * H, 2 * 2 * R * I * H, 0, 2 * R * H * I + 2 * T * H * Ish, 0]
    return names, nbytes, flops


def cpu_baseline_many(cfg, T, zipf_cfg, budget_s: float):
    """The reference CPU path for T-token blocks (c/qwen.c moe_prefill_grouped,
    compiled in place) on one layer of the same synthetic stack, Zipf column
    and constant feature included when the workload routes by Zipf; repeated
    blocks until the budget is spent, tok/s per layer scaled to the layer
    count of the GPU step."""
    H, E, K, I, Ish, fmt, layers, seed, _ = cfg
    from oracle import pyoracle as po
    o = po.Oracle()
    hl = o.host_layer(seed, 0, H, E, K, I, Ish, fmt)
    if zipf_cfg is not None:
        from shiftwing_amd import zipf
        hl.set_router_column(H - 1, zipf.zipf_column(E, zipf_cfg["beta"], seed, 0))
    threads = os.cpu_count() or 1
    try:
        ref = po.Reference()
        ref.set_threads(threads)
        rl = ref.layer(hl)
        run, kind, lib = rl.prefill, "reference", os.path.basename(ref.path)
    except Exception:
        o.set_threads(threads)
        run, kind, lib = (lambda x: o.moe_prefill(hl, x)), "port", "liboracle.so"

    def block(i):
        x = np.stack([o.synth_x(seed, 0, i * T + t, H) for t in range(T)])
        if zipf_cfg is not None:
            x[:, H - 1] = 1.0
        return x

    run(block(0))
    n, t0, i = 0, time.perf_counter(), 1
    while time.perf_counter() - t0 < budget_s and i < 64:
        run(block(i))
        n += 1
        i += 1
    dt = time.perf_counter() - t0
    per_block = dt / max(n, 1)
    return {"value": round(T / (per_block * layers), 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{n} blocks of {T} tokens through layer 0 of the same synthetic stack ({dt:.1f} s, "
                      f"{per_block * 1e3:.1f} ms per block-layer), scaled to {layers} layer(s) per step",
            "lib": lib}


def bench_many(args):
    """Configs 3 and 4: many tokens per MoE step through the many-token
    kernels (bucketing, grouped gate/up and down, combine)."""
    from shiftwing_amd import Backend, MoeLayer
    base, nl, T, use_zipf, desc = MANY[args.workload]
    H, E, K, I, Ish, fmt, layers_full, seed, _ = WORKLOADS[base]
    cfg = (H, E, K, I, Ish, fmt, nl, seed, desc)
    if T is None:
        T = args.batch
    if args.layers:
        nl = args.layers
    prefill = args.workload.startswith("prefill")
    be = Backend(0)
    lib = be.lib
    t0 = time.perf_counter()
    stack = []
    for l in range(nl):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, l)
        stack.append(L)
    be.sync()
    zipf_rec = apply_zipf(be, stack, cfg) if use_zipf else None
    gen_s = time.perf_counter() - t0
    resident = sum(L.nbytes() for L in stack)
    total = args.warmup + args.steps
    # activations: [layer][step][T][H] for the stack, [step][T][H] for prefill
    rows_per_layer = total * T
    xs = be.alloc((nl if not prefill else 1) * rows_per_layer * H * 4)
    for l in range(nl if not prefill else 1):
        off = l * rows_per_layer * H * 4
        done = 0
        while done < rows_per_layer:
            n = min(65535, rows_per_layer - done)
            be.check(lib.coli_cuda_synth_activations(be.ctx, C.c_void_p(xs.ptr + off + done * H * 4), n, H,
                                                     C.c_ulonglong(seed), l, done))
            done += n
    nrows = (nl if not prefill else 1) * rows_per_layer
    xh = np.empty((nrows, H), np.float32)
    be.check(lib.coli_cuda_download(be.ctx, xh.ctypes.data_as(C.c_void_p), xs.p, xh.nbytes), "download")
    be.sync()
    if prefill:  # bf16-valued activations (round to nearest even), passed as f32
        u = xh.view(np.uint32)
        u += 0x7FFF + ((u >> 16) & 1)
        u &= 0xFFFF0000
    if use_zipf:
        xh[:, H - 1] = 1.0
    be.check(lib.coli_cuda_upload(be.ctx, xs.p, xh.ctypes.data_as(C.c_void_p), xh.nbytes), "upload")
    be.sync()
    ys = be.alloc((nl if not prefill else 1) * T * H * 4)
    arr = (C.c_void_p * nl)(*[L.h.value for L in stack])

    def x_at(l, step):
        return C.c_void_p(xs.ptr + ((0 if prefill else l) * rows_per_layer + step * T) * H * 4)

    def run(step):
        if prefill:
            L = stack[step % nl]
            be.check(lib.coli_cuda_moe_forward(be.ctx, L.h, ys.p, x_at(0, step), T, None, None), "forward")
        else:
            be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, nl, ys.p, x_at(0, step), T,
                                                      rows_per_layer * H, T * H), "forward_layers")

    for s in range(args.warmup):
        run(s)
    be.sync()
    be.check(lib.coli_cuda_timer_start(be.ctx))
    for s in range(args.warmup, total):
        run(s)
    ms = C.c_float()
    be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)))
    ms_per_step = ms.value / args.steps
    layers_per_step = 1 if prefill else nl
    tok_s = T / (ms_per_step * 1e-3)

    # routing of the timed steps (untimed): distinct experts per layer-step
    di, dw = be.alloc(T * K * 4), be.alloc(T * K * 4)
    uniq = []
    for s in range(args.warmup, total):
        for l in ([s % nl] if prefill else range(nl)):
            be.check(lib.coli_cuda_moe_route(be.ctx, stack[l].h, x_at(l, s), T, di.p, dw.p), "route")
            idx = be.download(di, (T, K), np.int32)
            uniq.append(len(np.unique(idx)))
    U = float(np.mean(uniq))
    names, nbytes, flops = stage_model(H, E, K, I, Ish, fmt, T, U)
    layer_bytes = sum(nbytes)
    layer_flops = sum(flops)

    # per-stage device times (HIP events between the step's kernels)
    be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 1))
    for s in range(args.warmup, args.warmup + min(args.steps, 4)):
        run(s)
    be.sync()
    sms = (C.c_double * 8)()
    calls = C.c_ulonglong()
    be.check(lib.coli_cuda_moe_stage_times(be.ctx, sms, C.byref(calls)))
    be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 0))
    step_s = ms_per_step * 1e-3
    if calls.value:
        per = [sms[i] / calls.value for i in range(7)]
        dom = max(range(7), key=lambda i: per[i])
        kname, dom_bytes, dom_ms = f"stage {names[dom]}", nbytes[dom], per[dom]
    else:  # one token: the persistent decode kernel, one launch per step
        per = None
        kname, dom_bytes, dom_ms = "k_stack", layer_bytes * layers_per_step, ms_per_step
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
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
            "expert_format": f"int{fmt}-g128", "layers_per_step": layers_per_step, "tokens_per_step": T,
            "resident_layers": nl, "seed": seed, "resident_gb": round(resident / 1e9, 2),
            "zipf": zipf_rec,
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
            "traffic": None,
            "bytes_per_launch": int(dom_bytes),
            "avg_launch_us": round(dom_ms * 1e3, 3),
        },
        "mfma": {
            "flops_per_layer": int(layer_flops),
            "achieved_tflops": round(layer_flops * layers_per_step / step_s / 1e12, 3),
            "frac_bf16_peak": round(layer_flops * layers_per_step / step_s / 1e12 / BF16_PEAK_TFLOPS, 5),
            "int8_ops_issued_per_layer": int(2 * (flops[2] + flops[3] + flops[5])),
            "frac_int8_peak": round(2 * (flops[2] + flops[3] + flops[5]) * layers_per_step / step_s / 1e12
                                    / INT8_PEAK_TOPS, 5),
        },
        "step": {
            "distinct_experts_per_layer": round(U, 2),
            "algorithmic_bytes_per_layer": int(layer_bytes),
            "effective_gbs": round(layer_bytes * layers_per_step / step_s / 1e9, 1),
            "frac_of_peak": round(layer_bytes * layers_per_step / step_s / 1e9 / HBM_PEAK_GBS, 4),
            "stage_us": {names[i]: round(per[i] * 1e3, 2) for i in range(7)} if per else None,
            "stage_gbs": ({names[i]: round(nbytes[i] / (per[i] * 1e-3) / 1e9, 1) for i in range(7)
                           if nbytes[i] and per[i] > 0} if per else None),
            "weight_generation_s": round(gen_s, 1),
        },
    }
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline_many(cfg if prefill else (H, E, K, I, Ish, fmt, nl, seed, desc),
                                                       T, zipf_rec, args.cpu_seconds)
        except Exception as e:  # the CPU leg never hides the GPU number
            result["cpu_baseline"] = {"value": None, "error": str(e)}
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--workload", default="s397", choices=sorted(WORKLOADS) + sorted(MANY))
    ap.add_argument("--batch", type=int, default=8, help="tokens per step of --workload s397-batch")
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
    if args.workload in MANY:
        bench_many(args)
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
    zipf_rec = apply_zipf(be, stack, WORKLOADS[args.workload]) if args.workload in ZIPF_DECODE else None
    gen_s = time.perf_counter() - t0
    resident = sum(L.nbytes() for L in stack)
    total_steps = args.warmup + args.steps
    xs = be.alloc(layers * total_steps * H * 4)
    for l in range(layers):
        be.check(lib.coli_cuda_synth_activations(
            be.ctx, C.c_void_p(xs.ptr + l * total_steps * H * 4), total_steps, H, C.c_ulonglong(seed), l, 0))
    if zipf_rec is not None:
        set_constant_feature(be, xs, layers * total_steps, H)
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
            "resident_gb": round(resident / 1e9, 2), "zipf": zipf_rec,
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
