"""MoE decode benchmark on one MI355X.

Headline (the north-star config): a
Qwen3.5-397B-A17B-shaped MoE stack, 60 layers, hidden 4096, 512 routed experts
in grouped int3 (g128, uniform random codes, |N(0,0.01)| scales), top-10
softmax router (fp32 ~N(0,0.02)), one int8 shared expert (intermediate 1024);
all 157 GB of expert weights resident in HBM; batch-1 decode with seeded
N(0,1) activations per (step, layer).  A step is one decoded token through
every layer of the stack, layer l+1 starting after layer l's output is written
(strict decode order).  `value` is tokens/s with all inputs already in HBM.

The default run also times, in the same process, and reports under
"configs": configs[3] (continuous-batch decode on the same stack with Zipf(1.1)
routing, B = 1, 4, 8, 16, 32), configs[4] (a 512-token prefill chunk through
one S397 and one S35 layer) and configs[1] (the 40-layer S35 int4 stack,
batch-1 decode, Zipf routing).  `--workload` runs one of them alone.

Every result carries a roofline object for its dominant kernel (algorithmic
bytes per launch over the launch's duration, HIP events on the context
stream) and a cpu_baseline: the reference's own CPU MoE code (c/qwen.c
moe_forward / moe_prefill_grouped, compiled in place into oracle/_ref) on a
bounded sample of the same workload, with every usable host CPU and with 8
threads, next to the host CPU's model and physical core count.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import subprocess
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


def cpu_info():
    """The host CPU as lscpu describes it, and the CPUs this process may use
    (the GPU box gives a job a share of the host's CPUs)."""
    info = {"model": None, "physical_cores": None, "logical_cpus": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        info["model"] = kv.get("Model name")
        cps, sockets = kv.get("Core(s) per socket"), kv.get("Socket(s)")
        if cps and sockets and cps.isdigit() and sockets.isdigit():
            info["physical_cores"] = int(cps) * int(sockets)
    except Exception:
        pass
    return info


_HOST_LAYERS = {}


def host_layer(o, seed, l, H, E, K, I, Ish, fmt):
    key = (seed, l, H, E, K, I, Ish, fmt)
    if key not in _HOST_LAYERS:
        _HOST_LAYERS[key] = o.host_layer(seed, l, H, E, K, I, Ish, fmt)
    return _HOST_LAYERS[key]


def _timed(run_one, budget_s, max_n):
    run_one(0)  # warm the caches
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < max_n:
        n += run_one(n + 1)
    return n, time.perf_counter() - t0


def cpu_baseline(cfg, budget_s: float, zipf_rec=None):
    """The reference CPU path (c/qwen.c moe_forward, compiled in place into
    oracle/_ref) on a bounded sample: two layers of the same synthetic stack
    materialised on the host (identical bytes), tokens decoded until the time
    budget is spent, tok/s scaled to the full stack.  Timed with every usable
    host CPU, then again with 8 threads (the reference's 8-core desktop
    figures)."""
    H, E, K, I, Ish, fmt, layers, seed, _ = cfg
    from oracle import pyoracle as po
    o = po.Oracle()
    kind, ref = "port", None
    try:
        ref = po.Reference()
        kind = "reference"
    except Exception:
        pass
    sample_layers = 2
    hls = [host_layer(o, seed, l, H, E, K, I, Ish, fmt) for l in range(sample_layers)]
    if zipf_rec is not None:
        from shiftwing_amd import zipf
        for l, hl in enumerate(hls):
            hl.set_router_column(H - 1, zipf.zipf_column(E, zipf_rec["beta"], seed, l))
    rls = [ref.layer(hl) for hl in hls] if ref is not None else None

    def x_of(l, step):
        x = o.synth_x(seed, l, step, H)
        if zipf_rec is not None:
            x[H - 1] = 1.0
        return x

    def one(i):
        for l in range(sample_layers):
            x = x_of(l, i)
            rls[l].forward(x) if rls is not None else o.moe_forward(hls[l], x)
        return sample_layers

    info = cpu_info()
    out = {"unit": "tok/s", "kind": kind, "lib": os.path.basename(ref.path) if ref is not None else "liboracle.so",
           "cpu_model": info["model"], "physical_cores": info["physical_cores"],
           "logical_cpus": info["logical_cpus"]}
    for threads, key in ((info["usable_cpus"], "value"), (8, "value_8_threads")):
        (ref.set_threads if ref is not None else o.set_threads)(threads)
        n, dt = _timed(one, budget_s if key == "value" else budget_s / 2, 4096)
        out[key] = round(1.0 / (dt / n * layers), 3)
        if key == "value":
            out["cores"] = threads
            out["sample"] = (f"{n} token-layers over layers 0..{sample_layers - 1} of the same synthetic stack "
                             f"({dt:.1f} s, {dt / n * 1e3:.3f} ms per token-layer, {threads} threads), "
                             f"scaled to {layers} layers")
    if zipf_rec is not None:
        for l, hl in enumerate(hls):  # the cached layers go back to uniform routing
            hl.set_router_column(H - 1, _uniform_column(o, seed, l, H, E))
    return out


def _uniform_column(o, seed, l, H, E):
    from oracle import pyoracle as po
    r = np.zeros((E, H), np.float32)
    g = np.zeros(H, np.float32)
    o.lib.or_synth_router(seed, l, E, H, po.ptr(r, po.f32p), po.ptr(g, po.f32p))
    return r[:, H - 1].copy()


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


def cpu_baseline_many(cfg, T, zipf_rec, budget_s: float, layers_per_step: int):
    """The reference CPU path for T-token blocks (c/qwen.c moe_prefill_grouped,
    compiled in place) on layer 0 of the same synthetic stack, with the Zipf
    column and constant feature when the workload routes by Zipf; blocks
    repeated until the budget is spent, tok/s per layer scaled to the layer
    count of the GPU step.  Every usable host CPU, then 8 threads."""
    H, E, K, I, Ish, fmt, _, seed, _ = cfg
    from oracle import pyoracle as po
    o = po.Oracle()
    hl = host_layer(o, seed, 0, H, E, K, I, Ish, fmt)
    if zipf_rec is not None:
        from shiftwing_amd import zipf
        hl.set_router_column(H - 1, zipf.zipf_column(E, zipf_rec["beta"], seed, 0))
    ref = None
    try:
        ref = po.Reference()
        rl = ref.layer(hl)
        run, kind, lib = rl.prefill, "reference", os.path.basename(ref.path)
    except Exception:
        run, kind, lib = (lambda x: o.moe_prefill(hl, x)), "port", "liboracle.so"

    def block(i):
        x = np.stack([o.synth_x(seed, 0, i * T + t, H) for t in range(T)])
        if zipf_rec is not None:
            x[:, H - 1] = 1.0
        return x

    blocks = [block(i) for i in range(3)]

    def one(i):
        run(blocks[i % 3])
        return 1

    info = cpu_info()
    out = {"unit": "tok/s", "kind": kind, "lib": lib, "cpu_model": info["model"],
           "physical_cores": info["physical_cores"], "logical_cpus": info["logical_cpus"]}
    for threads, key in ((info["usable_cpus"], "value"), (8, "value_8_threads")):
        (ref.set_threads if ref is not None else o.set_threads)(threads)
        n, dt = _timed(one, budget_s if key == "value" else budget_s / 2, 64)
        out[key] = round(T / (dt / n * layers_per_step), 3)
        if key == "value":
            out["cores"] = threads
            out["sample"] = (f"{n} blocks of {T} tokens through layer 0 of the same synthetic stack ({dt:.1f} s, "
                             f"{dt / n * 1e3:.1f} ms per block-layer, {threads} threads), scaled to "
                             f"{layers_per_step} layer(s) per step")
    if zipf_rec is not None:
        hl.set_router_column(H - 1, _uniform_column(o, seed, 0, H, E))
    return out


ARITH = ("int3/int4 codes x two int8 activation digits on MFMA, fp32 group scaling; int8 IDOT shared expert; "
         "fp64-certified exact fp32 router")


def build_stack(be, name, n):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt, _, seed, _ = WORKLOADS[name]
    stack = []
    for l in range(n):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, l)
        stack.append(L)
    be.sync()
    return stack


def measure_decode(be, stack, cfg, steps, warmup, zipf_rec, workload_key, decode_kernels=1):
    """Batch-1 decode through the whole stack, one coli_cuda_moe_forward_layers
    call per token (strict decode order)."""
    H, E, K, I, Ish, fmt, layers, seed, desc = cfg
    lib = be.lib
    total = warmup + steps
    xs = be.alloc(layers * total * H * 4)
    for l in range(layers):
        be.check(lib.coli_cuda_synth_activations(
            be.ctx, C.c_void_p(xs.ptr + l * total * H * 4), total, H, C.c_ulonglong(seed), l, 0))
    if zipf_rec is not None:
        set_constant_feature(be, xs, layers * total, H)
    ys = be.alloc(layers * H * 4)
    arr = (C.c_void_p * layers)(*[L.h.value for L in stack])
    stats0 = [L.route_stats_full() for L in stack]

    def run(step):
        be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, layers, ys.p, C.c_void_p(xs.ptr + step * H * 4),
                                                  1, total * H, H), "forward_layers")

    for s in range(warmup):
        run(s)
    be.sync()
    be.check(lib.coli_cuda_timer_start(be.ctx))
    for s in range(warmup, total):
        run(s)
    ms = C.c_float()
    be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)))
    ms_per_step = ms.value / steps
    kb = kernel_bytes(H, E, K, I, Ish, fmt)
    step_bytes = sum(kb)
    if decode_kernels == 1:
        # one persistent kernel per step: HIP events on the context stream
        # right before and after single launches give its duration
        durs = []
        for s in range(warmup, warmup + min(steps, 16)):
            be.check(lib.coli_cuda_timer_start(be.ctx))
            run(s)
            m1 = C.c_float()
            be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(m1)))
            durs.append(m1.value)
        launch_ms = sum(durs) / len(durs)
        kname, launch_bytes, per_launch_layers = "k_stack", layers * step_bytes, layers
        kernel_us = {"k_stack": round(launch_ms * 1e3, 3), "per_layer": round(launch_ms * 1e3 / layers, 3)}
    else:
        be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 1))
        nst = min(steps, 8)
        for s in range(warmup, warmup + nst):
            run(s)
        be.sync()
        kms = (C.c_double * 3)()
        calls = C.c_ulonglong()
        be.check(lib.coli_cuda_moe_decode_times(be.ctx, kms, C.byref(calls)))
        be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 0))
        per_call = [kms[i] / max(calls.value, 1) for i in range(3)]
        dom = max(range(3), key=lambda i: per_call[i])
        kname, launch_bytes, per_launch_layers = KERNELS[dom], kb[dom], 1
        launch_ms = per_call[dom]
        kernel_us = {KERNELS[i]: round(per_call[i] * 1e3, 3) for i in range(3)}
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    stats = [L.route_stats_full() for L in stack]
    routed = sum(b[0] - a[0] for a, b in zip(stats0, stats))
    unc = sum(b[1] - a[1] for a, b in zip(stats0, stats))
    full = sum(b[2] - a[2] for a, b in zip(stats0, stats))
    return {
        "metric": METRIC, "value": round(steps / (ms.value / 1e3), 3), "unit": "tok/s",
        "ms_per_step": round(ms_per_step, 4), "steps": steps, "warmup": warmup,
        "config": {"workload": desc, "hidden": H, "experts": E, "topk": K, "intermediate": I,
                   "shared_intermediate": Ish, "expert_format": f"int{fmt}-g128", "layers": layers, "batch": 1,
                   "seed": seed, "resident_gb": round(sum(L.nbytes() for L in stack) / 1e9, 2), "zipf": zipf_rec,
                   "arithmetic": ARITH},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(workload_key, kname, per_launch_layers),
                     "bytes_per_launch": launch_bytes, "avg_launch_us": round(launch_ms * 1e3, 3)},
        "step": {"algorithmic_bytes_per_layer": step_bytes,
                 "effective_gbs": round(step_bytes * layers / (ms_per_step * 1e-3) / 1e9, 1),
                 "frac_of_peak": round(step_bytes * layers / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "kernel_us": kernel_us,
                 "router_not_certified": f"{unc}/{routed} token-layers ({full} needed every chain)"},
    }


STAMP_NAMES = ["router_done", "router_workgroup_barrier", "selection_done", "routed_gateup_done",
               "hidden_barrier_passed", "down_done", "layer_barrier_passed"]


def stack_stamps(be, stack, cfg, steps=8):
    """Per-stage stamps of the persistent decode kernel (coli_cuda_moe_stack_trace):
    median and slowest-workgroup microseconds from each layer's start, over the
    inner layers of `steps` further decode steps (after the timed region)."""
    H, E, K, I, Ish, fmt, layers, seed, desc = cfg
    lib = be.lib
    sm, lds = C.c_int(), C.c_int()
    be.check(lib.coli_cuda_device_limits(be.ctx, C.byref(sm), C.byref(lds)), "device_limits")
    NB, KS = sm.value, 8
    xs = be.alloc(layers * steps * H * 4)
    for l in range(layers):
        be.check(lib.coli_cuda_synth_activations(be.ctx, C.c_void_p(xs.ptr + l * steps * H * 4), steps, H,
                                                 C.c_ulonglong(seed + 1), l, 0))
    ys = be.alloc(layers * H * 4)
    arr = (C.c_void_p * layers)(*[L.h.value for L in stack])
    words = layers * NB * KS
    tr = be.alloc(words * 8)
    be.check(lib.coli_cuda_moe_stack_trace(be.ctx, tr.p, words))
    rel = []
    for s_ in range(steps):
        be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, layers, ys.p, C.c_void_p(xs.ptr + s_ * H * 4), 1,
                                                  steps * H, H), "forward_layers")
        be.sync()
        t = be.download(tr, (layers, NB, KS), np.uint64).astype(np.int64)
        rel.append((t[1:layers - 1] - t[1:layers - 1, :, 0:1]) / 100.0)
    be.check(lib.coli_cuda_moe_stack_trace(be.ctx, None, 0))
    r = np.stack(rel)
    out = {}
    for k, name in enumerate(STAMP_NAMES, start=1):
        v = r[..., k].ravel()
        out[name] = {"median_us": round(float(np.median(v)), 2), "max_us": round(float(v.max()), 2)}
    return out


def measure_many(be, stack, cfg, T, prefill, steps, warmup, zipf_rec, workload_key):
    """Configs 3 and 4: T tokens per MoE step through the many-token kernels
    (bucketing, grouped gate/up and down, combine); a prefill step is one
    layer (the resident copies used in turn), a batched-decode step every
    layer of the stack."""
    H, E, K, I, Ish, fmt, _, seed, desc = cfg
    lib = be.lib
    nl = len(stack)
    total = warmup + steps
    rows_per_layer = total * T
    nx = 1 if prefill else nl
    xs = be.alloc(nx * rows_per_layer * H * 4)
    for l in range(nx):
        off, done = l * rows_per_layer * H * 4, 0
        while done < rows_per_layer:
            n = min(65535, rows_per_layer - done)
            be.check(lib.coli_cuda_synth_activations(be.ctx, C.c_void_p(xs.ptr + off + done * H * 4), n, H,
                                                     C.c_ulonglong(seed), l, done))
            done += n
    xh = np.empty((nx * rows_per_layer, H), np.float32)
    be.check(lib.coli_cuda_download(be.ctx, xh.ctypes.data_as(C.c_void_p), xs.p, xh.nbytes), "download")
    be.sync()
    if prefill:  # bf16-valued activations (round to nearest even), passed as f32
        u = xh.view(np.uint32)
        u += 0x7FFF + ((u >> 16) & 1)
        u &= 0xFFFF0000
    if zipf_rec is not None:
        xh[:, H - 1] = 1.0
    be.check(lib.coli_cuda_upload(be.ctx, xs.p, xh.ctypes.data_as(C.c_void_p), xh.nbytes), "upload")
    be.sync()
    ys = be.alloc(nx * T * H * 4)
    arr = (C.c_void_p * nl)(*[L.h.value for L in stack])

    def x_at(l, step):
        return C.c_void_p(xs.ptr + ((0 if prefill else l) * rows_per_layer + step * T) * H * 4)

    def run(step):
        if prefill:
            be.check(lib.coli_cuda_moe_forward(be.ctx, stack[step % nl].h, ys.p, x_at(0, step), T, None, None),
                     "forward")
        else:
            be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, nl, ys.p, x_at(0, step), T, rows_per_layer * H,
                                                      T * H), "forward_layers")

    for s in range(warmup):
        run(s)
    be.sync()
    be.check(lib.coli_cuda_timer_start(be.ctx))
    for s in range(warmup, total):
        run(s)
    ms = C.c_float()
    be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)))
    ms_per_step = ms.value / steps
    layers_per_step = 1 if prefill else nl
    # routing of the timed steps (untimed): distinct experts per layer-step,
    # and how often the fp64 bounds left a token's top K to the exact chains
    di, dw = be.alloc(T * K * 4), be.alloc(T * K * 4)
    uniq = []
    stats0 = [L.route_stats_full() for L in stack]
    for s in range(warmup, total):
        for l in ([s % nl] if prefill else range(nl)):
            be.check(lib.coli_cuda_moe_route(be.ctx, stack[l].h, x_at(l, s), T, di.p, dw.p), "route")
            uniq.append(len(np.unique(be.download(di, (T, K), np.int32))))
    U = float(np.mean(uniq))
    stats1 = [L.route_stats_full() for L in stack]
    routed = sum(b[0] - a[0] for a, b in zip(stats0, stats1))
    unc = sum(b[1] - a[1] for a, b in zip(stats0, stats1))
    full = sum(b[2] - a[2] for a, b in zip(stats0, stats1))
    names, nbytes, flops = stage_model(H, E, K, I, Ish, fmt, T, U)
    layer_bytes, layer_flops = sum(nbytes), sum(flops)
    # per-stage device times (HIP events between the step's kernels)
    be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 1))
    for s in range(warmup, warmup + min(steps, 4)):
        run(s)
    be.sync()
    sms = (C.c_double * 8)()
    calls = C.c_ulonglong()
    be.check(lib.coli_cuda_moe_stage_times(be.ctx, sms, C.byref(calls)))
    be.check(lib.coli_cuda_moe_stage_timing(be.ctx, 0))
    step_s = ms_per_step * 1e-3
    if calls.value:
        per = [sms[i] / calls.value for i in range(7)]
        # the roofline's kernel: the longer of the two HBM-bound expert stages
        dom = max((names.index("routed_gateup"), names.index("down")), key=lambda i: per[i])
        kname, dom_bytes, dom_ms = f"stage {names[dom]}", nbytes[dom], per[dom]
    else:  # one token: the persistent decode kernel, one launch per step
        per = None
        kname, dom_bytes, dom_ms = "k_stack", layer_bytes * layers_per_step, ms_per_step
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    return {
        "value": round(T / step_s, 3), "unit": "tok/s", "ms_per_step": round(ms_per_step, 4), "steps": steps,
        "config": {"workload": desc, "tokens_per_step": T, "layers_per_step": layers_per_step,
                   "resident_layers": nl, "zipf": zipf_rec},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(workload_key, kname.replace("stage ", ""), 1),
                     "bytes_per_launch": int(dom_bytes), "avg_launch_us": round(dom_ms * 1e3, 3)},
        "mfma": {"flops_per_layer": int(layer_flops),
                 "achieved_tflops": round(layer_flops * layers_per_step / step_s / 1e12, 3),
                 "frac_bf16_peak": round(layer_flops * layers_per_step / step_s / 1e12 / BF16_PEAK_TFLOPS, 5),
                 "int8_ops_issued_per_layer": int(2 * (flops[2] + flops[3] + flops[5])),
                 "frac_int8_peak": round(2 * (flops[2] + flops[3] + flops[5]) * layers_per_step / step_s / 1e12
                                         / INT8_PEAK_TOPS, 5)},
        "step": {"distinct_experts_per_layer": round(U, 2), "algorithmic_bytes_per_layer": int(layer_bytes),
                 "router_not_certified": f"{unc}/{routed} token-layers ({full} needed every chain)",
                 "effective_gbs": round(layer_bytes * layers_per_step / step_s / 1e9, 1),
                 "frac_of_peak": round(layer_bytes * layers_per_step / step_s / 1e9 / HBM_PEAK_GBS, 4),
                 "stage_us": {names[i]: round(per[i] * 1e3, 2) for i in range(7)} if per else None,
                 "stage_gbs": ({names[i]: round(nbytes[i] / (per[i] * 1e-3) / 1e9, 1) for i in range(7)
                                if nbytes[i] and per[i] > 0} if per else None)},
    }


HEAD_SHAPE = (248320, 4096)  # vocab x hidden of the S397 model (c/fixtures/qwen3_5_config/config.json:9,98)


def measure_head(be, steps, warmup, batch=1):
    """The output head (the final norm and the int8 lm_head through IDOT,
    coli_cuda_output_head_q8) at the S397 model's vocab x hidden, for `batch`
    final rows per step: HIP events on the context stream around each call.
    The matrix bytes are a constant fill (timing does not depend on values;
    the GPU tests check the arithmetic)."""
    vocab, H = HEAD_SHAPE
    lib = be.lib
    q, sc = be.alloc(vocab * H), be.alloc(vocab * 4)
    be.check(lib.coli_cuda_memset(be.ctx, q.p, 0x35, vocab * H))
    be.check(lib.coli_cuda_synth_activations(be.ctx, sc.p, 1, vocab, C.c_ulonglong(7), 0, 0))
    x, w = be.alloc(batch * H * 4), be.alloc(H * 4)
    be.check(lib.coli_cuda_synth_activations(be.ctx, x.p, batch, H, C.c_ulonglong(8), 0, 0))
    be.check(lib.coli_cuda_synth_activations(be.ctx, w.p, 1, H, C.c_ulonglong(9), 0, 0))
    lg, hid = be.alloc(batch * vocab * 4), be.alloc(batch * H * 4)

    def run():
        be.check(lib.coli_cuda_output_head_q8(be.ctx, lg.p, hid.p, x.p, w.p, C.c_float(1e-6), batch, q.p, sc.p,
                                              vocab, H, H), "output_head_q8")

    for _ in range(warmup):
        run()
    be.sync()
    durs = []
    for _ in range(steps):
        be.check(lib.coli_cuda_timer_start(be.ctx))
        run()
        m = C.c_float()
        be.check(lib.coli_cuda_timer_stop(be.ctx, C.byref(m)))
        durs.append(m.value)
    ms = sum(durs) / len(durs)
    nbytes = vocab * H + vocab * 4 + batch * vocab * 4 + batch * H * 8  # rows, scales, logits, x and n
    achieved = nbytes / (ms * 1e-3) / 1e9
    for b in (q, sc, x, w, lg, hid):
        b.free()
    return {
        "metric": "output head calls/s (final norm + int8 lm_head, IDOT, bit-exact)", "value": round(1e3 / ms, 2),
        "unit": "calls/s", "ms_per_step": round(ms, 4), "steps": steps, "warmup": warmup,
        "config": {"workload": "f4: output head of the S397 model, vocab 248,320 x hidden 4096 int8 lm_head "
                               "(one f32 scale per row), final rmsnorm_zero", "vocab": vocab, "hidden": H,
                   "rows_per_call": batch},
        "roofline": {"bound": "hbm", "kernel": "k_head_norm + k_head_q8", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("output-head", "k_head_q8", 1), "bytes_per_launch": nbytes,
                     "avg_launch_us": round(ms * 1e3, 3)},
    }


def cpu_baseline_head(budget_s: float, batch=1):
    """The CPU path's output head (rmsnorm_zero + IDOT over the int8 lm_head)
    at the full vocab x hidden: the 1 GB matrix streams from host memory as
    it does in the reference (a row sample would sit in the CPU's cache)."""
    from oracle import pyoracle as po
    vocab, H = HEAD_SHAPE
    o = po.Oracle()
    kind, ref = "port", None
    try:
        ref = po.Reference()
        kind = "reference"
    except Exception:
        pass
    rows = vocab
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, (rows, H), dtype=np.int8)
    s = (np.abs(rng.standard_normal(rows)) * 0.01).astype(np.float32)
    x = rng.standard_normal((batch, H)).astype(np.float32)
    w = (rng.standard_normal(H) * 0.1).astype(np.float32)
    m = po.HostQMat(1, rows, H, 0, q=q, s=s)
    impl = ref if ref is not None else o

    def one(i):
        n = np.stack([impl.rmsnorm_zero(x[b], w, 1e-6) for b in range(batch)])
        impl.qmat_mul_batch(n, m, 1)
        return 1

    info = cpu_info()
    out = {"unit": "calls/s", "kind": kind, "cpu_model": info["model"], "physical_cores": info["physical_cores"]}
    for threads, key in ((info["usable_cpus"], "value"), (8, "value_8_threads")):
        impl.set_threads(threads)
        n, dt = _timed(one, budget_s if key == "value" else budget_s / 2, 200)
        out[key] = round(n / dt, 3)
        if key == "value":
            out["cores"] = threads
            out["sample"] = f"{n} calls over all {vocab} rows ({dt:.1f} s, {threads} threads)"
    return out


# f2: the S397 decoder's mixer layers (Qwen3.5-397B-A17B: hidden 4096; Gated
# DeltaNet 16 key / 64 value heads of 128, conv kernel 4; GQA 32 query / 2 kv
# heads of 256, rotary 64, theta 1e7), int4-g128 projections
MIXER_GDN = dict(hidden=4096, key_heads=16, value_heads=64, key_dim=128, value_dim=128, conv_kernel=4)
MIXER_GQA = dict(hidden=4096, query_heads=32, kv_heads=2, head_dim=256, rotary_dim=64)


def _rand_q4(rng, O, I, gs=128):
    rb = row_bytes(4, I, gs)
    return (rng.integers(0, 256, (O, rb), dtype=np.uint8),
            (np.abs(rng.standard_normal((O, (I + gs - 1) // gs))) * 0.005).astype(np.float32))


def _call_ms(be, run, steps, warmup):
    for _ in range(warmup):
        run()
    be.sync()
    durs = []
    for _ in range(steps):
        be.check(be.lib.coli_cuda_timer_start(be.ctx))
        run()
        m = C.c_float()
        be.check(be.lib.coli_cuda_timer_stop(be.ctx, C.byref(m)))
        durs.append(m.value)
    return sum(durs) / len(durs)


def measure_mixers(be, steps, warmup, batch=1, ctx_len=4096):
    """f2: one decode step of the S397 decoder's Gated DeltaNet layer
    (coli_cuda_gdn_slots_q4_f16_device, `batch` sequences in their own slots)
    and of its GQA attention layer at `ctx_len` cached positions
    (coli_cuda_gqa_slots_q4_f16_device), device-resident inputs and outputs,
    HIP events on the context stream.  Algorithmic bytes: every projection
    byte once, the recurrent state read and written, the KV prefix read."""
    from shiftwing_amd.mixers import DeviceAttn, DeviceGdn
    rng = np.random.default_rng(2024)
    lib = be.lib
    g = MIXER_GDN
    H, kh, vh, dk, dv, K = (g[k] for k in ("hidden", "key_heads", "value_heads", "key_dim", "value_dim",
                                           "conv_kernel"))
    cd, vd = 2 * kh * dk + vh * dv, vh * dv
    gdn = DeviceGdn(be, **g, group_size=128, eps=1e-6, qkv=_rand_q4(rng, cd, H), z=_rand_q4(rng, vd, H),
                    out=_rand_q4(rng, H, vd), conv=rng.standard_normal((cd, K)).astype(np.float32) * 0.5,
                    A_log=rng.standard_normal(vh).astype(np.float32) * 0.5,
                    dt_bias=rng.standard_normal(vh).astype(np.float32) * 0.5,
                    norm=np.ones(dv, np.float32), slots=batch)
    x = be.alloc(batch * H * 4)
    ab = be.alloc(batch * vh * 4)
    y = be.alloc(batch * H * 4)
    be.check(lib.coli_cuda_synth_activations(be.ctx, x.p, batch, H, C.c_ulonglong(31), 0, 0))
    be.check(lib.coli_cuda_synth_activations(be.ctx, ab.p, batch, vh, C.c_ulonglong(32), 0, 0))
    slot = np.arange(batch, dtype=np.int32)
    pos = np.full(batch, 7, np.int32)

    def run_gdn():
        be.check(lib.coli_cuda_gdn_slots_q4_f16_device(
            be.ctx, y.p, x.p, ab.p, ab.p, batch, C.c_void_p(slot.ctypes.data), C.c_void_p(pos.ctypes.data),
            *gdn._weights(), batch, H, kh, vh, dk, dv, K, 128, C.c_float(1e-6)), "gdn_slots_device")

    ms_gdn = _call_ms(be, run_gdn, steps, warmup)
    wbytes = sum(m.q.nbytes + m.s.nbytes for m in (gdn.qkv, gdn.z, gdn.out))
    gdn_bytes = wbytes + batch * (2 * vh * dk * dv * 4 + (K + 1) * cd * 4 + 2 * H * 4 + 2 * vh * 4)
    a = MIXER_GQA
    nh, nkv, hd, rd = (a[k] for k in ("query_heads", "kv_heads", "head_dim", "rotary_dim"))
    kvrows, ctxn = nkv * hd, nh * hd
    max_seq = ctx_len + 1
    att = DeviceAttn(be, **a, group_size=128, theta=1e7, eps=1e-6, q=_rand_q4(rng, 2 * ctxn, H),
                     k=_rand_q4(rng, kvrows, H), v=_rand_q4(rng, kvrows, H), o=_rand_q4(rng, H, ctxn), o_fmt=4,
                     q_norm=np.zeros(hd, np.float32), k_norm=np.zeros(hd, np.float32), max_seq=max_seq,
                     slots=batch)
    for sl in range(batch):
        off = sl * max_seq * kvrows * 4
        for buf, seed in ((att.k_cache, 33), (att.v_cache, 34)):
            be.check(lib.coli_cuda_synth_activations(be.ctx, C.c_void_p(buf.ptr + off), max_seq, kvrows,
                                                     C.c_ulonglong(seed), sl, 0))
    apos = np.full(batch, ctx_len, np.int32)

    def run_gqa():
        be.check(lib.coli_cuda_gqa_slots_q4_f16_device(
            be.ctx, y.p, x.p, batch, C.c_void_p(slot.ctypes.data), C.c_void_p(apos.ctypes.data), *att._weights(),
            batch, max_seq, *att._tail()), "gqa_slots_device")

    ms_gqa = _call_ms(be, run_gqa, steps, warmup)
    wq = sum(m.q.nbytes + m.s.nbytes for m in (att.q, att.k, att.v, att.o))
    gqa_bytes = wq + batch * (2 * (ctx_len + 1) * kvrows * 4 + 2 * H * 4)
    for b in (x, ab, y):
        b.free()

    def rl(nbytes, ms, kern):
        ach = nbytes / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "kernel": kern, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_call": int(nbytes),
                "avg_call_us": round(ms * 1e3, 2)}

    return {
        "metric": "mixer-layer decode steps/s (S397 Gated DeltaNet and GQA layers, int4 projections)",
        "unit": "steps/s", "steps": steps, "warmup": warmup,
        "config": {"workload": "f2: one decode step through the S397 decoder's Gated DeltaNet layer and its GQA "
                               f"attention layer at {ctx_len} cached positions, {batch} sequence(s), "
                               "device-resident activations", "batch": batch, "context": ctx_len,
                   **{f"gdn_{k}": v for k, v in MIXER_GDN.items()}, **{f"gqa_{k}": v for k, v in MIXER_GQA.items()}},
        "gdn": {"value": round(1e3 / ms_gdn, 2), "ms_per_step": round(ms_gdn, 4),
                "roofline": rl(gdn_bytes, ms_gdn, "k_mix_proj<4,CONV> + k_gdn_recur + k_mix_proj<4>")},
        "gqa": {"value": round(1e3 / ms_gqa, 2), "ms_per_step": round(ms_gqa, 4),
                "roofline": rl(gqa_bytes, ms_gqa, "k_mix_proj + k_gqa_prep + k_gqa_attn + k_gqa_combine "
                                                  "+ k_mix_proj")},
    }


def cpu_baseline_mixers(budget_s: float, ctx_len=4096):
    """The reference's own gdn_forward and attn_forward (c/qwen.c:3005, 3094,
    compiled in place into oracle/_ref) at the same shapes: one decode token,
    the attention layer at ctx_len cached positions."""
    from oracle import pyoracle as po
    try:
        lib, kind = po.Reference().lib, "reference"
    except Exception:
        lib, kind = None, "port"
    orc = po.Oracle()
    g = MIXER_GDN
    hg = po.HostGdn(5, g["hidden"], g["key_heads"], g["value_heads"], g["key_dim"], g["value_dim"], g["conv_kernel"])
    a = MIXER_GQA
    ha = po.HostAttn(6, a["hidden"], a["query_heads"], a["kv_heads"], a["head_dim"], a["rotary_dim"], o_fmt=4)
    x = np.random.default_rng(7).standard_normal(g["hidden"]).astype(np.float32)
    info = cpu_info()
    out = {"unit": "steps/s", "kind": kind, "cpu_model": info["model"], "physical_cores": info["physical_cores"],
           "cores": info["usable_cpus"]}
    if lib is not None:
        rg = po.RefMixer(lib, hg)
        ra = po.RefMixer(lib, ha, max_seq=ctx_len + 1)
        ra.k_cache[:] = np.random.default_rng(8).standard_normal(ra.k_cache.shape).astype(np.float32)
        ra.v_cache[:] = np.random.default_rng(9).standard_normal(ra.v_cache.shape).astype(np.float32)
        step_g = lambda i: rg.gdn(x, 7 + i)
        step_a = lambda i: ra.attn(x, ctx_len)
    else:
        cs, st = [v[0] for v in hg.new_state()]
        kc, vc = [v[0] for v in ha.new_cache(ctx_len + 1)]
        ab = np.zeros(g["value_heads"], np.float32)
        step_g = lambda i: po.oracle_gdn_step(orc, hg, x, ab, ab, 7 + i, cs, st)
        step_a = lambda i: po.oracle_attn_step(orc, ha, x, ctx_len, kc, vc)
    ng, dg = _timed(lambda i: (step_g(i), 1)[1], budget_s / 2, 200)
    na, da = _timed(lambda i: (step_a(i), 1)[1], budget_s / 2, 200)
    out["gdn_value"] = round(ng / dg, 3)
    out["gqa_value"] = round(na / da, 3)
    out["value"] = out["gdn_value"]
    out["sample"] = f"{ng} Gated DeltaNet steps in {dg:.1f} s, {na} attention steps at {ctx_len} positions in {da:.1f} s"
    return out


def progress(msg):
    """A progress line on stderr (the JSON result is the only stdout line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def with_cpu(result, args, fn):
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = fn()
        except Exception as e:  # the CPU leg never hides the GPU number
            result["cpu_baseline"] = {"value": None, "error": str(e)}
    return result


def headline(result, args, n_gpus=1):
    """The driver's fields around a config-2 decode result."""
    out = {"metric": METRIC, "value": result["value"], "unit": "tok/s", "n_gpus": n_gpus, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": result["ms_per_step"], "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic"}
    for k in ("config", "roofline", "step", "cpu_baseline"):
        if k in result:
            out[k] = result[k]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all",
                    choices=["all", "output-head", "mixers"] + sorted(WORKLOADS) + sorted(MANY),
                    help="all (default): config 2 is the headline; configs 1, 3 (B = 1..32) and 4 are timed in "
                         "the same run and reported under 'configs'")
    ap.add_argument("--batch", type=int, default=8, help="tokens per step of --workload s397-batch")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (testing)")
    ap.add_argument("--decode-kernels", type=int, default=1, choices=[0, 1, 2],
                    help="1: the persistent decode kernel, one launch per stack step (default); "
                         "2: the three per-layer decode kernels; 0: the many-token kernels for every "
                         "step size")
    ap.add_argument("--item-tokens", type=int, default=0, choices=[0, 8, 16],
                    help="many-token steps: tokens per expert item (0 automatic; for measurement)")
    ap.add_argument("--stamps", action="store_true",
                    help="--workload s397/s35: add the persistent kernel's per-stage stamps (measured after the "
                         "timed region) under step.stage_stamps")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="time a plain device-to-device copy of MIB MiB (the counter calibration kernel) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path's multi-GPU sharding is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    from shiftwing_amd import Backend
    be = Backend(0)
    be.set_decode_kernels(args.decode_kernels)
    be.check(be.lib.coli_cuda_moe_set_item_tokens(be.ctx, args.item_tokens), "set_item_tokens")
    t0 = time.perf_counter()

    def cfg_of(name, layers=None):
        H, E, K, I, Ish, fmt, nl, seed, desc = WORKLOADS[name]
        return (H, E, K, I, Ish, fmt, layers or args.layers or nl, seed, desc)

    if args.workload == "output-head":
        r = measure_head(be, args.steps, args.warmup, 1)
        r = with_cpu(r, args, lambda: cpu_baseline_head(args.cpu_seconds))
        print(json.dumps({"n_gpus": 1, "higher_is_better": True, "dtype": "int8", "data": "synthetic", **r}),
              flush=True)
        return
    if args.workload == "mixers":
        r = measure_mixers(be, args.steps, args.warmup, args.batch if args.batch != 8 else 1)
        r = with_cpu(r, args, lambda: cpu_baseline_mixers(args.cpu_seconds))
        print(json.dumps({"n_gpus": 1, "higher_is_better": True, "dtype": "f32", "data": "synthetic", **r}),
              flush=True)
        return
    if args.workload in MANY:
        base, nl, T, use_zipf, desc = MANY[args.workload]
        nl = args.layers or nl
        T = T or args.batch
        prefill = args.workload.startswith("prefill")
        stack = build_stack(be, base, nl)
        cfg = cfg_of(base, nl)[:8] + (desc,)
        zipf_rec = apply_zipf(be, stack, cfg) if use_zipf else None
        r = measure_many(be, stack, cfg, T, prefill, args.steps, args.warmup, zipf_rec, args.workload)
        r = with_cpu(r, args, lambda: cpu_baseline_many(cfg, T, zipf_rec, args.cpu_seconds, 1 if prefill else nl))
        print(json.dumps({"metric": METRIC, "n_gpus": 1, "warmup": args.warmup, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic", **r}),
              flush=True)
        return
    if args.workload == "s35":
        cfg = cfg_of("s35")
        stack = build_stack(be, "s35", cfg[6])
        zipf_rec = apply_zipf(be, stack, cfg)
        r = measure_decode(be, stack, cfg, args.steps, args.warmup, zipf_rec, "s35", args.decode_kernels)
        if args.stamps:
            r["step"]["stage_stamps"] = stack_stamps(be, stack, cfg)
        r = with_cpu(r, args, lambda: cpu_baseline(cfg, args.cpu_seconds, zipf_rec))
        print(json.dumps(headline(r, args)), flush=True)
        return

    # config 2, the headline: the S397 int3 stack, batch-1 decode, uniform routing
    cfg2 = cfg_of("s397")
    s397 = build_stack(be, "s397", cfg2[6])
    gen_s = time.perf_counter() - t0
    progress(f"S397 stack resident in {gen_s:.1f} s")
    r2 = measure_decode(be, s397, cfg2, args.steps, args.warmup, None, "s397", args.decode_kernels)
    progress(f"config 2 decode: {r2['value']} tok/s")
    if args.stamps:
        r2["step"]["stage_stamps"] = stack_stamps(be, s397, cfg2)
    r2["step"]["weight_generation_s"] = round(gen_s, 1)
    r2 = with_cpu(r2, args, lambda: cpu_baseline(cfg2, args.cpu_seconds))
    progress("config 2 CPU baseline done")
    line = headline(r2, args)
    if args.workload == "s397":
        print(json.dumps(line), flush=True)
        return
    configs = {}
    # config 4, S397: one 512-token prefill chunk through one layer (4 resident
    # copies used in turn), uniform routing
    d4 = MANY["prefill-s397"][4]
    c4 = cfg2[:8] + (d4,)
    p397 = measure_many(be, s397[:4], c4, 512, True, 8, 2, None, "prefill-s397")
    progress(f"config 4 S397 prefill: {p397['value']} tok/s")
    p397 = with_cpu(p397, args, lambda: cpu_baseline_many(c4, 512, None, args.cpu_seconds / 2, 1))
    # config 3: continuous-batch decode on the same stack with Zipf routing
    zipf397 = apply_zipf(be, s397, cfg2)
    d3 = MANY["s397-batch"][4]
    c3 = cfg2[:8] + (d3,)
    batch = {}
    for B in (1, 4, 8, 16, 32):
        rb = measure_many(be, s397, c3, B, False, 6, 2, zipf397, "s397-batch")
        if B in (4, 32):
            rb = with_cpu(rb, args, lambda: cpu_baseline_many(c3, B, zipf397, args.cpu_seconds / 2, len(s397)))
        batch[f"B{B}"] = rb
        progress(f"config 3 B={B}: {rb['value']} tok/s")
    configs["config3"] = batch
    for L in s397:
        L.close()
    del s397
    # the S35 stack: config 4 (S35 prefill, uniform routing), then config 1
    # (40-layer batch-1 decode with Zipf routing)
    cfg1 = cfg_of("s35")
    s35 = build_stack(be, "s35", cfg1[6])
    d4s = MANY["prefill-s35"][4]
    c4s = cfg1[:8] + (d4s,)
    p35 = measure_many(be, s35[:4], c4s, 512, True, 8, 2, None, "prefill-s35")
    progress(f"config 4 S35 prefill: {p35['value']} tok/s")
    p35 = with_cpu(p35, args, lambda: cpu_baseline_many(c4s, 512, None, args.cpu_seconds / 2, 1))
    configs["config4"] = {"s35": p35, "s397": p397}
    zipf35 = apply_zipf(be, s35, cfg1)
    r1 = measure_decode(be, s35, cfg1, args.steps, args.warmup, zipf35, "s35", args.decode_kernels)
    progress(f"config 1 decode: {r1['value']} tok/s")
    r1 = with_cpu(r1, args, lambda: cpu_baseline(cfg1, args.cpu_seconds, zipf35))
    configs["config1"] = r1
    for L in s35:
        L.close()
    del s35
    # f4: the output head after the last layer (one decode token)
    hd = measure_head(be, 10, 3)
    progress(f"output head: {hd['roofline']['avg_launch_us']} us per call")
    configs["output_head"] = with_cpu(hd, args, lambda: cpu_baseline_head(args.cpu_seconds / 2))
    # f2: the decoder's mixer layers around the MoE block (one decode token)
    mx = measure_mixers(be, 10, 3)
    progress(f"mixer layers: GDN {mx['gdn']['ms_per_step']} ms, GQA {mx['gqa']['ms_per_step']} ms per step")
    configs["mixers"] = with_cpu(mx, args, lambda: cpu_baseline_mixers(args.cpu_seconds / 2))
    line["configs"] = configs
    line["wall_s"] = round(time.perf_counter() - t0, 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
