"""The benchmarked call and the shared expert's bit-exact contract, against the
CPU checker (oracle/, the C restatement of c/qwen.c pinned to the compiled
reference).

- The call bench.py times: coli_cuda_moe_forward_layers with one token and no
  route outputs, over a multi-layer S397 int3 stack.  Without route outputs the
  persistent kernel takes a certified expert set whose internal order the
  bounds cannot settle as it is (only the combine's rounding order depends on
  it), so steered near-ties inside the top K, at the K|K+1 boundary and
  three-way ties go through that branch and the exact paths.  Each layer's
  output is checked against moe_forward (c/qwen.c:3717-3739) within max-abs
  1e-3 x RMS: routing a wrong expert moves the output by about one expert's
  weight, hundreds of times the tolerance.
- an S35 int4 stack with Zipf(1.1) routing through the same call.
- The shared expert (c/qwen.c:1696-1705, 1765-1768, 3737): with every routed
  expert's scales at zero the routed terms are exactly zero, and with the
  shared gate row at zero the gate is sigmoid(0) = 0.5 exactly, so the layer
  output must equal the reference's shared-expert vector times 0.5 bit for
  bit.  That pins the IDOT quantisation of x, the int32 gate/up dots, the
  SwiGLU (glibc expf), the quantisation of the hidden vector and the int32
  down dots on every product kernel: persistent, three-kernel, many-token and
  the stack call.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

S397 = (4096, 512, 10, 1024, 1024, 3)
S35 = (2048, 256, 8, 512, 512, 4)


def _steer(router_w, x, pairs):
    """x moved (least-norm) so that logit(a) - logit(b) = gap in fp64 for each
    (a, b, gap) in pairs."""
    W = router_w.astype(np.float64)
    D = np.stack([W[a] - W[b] for a, b, _ in pairs])
    g = np.array([gap for _, _, gap in pairs])
    xd = x.astype(np.float64)
    r = D @ xd - g
    xd = xd - D.T @ np.linalg.solve(D @ D.T, r)
    return xd.astype(np.float32)


def _order(hl, x):
    return np.argsort(-(hl.router_w.astype(np.float64) @ x.astype(np.float64)), kind="stable")


# (name, pairs of ranks with their fp64 logit gaps)
CASES = [
    ("plain", []),
    ("tie inside top K (ranks 2|3)", [(2, 3, 1e-6)]),
    ("exact tie inside top K (ranks 0|1)", [(0, 1, 0.0)]),
    ("boundary K-1|K", [("K-1", "K", 1e-6)]),
    ("three-way inside top K (ranks 4|5|6)", [(4, 5, 2e-7), (5, 6, 3e-7)]),
    ("three-way at the boundary (K-2|K-1|K)", [("K-2", "K-1", 1e-6), ("K-1", "K", 5e-7)]),
    ("wide boundary gap", [("K-1", "K", 3e-5)]),
]


def _rank(r, K):
    return {"K": K, "K-1": K - 1, "K-2": K - 2}.get(r, r)


def _stack(be, shape, seed, n):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    layers = []
    for l in range(n):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, l)
        layers.append(L)
    return layers


def _stack_call(be, layers, xs):
    """The bench's call: one token per layer, no route outputs."""
    n, H = xs.shape
    dx = be.upload(np.ascontiguousarray(xs, np.float32))
    dy = be.alloc(n * H * 4)
    arr = (C.c_void_p * n)(*[L.h.value for L in layers])
    be.check(be.lib.coli_cuda_moe_forward_layers(be.ctx, arr, n, dy.p, dx.p, 1, H, H), "forward_layers")
    return be.download(dy, (n, H), np.float32)


def test_bench_call_s397_stack_vs_oracle(be, oracle):
    """coli_cuda_moe_forward_layers(tokens=1, no route outputs) over three
    S397 int3 layers, every step's output per layer against moe_forward."""
    H, E, K, I, Ish, fmt = S397
    seed, n = 397, 3
    hls = [oracle.host_layer(seed, l, H, E, K, I, Ish, fmt) for l in range(n)]
    layers = _stack(be, S397, seed, n)
    as_is = 0
    try:
        for step, (name, pairs) in enumerate(CASES):
            xs = np.zeros((n, H), np.float32)
            for l in range(n):
                x0 = oracle.synth_x(seed, l, step, H)
                if pairs:
                    o = _order(hls[l], x0)
                    x0 = _steer(hls[l].router_w, x0,
                                [(int(o[_rank(a, K)]), int(o[_rank(b, K)]), gap) for a, b, gap in pairs])
                xs[l] = x0
            print(f"[bench call s397] step {step}: {name}", flush=True)
            before = [L.route_stats_full() for L in layers]
            got = _stack_call(be, layers, xs)
            after = [L.route_stats_full() for L in layers]
            for l in range(n):
                want, tr = oracle.moe_forward(hls[l], xs[l], trace=True)
                assert_close_rms(got[l], want, 1e-3, f"step {step} ({name}) layer {l}")
                # the same input with route outputs: indices must be router_topk's
                y1, idx, w = layers[l].forward_host(xs[l])
                assert np.array_equal(idx[0], tr["idx"]), (step, l, idx[0], tr["idx"])
                assert_close_rms(y1[0], want, 1e-3, f"step {step} ({name}) layer {l}, route outputs")
                uncert_stack = after[l][1] - before[l][1]
                uncert_routes = layers[l].route_stats_full()[1] - after[l][1]
                if uncert_routes > uncert_stack:
                    as_is += 1  # this layer's order was uncertain, its set certified
    finally:
        for L in layers:
            L.close()
    print(f"layer-steps through the uncertain-order branch: {as_is}", flush=True)
    assert as_is > 0, "no steered case took the certified-set, uncertain-order branch"


def test_config1_s35_zipf_stack_vs_oracle(be, oracle):
    """configs[1] on four S35 int4 layers: Zipf(1.1) routing through the
    router column H-1 (x[H-1] = 1), the bench's stack call, every layer
    against moe_forward."""
    from shiftwing_amd import zipf
    H, E, K, I, Ish, fmt = S35
    seed, n = 35, 4
    beta, _ = zipf.calibrate_beta(H, E, K)
    layers = _stack(be, S35, seed, n)
    hls = []
    for l in range(n):
        col = zipf.apply_to_layer(be, layers[l], beta, seed, l)
        hl = oracle.host_layer(seed, l, H, E, K, I, Ish, fmt)
        hl.set_router_column(H - 1, col)
        hls.append(hl)
    hot = []
    try:
        for step in range(8):
            xs = np.stack([oracle.synth_x(seed, l, step, H) for l in range(n)])
            xs[:, H - 1] = 1.0
            print(f"[config1 s35 zipf] step {step}", flush=True)
            got = _stack_call(be, layers, xs)
            for l in range(n):
                want, tr = oracle.moe_forward(hls[l], xs[l], trace=True)
                assert_close_rms(got[l], want, 1e-3, f"s35 zipf step {step} layer {l}")
                rank = zipf.zipf_rank_of_expert(E, seed, l)
                hot.append(np.mean(rank[tr["idx"]] < 16))
    finally:
        for L in layers:
            L.close()
    # skewed routing: the 16 hottest of 256 ranks take far more than 16/256
    assert np.mean(hot) > 0.2, np.mean(hot)


def _zero_routed_and_gate(be, L, hl):
    """Every routed expert's scales to zero (codes kept), the shared gate row
    to zero; router and shared expert as synthesised."""
    H, E, I = hl.H, hl.E, hl.I
    zg = np.zeros_like(hl.gsc[0])
    zd = np.zeros_like(hl.dsc[0])
    bufs = [be.upload(hl.gq[0]), be.upload(zg), be.upload(hl.uq[0]), be.upload(zg),
            be.upload(hl.dq[0]), be.upload(zd)]
    for e in range(E):
        L.set_expert(e, *bufs)
    keep = [be.upload(hl.router_w), be.upload(np.zeros(H, np.float32))]
    L.set_router(*keep)
    be.sync()


def _shared_half(oracle, hl, x):
    """The reference's shared-expert vector (IDOT, c/qwen.c:3737) times 0.5."""
    _, tr = oracle.moe_forward(hl, x, trace=True)
    return (tr["shared"].astype(np.float32) * np.float32(0.5)).astype(np.float32)


def _assert_bitexact(got, want, what):
    assert not np.isnan(got).any(), what
    bad = np.where(got != want)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} values differ, first rows "
                           f"{bad[:8].tolist()} got {got[bad[:4]].tolist()} want {want[bad[:4]].tolist()}")


@pytest.mark.parametrize("shape,seed", [(S35, 35), (S397, 397)], ids=["s35", "s397"])
def test_shared_expert_bitexact_every_path(be, oracle, shape, seed):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(seed, 0, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(seed, 0)
    _zero_routed_and_gate(be, L, hl)
    L2 = MoeLayer(be, H, E, K, I, Ish, fmt)  # a second, identical layer for the stack call
    L2.synthesize(seed, 0)
    _zero_routed_and_gate(be, L2, hl)
    xs = np.stack([oracle.synth_x(seed, 0, t, H) for t in range(4)])
    want = np.stack([_shared_half(oracle, hl, xs[t]) for t in range(4)])
    try:
        for mode, name in ((1, "persistent"), (2, "three-kernel"), (0, "many-token, one token")):
            be.set_decode_kernels(mode)
            for t in range(2):
                print(f"[shared bit-exact] {shape[0]} {name} token {t}", flush=True)
                y, _, _ = L.forward_host(xs[t])
                _assert_bitexact(y[0], want[t], f"{name} token {t}")
        be.set_decode_kernels(1)
        print(f"[shared bit-exact] {shape[0]} many-token, 4 tokens", flush=True)
        y, _, _ = L.forward_host(xs)
        for t in range(4):
            _assert_bitexact(y[t], want[t], f"many-token block token {t}")
        print(f"[shared bit-exact] {shape[0]} stack call", flush=True)
        got = _stack_call(be, [L, L2], xs[:2])
        for t in range(2):
            _assert_bitexact(got[t], want[t], f"stack call layer {t}")
    finally:
        be.set_decode_kernels(1)
        L.close()
        L2.close()
