"""The decode step's three router selection paths against router_topk on the
reference's fp32 logits (oracle, c/qwen.c:3421).

Inputs are steered so that two neighbouring experts' logits differ by a
chosen gap: wide gaps are certified by the fp64 bounds, middling gaps need the
exact chains of the ambiguous experts only, near-ties need the reference's full
serial computation.  Every path must give router_topk's indices bit for bit
and the layer output within max-abs 1e-3 x RMS."""
import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

GAPS = [1e-2, 3e-5, 1e-5, 4e-6, 1e-6, 0.0]


def _steer(router_w: np.ndarray, x: np.ndarray, a: int, b: int, gap: float) -> np.ndarray:
    """x moved along (w_a - w_b) so that the fp64 logit difference is `gap`."""
    d = router_w[a].astype(np.float64) - router_w[b].astype(np.float64)
    xd = x.astype(np.float64)
    t = (d @ xd - gap) / (d @ d)
    return (xd - t * d).astype(np.float32)


def _run_cases(be, oracle, shape, seeds):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    seen = {"certified": 0, "targeted": 0, "full": 0}
    for seed in seeds:
        hl = oracle.host_layer(seed, 1, H, E, K, I, Ish, fmt)
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, 1)
        for step, rank in enumerate((K - 1, 0)):
            x0 = oracle.synth_x(seed, 1, step, H)
            order = np.argsort(-(hl.router_w.astype(np.float64) @ x0.astype(np.float64)), kind="stable")
            a, b = int(order[rank]), int(order[rank + 1])
            for gap in GAPS:
                x = _steer(hl.router_w, x0, a, b, gap)
                print(f"[router paths] H{H} E{E} seed {seed} rank {rank} gap {gap:g}", flush=True)
                before = L.route_stats_full()
                want, tr = oracle.moe_forward(hl, x, trace=True)
                y, idx, w = L.forward_host(x)
                after = L.route_stats_full()
                fb, full = after[1] - before[1], after[2] - before[2]
                seen["full" if full else ("targeted" if fb else "certified")] += 1
                assert np.array_equal(idx[0], tr["idx"]), (seed, rank, gap, idx[0], tr["idx"])
                assert np.max(np.abs(w[0] - tr["weight"])) <= 1e-5, (seed, rank, gap)
                assert_close_rms(y[0], want, 1e-3, f"seed {seed} rank {rank} gap {gap:g}")
        L.close()
    return seen


def test_router_paths_small(be, oracle):
    seen = _run_cases(be, oracle, (512, 32, 4, 128, 128, 4), seeds=[11, 12, 13])
    print("paths taken:", seen, flush=True)
    assert seen["certified"] > 0 and seen["targeted"] > 0 and seen["full"] > 0, seen


def test_router_paths_s35_shape(be, oracle):
    seen = _run_cases(be, oracle, (2048, 256, 8, 512, 512, 4), seeds=[35])
    print("paths taken:", seen, flush=True)
    assert seen["targeted"] > 0, seen


def test_decode_kernels_agree_with_many_token_kernels(be, oracle):
    """One token through the decode kernels and through the many-token
    kernels: same indices, outputs within the tolerance of each other."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = 2048, 256, 8, 512, 512, 3
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(77, 3)
    try:
        for t in range(12):
            x = oracle.synth_x(77, 3, t, H)
            be.set_decode_kernels(True)
            y1, i1, w1 = L.forward_host(x)
            be.set_decode_kernels(False)
            y2, i2, w2 = L.forward_host(x)
            assert np.array_equal(i1, i2), t
            assert np.max(np.abs(w1 - w2)) <= 1e-5
            assert_close_rms(y1[0], y2[0], 1e-3, f"decode vs many-token t={t}")
    finally:
        be.set_decode_kernels(True)
        L.close()


@pytest.mark.parametrize("shape", [(2048, 256, 8, 512, 512, 3), (4096, 512, 10, 1024, 1024, 3),
                                   (512, 32, 4, 256, 128, 4)])
def test_persistent_agrees_with_three_kernel_decode(be, oracle, shape):
    """The persistent decode kernel and the three per-layer decode kernels:
    same indices, weights within 1e-5, outputs within the tolerance of each
    other (they quantise the routed hidden vector per 16 and per 128 values)."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(91, 2)
    try:
        for t in range(6):
            print(f"[persistent vs three-kernel] H{H} token {t}", flush=True)
            x = oracle.synth_x(91, 2, t, H)
            be.set_decode_kernels(1)
            y1, i1, w1 = L.forward_host(x)
            be.set_decode_kernels(2)
            y2, i2, w2 = L.forward_host(x)
            assert np.array_equal(i1, i2), t
            assert np.max(np.abs(w1 - w2)) <= 1e-5
            assert_close_rms(y1[0], y2[0], 1e-3, f"persistent vs three-kernel t={t}")
    finally:
        be.set_decode_kernels(1)
        L.close()


def test_stack_forward_equals_per_layer_calls(be):
    """coli_cuda_moe_forward_layers over a stack == one forward per layer."""
    import ctypes as C
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt, n = 1024, 64, 6, 256, 256, 3, 3
    layers = []
    for l in range(n):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(5, l)
        layers.append(L)
    lib = be.lib
    xs = be.alloc(n * 2 * H * 4)
    be.check(lib.coli_cuda_synth_activations(be.ctx, xs.p, 2 * n, H, C.c_ulonglong(5), 0, 0))
    ys = be.alloc(n * H * 4)
    arr = (C.c_void_p * n)(*[L.h.value for L in layers])
    for step in range(2):
        x0 = C.c_void_p(xs.ptr + step * H * 4)
        be.check(lib.coli_cuda_moe_forward_layers(be.ctx, arr, n, ys.p, x0, 1, 2 * H, H))
        got = be.download(ys, (n, H), np.float32)
        for l, L in enumerate(layers):
            y1 = be.alloc(H * 4)
            xl = C.c_void_p(xs.ptr + (l * 2 * H + step * H) * 4)
            be.check(lib.coli_cuda_moe_forward(be.ctx, L.h, y1.p, xl, 1, None, None))
            want = be.download(y1, (H,), np.float32)
            assert np.array_equal(got[l].view(np.uint32), want.view(np.uint32)), (step, l)
    for L in layers:
        L.close()


def test_router_paths_many_token_kernels(be, oracle):
    """The same steered cases through the many-token kernels (one wave per
    token certifies; targeted exact chains of the ambiguous experts; every
    chain and the router_topk replica when those do not settle the order)."""
    be.set_decode_kernels(0)
    try:
        seen = _run_cases(be, oracle, (512, 32, 4, 128, 128, 4), seeds=[11, 12, 13])
    finally:
        be.set_decode_kernels(1)
    print("paths taken:", seen, flush=True)
    assert seen["certified"] > 0 and seen["targeted"] > 0 and seen["full"] > 0, seen


@pytest.mark.parametrize("shape", [(2048, 256, 8, 512, 512, 4), (4096, 512, 10, 1024, 1024, 3)],
                         ids=["s35", "s397"])
def test_router_gemm_path_steered_block(be, oracle, shape):
    """Blocks of at least 64 tokens route through the fp64 MFMA GEMM with the
    a-priori bound, tightened for the experts near each token's top K.  An
    80-token block (two full 32-token tiles and a partial one) whose tokens
    carry steered gaps (every GAPS value at the
    K|K+1 boundary and inside the top K, plus unsteered tokens) must give
    router_topk's indices for every token (c/qwen.c:3421) and outputs within
    max-abs 1e-3 x RMS of moe_prefill_grouped."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    seed = 61
    hl = oracle.host_layer(seed, 4, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(seed, 4)
    xs = []
    for t in range(80):
        x0 = oracle.synth_x(seed, 4, t, H)
        case = t % (2 * len(GAPS) + 2)
        if case < 2 * len(GAPS):
            rank = K - 1 if case < len(GAPS) else 0
            order = np.argsort(-(hl.router_w.astype(np.float64) @ x0.astype(np.float64)), kind="stable")
            x0 = _steer(hl.router_w, x0, int(order[rank]), int(order[rank + 1]), GAPS[case % len(GAPS)])
        xs.append(x0)
    x = np.stack(xs)
    print(f"[router gemm] H{H} E{E} block of 80", flush=True)
    before = L.route_stats_full()
    try:
        want, tr = oracle.moe_prefill(hl, x, trace=True)
        y, idx, w = L.forward_host(x)
        after = L.route_stats_full()
    finally:
        L.close()
    bad = [t for t in range(80) if not np.array_equal(idx[t], tr["idx"][t])]
    assert not bad, f"tokens {bad[:8]}: {idx[bad[0]]} vs {tr['idx'][bad[0]]}"
    assert np.max(np.abs(w - tr["weight"])) <= 1e-5
    assert_close_rms(y, want, 1e-3, f"router gemm block H{H}")
    print("route stats delta:", [a - b for a, b in zip(after, before)], flush=True)
    assert after[1] - before[1] > 0  # the near-ties took the exact chains
