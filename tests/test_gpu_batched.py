"""Many-token MoE steps at the batched-decode and prefill workloads, through
the C ABI, against the CPU checker (oracle/, the C restatement of
c/qwen.c moe_prefill_grouped, pinned against the compiled reference).

- Continuous-batch decode on S397 shapes with Zipf(1.1) routing (the router
  column H-1 carries beta*log p, x[t, H-1] = 1): B = 4 and 32 tokens.
- A 512-token prefill chunk through one S35 and one S397 layer with
  bf16-valued N(0,1) activations.
- A batched stack call equals per-layer calls bit for bit.

Contract: router indices (rank order included) bit-exact; the device
bucketing of those indices equals the reference's stable order; outputs within
max-abs 1e-3 x RMS of the reference path."""
import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

S397 = (4096, 512, 10, 1024, 1024, 3)
S35 = (2048, 256, 8, 512, 512, 4)


def _bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).copy()
    u += 0x7FFF + ((u >> 16) & 1)
    u &= 0xFFFF0000
    return u.view(np.float32)


def _pair(be, oracle, shape, seed, layer, beta=None):
    from shiftwing_amd import MoeLayer, zipf
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(seed, layer, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(seed, layer)
    if beta is not None:
        col = zipf.apply_to_layer(be, L, beta, seed, layer)
        hl.set_router_column(H - 1, col)
    return hl, L


def _check_bucket(be, oracle, idx, E):
    T, K = idx.shape
    d_idx = be.upload(np.ascontiguousarray(idx, np.int32))
    off, tok, slot = be.alloc((E + 1) * 4), be.alloc(T * K * 4), be.alloc(T * K * 4)
    be.check(be.lib.coli_cuda_moe_bucket(be.ctx, d_idx.p, T, K, E, off.p, tok.p, slot.p), "bucket")
    o_off, o_tok, o_slot = oracle.bucket(np.ascontiguousarray(idx, np.int32), E)
    g_off = be.download(off, (E + 1,), np.int32)
    n = int(g_off[E])
    assert np.array_equal(g_off, o_off)
    assert np.array_equal(be.download(tok, (T * K,), np.int32)[:n], o_tok)
    assert np.array_equal(be.download(slot, (T * K,), np.int32)[:n], o_slot)


@pytest.mark.parametrize("B", [4, 8, 16, 32])
def test_batched_decode_zipf_s397(be, oracle, B):
    from shiftwing_amd import zipf
    H, E, K = S397[:3]
    beta, _ = zipf.calibrate_beta(H, E, K)
    hl, L = _pair(be, oracle, S397, 397, 3, beta)
    x = np.stack([oracle.synth_x(397, 3, 1000 + t, H) for t in range(B)])
    x[:, H - 1] = 1.0
    print(f"[zipf s397] B={B} beta={beta:.4f}", flush=True)
    want, tr = oracle.moe_prefill(hl, x, trace=True)
    y, idx, w = L.forward_host(x)
    assert np.array_equal(idx, tr["idx"])
    assert np.max(np.abs(w - tr["weight"])) <= 1e-5
    assert_close_rms(y, want, 1e-3, f"zipf batch B={B}")
    _check_bucket(be, oracle, idx, E)
    # the routing is skewed: the hottest ranks take a large share of the routes
    rank = zipf.zipf_rank_of_expert(E, 397, 3)
    top_share = np.mean(rank[idx] < 32)
    assert top_share > 0.2, top_share  # uniform routing would give 32/512 = 0.0625


@pytest.mark.parametrize("shape,seed", [(S35, 35), (S397, 397)], ids=["s35", "s397"])
def test_prefill_512(be, oracle, shape, seed):
    H = shape[0]
    oracle.set_threads(16)
    hl, L = _pair(be, oracle, shape, seed, 1)
    x = _bf16(np.stack([oracle.synth_x(seed, 1, t, H) for t in range(512)]))
    print(f"[prefill 512] H={H}", flush=True)
    want, tr = oracle.moe_prefill(hl, x, trace=True)
    y, idx, w = L.forward_host(x)
    assert np.array_equal(idx, tr["idx"])
    assert np.max(np.abs(w - tr["weight"])) <= 1e-5
    assert_close_rms(y, want, 1e-3, f"prefill 512 H={H}")
    _check_bucket(be, oracle, idx, shape[1])


def test_batched_stack_equals_layer_calls(be):
    """coli_cuda_moe_forward_layers with 8 tokens over 3 layers (strided x and
    y) equals three coli_cuda_moe_forward calls without route outputs bit for
    bit, and calls with route outputs (whose routes are in router_topk's exact
    order, where a stack call may keep a certified set in the order of its
    bounds) within max-abs 1e-3 x RMS."""
    import ctypes as C

    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = S35
    T, nl = 8, 3
    layers = []
    for l in range(nl):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(77, l)
        layers.append(L)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((nl, T, H)).astype(np.float32)
    dx = be.upload(x)
    dy = be.alloc(x.nbytes)
    arr = (C.c_void_p * nl)(*[L.h.value for L in layers])
    be.check(be.lib.coli_cuda_moe_forward_layers(be.ctx, arr, nl, dy.p, dx.p, T, T * H, T * H), "forward_layers")
    ys = be.download(dy, (nl, T, H), np.float32)
    for l in range(nl):
        dxl, dyl = be.upload(x[l]), be.alloc(x[l].nbytes)
        be.check(be.lib.coli_cuda_moe_forward(be.ctx, layers[l].h, dyl.p, dxl.p, T, None, None), "forward")
        y0 = be.download(dyl, (T, H), np.float32)
        assert np.array_equal(ys[l].view(np.uint32), y0.view(np.uint32)), l
        y1, _, _ = layers[l].forward_host(x[l])
        assert_close_rms(ys[l], y1, 1e-3, f"stack layer {l} against a call with route outputs")


@pytest.mark.parametrize("T", [2, 3, 5])
def test_small_batch_stack_runs_token_by_token(be, oracle, T):
    """coli_cuda_moe_forward_layers with 2 tokens runs the persistent decode
    kernel once per token: bit for bit the one-token calls.  From 3 tokens the
    many-token step runs.  Either way each layer is within the tolerance of
    the oracle's moe_forward (c/qwen.c:3717-3739)."""
    import ctypes as C

    from conftest import assert_close_rms
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = S35
    nl = 2
    layers, hls = [], []
    for l in range(nl):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(91, l)
        layers.append(L)
        hls.append(oracle.host_layer(91, l, H, E, K, I, Ish, fmt))
    rng = np.random.default_rng(T)
    x = rng.standard_normal((nl, T, H)).astype(np.float32)
    dx = be.upload(x)
    dy = be.alloc(x.nbytes)
    arr = (C.c_void_p * nl)(*[L.h.value for L in layers])
    print(f"[small batch stack] T={T}", flush=True)
    be.check(be.lib.coli_cuda_moe_forward_layers(be.ctx, arr, nl, dy.p, dx.p, T, T * H, T * H), "forward_layers")
    ys = be.download(dy, (nl, T, H), np.float32)
    for t in range(T):
        d1 = be.alloc(nl * H * 4)
        dxt = be.upload(np.ascontiguousarray(x[:, t, :]))
        be.check(be.lib.coli_cuda_moe_forward_layers(be.ctx, arr, nl, d1.p, dxt.p, 1, H, H), "forward_layers 1")
        y1 = be.download(d1, (nl, H), np.float32)
        if T <= 2:
            assert np.array_equal(ys[:, t, :].view(np.uint32), y1.view(np.uint32)), t
    for l in range(nl):
        for t in range(T):
            want = oracle.moe_forward(hls[l], x[l, t])
            assert_close_rms(ys[l, t], want, 1e-3, f"layer {l} token {t}")


@pytest.mark.parametrize("shape,T", [((512, 32, 4, 128, 128, 3), 4100), ((512, 1024, 8, 128, 128, 4), 1300)],
                         ids=["E32_T4100", "E1024_T1300"])
def test_long_block_runs_in_steps(be, oracle, shape, T):
    """A block longer than one step (2048 tokens, or fewer when the bucketing
    map of many experts fills the LDS: 1184 at E = 1024) runs as balanced
    steps; every token's routes and output still match moe_prefill_grouped
    (c/qwen.c:4141-4206) on the whole block."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    oracle.set_threads(16)
    hl = oracle.host_layer(63, 1, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(63, 1)
    x = np.stack([oracle.synth_x(63, 1, t, H) for t in range(T)])
    print(f"[long block] E={E} T={T}", flush=True)
    want, tr = oracle.moe_prefill(hl, x, trace=True)
    y, idx, w = L.forward_host(x)
    assert np.array_equal(idx, tr["idx"])
    assert np.max(np.abs(w - tr["weight"])) <= 1e-5
    assert_close_rms(y, want, 1e-3, f"long block E={E} T={T}")
    L.close()


def test_bucket_limit_follows_the_lds_map(be, oracle):
    """coli_cuda_moe_bucket takes as many tokens as the E x T map fits in
    160 KiB (1184 tokens at 1024 experts) and rejects one more with a message,
    before any launch."""
    rng = np.random.default_rng(12)
    E, K = 1024, 8
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(1184)]).astype(np.int32)
    _check_bucket(be, oracle, idx, E)
    d = be.alloc(1185 * K * 4)
    rc = be.lib.coli_cuda_moe_bucket(be.ctx, d.p, 1185, K, E, d.p, d.p, d.p)
    assert rc == -1 and "1184 tokens" in be.last_error(), be.last_error()


ITEM_CASES = [
    ("s35_T200", S35, 35, 200, None),
    ("s397_zipf_B32", S397, 397, 32, "zipf"),
    ("s397_T64", S397, 397, 64, None),
    ("ragged_T64", (384, 32, 8, 257, 129, 4), 13, 64, None),
    ("I1152_T50", (512, 16, 4, 1152, 128, 3), 11, 50, None),
    ("H4224_T40", (4224, 16, 4, 256, 128, 4), 11, 40, None),
]


@pytest.mark.parametrize("items", [8, 16])
@pytest.mark.parametrize("name,shape,seed,T,routing", ITEM_CASES, ids=[c[0] for c in ITEM_CASES])
def test_item_kernels_vs_oracle(be, oracle, items, name, shape, seed, T, routing):
    """Both routed-expert kernel families of the many-token step against
    moe_prefill_grouped (c/qwen.c:4141-4206): items of 8 tokens (k split over
    the waves) and of 16 tokens (one read of each tile per 16 tokens, digits
    staged in LDS), forced through coli_cuda_moe_set_item_tokens.  Hot Zipf
    experts span several 16-token items; ragged I, I > 1024 and H > 4096
    cover the padding, more than 8 down groups and more than 32 hidden groups."""
    from shiftwing_amd import zipf
    H, E, K = shape[:3]
    beta = zipf.calibrate_beta(H, E, K)[0] if routing == "zipf" else None
    hl, L = _pair(be, oracle, shape, seed, 2, beta)
    x = np.stack([oracle.synth_x(seed, 2, 500 + t, H) for t in range(T)])
    if beta is not None:
        x[:, H - 1] = 1.0
    print(f"[item kernels] {name} items of {items}", flush=True)
    be.check(be.lib.coli_cuda_moe_set_item_tokens(be.ctx, items), "set_item_tokens")
    try:
        want, tr = oracle.moe_prefill(hl, x, trace=True)
        y, idx, w = L.forward_host(x)
    finally:
        be.check(be.lib.coli_cuda_moe_set_item_tokens(be.ctx, 0), "set_item_tokens")
        L.close()
    assert np.array_equal(idx, tr["idx"])
    assert_close_rms(y, want, 1e-3, f"{name} items of {items}")


def test_item_tokens_rejects_other_sizes(be):
    assert be.lib.coli_cuda_moe_set_item_tokens(be.ctx, 12) == -1
    assert "automatic" in be.last_error()
