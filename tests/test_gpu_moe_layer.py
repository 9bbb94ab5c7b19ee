"""The fused MoE step (coli_cuda_moe_forward) against the reference CPU layer.

Golden fixtures hold the compiled reference's outputs (moe_forward per token,
moe_prefill_grouped for the token block) for synthetic layers that both sides
regenerate from the seed; the oracle (C restatement) covers random seeds.
Contract: router indices bit-exact; outputs within max-abs 1e-3 x RMS."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, assert_close_rms

pytestmark = pytest.mark.gpu

LAYERS = ["small_q4", "small_q3", "ragged_q4", "ragged_q3", "s35_q4", "s397_q3", "small_q2", "ragged_q2"]


def _load(name):
    g = np.load(os.path.join(GOLDEN, f"layer_{name}.npz"))
    H, E, K, I, Ish, fmt, gs, seed, layer, T = (int(v) for v in g["cfg"])
    return g, dict(H=H, E=E, K=K, I=I, Ish=Ish, fmt=fmt, gs=gs, seed=seed, layer=layer, T=T)


def _device_layer(be, c):
    from shiftwing_amd import MoeLayer
    L = MoeLayer(be, c["H"], c["E"], c["K"], c["I"], c["Ish"], c["fmt"], c["gs"])
    L.synthesize(c["seed"], c["layer"])
    return L


def _pad_ok(c):
    """Shapes the fused layer takes: any I and shared I (held padded to the
    row tiles), H a multiple of 64."""
    return c["H"] % 64 == 0


@pytest.mark.parametrize("name", LAYERS)
def test_decode_matches_reference(be, name):
    g, c = _load(name)
    if not _pad_ok(c):
        pytest.skip("shape outside the fused path's tiling (H%64, I%16, I_sh%64)")
    L = _device_layer(be, c)
    for t in range(c["T"]):
        print(f"[{name}] decode token {t}", flush=True)
        y, idx, w = L.forward_host(g["x"][t])
        assert np.array_equal(idx[0], g["idx"][t]), (t, idx[0], g["idx"][t])
        assert np.max(np.abs(w[0] - g["weight"][t])) <= 1e-4
        assert_close_rms(y[0], g["decode"][t], 1e-3, f"{name} decode t={t}")


def test_decode_repeats_bit_identical_s397(be):
    """The S397 golden tokens, again and again through the persistent kernel:
    every repetition bit-identical to the first and within the tolerance (a
    race between the waves of one workgroup shows as one wrong 16-row tile
    in a few repetitions, not in every one)."""
    g, c = _load("s397_q3")
    L = _device_layer(be, c)
    first = {}
    for rep in range(12):
        for t in range(c["T"]):
            y, idx, w = L.forward_host(g["x"][t])
            assert np.array_equal(idx[0], g["idx"][t]), (rep, t)
            if rep == 0:
                assert_close_rms(y[0], g["decode"][t], 1e-3, f"s397 decode t={t}")
                first[t] = y[0].copy()
            else:
                bad = np.where(y[0].view(np.uint32) != first[t].view(np.uint32))[0]
                assert bad.size == 0, f"repetition {rep} t={t}: rows {bad[:16].tolist()} differ"


@pytest.mark.parametrize("name", LAYERS)
def test_prefill_matches_reference(be, name):
    g, c = _load(name)
    if not _pad_ok(c):
        pytest.skip("shape outside the fused path's tiling")
    L = _device_layer(be, c)
    print(f"[{name}] prefill T={c['T']}", flush=True)
    y, idx, w = L.forward_host(g["x"])
    assert np.array_equal(idx, g["idx"])
    assert_close_rms(y, g["prefill"], 1e-3, f"{name} prefill")


def test_exact_router_mode_bitexact_weights(be, oracle):
    """Router mode 1 runs the serial fp32 chain for every token: indices and
    weights equal router_topk over the reference's logits bit for bit."""
    g, c = _load("s35_q4")
    L = _device_layer(be, c)
    L.set_router_mode(1)
    for t in range(c["T"]):
        y, idx, w = L.forward_host(g["x"][t])
        assert np.array_equal(idx[0], g["idx"][t])
        assert np.array_equal(w[0].view(np.uint32), g["weight"][t].view(np.uint32))
        assert_close_rms(y[0], g["decode"][t], 1e-3, "exact-router decode")
    tok, fb = L.route_stats()
    assert tok == c["T"] and fb == c["T"]


@pytest.mark.parametrize("shape", [(256, 16, 4, 128, 128, 3), (384, 32, 8, 257, 129, 4), (384, 32, 8, 200, 100, 3),
                                   (384, 32, 8, 257, 129, 2)],
                         ids=["small_q3", "ragged_q4", "ragged_q3", "ragged_q2"])
def test_upload_path_equals_device_synthesis(be, oracle, shape):
    """Weights uploaded in the container layout (set_router / set_shared_q8 /
    set_expert, repacked on device) give the same result as device synthesis,
    also for a ragged I and shared I (held padded to the row tiles), one
    token (decode kernels) and three (many-token kernels)."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(21, 2, H, E, K, I, Ish, fmt)
    A = MoeLayer(be, H, E, K, I, Ish, fmt)
    A.synthesize(21, 2)
    B = MoeLayer(be, H, E, K, I, Ish, fmt)
    keep = [be.upload(hl.router_w), be.upload(hl.shared_gate_row)]
    B.set_router(*keep)
    sh = [be.upload(a) for a in (hl.shared_gate.q, hl.shared_gate.s, hl.shared_up.q, hl.shared_up.s,
                                 hl.shared_down.q, hl.shared_down.s)]
    B.set_shared_q8(*sh)
    for e in range(E):
        bufs = [be.upload(a) for a in (hl.gq[e], hl.gsc[e], hl.uq[e], hl.usc[e], hl.dq[e], hl.dsc[e])]
        B.set_expert(e, *bufs)
        be.sync()
    x = np.stack([oracle.synth_x(21, 2, t, H) for t in range(3)])
    ya, ia, _ = A.forward_host(x)
    yb, ib, _ = B.forward_host(x)
    assert np.array_equal(ia, ib)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
    want = oracle.moe_prefill(hl, x)
    assert_close_rms(ya, want, 1e-3, "upload path vs oracle")
    y1a, i1a, _ = A.forward_host(x[0])
    y1b, i1b, _ = B.forward_host(x[0])
    assert np.array_equal(i1a, i1b) and np.array_equal(y1a.view(np.uint32), y1b.view(np.uint32))
    want1, tr = oracle.moe_forward(hl, x[0], trace=True)
    assert np.array_equal(i1a[0], tr["idx"])
    assert_close_rms(y1a[0], want1, 1e-3, "upload path vs oracle, one token")
    A.close()
    B.close()


def test_int2_layer_equals_int4_layer_of_widened_codes(be, oracle):
    """An int2 layer (expert_format 2) is an int4 layer whose codes are the
    int2 codes widened as the reference's q2_expand_q4 does (c/qwen.c:567-575:
    nibble 5 + 2c, the same value 2c - 3), widened here on the host: both
    give the same bits for one token and for a block."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish = 512, 16, 4, 256, 128
    hl = oracle.host_layer(31, 1, H, E, K, I, Ish, 2)

    def widen(q):
        c = [(q >> (2 * k)) & 3 for k in range(4)]
        n = [(5 + 2 * ck).astype(np.uint8) for ck in c]
        out = np.empty(q.shape[:-1] + (2 * q.shape[-1],), np.uint8)
        out[..., 0::2] = n[0] | (n[1] << 4)
        out[..., 1::2] = n[2] | (n[3] << 4)
        return out

    A = MoeLayer(be, H, E, K, I, Ish, 2)
    A.synthesize(31, 1)
    B = MoeLayer(be, H, E, K, I, Ish, 4)
    keep = [be.upload(hl.router_w), be.upload(hl.shared_gate_row)]
    B.set_router(*keep)
    sh = [be.upload(a) for a in (hl.shared_gate.q, hl.shared_gate.s, hl.shared_up.q, hl.shared_up.s,
                                 hl.shared_down.q, hl.shared_down.s)]
    B.set_shared_q8(*sh)
    for e in range(E):
        bufs = [be.upload(np.ascontiguousarray(a)) for a in (widen(hl.gq[e]), hl.gsc[e], widen(hl.uq[e]),
                                                               hl.usc[e], widen(hl.dq[e]), hl.dsc[e])]
        B.set_expert(e, *bufs)
        be.sync()
    try:
        x = np.stack([oracle.synth_x(31, 1, t, H) for t in range(6)])
        for rows in (x[:1], x):
            ya, ia, _ = A.forward_host(rows)
            yb, ib, _ = B.forward_host(rows)
            assert np.array_equal(ia, ib)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
        want, tr = oracle.moe_prefill(hl, x, trace=True)
        y, idx, _ = A.forward_host(x)
        assert np.array_equal(idx, tr["idx"])
        assert_close_rms(y, want, 1e-3, "int2 layer vs oracle")
    finally:
        A.close()
        B.close()


@pytest.mark.parametrize("seed", [101, 202, 303])
def test_random_seeds_vs_oracle_s35(be, oracle, seed):
    H, E, K, I, Ish, fmt = 2048, 256, 8, 512, 512, 4
    hl = oracle.host_layer(seed, 5, H, E, K, I, Ish, fmt)
    from shiftwing_amd import MoeLayer
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(seed, 5)
    for t in range(4):
        x = oracle.synth_x(seed, 5, t, H)
        want, tr = oracle.moe_forward(hl, x, trace=True)
        y, idx, w = L.forward_host(x)
        assert np.array_equal(idx[0], tr["idx"])
        assert_close_rms(y[0], want, 1e-3, f"seed {seed} t {t}")


def test_shapes_interleaved_in_one_context(be):
    """Layers of different shapes served by one context, in both router
    modes, in an order that reuses the context workspace across shapes."""
    order = ["s397_q3", "s35_q4", "small_q3", "s397_q3", "s35_q4"]
    layers = {}
    for i, name in enumerate(order):
        g, c = _load(name)
        if name not in layers:
            layers[name] = _device_layer(be, c)
        L = layers[name]
        L.set_router_mode(i % 2)
        print(f"[interleave] {name} mode {i % 2}", flush=True)
        y, idx, w = L.forward_host(g["x"][0])
        assert np.array_equal(idx[0], g["idx"][0]), name
        assert_close_rms(y[0], g["decode"][0], 1e-3, f"interleaved {name}")


WIDE = [(512, 16, 4, 1152, 128, 4), (512, 16, 4, 1152, 128, 3), (4224, 16, 4, 256, 128, 4),
        (4224, 16, 4, 256, 128, 3)]


@pytest.mark.parametrize("shape", WIDE, ids=["I1152_q4", "I1152_q3", "H4224_q4", "H4224_q3"])
def test_wide_shapes_vs_oracle(be, oracle, shape):
    """Shapes past the common tiles: I > 1024 (more than 8 down groups per row:
    the many-token k_down instead of k_down_split) and H > 4096 (more groups
    per wave than one batch: k_expert_gateup's batched variant; the stack
    kernel's one-output-tile-per-workgroup limit sends one token to the
    three-kernel decode path).  One token and a 40-token block against
    moe_forward / moe_prefill_grouped."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(11, 0, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(11, 0)
    try:
        for t in range(2):
            x = oracle.synth_x(11, 0, t, H)
            want, tr = oracle.moe_forward(hl, x, trace=True)
            y, idx, _ = L.forward_host(x)
            assert np.array_equal(idx[0], tr["idx"]), t
            assert_close_rms(y[0], want, 1e-3, f"{shape} token {t}")
        T = 40
        xs = np.stack([oracle.synth_x(11, 0, 10 + t, H) for t in range(T)])
        want = oracle.moe_prefill(hl, xs)
        y, idx, _ = L.forward_host(xs)
        assert_close_rms(y, want, 1e-3, f"{shape} block of {T}")
    finally:
        L.close()
