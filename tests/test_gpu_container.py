"""The converted-snapshot loader on the GPU: a container written in the
reference's conventions (tests/st_writer.py) from the CPU checker's synthetic
layers is loaded into an HBM-resident layer (coli_cuda_moe_layer_load).  The
loaded layer must equal the same layer synthesised on the device bit for bit
(int4 experts from the main payloads, int3 from the .q3 sidecar, int2 from
.qtype 2 payloads or .q2 sidecars), and match
moe_forward / moe_prefill_grouped (c/qwen.c:3717-3739, 4141-4206)."""
import ctypes as C

import numpy as np
import pytest

import st_writer
from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

SHAPE = (512, 16, 4, 256, 128)  # H, E, K, I, Ish


def _load(be, d, layer, K, sidecar, H):
    from shiftwing_amd import Container, MoeLayer
    c = Container(d)
    try:
        return MoeLayer.load(be, c, layer, K, int(sidecar))
    finally:
        c.close()


def test_container_load_equals_device_synthesis(be, oracle, tmp_path):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish = SHAPE
    hl4 = oracle.host_layer(9, 2, H, E, K, I, Ish, 4)
    hl3 = oracle.host_layer(9, 2, H, E, K, I, Ish, 3)
    st_writer.write_split(str(tmp_path), st_writer.moe_layer_tensors(hl4, 2, "model.language_model.", q3=hl3), 3)
    x = np.stack([oracle.synth_x(9, 2, t, H) for t in range(5)])
    for use_q3, hl, fmt in ((0, hl4, 4), (1, hl3, 3)):
        print(f"[container] load use_q3={use_q3}", flush=True)
        Lc = _load(be, str(tmp_path), 2, K, use_q3, H)
        Ls = MoeLayer(be, H, E, K, I, Ish, fmt)
        Ls.synthesize(9, 2)
        for rows in (x[:1], x):
            yc, ic, _ = Lc.forward_host(rows)
            ys, is_, _ = Ls.forward_host(rows)
            assert np.array_equal(ic, is_)
            assert np.array_equal(yc.view(np.uint32), ys.view(np.uint32))
        want, tr = oracle.moe_prefill(hl, x, trace=True)
        y, idx, _ = Lc.forward_host(x)
        assert np.array_equal(idx, tr["idx"])
        assert_close_rms(y, want, 1e-3, f"container use_q3={use_q3}")
        Lc.close()
        Ls.close()


def test_container_bf16_router(be, oracle, tmp_path):
    """A BF16 router (the reference reads it through st_read_f32, c/st.h) is
    widened to f32 on load: routing equals router_topk over the widened
    router."""
    H, E, K, I, Ish = SHAPE
    hl = oracle.host_layer(10, 0, H, E, K, I, Ish, 4)
    st_writer.write_split(str(tmp_path), st_writer.moe_layer_tensors(hl, 0, router_bf16=True), 2)
    hl.router_w[...] = st_writer.bf16_values(hl.router_w)
    Lc = _load(be, str(tmp_path), 0, K, 0, H)
    x = np.stack([oracle.synth_x(10, 0, t, H) for t in range(3)])
    want, tr = oracle.moe_prefill(hl, x, trace=True)
    y, idx, _ = Lc.forward_host(x)
    assert np.array_equal(idx, tr["idx"])
    assert_close_rms(y, want, 1e-3, "container bf16 router")
    Lc.close()


def test_container_int2_loads(be, oracle, tmp_path):
    """int2 routed experts as the reference reads them (c/qwen.c:2207-2212,
    2244-2246): .qtype 2 main payloads (sidecar 0) and .q2 sidecars (sidecar
    2, EXPERT_Q2=1).  Loaded, they equal the same int2 layer synthesised on the
    device bit for bit, and match moe_forward / moe_prefill_grouped over the
    int2 layer; the .q2 directory's main payloads (sidecar 0) are its int4
    layer."""
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish = SHAPE
    hl4 = oracle.host_layer(8, 1, H, E, K, I, Ish, 4)
    hl2 = oracle.host_layer(8, 1, H, E, K, I, Ish, 2)
    st_writer.write_split(str(tmp_path / "q2main"), st_writer.moe_layer_tensors(hl2, 1), parts=2)
    st_writer.write_split(str(tmp_path / "q2side"), st_writer.moe_layer_tensors(hl4, 1, q2=hl2), parts=2)
    x = np.stack([oracle.synth_x(8, 1, t, H) for t in range(5)])
    Ls = MoeLayer(be, H, E, K, I, Ish, 2)
    Ls.synthesize(8, 1)
    want, tr = oracle.moe_prefill(hl2, x, trace=True)
    want1, tr1 = oracle.moe_forward(hl2, x[0], trace=True)
    for d, sidecar in (("q2main", 0), ("q2side", 2)):
        print(f"[container int2] {d} sidecar {sidecar}", flush=True)
        Lc = _load(be, str(tmp_path / d), 1, K, sidecar, H)
        try:
            for rows in (x[:1], x):
                yc, ic, _ = Lc.forward_host(rows)
                ys, is_, _ = Ls.forward_host(rows)
                assert np.array_equal(ic, is_)
                assert np.array_equal(yc.view(np.uint32), ys.view(np.uint32))
            y, idx, _ = Lc.forward_host(x)
            assert np.array_equal(idx, tr["idx"])
            assert_close_rms(y, want, 1e-3, f"{d} int2 block")
            y1, i1, _ = Lc.forward_host(x[0])
            assert np.array_equal(i1[0], tr1["idx"])
            assert_close_rms(y1[0], want1, 1e-3, f"{d} int2 token")
        finally:
            Lc.close()
    Ls.close()
    Lc = _load(be, str(tmp_path / "q2side"), 1, K, 0, H)
    want4, tr4 = oracle.moe_forward(hl4, x[0], trace=True)
    y, idx, _ = Lc.forward_host(x[0])
    assert np.array_equal(idx[0], tr4["idx"])
    assert_close_rms(y[0], want4, 1e-3, "q2side main payload")
    Lc.close()


def test_container_int2_sidecars_with_an_int4_fallback(be, oracle, tmp_path):
    """EXPERT_Q2=1 takes an expert's .q2 sidecar where it has one, else its
    int4 payload (c/qwen.c:2207-2214): with the last expert's sidecar
    missing, the loaded layer mixes int2 and int4 experts (both held as int4
    records) and matches moe_forward / moe_prefill_grouped over the same
    mixed layer."""
    H, E, K, I, Ish = SHAPE
    hl4 = oracle.host_layer(12, 1, H, E, K, I, Ish, 4)
    mix = oracle.host_layer(12, 1, H, E, K, I, Ish, 2)
    t = st_writer.moe_layer_tensors(hl4, 1, q2=mix)
    for nm in ("gate", "up", "down"):
        base = f"layers.1.mlp.experts.{E - 1}.{nm}_proj.weight.q2"
        for sfx in ("", ".qs", ".qtype"):
            del t[base + sfx]
    st_writer.write_split(str(tmp_path), t, parts=2)
    # the CPU checker's layer: int2 experts but the last, which is int4
    mix._g[E - 1], mix._u[E - 1], mix._d[E - 1] = hl4.gate[E - 1].st, hl4.up[E - 1].st, hl4.down[E - 1].st
    # tokens 1, 4 and 5 route to the last (int4) expert
    x = np.stack([oracle.synth_x(12, 1, t_, H) for t_ in range(6)])
    Lc = _load(be, str(tmp_path), 1, K, 2, H)
    try:
        want, tr = oracle.moe_prefill(mix, x, trace=True)
        y, idx, _ = Lc.forward_host(x)
        assert np.array_equal(idx, tr["idx"])
        assert_close_rms(y, want, 1e-3, "int2 + int4 fallback block")
        assert E - 1 in set(np.asarray(tr["idx"]).ravel().tolist())
        for r in range(2):
            w1, tr1 = oracle.moe_forward(mix, x[r], trace=True)
            y1, i1, _ = Lc.forward_host(x[r])
            assert np.array_equal(i1[0], tr1["idx"])
            assert_close_rms(y1[0], w1, 1e-3, f"int2 + int4 fallback token {r}")
    finally:
        Lc.close()


def test_container_load_refusals(be, oracle, tmp_path):
    """Layers the device layer does not take return -1 with a message from
    coli_cuda_moe_layer_load, and nothing is created: int4 experts in groups
    of 64 (read by the reference's CPU path, c/qwen.c:2244-2254), and a shared
    expert tagged int8 with two scales per row (more than the one per row an
    int8 matrix uses, c/qwen.c:1765-1768)."""
    H, E, K, I, Ish = SHAPE
    hl = oracle.host_layer(6, 1, H, E, K, I, Ish, 4)
    hl64 = oracle.host_layer(6, 1, H, E, K, I, Ish, 4, gs=64)
    st_writer.write_split(str(tmp_path / "g64"), st_writer.moe_layer_tensors(hl64, 1), parts=1)
    t = st_writer.moe_layer_tensors(hl, 1)
    t["layers.1.mlp.shared_expert.down_proj.weight.qs"] = np.repeat(
        np.asarray(hl.shared_down.s, np.float32)[:, None], 2, axis=1)
    st_writer.write_split(str(tmp_path / "i8two"), t, parts=1)
    from shiftwing_amd import Container
    for d, sidecar, msg in (("g64", 0, "groups of 64"), ("i8two", 0, "2 scales per row")):
        print(f"[container refusal] {d}", flush=True)
        c = Container(str(tmp_path / d))
        try:
            h = C.c_void_p()
            rc = be.lib.coli_cuda_moe_layer_load(be.ctx, c.h, 1, K, sidecar, C.byref(h))
            err = be.lib.coli_cuda_last_error().decode()
            assert rc == -1 and not h.value, (d, rc)
            assert msg in err, (d, err)
        finally:
            c.close()
