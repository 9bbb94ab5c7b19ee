"""The converted-snapshot loader on the GPU: a container written in the
reference's conventions (tests/st_writer.py) from the CPU checker's synthetic
layers is loaded into an HBM-resident layer (coli_cuda_moe_layer_load).  The
loaded layer must equal the same layer synthesised on the device bit for bit
(int4 experts from the main payloads, int3 from the .q3 sidecar), and match
moe_forward / moe_prefill_grouped (c/qwen.c:3717-3739, 4141-4206)."""
import ctypes as C

import numpy as np
import pytest

import st_writer
from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

SHAPE = (512, 16, 4, 256, 128)  # H, E, K, I, Ish


def _load(be, d, layer, K, use_q3, H):
    from shiftwing_amd import Container, MoeLayer
    c = Container(d)
    try:
        return MoeLayer.load(be, c, layer, K, bool(use_q3))
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
