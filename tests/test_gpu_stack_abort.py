"""The persistent decode kernel's timeout path, forced from the host.

The kernel needs every workgroup resident at once; one that never runs would
leave the others waiting at the grid exchanges.  Every such wait is bounded:
on expiry it raises an abort word that all workgroups read, every workgroup
leaves, and the next coli_cuda_sync reports the abort after clearing the
kernel's device state (counters, tagged records, call state).

coli_cuda_moe_stack_drill keeps the last workgroups of the next launch out, as
a workgroup that never became resident would be, and shortens the wait limit
so the drill takes a millisecond.  Every kernel still exits normally: the
present workgroups time out on the absent ones' router records.  The test
checks that the call reports the abort and that the calls after it give the
results of the calls before it, bit for bit, and the reference's within
tolerance (moe_forward, c/qwen.c:3717-3739; router_topk indices)."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

S35 = (2048, 256, 8, 512, 512, 4)


def _stack_call(be, layers, xs):
    n, H = xs.shape
    dx = be.upload(np.ascontiguousarray(xs, np.float32))
    dy = be.alloc(n * H * 4)
    arr = (C.c_void_p * n)(*[L.h.value for L in layers])
    be.check(be.lib.coli_cuda_moe_forward_layers(be.ctx, arr, n, dy.p, dx.p, 1, H, H), "forward_layers")
    return be.download(dy, (n, H), np.float32)


def test_drill_rejects_bad_arguments(be):
    assert be.lib.coli_cuda_moe_stack_drill(be.ctx, -1, 100) == -1
    assert "absent" in be.last_error()
    assert be.lib.coli_cuda_moe_stack_drill(be.ctx, 1, 0) == -1
    assert "wait limit" in be.last_error()
    assert be.lib.coli_cuda_moe_stack_drill(be.ctx, 1, 2000001) == -1
    assert be.lib.coli_cuda_moe_stack_drill(be.ctx, 1 << 20, 100) == -1
    be.check(be.lib.coli_cuda_moe_stack_drill(be.ctx, 0, 0), "disarm")


def test_abort_drill_then_recovery(be, oracle):
    from shiftwing_amd import HipError, MoeLayer
    H, E, K, I, Ish, fmt = S35
    seed, n = 35, 3
    be.set_decode_kernels(1)
    layers = []
    for l in range(n):
        L = MoeLayer(be, H, E, K, I, Ish, fmt)
        L.synthesize(seed, l)
        layers.append(L)
    hls = [oracle.host_layer(seed, l, H, E, K, I, Ish, fmt) for l in range(n)]
    xs = np.stack([oracle.synth_x(seed, l, 5, H) for l in range(n)])
    try:
        print("[abort drill] calls before the drill", flush=True)
        good = _stack_call(be, layers, xs)
        assert np.array_equal(_stack_call(be, layers, xs).view(np.uint32), good.view(np.uint32))
        for l in range(n):
            assert_close_rms(good[l], oracle.moe_forward(hls[l], xs[l]), 1e-3, f"layer {l}")
        # one workgroup out; half of them out, with a shorter limit
        for absent, us in [(1, 1000), (100, 200)]:
            print(f"[abort drill] {absent} workgroups out, {us} us waits", flush=True)
            be.check(be.lib.coli_cuda_moe_stack_drill(be.ctx, absent, us), "drill")
            with pytest.raises(HipError, match="aborted"):
                _stack_call(be, layers, xs)
            be.sync()  # the report was consumed: the context is clean
            print("[abort drill] the call after it", flush=True)
            again = _stack_call(be, layers, xs)
            assert np.array_equal(again.view(np.uint32), good.view(np.uint32)), absent
            # and a single-layer call with route outputs (the same kernel)
            y1, idx, _ = layers[1].forward_host(xs[1])
            want, tr = oracle.moe_forward(hls[1], xs[1], trace=True)
            assert np.array_equal(idx[0], tr["idx"])
            assert_close_rms(y1[0], want, 1e-3, "layer 1 after the drill")
    finally:
        for L in layers:
            L.close()
