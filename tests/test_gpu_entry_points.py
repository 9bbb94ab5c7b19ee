"""The Part 1 entry points that neither the reference's own GPU test
(c/tests/test_backend_cuda.c, run unmodified by test_gpu_reference_glue.py)
nor the MoE tests call: the batched GEMMs, sigmoid_axpy, copy/memset, the
fp32-activation grouped MLPs, and the context queries.

Data follow the reference test's recipe (c/tests/test_backend_cuda.c:131-300:
N=2053, ROWS=37, COLS=1027, GS=128, padded int8 rows of COLS+5 bytes, scales
2^k) and its tolerances (:546-555: 2e-4 for the fp32 GEMVs, 1e-7 for axpy).
The GEMM references are the float64 sums of the dequantised rows (the layouts
the oracle pins: low nibble first, code-8; c/qwen.c:1706-1716)."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

N, ROWS, COLS, GS = 2053, 37, 1027, 128
NG = (COLS + GS - 1) // GS
RB4 = NG * (GS // 2)
RB8 = COLS + 5


def _x(batch):
    i = np.arange(N, dtype=np.float32)
    x = (np.sin(i * 13 + 1) * 0.125).astype(np.float32)
    return np.stack([x[:COLS] + np.float32(0.125 * b) for b in range(batch)]).astype(np.float32)


def _q8():
    r = np.arange(ROWS)[:, None]
    i = np.arange(COLS)[None, :]
    q = np.zeros((ROWS, RB8), np.int8)
    q[:, :COLS] = (((r * 29 + i * 11) % 255) - 127).astype(np.int8)
    s = np.ldexp(np.float32(1), (np.arange(ROWS) % 7) - 9).astype(np.float32)
    return q, s


def _q4():
    q = np.zeros((ROWS, RB4), np.uint8)
    for r in range(ROWS):
        codes = (r * 3 + np.arange(RB4 * 2) * 13) % 16
        q[r] = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    s = np.array([[np.ldexp(1.0, ((r + g) % 7) - 7) for g in range(NG)] for r in range(ROWS)], np.float32)
    return q, s


def _deq4(q, s, cols):
    codes = np.empty((q.shape[0], q.shape[1] * 2), np.int64)
    codes[:, 0::2] = q & 15
    codes[:, 1::2] = q >> 4
    w = (codes[:, :cols] - 8).astype(np.float64)
    return w * np.repeat(s.astype(np.float64), GS, axis=1)[:, :cols]


def test_q8_gemm_batch(be):
    q, s = _q8()
    x = _x(3)
    dq, ds, dx, dy = be.upload(q), be.upload(s), be.upload(x), be.alloc(3 * ROWS * 4)
    be.check(be.lib.coli_cuda_q8_gemm(be.ctx, dy.p, dx.p, 3, dq.p, ds.p, ROWS, COLS, RB8), "q8_gemm")
    got = be.download(dy, (3, ROWS), np.float32)
    want = x.astype(np.float64) @ (q[:, :COLS].astype(np.float64) * s[:, None]).T
    assert np.max(np.abs(got - want)) < 2e-4
    # each sample equals the single-sample GEMV within the same tolerance
    for b in range(3):
        dxb, dyb = be.upload(x[b]), be.alloc(ROWS * 4)
        be.check(be.lib.coli_cuda_q8_gemv(be.ctx, dyb.p, dxb.p, dq.p, ds.p, ROWS, COLS, RB8), "q8_gemv")
        assert np.max(np.abs(be.download(dyb, (ROWS,), np.float32) - got[b])) < 2e-4


def test_q4_gemm_batch(be):
    q, s = _q4()
    x = _x(3)
    dq, ds, dx, dy = be.upload(q), be.upload(s), be.upload(x), be.alloc(3 * ROWS * 4)
    be.check(be.lib.coli_cuda_q4_gemm(be.ctx, dy.p, dx.p, 3, dq.p, ds.p, ROWS, COLS, GS, RB4, NG), "q4_gemm")
    got = be.download(dy, (3, ROWS), np.float32)
    want = x.astype(np.float64) @ _deq4(q, s, COLS).T
    assert np.max(np.abs(got - want)) < 2e-4


@pytest.mark.parametrize("gs", [32, 64])
def test_q4_gemm_other_group_sizes(be, gs):
    """The Part 1 GEMMs take the group size as an argument, as the reference's
    kernels do (c/backend_cuda.cu:485-496: sr[i / group_size]); the CPU path
    derives it as rb*2/ng (c/qwen.c:2253).  A layer quantised in groups other
    than 128 therefore runs on these entry points."""
    ng = (COLS + gs - 1) // gs
    rb = ng * (gs // 2)
    q = np.zeros((ROWS, rb), np.uint8)
    for r in range(ROWS):
        codes = (r * 5 + np.arange(rb * 2) * 7) % 16
        q[r] = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    s = np.array([[np.ldexp(1.0, ((r + 2 * g) % 7) - 7) for g in range(ng)] for r in range(ROWS)], np.float32)
    x = _x(2)
    dq, ds, dx, dy = be.upload(q), be.upload(s), be.upload(x), be.alloc(2 * ROWS * 4)
    be.check(be.lib.coli_cuda_q4_gemm(be.ctx, dy.p, dx.p, 2, dq.p, ds.p, ROWS, COLS, gs, rb, ng), "q4_gemm")
    got = be.download(dy, (2, ROWS), np.float32)
    codes = np.empty((ROWS, rb * 2), np.int64)
    codes[:, 0::2] = q & 15
    codes[:, 1::2] = q >> 4
    w = (codes[:, :COLS] - 8).astype(np.float64) * np.repeat(s.astype(np.float64), gs, axis=1)[:, :COLS]
    want = x.astype(np.float64) @ w.T
    assert np.max(np.abs(got - want)) < 2e-4


def test_sigmoid_axpy_copy_memset(be, oracle):
    i = np.arange(N, dtype=np.float32)
    y0 = (np.cos(i * 7 + 2) * 0.0625).astype(np.float32)
    x = (np.sin(i * 17 + 4) * 0.25).astype(np.float32)
    for logit in (np.float32(-1.75), np.float32(0.0), np.float32(3.5)):
        dy, dx, dl = be.upload(y0), be.upload(x), be.upload(np.array([logit], np.float32))
        be.check(be.lib.coli_cuda_sigmoid_axpy(be.ctx, dy.p, dx.p, dl.p, N), "sigmoid_axpy")
        got = be.download(dy, (N,), np.float32)
        # y += sigmoid(logit) * x, the gate by the reference's sigmoidf_stable
        g = oracle.sigmoid_batch(np.array([logit], np.float32))[0]
        want = (y0 + np.float32(g) * x).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), logit
    dc = be.alloc(N * 4)
    be.check(be.lib.coli_cuda_memset(be.ctx, dc.p, 0x5A, N * 4), "memset")
    assert np.all(be.download(dc, (N * 4,), np.uint8) == 0x5A)
    be.check(be.lib.coli_cuda_copy(be.ctx, dc.p, dx.p, N * 4), "copy")
    assert np.array_equal(be.download(dc, (N,), np.float32).view(np.uint32), x.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 3])
def test_grouped_mlp_fp32_activations(be, oracle, bits):
    """coli_cuda_grouped_q{4,3}_mlp (fp32 x): sum_j w_j * down_j(silu(gate_j x) * up_j x)
    against the oracle's expert MLP (c/qwen.c:1755-1773) on host-synthesised experts."""
    H, E, K, I, Ish = 1024, 8, 3, 384, 256
    hl = oracle.host_layer(77, 0, H, E, K, I, Ish, bits)
    from oracle.pyoracle import HostQMat
    experts = [2, 5, 7]
    w = np.array([0.5, 0.3125, 0.1875], np.float32)
    x = oracle.synth_x(77, 0, 1, H)
    want = np.zeros(H, np.float64)
    keep = []
    ptrs = {k: (C.c_void_p * K)() for k in ("gq", "gs", "uq", "us", "dq", "ds")}
    for j, e in enumerate(experts):
        g = HostQMat(bits, I, H, 128, q=hl.gq[e], s=hl.gsc[e])
        u = HostQMat(bits, I, H, 128, q=hl.uq[e], s=hl.usc[e])
        d = HostQMat(bits, H, I, 128, q=hl.dq[e], s=hl.dsc[e])
        out = np.zeros(H, np.float32)
        oracle.lib.or_mlp_one(out.ctypes.data_as(C.POINTER(C.c_float)), x.ctypes.data_as(C.POINTER(C.c_float)),
                              C.byref(g.st), C.byref(u.st), C.byref(d.st), I)
        want += float(w[j]) * out.astype(np.float64)
        for k, a in (("gq", hl.gq[e]), ("gs", hl.gsc[e]), ("uq", hl.uq[e]), ("us", hl.usc[e]),
                     ("dq", hl.dq[e]), ("ds", hl.dsc[e])):
            b = be.upload(np.ascontiguousarray(a))
            keep.append(b)
            ptrs[k][j] = b.p
    dx, dy = be.upload(x), be.alloc(H * 4)
    fn = be.lib.coli_cuda_grouped_q4_mlp if bits == 4 else be.lib.coli_cuda_grouped_q3_mlp
    rbh, rbi = hl.gq.shape[2], hl.dq.shape[2]
    be.check(fn(be.ctx, dy.p, dx.p, ptrs["gq"], ptrs["gs"], ptrs["uq"], ptrs["us"], ptrs["dq"], ptrs["ds"],
                w.ctypes.data_as(C.c_void_p), K, H, I, 128, rbh, (H + 127) // 128, rbi, (I + 127) // 128),
             "grouped mlp")
    got = be.download(dy, (H,), np.float32)
    assert_close_rms(got, want, 1e-4, f"grouped q{bits} fp32")


def test_context_queries(be):
    sm, lds = C.c_int(), C.c_int()
    be.check(be.lib.coli_cuda_device_limits(be.ctx, C.byref(sm), C.byref(lds)), "device_limits")
    assert sm.value >= 1 and lds.value >= 64 * 1024
    assert be.lib.coli_cuda_async_alloc_enabled(be.ctx) in (0, 1)
    free, total = be.memory_info()
    assert 0 < free <= total
    name = be.device_name()
    assert name and ("gfx" in name or "MI" in name), name
    be.check(be.lib.coli_cuda_timer_start(be.ctx), "timer_start")
    d = be.alloc(1 << 20)
    be.check(be.lib.coli_cuda_memset(be.ctx, d.p, 0, 1 << 20), "memset")
    ms = C.c_float(-1.0)
    be.check(be.lib.coli_cuda_timer_stop(be.ctx, C.byref(ms)), "timer_stop")
    assert ms.value >= 0.0
    # page-locking existing host memory is not available here: -1 with a message
    buf = (C.c_char * 4096)()
    assert be.lib.coli_cuda_host_register(be.ctx, buf, 4096) == -1
    assert be.last_error()
    be.lib.coli_cuda_host_unregister(be.ctx, buf)
