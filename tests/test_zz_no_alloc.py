"""coli_cuda_idot_q8_gemm_noalloc: the IDOT GEMM with its activation scratch in
a fixed per-device array instead of an allocation.  It must give
coli_cuda_idot_q8_gemm's results bit for bit (which match the reference's IDOT,
c/qwen.c:1696-1705, 1765-1768), on consecutive calls whose second input is
smaller than the first (the array keeps the last call's contents), and reject
sizes beyond the array with an error before touching the device."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(rng, B, O, I, row_bytes):
    q = rng.integers(-127, 128, (O, row_bytes), dtype=np.int8)
    s = np.abs(rng.standard_normal(O) * 0.01).astype(np.float32)
    x = (rng.standard_normal((B, I)) * 2).astype(np.float32)
    return q, s, x


def _run(be, fn, q, s, x, O, I, row_bytes):
    B = x.shape[0]
    dq, ds, dx, dy = be.upload(q), be.upload(s), be.upload(x), be.alloc(B * O * 4)
    be.check(fn(be.ctx, dy.p, dx.p, B, dq.p, ds.p, O, I, row_bytes), fn.__name__)
    return be.download(dy, (B, O), np.float32)


def test_noalloc_idot_equals_idot_gemm(be, oracle):
    from oracle.pyoracle import HostQMat
    rng = np.random.default_rng(17)
    # the second call is smaller than the first: stale bytes of the first call
    # lie past its end in the fixed array
    for B, O, I, rb in [(24, 96, 4096, 4100), (3, 33, 1027, 1027), (1, 512, 2048, 2048), (7, 17, 130, 136)]:
        print(f"[no-alloc idot] B={B} O={O} I={I}", flush=True)
        q, s, x = _case(rng, B, O, I, rb)
        want = _run(be, be.lib.coli_cuda_idot_q8_gemm, q, s, x, O, I, rb)
        got = _run(be, be.lib.coli_cuda_idot_q8_gemm_noalloc, q, s, x, O, I, rb)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (B, O, I)
        m = HostQMat(1, O, I, 0, q=np.ascontiguousarray(q[:, :I]), s=s)
        ref = oracle.qmat_mul_batch(x, m, 1)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (B, O, I)


def test_noalloc_idot_rejects_oversize(be):
    # 300 x 4096 int8 activations exceed the 1 MiB array
    y = be.alloc(4)
    rc = be.lib.coli_cuda_idot_q8_gemm_noalloc(be.ctx, y.p, y.p, 300, y.p, y.p, 1, 4096, 4096)
    assert rc == -1
    assert "scratch" in be.last_error(), be.last_error()
