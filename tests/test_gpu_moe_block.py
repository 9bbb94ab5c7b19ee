"""coli_cuda_moe_block: the MoE half of a decoder layer on the residual stream,
n = rmsnorm_zero(x, post_norm) then x += MoE(n) (c/qwen.c:1780-1784,
4593-4596), against the CPU checker.

- n must be the CPU path's bit for bit: rmsnorm_zero's serial fp32 sum of
  squares (or_rmsnorm_zero, pinned to the compiled reference).  A parallel sum
  rounds differently in the last bits, and the router then sees another input.
- The routes chosen on the block's n must be router_topk's on the reference's
  n (c/qwen.c:3421-3426), bit for bit, including near-ties steered through the
  norm: the residual input is built so that n's logits of two neighbouring
  experts differ by a tiny fp64 gap, so the choice between them is decided by
  the last bits of n.
- The updated residual stream is within max-abs 1e-3 x RMS of x + MoE(n)
  (moe_forward for one token, moe_prefill_grouped for several).
T = 1 (the persistent decode kernel) and T = 7 (the many-token kernels) at the
S35 and S397 shapes."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

S397 = (4096, 512, 10, 1024, 1024, 3)
S35 = (2048, 256, 8, 512, 512, 4)
EPS = 1e-6
# (rank a, rank b, fp64 logit gap of n) per steered token; None = unsteered
STEER = [None, ("K-1", "K", 1e-6), ("K-1", "K", 1e-7), ("K-1", "K", 0.0), (2, 3, 3e-7), (0, 1, 0.0),
         ("K-1", "K", 3e-8)]


def _rank(r, K):
    return {"K": K, "K-1": K - 1}.get(r, r)


def _residual_with_tie(oracle, hl, n0, w, steer, scale):
    """A residual-stream row x whose rmsnorm_zero(x, w) has the steered gap:
    n0 is moved (least norm) so that logit(a) - logit(b) = gap in fp64, then
    x = scale * n / (1 + w); the norm's scale factor keeps the gap's size
    relative to the logits, and the rounding of x and of the norm decides it."""
    n = n0.astype(np.float64)
    if steer is not None:
        K = hl.K
        Wr = hl.router_w.astype(np.float64)
        order = np.argsort(-(Wr @ n), kind="stable")
        a, b = int(order[_rank(steer[0], K)]), int(order[_rank(steer[1], K)])
        d = Wr[a] - Wr[b]
        n = n - ((d @ n - steer[2]) / (d @ d)) * d
    return (scale * n / (1.0 + w.astype(np.float64))).astype(np.float32)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("shape,T", [(S35, 1), (S35, 7), (S397, 1), (S397, 7), ((512, 32, 4, 256, 128, 3), 300)],
                         ids=["s35_T1", "s35_T7", "s397_T1", "s397_T7", "small_T300"])
def test_moe_block_norm_routes_and_output(be, oracle, shape, T):
    from shiftwing_amd import MoeLayer
    H, E, K, I, Ish, fmt = shape
    seed = 44 + T
    hl = oracle.host_layer(seed, 1, H, E, K, I, Ish, fmt)
    L = MoeLayer(be, H, E, K, I, Ish, fmt)
    L.synthesize(seed, 1)
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(H) * 0.1).astype(np.float32)
    try:
        for rep in range(4 if T == 1 else 1):
            xs = []
            for t in range(T):
                steer = STEER[(rep + t) % len(STEER)]
                n0 = oracle.synth_x(seed, 1, rep * T + t, H)
                xs.append(_residual_with_tie(oracle, hl, n0, w, steer, 2.5 + 0.5 * (t % 3)))
            x = np.stack(xs)
            print(f"[moe block] H{H} E{E} T{T} rep {rep}", flush=True)
            n_want = oracle.rmsnorm_zero(x, w, EPS)
            moe = oracle.moe_forward(hl, n_want[0])[None] if T == 1 else oracle.moe_prefill(hl, n_want)
            dx, dw = be.upload(x), be.upload(w)
            dn, di, dwt = be.alloc(T * H * 4), be.alloc(T * K * 4), be.alloc(T * K * 4)
            be.check(be.lib.coli_cuda_moe_block_ex(be.ctx, L.h, dx.p, dw.p, C.c_float(EPS), T, dn.p, di.p, dwt.p),
                     "moe_block_ex")
            got_x = be.download(dx, (T, H), np.float32)
            got_n = be.download(dn, (T, H), np.float32)
            got_i = be.download(di, (T, K), np.int32)
            got_w = be.download(dwt, (T, K), np.float32)
            bad = np.nonzero(_bits(got_n) != _bits(n_want))
            assert bad[0].size == 0, f"n differs from rmsnorm_zero at {bad[0].size} places, first {bad[0][:4]} {bad[1][:4]}"
            for t in range(T):
                _, tr = oracle.moe_forward(hl, n_want[t], trace=True)
                assert np.array_equal(got_i[t], tr["idx"]), (rep, t, got_i[t], tr["idx"])
                assert np.max(np.abs(got_w[t] - tr["weight"])) <= 1e-5, (rep, t)
            assert_close_rms(got_x.astype(np.float64) - x, moe, 1e-3, f"moe block T={T} rep {rep}")
            assert np.max(np.abs(got_x - (x + moe))) <= 1e-3 * float(np.sqrt(np.mean(moe.astype(np.float64) ** 2))) + 1e-6
            # the plain block call (no route outputs: a one-token step may keep a
            # certified set's order as it is, so only the combine's rounding may differ)
            dx2 = be.upload(x)
            be.check(be.lib.coli_cuda_moe_block(be.ctx, L.h, dx2.p, dw.p, C.c_float(EPS), T), "moe_block")
            got2 = be.download(dx2, (T, H), np.float32)
            assert_close_rms(got2.astype(np.float64) - x, moe, 1e-3, f"plain moe block T={T} rep {rep}")
    finally:
        L.close()


def test_rmsnorm_zero_entry_points_bitexact(be, oracle):
    """coli_cuda_rmsnorm_zero{,_batch} (c/backend_cuda.h:46-49) give the CPU
    path's rmsnorm_zero bit for bit, at sizes below, at and above the LDS
    chunk of squares (4096) and not a multiple of 64."""
    rng = np.random.default_rng(5)
    for n in (1, 63, 1027, 2048, 4096, 4097, 9000):
        x = (rng.standard_normal((3, n)) * 2).astype(np.float32)
        w = (rng.standard_normal(n) * 0.1).astype(np.float32)
        want = oracle.rmsnorm_zero(x, w, EPS)
        dx, dw, dy = be.upload(x), be.upload(w), be.alloc(3 * n * 4)
        be.check(be.lib.coli_cuda_rmsnorm_zero_batch(be.ctx, dy.p, dx.p, dw.p, 3, n, C.c_float(EPS)), "batch")
        assert np.array_equal(_bits(be.download(dy, (3, n), np.float32)), _bits(want)), n
        be.check(be.lib.coli_cuda_rmsnorm_zero(be.ctx, dy.p, dx.p, dw.p, n, C.c_float(EPS)), "one row")
        assert np.array_equal(_bits(be.download(dy, (n,), np.float32)), _bits(want[0])), n
