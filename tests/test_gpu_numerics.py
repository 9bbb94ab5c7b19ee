"""Bit-exact device arithmetic against the host: glibc expf (through the
reference's sigmoidf_stable / siluf, c/qwen.c:307-308), IDOT int8 dots
(c/qwen.c:1696-1705) and router_topk (c/qwen.c:3421-3426)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def test_sigmoid_exhaustive_matches_glibc(be, oracle):
    """Every float32 bit pattern: coli_cuda_sigmoid == sigmoidf_stable.  This
    exercises expf on every non-positive float (x>=0 uses expf(-x), x<0 uses
    expf(x)), the whole domain the router softmax and SiLU use."""
    n = 1 << 26
    dx = be.alloc(n * 4)
    dy = be.alloc(n * 4)
    bad = 0
    for chunk in range(64):
        bits = np.arange(chunk * n, (chunk + 1) * n, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        be.check(be.lib.coli_cuda_upload(be.ctx, dx.p, x.ctypes.data_as(C.c_void_p), x.nbytes))
        be.check(be.lib.coli_cuda_sigmoid(be.ctx, dy.p, dx.p, n))
        got = be.download(dy, (n,), np.float32)
        want = oracle.sigmoid_batch(x)
        bad += int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
    assert bad == 0


def test_silu_mul_matches_host(be, oracle):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(1 << 20) * 8).astype(np.float32)
    u = rng.standard_normal(1 << 20).astype(np.float32)
    dg, du, dy = be.upload(g), be.upload(u), be.alloc(g.nbytes)
    be.check(be.lib.coli_cuda_silu_mul(be.ctx, dy.p, dg.p, du.p, g.size))
    got = be.download(dy, g.shape, np.float32)
    want = np.array([oracle.lib.or_siluf(float(v)) for v in g[:4096]], np.float32) * u[:4096]
    assert np.array_equal(got[:4096].view(np.uint32), want.view(np.uint32))


def _router(be, logits, K):
    T, E = logits.shape
    dl = be.upload(np.ascontiguousarray(logits, np.float32))
    di, dw = be.alloc(T * K * 4), be.alloc(T * K * 4)
    be.check(be.lib.coli_cuda_router_topk(be.ctx, dl.p, T, E, K, di.p, dw.p))
    return be.download(di, (T, K), np.int32), be.download(dw, (T, K), np.float32)


def test_router_topk_reference_fixture(be):
    """c/fixtures/router.json (c/tests/test_router.c): indices exact, weights 2e-6."""
    fx = json.load(open(os.path.join(GOLDEN, "router.json")))
    logits = np.array(fx["logits"], np.float32)
    idx, w = _router(be, logits, 2)
    assert np.array_equal(idx, np.array(fx["indices"]))
    assert np.max(np.abs(w - np.array(fx["weights"], np.float32))) <= 2e-6


def test_router_topk_golden_bitexact(be):
    g = np.load(os.path.join(GOLDEN, "router_topk.npz"))
    for i in range(len(g["E"])):
        E, K = int(g["E"][i]), int(g["K"][i])
        idx, w = _router(be, g["logits"][i:i + 1, :E], K)
        assert np.array_equal(idx[0], g["idx"][i, :K]), i
        assert np.array_equal(w[0].view(np.uint32), g["weight"][i, :K].view(np.uint32)), i


def test_idot_gemm_bitexact(be, oracle):
    from oracle.pyoracle import HostQMat
    rng = np.random.default_rng(5)
    for B, O, I in [(1, 17, 1027), (5, 64, 4096), (3, 33, 130)]:
        q = rng.integers(-127, 128, (O, I), dtype=np.int8)
        s = np.abs(rng.standard_normal(O) * 0.01).astype(np.float32)
        x = (rng.standard_normal((B, I)) * 2).astype(np.float32)
        m = HostQMat(1, O, I, 0, q=q, s=s)
        want = oracle.qmat_mul_batch(x, m, 1)
        dq, ds, dx, dy = be.upload(q), be.upload(s), be.upload(x), be.alloc(B * O * 4)
        be.check(be.lib.coli_cuda_idot_q8_gemm(be.ctx, dy.p, dx.p, B, dq.p, ds.p, O, I, I))
        got = be.download(dy, (B, O), np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (B, O, I)


def test_bucket_matches_reference_order(be, oracle):
    rng = np.random.default_rng(9)
    for T, K, E in [(1, 8, 256), (7, 4, 16), (32, 10, 512), (512, 10, 512), (513, 8, 256)]:
        idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        off, tok, slot = oracle.bucket(idx, E)
        di = be.upload(idx)
        do, dt, ds = be.alloc((E + 1) * 4), be.alloc(T * K * 4), be.alloc(T * K * 4)
        be.check(be.lib.coli_cuda_moe_bucket(be.ctx, di.p, T, K, E, do.p, dt.p, ds.p))
        assert np.array_equal(be.download(do, (E + 1,), np.int32), off)
        assert np.array_equal(be.download(dt, (T * K,), np.int32)[:len(tok)], tok)
        assert np.array_equal(be.download(ds, (T * K,), np.int32)[:len(slot)], slot)


def test_bucket_repeated_experts_match_reference(be, oracle):
    """Lists that name an expert twice take the reference's first matching k
    (moe_prefill_route_gather, c/qwen.c:3956-3968): a step of repeats on few
    experts, and a step where one token of many repeats an expert (the device
    checks first occurrences only when some list repeats)."""
    rng = np.random.default_rng(21)
    many = np.stack([rng.choice(512, 10, replace=False) for _ in range(300)]).astype(np.int32)
    many[137, 6] = many[137, 2]
    for idx, E in [(rng.integers(0, 6, (40, 5)).astype(np.int32), 6), (many, 512)]:
        T, K = idx.shape
        off, tok, slot = oracle.bucket(idx, E)
        di = be.upload(idx)
        do, dt, ds = be.alloc((E + 1) * 4), be.alloc(T * K * 4), be.alloc(T * K * 4)
        be.check(be.lib.coli_cuda_moe_bucket(be.ctx, di.p, T, K, E, do.p, dt.p, ds.p))
        assert np.array_equal(be.download(do, (E + 1,), np.int32), off)
        assert np.array_equal(be.download(dt, (T * K,), np.int32)[:len(tok)], tok)
        assert np.array_equal(be.download(ds, (T * K,), np.int32)[:len(slot)], slot)
