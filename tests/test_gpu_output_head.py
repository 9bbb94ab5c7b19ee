"""coli_cuda_output_head_q8 against the CPU path's output head, bit for bit.

The reference's output (c/qwen.c:4505-4516 for B rows, 4613-4616 for one
token) is rmsnorm_zero with the final norm (c/qwen.c:1780-1784) followed by
the int8 lm_head through qmat_mul_ex / qmat_mul_batch with IDOT
(c/qwen.c:1696-1705, 1765-1768, 3313-3319).  The oracle restates both and is
pinned bit-exact to the compiled reference (tests/test_oracle_cpu.py:
rmsnorm, IDOT and the qmat goldens).  Shapes: the fast path (hidden % 16,
aligned rows), padded rows, more than four rows (two passes), a hidden size
that is not a multiple of 16 (the any-shape kernel), and the full S397 head
(vocab 248,320 x 4096, c/fixtures/qwen3_5_config/config.json:9,98)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS = np.float32(1e-6)


def _case(rng, vocab, cols, rb, batch):
    q = np.zeros((vocab, rb), np.int8)
    q[:, :cols] = rng.integers(-127, 128, (vocab, cols), dtype=np.int8)
    s = (np.abs(rng.standard_normal(vocab)) * 0.01).astype(np.float32)
    x = (rng.standard_normal((batch, cols)) * 2).astype(np.float32)
    w = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    return q, s, x, w


def _want(oracle, q, s, x, w, cols):
    from oracle.pyoracle import HostQMat
    n = np.stack([oracle.rmsnorm_zero(x[b], w, float(EPS)) for b in range(x.shape[0])])
    m = HostQMat(1, q.shape[0], cols, 0, q=np.ascontiguousarray(q[:, :cols]), s=s)
    return n, oracle.qmat_mul_batch(n, m, 1)


def _run(be, q, s, x, w, vocab, cols, rb):
    B = x.shape[0]
    dq, ds, dx, dw = be.upload(q), be.upload(s), be.upload(x), be.upload(w)
    dl, dh = be.alloc(B * vocab * 4), be.alloc(B * cols * 4)
    be.check(be.lib.coli_cuda_output_head_q8(be.ctx, dl.p, dh.p, dx.p, dw.p, float(EPS), B, dq.p, ds.p, vocab, cols, rb),
             "output_head_q8")
    return be.download(dh, (B, cols), np.float32), be.download(dl, (B, vocab), np.float32)


@pytest.mark.parametrize("vocab,cols,rb,batch", [(5003, 4096, 4096, 1), (5003, 4096, 4096, 3),
                                                 (777, 2048, 2064, 6), (1000, 1000, 1000, 2),
                                                 (4099, 5120, 5120, 1), (333, 64, 64, 5)])
def test_output_head_bitexact(be, oracle, vocab, cols, rb, batch):
    rng = np.random.default_rng(vocab + cols + batch)
    q, s, x, w = _case(rng, vocab, cols, rb, batch)
    print(f"[output head] vocab {vocab} hidden {cols} rows {batch}", flush=True)
    hid, lg = _run(be, q, s, x, w, vocab, cols, rb)
    n, want = _want(oracle, q, s, x, w, cols)
    assert np.array_equal(hid.view(np.uint32), n.view(np.uint32))
    bad = np.argwhere(lg.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} logits differ, first {bad[:4].tolist()}"


def test_output_head_full_s397(be, oracle):
    """The full head: every logit bit-exact, so the greedy token is the CPU
    path's."""
    vocab, cols = 248320, 4096
    rng = np.random.default_rng(248320)
    print("[output head] full S397 head: generating 1 GB of int8 rows", flush=True)
    q, s, x, w = _case(rng, vocab, cols, cols, 1)
    hid, lg = _run(be, q, s, x, w, vocab, cols, cols)
    print("[output head] full S397 head: oracle", flush=True)
    n, want = _want(oracle, q, s, x, w, cols)
    assert np.array_equal(hid.view(np.uint32), n.view(np.uint32))
    assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))
    assert int(np.argmax(lg[0])) == int(np.argmax(want[0]))


def test_output_head_rejects_bad_arguments(be):
    y = be.alloc(64)
    assert be.lib.coli_cuda_output_head_q8(be.ctx, y.p, None, y.p, y.p, float(EPS), 1, y.p, y.p, 4, 16, 8) == -1
    assert "invalid argument" in be.last_error()
    assert be.lib.coli_cuda_output_head_q8(be.ctx, y.p, None, y.p, y.p, float(EPS), 1, y.p, y.p, 4, 20000, 20000) == -1
    assert "16384" in be.last_error()
