"""The oracle (oracle/moe_oracle.c, a C restatement of the reference CPU MoE
path) pinned without a GPU.

What pins it (each check chosen so that a plausible slip fails one of them):
  * golden vectors written by the compiled reference (tests/golden/*.npz,
    made by tests/golden/make_golden.py from c/qwen.c compiled in place):
    router_topk, the int8/int4/int3 row dots (IDOT on and off, single and
    batched), and whole layers (moe_forward decode, moe_prefill_grouped);
  * the reference's own router fixture c/fixtures/router.json (indices exact,
    weights within 2e-6 as in c/tests/test_router.c);
  * byte-layout known answers from c/tests/test_convert_qwen.py:283-290 and
    c/quant.h:167-209, and a brute-force fp64 dequantised dot (closed form);
  * integer identities (IDOT dots are exact int32; bucketing is a stable
    counting sort) and the tie rule of router_topk (lowest index first);
  * the compiled reference itself (oracle/_ref) on fresh seeds, when built.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

LAYERS = ["small_q4", "small_q3", "ragged_q4", "ragged_q3", "s35_q4", "s397_q3", "small_q2", "ragged_q2"]


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- router_topk
def test_router_topk_golden_bitexact(oracle):
    g = np.load(os.path.join(GOLDEN, "router_topk.npz"))
    for c in range(len(g["E"])):
        E, K = int(g["E"][c]), int(g["K"][c])
        idx, w = oracle.router_topk(g["logits"][c, :E].copy(), K)
        assert np.array_equal(idx, g["idx"][c, :K]), c
        assert np.array_equal(_bits(w), _bits(g["weight"][c, :K])), c


def test_router_topk_reference_fixture(oracle):
    """c/fixtures/router.json: indices exact, weights within 2e-6."""
    j = json.load(open(os.path.join(GOLDEN, "router.json")))
    logits = np.asarray(j["logits"], np.float32)
    K = int(j["top_k"])
    want_i = np.asarray(j["indices"], np.int32)
    want_w = np.asarray(j["weights"], np.float32)
    logits = logits.reshape(-1, logits.shape[-1])
    want_i = want_i.reshape(len(logits), -1)
    want_w = want_w.reshape(len(logits), -1)
    for t in range(len(logits)):
        idx, w = oracle.router_topk(logits[t].copy(), K)
        assert np.array_equal(idx, want_i[t])
        assert np.max(np.abs(w - want_w[t])) <= 2e-6


def test_router_topk_closed_forms(oracle):
    rng = np.random.default_rng(5)
    # distinct, well separated logits: indices are the descending sort, the
    # weights the renormalised softmax of the top K
    for E, K in [(16, 4), (256, 8), (512, 10)]:
        lg = (rng.permutation(E).astype(np.float32) * 0.05).astype(np.float32)
        idx, w = oracle.router_topk(lg.copy(), K)
        want = np.argsort(-lg, kind="stable")[:K]
        assert np.array_equal(idx, want)
        p = np.exp(lg[want].astype(np.float64) - lg.max())
        assert np.max(np.abs(w - p / p.sum())) <= 1e-6
        assert abs(float(np.sum(w, dtype=np.float64)) - 1.0) <= 1e-6
    # equal logits: lowest index first
    lg = np.zeros(32, np.float32)
    lg[[3, 17, 9]] = 2.0
    idx, w = oracle.router_topk(lg.copy(), 5)
    assert list(idx[:3]) == [3, 9, 17] and list(idx[3:]) == [0, 1]


# ---------------------------------------------------------------- row dots
def _qmat_cases():
    g = np.load(os.path.join(GOLDEN, "qmat.npz"))
    keys = sorted({k.rsplit("_", 1)[0] for k in g.files if k.endswith("_q")})
    return g, keys


def test_qmat_golden_bitexact(oracle):
    from oracle.pyoracle import HostQMat
    g, keys = _qmat_cases()
    assert keys
    for k in keys:
        fmt, I = int(k.split("_")[0][1:]), int(k.split("_")[1][1:])
        q, s = g[k + "_q"], g[k + "_s"]
        m = HostQMat(fmt, q.shape[0], I, 0 if fmt == 1 else 128, q=q, s=s)
        assert np.array_equal(_bits(oracle.qmat_mul(g[k + "_x"], m, 1)), _bits(g[k + "_y"])), k
        assert np.array_equal(_bits(oracle.qmat_mul(g[k + "_x"], m, 0)), _bits(g[k + "_y_noidot"])), k
        assert np.array_equal(_bits(oracle.qmat_mul_batch(g[k + "_X"], m)), _bits(g[k + "_Y"])), k


def test_qmat_q2_golden_bitexact(oracle):
    """int2 rows (dot_q2_group, c/qwen.c:1717-1724) bit for bit against the
    compiled reference's qmat_mul, ragged widths included."""
    from oracle.pyoracle import HostQMat
    g = np.load(os.path.join(GOLDEN, "qmat_q2.npz"))
    keys = sorted({k.rsplit("_", 1)[0] for k in g.files if k.endswith("_q")})
    assert keys
    for k in keys:
        I = int(k.split("_")[1][1:])
        q, s = g[k + "_q"], g[k + "_s"]
        m = HostQMat(2, q.shape[0], I, 128, q=q, s=s)
        assert np.array_equal(_bits(oracle.qmat_mul(g[k + "_x"], m, 1)), _bits(g[k + "_y"])), k
        # and up to rounding the brute-force dequantisation
        w = _dequant(2, q, s, I)
        x = g[k + "_x"].astype(np.float64)
        got = oracle.qmat_mul(g[k + "_x"], m, 0)
        assert np.all(np.abs(got - w @ x) <= 1e-5 * (np.abs(w) @ np.abs(x) + 1e-30)), k


def test_q2_group_known_answers_and_exact_sums(oracle):
    """int2 layout: byte 0b11100100 holds codes 0, 1, 2, 3 (lowest bits
    first), values 2c - 3 = -3, -1, 1, 3.  With small-integer activations
    every partial sum is exact, so any order gives sum x_i (2 c_i - 3)
    exactly: random codes pin the bit positions and the value map."""
    import ctypes as C
    L = oracle.lib
    w = np.array([0b11100100], np.uint8)
    x = np.array([1, 10, 100, 1000], np.float32)
    assert L.or_dot_q2_group(w.ctypes.data, x.ctypes.data_as(C.POINTER(C.c_float)), 4) == 3087.0
    rng = np.random.default_rng(4)
    for n in (1, 5, 64, 128):
        q = rng.integers(0, 256, (n + 3) // 4, dtype=np.uint8)
        xi = rng.integers(-8, 9, n).astype(np.float32)
        codes = (q[np.arange(n) >> 2] >> (2 * (np.arange(n) & 3))) & 3
        want = float(np.sum(xi.astype(np.int64) * (2 * codes.astype(np.int64) - 3)))
        got = L.or_dot_q2_group(q.ctypes.data, xi.ctypes.data_as(C.POINTER(C.c_float)), n)
        assert got == want, n


def test_q2_group_matches_compiled_reference(oracle):
    """Random groups (lengths 1..128, activations of three magnitudes):
    or_dot_q2_group equals the compiled dot_q2_group bit for bit (gcc keeps
    the scalar loop in order and contracts it into an FMA chain)."""
    import ctypes as C
    from oracle.pyoracle import Reference
    try:
        ref = Reference()
    except Exception as e:  # not built (no reference sources here)
        pytest.skip(f"compiled reference not available: {e}")
    rng = np.random.default_rng(6)
    f32p = C.POINTER(C.c_float)
    for n in (1, 3, 4, 31, 64, 127, 128):
        for _ in range(100):
            q = rng.integers(0, 256, (n + 3) // 4, dtype=np.uint8)
            x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 1e3])).astype(np.float32)
            a = oracle.lib.or_dot_q2_group(q.ctypes.data, x.ctypes.data_as(f32p), n)
            b = ref.lib.ref_dot_q2_group(q.ctypes.data, x.ctypes.data_as(f32p), n)
            assert _bits(a) == _bits(b), n


def _dequant(fmt, q, s, I, gs=128):
    """Brute-force dequantisation from the byte layouts (fp64)."""
    O = q.shape[0]
    w = np.zeros((O, I), np.float64)
    for o in range(O):
        for i in range(I):
            if fmt == 1:
                w[o, i] = float(q[o, i]) * float(s[o])
                continue
            if fmt == 4:
                byte = int(q[o, i >> 1])
                code = (byte & 15) if (i & 1) == 0 else (byte >> 4)
                v = code - 8
            elif fmt == 2:
                v = 2 * ((int(q[o, i >> 2]) >> (2 * (i & 3))) & 3) - 3
            else:
                j, k = i // 8, i % 8
                word = int(q[o, 3 * j]) | int(q[o, 3 * j + 1]) << 8 | int(q[o, 3 * j + 2]) << 16
                v = ((word >> (3 * k)) & 7) - 4
            w[o, i] = v * float(s[o, i // gs])
    return w


def test_qmat_matches_bruteforce_dequant(oracle):
    """The row dots equal x . dequant(W) up to fp32 rounding: pins nibble
    order, triplet bit order, code offsets and the per-group scale index."""
    from oracle.pyoracle import HostQMat
    g, keys = _qmat_cases()
    for k in keys:
        fmt, I = int(k.split("_")[0][1:]), int(k.split("_")[1][1:])
        q, s, x = g[k + "_q"], g[k + "_s"], g[k + "_x"]
        w = _dequant(fmt, q, s, I)
        want = w @ x.astype(np.float64)
        m = HostQMat(fmt, q.shape[0], I, 0 if fmt == 1 else 128, q=q, s=s)
        got = oracle.qmat_mul(x, m, 0)
        scale = np.abs(w) @ np.abs(x.astype(np.float64)) + 1e-30
        assert np.all(np.abs(got - want) <= 1e-5 * scale), k


def test_layout_known_answers(oracle):
    """int3: codes [-4..3] with scale 1 pack to 88 C6 FA
    (c/tests/test_convert_qwen.py:283-290); int4: byte 0x71 holds values
    (1-8, 7-8) = (-7, -1), low nibble first (c/quant.h:167-209)."""
    from oracle.pyoracle import HostQMat
    q3 = np.zeros((1, 48), np.uint8)
    q3[0, :3] = [0x88, 0xC6, 0xFA]
    s3 = np.ones((1, 1), np.float32)
    m3 = HostQMat(3, 1, 8, 128, q=q3, s=s3)
    for i in range(8):
        x = np.zeros(8, np.float32)
        x[i] = 1.0
        assert oracle.qmat_mul(x, m3, 0)[0] == float(i - 4)
    q4 = np.zeros((1, 64), np.uint8)
    q4[0, 0] = 0x71
    m4 = HostQMat(4, 1, 2, 128, q=q4, s=np.ones((1, 1), np.float32))
    assert oracle.qmat_mul(np.array([1, 0], np.float32), m4, 0)[0] == -7.0
    assert oracle.qmat_mul(np.array([0, 1], np.float32), m4, 0)[0] == -1.0


def test_idot_is_exact_integer_dot(oracle):
    """IDOT: x -> (q, sx) by qrow_i8; y_o = ((float)sum q*w) * s_o * sx with an
    exact integer sum (checked against int64)."""
    from oracle.pyoracle import HostQMat
    rng = np.random.default_rng(9)
    O, I = 7, 4099
    w = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = np.abs(rng.standard_normal(O)).astype(np.float32) * 0.01
    x = rng.standard_normal(I).astype(np.float32)
    q, sx = oracle.qrow_i8(x)
    assert q.dtype == np.int8 and np.max(np.abs(q.astype(np.int32))) <= 127
    dot = w.astype(np.int64) @ q.astype(np.int64)
    assert np.all(np.abs(dot) < 2 ** 31)
    want = (dot.astype(np.float32) * s) * np.float32(sx)
    got = oracle.qmat_mul(x, HostQMat(1, O, I, 0, q=w, s=s), 1)
    assert np.array_equal(_bits(got), _bits(want))


# ---------------------------------------------------------------- bucketing
def test_bucket_is_stable_counting_sort(oracle):
    rng = np.random.default_rng(3)
    for T, K, E in [(1, 8, 256), (7, 4, 16), (32, 10, 512), (512, 8, 256)]:
        idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        off, tok, slot = oracle.bucket(idx, E)
        # experts ascending; within an expert tokens ascending, slot = first k
        want_tok, want_slot, want_off = [], [], [0]
        for e in range(E):
            for t in range(T):
                ks = np.nonzero(idx[t] == e)[0]
                if len(ks):
                    want_tok.append(t)
                    want_slot.append(int(ks[0]))
            want_off.append(len(want_tok))
        assert np.array_equal(off, want_off)
        assert np.array_equal(tok, want_tok) and np.array_equal(slot, want_slot)


def test_bucket_matches_compiled_route_gather(oracle):
    """or_bucket against the reference's own moe_prefill_route_gather
    (c/qwen.c:3956-3968, compiled in place), walked over the experts in
    ascending id as moe_prefill_grouped does: the same offsets and tokens in
    the same order, each gathered row the token's, each weight the token's
    first route to that expert (also when a row repeats an expert, where the
    reference's loop stops at the first match)."""
    from oracle.pyoracle import Reference
    try:
        ref = Reference()
    except Exception as e:  # not built (no reference sources here)
        pytest.skip(f"compiled reference not available: {e}")
    rng = np.random.default_rng(31)
    cases = []
    for T, K, E in [(1, 8, 256), (7, 4, 16), (33, 10, 512), (300, 8, 256)]:
        cases.append(np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32))
    dup = rng.integers(0, 6, (40, 5)).astype(np.int32)  # repeats within a row, unused experts
    cases.append(dup)
    for idx in cases:
        T, K = idx.shape
        E = 6 if idx is dup else int(idx.max()) + 1 + (idx is not dup) * 3
        weight = rng.random((T, K)).astype(np.float32)
        off, tok, slot = oracle.bucket(idx, E)
        roff, rtok, rwt, rxb = ref.route_gather_all(idx, weight, E)
        assert np.array_equal(off, roff) and np.array_equal(tok, rtok), (T, K, E)
        assert np.array_equal(rxb, rtok.astype(np.float32))
        assert np.array_equal(rwt, weight[tok, slot])
        for e in range(E):
            for n in range(off[e], off[e + 1]):
                assert idx[tok[n], slot[n]] == e and e not in idx[tok[n], :slot[n]]


# ---------------------------------------------------------------- layers
def _layer(oracle, name):
    g = np.load(os.path.join(GOLDEN, f"layer_{name}.npz"))
    H, E, K, I, Ish, fmt, gs, seed, layer, T = (int(v) for v in g["cfg"])
    return g, oracle.host_layer(seed, layer, H, E, K, I, Ish, fmt, gs)


@pytest.mark.parametrize("name", LAYERS)
def test_layer_golden_bitexact(oracle, name):
    """moe_forward per token and moe_prefill_grouped over the block, bit for
    bit against the compiled reference (same synthetic weights by seed)."""
    g, hl = _layer(oracle, name)
    for t in range(len(g["x"])):
        y, tr = oracle.moe_forward(hl, g["x"][t], trace=True)
        assert np.array_equal(tr["idx"], g["idx"][t]), (name, t)
        assert np.array_equal(_bits(tr["weight"]), _bits(g["weight"][t])), (name, t)
        assert np.array_equal(_bits(tr["logits"]), _bits(g["logits"][t])), (name, t)
        assert np.array_equal(_bits(y), _bits(g["decode"][t])), (name, t)
    yp = oracle.moe_prefill(hl, g["x"])
    assert np.array_equal(_bits(yp), _bits(g["prefill"])), name


def test_decode_equals_single_token_prefill(oracle):
    """Batched == single (c/tests/test_quant_matmul.c:72-86) at the layer
    level: a one-token prefill block is the decode step up to the combine's
    contraction (fma chain vs mul-then-add), here within 1e-6 x RMS."""
    g, hl = _layer(oracle, "small_q3")
    for t in range(3):
        a = oracle.moe_forward(hl, g["x"][t])
        b = oracle.moe_prefill(hl, g["x"][t:t + 1])[0]
        assert np.max(np.abs(a - b)) <= 1e-6 * float(np.sqrt(np.mean(a.astype(np.float64) ** 2)))


def test_oracle_matches_compiled_reference(oracle):
    """Fresh seeds through the compiled reference (oracle/_ref, built from the
    reference's own c/qwen.c where /root/reference is present)."""
    from oracle.pyoracle import Reference
    try:
        ref = Reference()
    except Exception as e:  # not built (no reference sources here)
        pytest.skip(f"compiled reference not available: {e}")
    for (H, E, K, I, Ish, fmt, seed) in [(256, 16, 4, 128, 128, 4, 71), (384, 32, 8, 257, 129, 3, 72),
                                         (1024, 64, 6, 256, 256, 3, 73)]:
        hl = oracle.host_layer(seed, 2, H, E, K, I, Ish, fmt)
        rl = ref.layer(hl)
        X = np.stack([oracle.synth_x(seed, 2, t, H) for t in range(4)])
        for t in range(4):
            assert np.array_equal(_bits(oracle.moe_forward(hl, X[t])), _bits(rl.forward(X[t]))), (seed, t)
        assert np.array_equal(_bits(oracle.moe_prefill(hl, X)), _bits(rl.prefill(X))), seed


def test_rmsnorm_zero_matches_compiled_reference_and_closed_form(oracle):
    """or_rmsnorm_zero (c/qwen.c:1780-1784): bit-exact with the compiled
    reference where oracle/_ref is built; a constant row c gives
    c / sqrt(c^2 + eps) * (1 + w) exactly as the reference's float steps
    compute it; a fused multiply-add chain (a plausible mistake) does not
    match the reference on random rows."""
    import numpy as np
    rng = np.random.default_rng(8)
    x = np.full(64, 0.75, np.float32)
    w = (rng.standard_normal(64) * 0.1).astype(np.float32)
    got = oracle.rmsnorm_zero(x, w, 1e-6)
    ms = np.float32(0)
    for v in x:
        ms = np.float32(ms + np.float32(v * v))
    r = np.float32(1) / np.sqrt(np.float32(ms / np.float32(64) + np.float32(1e-6)))
    assert np.array_equal(got, (x * r).astype(np.float32) * (np.float32(1) + w))
    try:
        from oracle.pyoracle import Reference
        ref = Reference()
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built")
    fma_differs = 0
    for n in (4096, 2048, 1027):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = (rng.standard_normal(n) * 0.1).astype(np.float32)
        a, b = oracle.rmsnorm_zero(x, w, 1e-6), ref.rmsnorm_zero(x, w, 1e-6)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), n
        ms = np.float32(0)
        for v in x:  # fused chain: one rounding per term
            ms = np.float32(np.float64(v) * np.float64(v) + np.float64(ms))
        r = np.float32(1) / np.sqrt(np.float32(ms / np.float32(n) + np.float32(1e-6)))
        fma_differs += not np.array_equal(((x * r) * (np.float32(1) + w)).astype(np.float32), b)
    assert fma_differs > 0


# ------------------------------------------- the mixer layers around the MoE
def _avx512_reference():
    """The compiled reference when it is an AVX-512 build (the lane structure
    the oracle's grouped dots restate), else None."""
    from oracle.pyoracle import Reference, ref_lib_candidates
    c = [p for p in ref_lib_candidates() if p.endswith(("libref_native.so", "libref_v4.so"))]
    return Reference(c[0]) if c else None


def test_gdn_and_attention_match_compiled_reference():
    """or_gdn_forward / or_attn_forward (c/qwen.c:3005, 2907, 3094, 3031)
    against the reference's own gdn_forward and attn_forward compiled in place:
    bit for bit over several decode steps with the state carried, including
    the gate projections a and b and every conv and recurrent state word.
    The restatement's unfused sums (q/k norms, memory read-out, output sum)
    and fused updates are the ones gcc emits for c/qwen.c at its flags; a
    plausible slip (a fused sum, a dropped 1/sqrt(dk), the rotation sign)
    breaks the equality."""
    from oracle import pyoracle as po
    ref = _avx512_reference()
    if ref is None:
        pytest.skip("no AVX-512 build of the compiled reference (oracle/_ref)")
    orc = po.Oracle()
    rng = np.random.default_rng(101)
    g = po.HostGdn(7, 512, 2, 8, 128, 128)
    rm = po.RefMixer(ref.lib, g)
    cs, st = [a[0] for a in g.new_state()]
    for pos in range(6):
        x = rng.standard_normal(512).astype(np.float32)
        want, a, b = rm.gdn(x, pos)
        a2, b2 = po.oracle_gdn_gates(orc, g, x)
        assert np.array_equal(_bits(a), _bits(a2)) and np.array_equal(_bits(b), _bits(b2))
        got = po.oracle_gdn_step(orc, g, x, a, b, pos, cs, st)
        assert np.array_equal(_bits(got), _bits(want)), pos
        assert np.array_equal(_bits(st), _bits(rm.state)) and np.array_equal(_bits(cs), _bits(rm.conv_state))
    for o_fmt in (1, 4):
        at = po.HostAttn(8 + o_fmt, 512, 4, 2, 256, 64, o_fmt=o_fmt)
        ra = po.RefMixer(ref.lib, at, max_seq=24)
        kc, vc = [a[0] for a in at.new_cache(24)]
        for pos in range(20):
            x = rng.standard_normal(512).astype(np.float32)
            want = ra.attn(x, pos)
            got = po.oracle_attn_step(orc, at, x, pos, kc, vc)
            assert np.array_equal(_bits(got), _bits(want)), (o_fmt, pos)
        assert np.array_equal(_bits(kc), _bits(ra.k_cache)) and np.array_equal(_bits(vc), _bits(ra.v_cache))


def test_gdn_first_step_closed_form(oracle):
    """From a zero state the delta rule gives S = beta k_hat v^T, so the
    pre-norm output of value head h is beta (k_hat . q_hat) / sqrt(dk) v_h;
    with the conv kernel K = 1 (tap weight w) the mixer value of a channel is
    silu(w raw), raw = W x.  fp32 weights (format 0) and the identity out
    projection expose the gated RMS-normed core directly.  Checked in fp64
    against the oracle's fp32 path."""
    from oracle import pyoracle as po
    H, kh, vh, dk, dv = 64, 1, 2, 16, 16
    rng = np.random.default_rng(5)
    g = po.HostGdn(3, 512, 2, 4, 128, 128)  # a template; every field is replaced below
    cd, vd = 2 * kh * dk + vh * dv, vh * dv
    Wqkv = rng.standard_normal((cd, H)).astype(np.float32) * 0.2
    Wz = rng.standard_normal((vd, H)).astype(np.float32) * 0.2
    Wo = np.eye(H, vd, dtype=np.float32)
    conv = np.full((cd, 1), 0.75, np.float32)
    A_log = np.array([0.3, -0.2], np.float32)
    dt_bias = np.array([0.1, 0.4], np.float32)
    norm = (1 + rng.standard_normal(dv) * 0.1).astype(np.float32)
    keep = [Wqkv, Wz, Wo, conv, A_log, dt_bias, norm]
    g.H, g.kh, g.vh, g.dk, g.dv, g.K = H, kh, vh, dk, dv, 1
    g.qkv, g.z, g.out = po.HostQMat(0, cd, H, f=Wqkv), po.HostQMat(0, vd, H, f=Wz), po.HostQMat(0, H, vd, f=Wo)
    g.st = po.OrGdn(H, kh, vh, dk, dv, 1, 1e-6, g.qkv.st, g.z.st, g.a.st, g.b.st, g.out.st,
                    po.ptr(conv, po.f32p), po.ptr(A_log, po.f32p), po.ptr(dt_bias, po.f32p), po.ptr(norm, po.f32p))
    x = rng.standard_normal(H).astype(np.float32)
    a = np.array([0.5, -1.0], np.float32)
    b = np.array([0.2, 1.5], np.float32)
    cs = np.zeros((1, cd), np.float32)
    st = np.zeros((vh, dk, dv), np.float32)
    out = po.oracle_gdn_step(oracle, g, x, a, b, 0, cs, st)
    x64 = x.astype(np.float64)
    raw = Wqkv.astype(np.float64) @ x64
    mix = 0.75 * raw / (1 + np.exp(-0.75 * raw))
    q, k, v = mix[:dk], mix[dk:2 * dk], mix[2 * dk:]
    qh = q / np.sqrt(q @ q + 1e-6) / np.sqrt(dk)
    kh_ = k / np.sqrt(k @ k + 1e-6)
    z = Wz.astype(np.float64) @ x64
    core = np.zeros(vd)
    for h in range(vh):
        beta = 1 / (1 + np.exp(-b[h]))
        o = beta * (kh_ @ qh) * v[h * dv:(h + 1) * dv]
        r = 1 / np.sqrt(np.mean(o * o) + 1e-6)
        zz = z[h * dv:(h + 1) * dv]
        core[h * dv:(h + 1) * dv] = o * r * norm * zz / (1 + np.exp(-zz))
        # the state after one step is beta k_hat v^T (the decay multiplies zeros)
        assert np.allclose(st[h], beta * np.outer(kh_, v[h * dv:(h + 1) * dv]), rtol=2e-4, atol=1e-6)
    assert np.allclose(out, Wo.astype(np.float64) @ core, rtol=2e-4, atol=1e-5)
    del keep


def test_attention_first_position_closed_form(oracle):
    """At position 0 the softmax has one key, so the context of query head h is
    v_{kv(h)} * sigmoid(gate_h) and the output is W_o of that, whatever q, k
    and the rotation are; the cache row 0 holds the RMS-normed, rotated k
    (at position 0 the rotation is the identity) and the raw v."""
    from oracle import pyoracle as po
    rng = np.random.default_rng(6)
    at = po.HostAttn(12, 256, 4, 2, 64, 16, o_fmt=4)
    kc, vc = [a[0] for a in at.new_cache(4)]
    x = rng.standard_normal(256).astype(np.float32)
    out = po.oracle_attn_step(oracle, at, x, 0, kc, vc)
    qp = oracle.qmat_mul(x, at.q, 0).astype(np.float64)
    v = oracle.qmat_mul(x, at.v, 0).astype(np.float64)
    k = oracle.qmat_mul(x, at.k, 0).astype(np.float64)
    ctx = np.zeros(at.nh * at.hd)
    for h in range(at.nh):
        gate = qp[h * 2 * at.hd + at.hd:(h + 1) * 2 * at.hd]
        kv = h // (at.nh // at.nkv)
        ctx[h * at.hd:(h + 1) * at.hd] = v[kv * at.hd:(kv + 1) * at.hd] / (1 + np.exp(-gate))
    want = oracle.qmat_mul(ctx.astype(np.float32), at.o, 0)
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6)
    assert np.array_equal(vc[0], v.astype(np.float32))
    for h in range(at.nkv):
        kh_ = k[h * at.hd:(h + 1) * at.hd]
        kn = kh_ / np.sqrt(np.mean(kh_ * kh_) + 1e-6) * (1 + at.k_norm.astype(np.float64))
        assert np.allclose(kc[0, h * at.hd:(h + 1) * at.hd], kn, rtol=1e-5, atol=1e-6)
