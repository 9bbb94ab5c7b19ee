"""The reference's own host code driving this library on the GPU.

oracle/_ref holds reference sources compiled in place against
libshiftwing_moe.so in place of backend_cuda.o (`make -C oracle ref-hip`;
c/Makefile:124-125, 148-149 with CUDA=1):

- _ref/test_backend_cuda: the reference's GPU test, c/tests/test_backend_cuda.c,
  unmodified.  It checks every Part 1 compute entry point against a scalar
  host reference on non-power-of-two shapes (N=2053, ROWS=37, COLS=1027,
  padded int8 rows), batch against single calls, q3 native against expanded q4
  at the 397B expert shape, and the stage profiler's transaction count, with
  the reference's tolerances (c/tests/test_backend_cuda.c:546-555).
- _ref/libref_hip.so: the reference's GPU glue (c/qwen.c:462-1474, 3741-3809)
  behind moe_forward and moe_cuda_block, run on synthetic layers and checked
  against the same layer on the reference's CPU path, with the shared expert
  in the fp32 arithmetic the reference's GPU path uses for it.

The binaries are built here (the reference tree is not on the GPU box) and
travel with the tree; a test skips when they were not built."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT, assert_close_rms

pytestmark = pytest.mark.gpu

REF = os.path.join(ROOT, "oracle", "_ref")
TEST_BIN = os.path.join(REF, "test_backend_cuda")
GLUE_LIB = os.path.join(REF, "libref_hip.so")


def test_reference_backend_test_passes():
    if not os.path.exists(TEST_BIN):
        pytest.skip("oracle/_ref/test_backend_cuda not built (make -C oracle ref-hip)")
    print("[reference GPU test] c/tests/test_backend_cuda.c against libshiftwing_moe.so", flush=True)
    r = subprocess.run([TEST_BIN], capture_output=True, text=True, timeout=240)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0, f"reference GPU test failed (rc {r.returncode})"
    line = [l for l in r.stdout.splitlines() if "maxdiff" in l]
    assert line, r.stdout
    diffs = {k: float(v) for k, v in re.findall(r"([\w-]+)(?: maxdiff)?=([0-9.eE+-]+)", line[0])}
    print("reference test diffs:", diffs, flush=True)


class Glue:
    """ctypes view of oracle/_ref/libref_hip.so."""

    def __init__(self):
        from oracle.pyoracle import OrLayer, f32p
        lib = C.CDLL(GLUE_LIB)
        lib.ref_cuda_start.restype = C.c_int
        lib.ref_cuda_set_f16.argtypes = [C.c_int]
        lib.ref_cuda_counters.argtypes = [C.POINTER(C.c_ulonglong)]
        lib.ref_layer_create.restype = C.c_void_p
        lib.ref_layer_create.argtypes = [C.POINTER(OrLayer)]
        lib.ref_layer_destroy.argtypes = [C.c_void_p]
        lib.ref_moe_forward.argtypes = [C.c_void_p, f32p, f32p]
        lib.ref_moe_cuda_block.restype = C.c_int
        lib.ref_moe_cuda_block.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        lib.ref_sw_register.restype = C.c_int
        lib.ref_sw_register.argtypes = [C.c_void_p]
        lib.ref_sw_forward.restype = C.c_int
        lib.ref_sw_forward.argtypes = [C.c_void_p, f32p, C.c_int, f32p, C.POINTER(C.c_int)]
        lib.ref_sw_forward_device.restype = C.c_int
        lib.ref_sw_forward_device.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        lib.ref_hooked_moe_forward.restype = C.c_int
        lib.ref_hooked_moe_forward.argtypes = [C.c_void_p, f32p, f32p]
        lib.ref_hooked_moe_prefill.restype = C.c_int
        lib.ref_hooked_moe_prefill.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        lib.ref_sw_disabled.restype = C.c_int
        self.lib = lib
        self.f32p = f32p

    def counters(self):
        out = (C.c_ulonglong * 7)()
        self.lib.ref_cuda_counters(out)
        keys = ["active", "failed", "grouped", "grouped_kernel", "batch", "mlp", "q3_native"]
        return dict(zip(keys, [int(v) for v in out]))

    def forward(self, h, x, H):
        from oracle.pyoracle import ptr
        out = np.zeros(H, np.float32)
        self.lib.ref_moe_forward(h, ptr(x, self.f32p), ptr(out, self.f32p))
        return out

    def sw_forward(self, h, x, K):
        from oracle.pyoracle import ptr
        T, H = x.shape
        out = np.zeros((T, H), np.float32)
        idx = np.zeros((T, K), np.int32)
        used = self.lib.ref_sw_forward(h, ptr(np.ascontiguousarray(x), self.f32p), T, ptr(out, self.f32p),
                                       ptr(idx, C.POINTER(C.c_int)))
        return used, out, idx

    def block(self, h, x):
        from oracle.pyoracle import ptr
        T, H = x.shape
        out = np.zeros((T, H), np.float32)
        used = self.lib.ref_moe_cuda_block(h, ptr(np.ascontiguousarray(x), self.f32p), T, ptr(out, self.f32p))
        return used, out


def _with_fp32_shared(oracle, hl, x, want, trace):
    """The reference CPU output with its shared expert recomputed in the fp32
    arithmetic its CUDA glue uses (q8 rows x fp32 activations, qmat_mul_ex
    with IDOT off, c/qwen.c:1757, 1765): the reference's GPU path runs the
    int8 shared expert through coli_cuda_q8_gemv / shared_q8_mlp_batch, not
    through IDOT, so its output differs from the CPU path's by the int8
    activation quantisation (about 1% of the shared term here)."""
    x = np.atleast_2d(x)
    want = np.atleast_2d(want).astype(np.float64)
    sh_idot = np.atleast_2d(trace["shared"]).astype(np.float64)
    sg = np.atleast_1d(trace["sgate"]).astype(np.float64)
    out = np.empty_like(want)
    for t in range(x.shape[0]):
        g = oracle.qmat_mul(x[t], hl.shared_gate, 0)
        u = oracle.qmat_mul(x[t], hl.shared_up, 0)
        h = np.array([oracle.lib.or_siluf(float(v)) for v in g], np.float32) * u
        sh = oracle.qmat_mul(h.astype(np.float32), hl.shared_down, 0).astype(np.float64)
        out[t] = want[t] - sg[t] * sh_idot[t] + sg[t] * sh
    return out


@pytest.fixture(scope="module")
def glue():
    if not os.path.exists(GLUE_LIB):
        pytest.skip("oracle/_ref/libref_hip.so not built (make -C oracle ref-hip)")
    # the reference's switches (c/qwen.c:533-536, 1168-1169): device backend on,
    # fp16 activations, q3 experts uploaded natively (not expanded to q4)
    os.environ.update({"COLI_CUDA": "1", "CUDA_DENSE": "1", "CUDA_F16": "1", "Q3_NATIVE": "1"})
    g = Glue()
    assert g.lib.ref_cuda_start() == 1, "the reference glue could not start the device backend"
    yield g
    g.lib.ref_cuda_stop()


@pytest.mark.parametrize("shape,seed", [((2048, 256, 8, 512, 512, 4), 35), ((4096, 512, 10, 1024, 1024, 3), 397),
                                        ((2048, 256, 8, 512, 512, 2), 36)],
                         ids=["s35_q4", "s397_q3", "s35_q2"])
def test_reference_glue_moe_forward(glue, oracle, shape, seed):
    """moe_forward with the device backend active: the reference routes on the
    host and runs cuda_experts_try (c/qwen.c:1270) -> coli_cuda_grouped_q{4,3}_mlp_f16
    and the q8 shared expert via cuda_mlp_try (q8_gemv, silu_mul) on this
    library.  fp16 activations (CUDA_F16=1), then fp32 (per-expert q4/q3 gemv
    + silu_mul + axpy).  int2 experts reach the q4 kernels widened by the
    reference's own upload (q2_expand_q4, c/qwen.c:567-575)."""
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(seed, 2, H, E, K, I, Ish, fmt)
    h = glue.lib.ref_layer_create(C.byref(hl.st))
    try:
        for f16, tol in ((1, 5e-3), (0, 1e-4)):
            glue.lib.ref_cuda_set_f16(f16)
            for t in range(3):
                print(f"[reference glue] {shape[0]} f16={f16} token {t}", flush=True)
                x = oracle.synth_x(seed, 2, t, H)
                before = glue.counters()
                got = glue.forward(h, x, H)
                after = glue.counters()
                assert after["active"] == 1 and after["failed"] == 0, after
                assert after["grouped"] == before["grouped"] + 1, (before, after)
                if f16:
                    assert after["grouped_kernel"] == before["grouped_kernel"] + 1
                    if fmt == 3:
                        assert after["q3_native"] == before["q3_native"] + 1
                want, tr = oracle.moe_forward(hl, x, trace=True)
                want = _with_fp32_shared(oracle, hl, x, want, tr)[0]
                assert_close_rms(got, want, tol, f"reference glue f16={f16} t={t}")
    finally:
        glue.lib.ref_layer_destroy(h)


def test_reference_glue_speculative_block(glue, oracle):
    """moe_cuda_block (c/qwen.c:3741) for T = 2, 4 and 8 tokens: host routing,
    route dedup, coli_cuda_grouped_q4_mlp_batch_f16 and the batched int8 shared
    expert (coli_cuda_shared_q8_mlp_batch with host gate scales) on this
    library, against moe_prefill_grouped on the CPU."""
    H, E, K, I, Ish, fmt = 2048, 64, 8, 512, 512, 4
    hl = oracle.host_layer(41, 1, H, E, K, I, Ish, fmt)
    h = glue.lib.ref_layer_create(C.byref(hl.st))
    glue.lib.ref_cuda_set_f16(1)
    try:
        for T in (2, 4, 8):
            print(f"[reference glue] speculative block T={T}", flush=True)
            x = np.stack([oracle.synth_x(41, 1, 100 + t, H) for t in range(T)])
            before = glue.counters()
            used, got = glue.block(h, x)
            after = glue.counters()
            assert used == 1 and after["failed"] == 0, (used, after)
            assert after["batch"] == before["batch"] + 1
            want, tr = oracle.moe_prefill(hl, x, trace=True)
            want = _with_fp32_shared(oracle, hl, x, want, tr)
            assert_close_rms(got, want, 5e-3, f"speculative block T={T}")
    finally:
        glue.lib.ref_layer_destroy(h)


@pytest.mark.parametrize("shape,seed", [((2048, 256, 8, 512, 512, 4), 35), ((4096, 512, 10, 1024, 1024, 3), 397),
                                        ((2048, 256, 8, 512, 512, 2), 36)],
                         ids=["s35_q4", "s397_q3", "s35_q2"])
def test_bridge_device_moe_step(glue, oracle, shape, seed):
    """shiftwing_amd/integration/sw_qwen_bridge.inc compiled into the reference
    engine: sw_moe_register copies a loaded MoeW (router, shared expert, every
    routed expert) into an HBM-resident layer, and sw_moe_try runs the MoE step
    on the device for T tokens.  Checked against moe_forward (T = 1) and
    moe_prefill_grouped (T > 1) on the CPU: router indices exact (rank order
    included), outputs within max-abs 1e-3 x RMS."""
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(seed, 4, H, E, K, I, Ish, fmt)
    h = glue.lib.ref_layer_create(C.byref(hl.st))
    try:
        print(f"[bridge] register {shape}", flush=True)
        assert glue.lib.ref_sw_register(h) == 1
        for T in (1, 4, 37):
            print(f"[bridge] {shape[0]} T={T}", flush=True)
            x = np.stack([oracle.synth_x(seed, 4, 200 + t, H) for t in range(T)])
            used, got, idx = glue.sw_forward(h, x, K)
            assert used == 1 and glue.counters()["failed"] == 0
            if T == 1:
                want, tr = oracle.moe_forward(hl, x[0], trace=True)
                want, want_idx = want[None], tr["idx"][None]
            else:
                want, tr = oracle.moe_prefill(hl, x, trace=True)
                want_idx = tr["idx"]
            assert np.array_equal(idx, want_idx), (T, idx, want_idx)
            assert_close_rms(got, want, 1e-3, f"bridge T={T}")
    finally:
        glue.lib.ref_layer_destroy(h)


@pytest.mark.parametrize("shape,seed", [((2048, 256, 8, 512, 512, 4), 35), ((4096, 512, 10, 1024, 1024, 3), 397)],
                         ids=["s35_q4", "s397_q3"])
def test_bridge_device_activations_and_hooks(glue, oracle, shape, seed):
    """The bridge's two other ways in, on a registered reference MoeW layer:
    sw_moe_try_device on activations in device memory (the resident decode
    loop's replacement of cuda_resident_moe_try, c/qwen.c:3825-3954, 4404-4522)
    for T = 1 and 4; and moe_forward / moe_prefill_grouped (c/qwen.c:3717, 4141)
    with the integration patch's hook as their first statement, which must take
    the device step.  Outputs within max-abs 1e-3 x RMS of the CPU path; the
    bridge stays on."""
    from oracle.pyoracle import ptr
    H, E, K, I, Ish, fmt = shape
    hl = oracle.host_layer(seed, 5, H, E, K, I, Ish, fmt)
    h = glue.lib.ref_layer_create(C.byref(hl.st))
    f32p = glue.f32p
    try:
        assert glue.lib.ref_sw_register(h) == 1
        for T in (1, 4):
            print(f"[bridge device] {shape[0]} T={T}", flush=True)
            x = np.ascontiguousarray(np.stack([oracle.synth_x(seed, 5, 300 + t, H) for t in range(T)]))
            out = np.zeros((T, H), np.float32)
            assert glue.lib.ref_sw_forward_device(h, ptr(x, f32p), T, ptr(out, f32p)) == 1
            want = oracle.moe_forward(hl, x[0])[None] if T == 1 else oracle.moe_prefill(hl, x)
            assert_close_rms(out, want, 1e-3, f"sw_moe_try_device T={T}")
            hooked = np.zeros((T, H), np.float32)
            if T == 1:
                used = glue.lib.ref_hooked_moe_forward(h, ptr(x[0], f32p), ptr(hooked[0], f32p))
            else:
                used = glue.lib.ref_hooked_moe_prefill(h, ptr(x, f32p), T, ptr(hooked, f32p))
            assert used == 1, T
            assert_close_rms(hooked, want, 1e-3, f"hooked T={T}")
        assert glue.lib.ref_sw_disabled() == 0 and glue.counters()["failed"] == 0
    finally:
        glue.lib.ref_layer_destroy(h)


def test_bridge_registers_layers_mixing_int2_and_int4_experts(glue, oracle):
    """A reference layer as EXPERT_Q2=1 leaves it when only some experts have
    .q2 sidecars (c/qwen.c:2207-2214): int2 experts with int4 ones (here the
    first and the last, expert 0 deciding the layer's format).  sw_moe_register
    takes it (both held as int4 records, each expert given in its own format),
    and the device step matches moe_forward / moe_prefill_grouped over the
    same mixed layer; the tokens route to both kinds."""
    H, E, K, I, Ish = 2048, 64, 8, 512, 512
    hl4 = oracle.host_layer(44, 2, H, E, K, I, Ish, 4)
    mix = oracle.host_layer(44, 2, H, E, K, I, Ish, 2)
    for e in (0, E - 1):
        mix._g[e], mix._u[e], mix._d[e] = hl4.gate[e].st, hl4.up[e].st, hl4.down[e].st
    h = glue.lib.ref_layer_create(C.byref(mix.st))
    try:
        assert glue.lib.ref_sw_register(h) == 1
        x = np.stack([oracle.synth_x(44, 2, 400 + t, H) for t in range(5)])
        for T in (1, 5):
            print(f"[bridge int2+int4] T={T}", flush=True)
            used, got, idx = glue.sw_forward(h, x[:T], K)
            assert used == 1 and glue.counters()["failed"] == 0
            if T == 1:
                want, tr = oracle.moe_forward(mix, x[0], trace=True)
                want, want_idx = want[None], tr["idx"][None]
            else:
                want, tr = oracle.moe_prefill(mix, x, trace=True)
                want_idx = tr["idx"]
                assert {0, E - 1} <= set(np.asarray(want_idx).ravel().tolist())
            assert np.array_equal(idx, want_idx), (T, idx, want_idx)
            assert_close_rms(got, want, 1e-3, f"bridge int2+int4 T={T}")
    finally:
        glue.lib.ref_layer_destroy(h)


def test_bridge_declines_layers_it_does_not_take(glue, oracle):
    """A reference layer whose routed experts use groups of 64 (which the
    reference's CPU path computes, c/qwen.c:1706-1716 with gs = 64) is not
    registered: sw_moe_register returns 0, the hooked moe_forward and
    moe_prefill_grouped run the reference's own body (bit for bit with the
    compiled reference's CPU path), sw_moe_try_device declines, and the bridge
    stays on for other layers."""
    from oracle.pyoracle import ptr
    H, E, K, I, Ish = 512, 16, 4, 256, 128
    hl = oracle.host_layer(8, 2, H, E, K, I, Ish, 4, gs=64)
    h = glue.lib.ref_layer_create(C.byref(hl.st))
    f32p = glue.f32p
    try:
        assert glue.lib.ref_sw_register(h) == 0
        x = np.ascontiguousarray(np.stack([oracle.synth_x(8, 2, t, H) for t in range(3)]))
        one = np.zeros(H, np.float32)
        assert glue.lib.ref_hooked_moe_forward(h, ptr(x[0], f32p), ptr(one, f32p)) == 0
        many = np.zeros((3, H), np.float32)
        assert glue.lib.ref_hooked_moe_prefill(h, ptr(x, f32p), 3, ptr(many, f32p)) == 0
        assert glue.lib.ref_sw_forward_device(h, ptr(x, f32p), 3, ptr(many.copy(), f32p)) == 0
        # the same library's unhooked reference functions, bit for bit
        assert np.array_equal(one.view(np.uint32), glue.forward(h, x[0], H).view(np.uint32))
        plain = np.zeros((3, H), np.float32)
        glue.lib.ref_moe_prefill_grouped.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        glue.lib.ref_moe_prefill_grouped(h, ptr(x, f32p), 3, ptr(plain, f32p))
        assert np.array_equal(many.view(np.uint32), plain.view(np.uint32))
        assert_close_rms(many, oracle.moe_prefill(hl, x), 5e-3, "declined prefill against the CPU checker")
        assert glue.lib.ref_sw_disabled() == 0
    finally:
        glue.lib.ref_layer_destroy(h)


def test_reference_glue_mixers(glue, oracle):
    """The reference's own mixer layers with its device switches on (CUDA_GDN
    and CUDA_ATTN default on, c/qwen.c:868, 919; CUDA_SPEC_GDN=1 for the
    speculative block, 912): gdn_forward -> cuda_gdn_try ->
    coli_cuda_gdn_decode_q4_f16, gdn_decode_block -> cuda_gdn_block_try ->
    coli_cuda_gdn_block_q4_f16, attn_forward -> cuda_attn_try ->
    coli_cuda_gqa_decode_q4_f16 and attn_prefill_layer ->
    cuda_attn_prefill_try -> coli_cuda_gqa_prefill_q4_f16, each on this
    library with the state kept on the device between calls, against the
    oracle's CPU restatement of the same layers (bit-exact with c/qwen.c)."""
    from oracle import pyoracle as po
    lib = glue.lib
    lib.ref_cuda_mixer_counters.argtypes = [C.POINTER(C.c_ulonglong)]

    def counters():
        out = (C.c_ulonglong * 3)()
        lib.ref_cuda_mixer_counters(out)
        return [int(v) for v in out]

    glue.lib.ref_cuda_set_f16(1)
    os.environ["CUDA_SPEC_GDN"] = "1"
    rng = np.random.default_rng(93)
    g = po.HostGdn(91, 2048, 16, 32, 128, 128)
    rm = po.RefMixer(lib, g)
    cs, st = [a[0] for a in g.new_state()]
    try:
        for pos in range(4):
            print(f"[reference glue] gdn_forward pos {pos}", flush=True)
            x = rng.standard_normal(2048).astype(np.float32)
            before = counters()
            got, a, b = rm.gdn(x, pos)
            assert counters()[0] == before[0] + 1, "gdn_forward did not take the device path"
            want = po.oracle_gdn_step(oracle, g, x, a, b, pos, cs, st)
            assert_close_rms(got, want, 1e-3, f"reference gdn_forward pos {pos}")
        X = rng.standard_normal((3, 2048)).astype(np.float32)
        print("[reference glue] gdn_decode_block T=3 from 4", flush=True)
        before = counters()
        got = rm.gdn_block(X, 4)
        assert counters()[0] == before[0] + 3, "gdn_decode_block did not take the device block path"
        for t in range(3):
            a, b = po.oracle_gdn_gates(oracle, g, X[t])
            want = po.oracle_gdn_step(oracle, g, X[t], a, b, 4 + t, cs, st)
            assert_close_rms(got[t], want, 1e-3, f"reference gdn_decode_block token {t}")
    finally:
        rm.close()
        os.environ.pop("CUDA_SPEC_GDN", None)

    at = po.HostAttn(92, 2048, 16, 2, 256, 64, o_fmt=1)
    ra = po.RefMixer(lib, at, max_seq=64)
    kc, vc = [a[0] for a in at.new_cache(64)]
    try:
        for pos in range(20):
            x = rng.standard_normal(2048).astype(np.float32)
            before = counters()
            got = ra.attn(x, pos)
            assert counters()[1] == before[1] + 1, "attn_forward did not take the device path"
            want = po.oracle_attn_step(oracle, at, x, pos, kc, vc)
            assert_close_rms(got, want, 1e-3, f"reference attn_forward pos {pos}")
        print("[reference glue] attn_prefill_layer 20 rows from 20", flush=True)
        X = rng.standard_normal((20, 2048)).astype(np.float32)
        before = counters()
        got = ra.attn_prefill(X, 20)
        assert counters()[2] == before[2] + 1, "attn_prefill_layer did not take the device prefill path"
        for r in range(20):
            want = po.oracle_attn_step(oracle, at, X[r], 20 + r, kc, vc)
            assert_close_rms(got[r], want, 1e-3, f"reference attn_prefill_layer row {20 + r}")
    finally:
        ra.close()
