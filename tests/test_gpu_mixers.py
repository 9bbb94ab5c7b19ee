"""The mixer layers either side of the MoE block on the device against the
oracle's restatement of the reference CPU path (or_gdn_forward /
or_attn_forward, pinned bit for bit to the compiled c/qwen.c in
tests/test_oracle_cpu.py):

- Gated DeltaNet (coli_cuda_gdn_*, c/backend_cuda.h:149-193): decode steps
  with the conv ring and recurrent state carried on the device, blocks of
  2..8 tokens against the same tokens stepped one by one (gdn_decode_block,
  c/qwen.c:4642), and slot batches with distinct and repeated slots;
- gated GQA attention (coli_cuda_gqa_*, c/backend_cuda.h:194-236): decode
  steps across several 16-key blocks and key splits, o in int8 and int4,
  prefill in row tiles continued by decode, and slot batches.

Shapes are the Qwen3.5-35B-A3B and 397B-A17B mixer layers (hidden 2048 / 4096,
16 key heads, 32 / 64 value heads of 128, conv kernel 4; 16 / 32 query heads,
2 kv heads, head_dim 256, rotary 64, theta 1e7), weights random.  Tolerance:
max |got - want| <= 1e-3 x RMS(want) on outputs; states
and caches within 1e-3 of their RMS."""
import numpy as np
import pytest

from conftest import assert_close_rms

pytestmark = pytest.mark.gpu

GDN_SHAPES = {"s35": (2048, 16, 32), "s397": (4096, 16, 64)}
ATTN_SHAPES = {"s35": (2048, 16), "s397": (4096, 32)}


def _dev_gdn(be, g, slots=1):
    from shiftwing_amd.mixers import DeviceGdn
    return DeviceGdn(be, hidden=g.H, key_heads=g.kh, value_heads=g.vh, key_dim=g.dk, value_dim=g.dv,
                     conv_kernel=g.K, group_size=g.gs, eps=g.eps, qkv=(g.qkv.q, g.qkv.s), z=(g.z.q, g.z.s),
                     out=(g.out.q, g.out.s), conv=g.conv, A_log=g.A_log, dt_bias=g.dt_bias, norm=g.norm, slots=slots)


def _dev_attn(be, at, max_seq, slots=1):
    from shiftwing_amd.mixers import DeviceAttn
    return DeviceAttn(be, hidden=at.H, query_heads=at.nh, kv_heads=at.nkv, head_dim=at.hd, rotary_dim=at.rd,
                      group_size=at.gs, theta=at.theta, eps=at.eps, q=(at.q.q, at.q.s), k=(at.k.q, at.k.s),
                      v=(at.v.q, at.v.s), o=(at.o.q, at.o.s), o_fmt=at.o_fmt, q_norm=at.q_norm, k_norm=at.k_norm,
                      max_seq=max_seq, slots=slots)


def _x(rng, n, H):
    return rng.standard_normal((n, H)).astype(np.float32)


def _close_state(got, want, what):
    assert_close_rms(got.ravel(), want.ravel(), 1e-3, what)


@pytest.mark.parametrize("shape", ["s35", "s397"])
def test_gdn_decode_steps(be, oracle, shape):
    from oracle import pyoracle as po
    H, kh, vh = GDN_SHAPES[shape]
    g = po.HostGdn(11, H, kh, vh, 128, 128)
    dev = _dev_gdn(be, g)
    cs, st = [a[0] for a in g.new_state()]
    rng = np.random.default_rng(12)
    for pos in range(6):
        print(f"[gdn decode] {shape} pos {pos}", flush=True)
        x = _x(rng, 1, H)[0]
        a, b = po.oracle_gdn_gates(oracle, g, x)
        want = po.oracle_gdn_step(oracle, g, x, a, b, pos, cs, st)
        got = dev.decode(x, a, b, pos)
        assert_close_rms(got, want, 1e-3, f"gdn decode {shape} pos {pos}")
    dcs, dst = dev.read_state()
    _close_state(dcs[0], cs, "conv state")
    _close_state(dst[0], st, "recurrent state")


def test_gdn_block_matches_token_steps(be, oracle):
    """coli_cuda_gdn_block_q4_f16 for T = 2, 5, 8 continuing one state
    (gdn_decode_block, c/qwen.c:4642) against the oracle stepped token by
    token: the ring index is absolute, so blocks start mid-ring."""
    from oracle import pyoracle as po
    H, kh, vh = GDN_SHAPES["s35"]
    g = po.HostGdn(21, H, kh, vh, 128, 128)
    dev = _dev_gdn(be, g)
    cs, st = [a[0] for a in g.new_state()]
    rng = np.random.default_rng(22)
    pos = 0
    for T in (2, 5, 8, 1):
        print(f"[gdn block] T={T} from {pos}", flush=True)
        X = _x(rng, T, H)
        AB = [po.oracle_gdn_gates(oracle, g, X[t]) for t in range(T)]
        A = np.stack([ab[0] for ab in AB])
        Bv = np.stack([ab[1] for ab in AB])
        want = np.stack([po.oracle_gdn_step(oracle, g, X[t], A[t], Bv[t], pos + t, cs, st) for t in range(T)])
        got = dev.block(X, A, Bv, pos) if T > 1 else dev.decode(X[0], A[0], Bv[0], pos)[None]
        assert_close_rms(got, want, 1e-3, f"gdn block T={T}")
        pos += T
    dcs, dst = dev.read_state()
    _close_state(dst[0], st, "recurrent state after blocks")


@pytest.mark.parametrize("device_io", [False, True], ids=["host_io", "device_io"])
def test_gdn_slots(be, oracle, device_io):
    """coli_cuda_gdn_slots_q4_f16[_device]: four slots at different positions,
    then a batch where one slot appears twice (its two tokens run in order)."""
    from oracle import pyoracle as po
    H, kh, vh = GDN_SHAPES["s397"]
    g = po.HostGdn(31, H, kh, vh, 128, 128)
    nslots = 4
    dev = _dev_gdn(be, g, slots=nslots)
    CS, ST = g.new_state(nslots)
    rng = np.random.default_rng(32)
    nextpos = [0] * nslots
    for batch in ([0, 1, 2, 3], [2, 0, 3], [1, 1, 3, 0, 2]):
        print(f"[gdn slots] device_io={device_io} slots {batch}", flush=True)
        X = _x(rng, len(batch), H)
        pos = []
        for s in batch:
            pos.append(nextpos[s])
            nextpos[s] += 1
        AB = [po.oracle_gdn_gates(oracle, g, X[r]) for r in range(len(batch))]
        A = np.stack([ab[0] for ab in AB])
        Bv = np.stack([ab[1] for ab in AB])
        want = np.stack([po.oracle_gdn_step(oracle, g, X[r], A[r], Bv[r], pos[r], CS[s], ST[s])
                         for r, s in enumerate(batch)])
        got = dev.slots_step(X, A, Bv, batch, pos, device_io=device_io)
        assert_close_rms(got, want, 1e-3, f"gdn slots {batch}")
    dcs, dst = dev.read_state()
    for s in range(nslots):
        _close_state(dst[s], ST[s], f"recurrent state slot {s}")


def test_gdn_rejects_bad_arguments(be):
    from oracle import pyoracle as po
    from shiftwing_amd import HipError
    g = po.HostGdn(41, 512, 2, 4, 128, 128)
    dev = _dev_gdn(be, g, slots=2)
    x = np.zeros((2, 512), np.float32)
    a = np.zeros((2, 4), np.float32)
    with pytest.raises(HipError, match="invalid slot"):
        dev.slots_step(x, a, a, [0, 2], [0, 0])
    with pytest.raises(HipError, match="invalid argument"):
        dev.block(np.zeros((9, 512), np.float32), np.zeros((9, 4), np.float32), np.zeros((9, 4), np.float32), 0)


@pytest.mark.parametrize("shape,o_fmt", [("s35", 1), ("s397", 4)], ids=["s35_o8", "s397_o4"])
def test_gqa_decode_steps(be, oracle, shape, o_fmt):
    """Decode at positions 0..39: one to three 16-key blocks, more splits than
    blocks at first, the key-split merge later."""
    from oracle import pyoracle as po
    H, nh = ATTN_SHAPES[shape]
    at = po.HostAttn(51, H, nh, 2, 256, 64, o_fmt=o_fmt)
    max_seq = 64
    dev = _dev_attn(be, at, max_seq)
    kc, vc = [a[0] for a in at.new_cache(max_seq)]
    rng = np.random.default_rng(52)
    for pos in range(40):
        x = _x(rng, 1, H)[0]
        want = po.oracle_attn_step(oracle, at, x, pos, kc, vc)
        got = dev.decode(x, pos)
        if pos % 8 == 0 or pos in (15, 16, 17, 39):
            print(f"[gqa decode] {shape} o{o_fmt} pos {pos}", flush=True)
        assert_close_rms(got, want, 1e-3, f"gqa decode {shape} pos {pos}")
    dk, dvv = dev.read_cache()
    _close_state(dk[0, :40], kc[:40], "k cache")
    _close_state(dvv[0, :40], vc[:40], "v cache")


def test_gqa_prefill_then_decode(be, oracle):
    """coli_cuda_gqa_prefill_q4_f16 over 37 rows (three projection tiles) and
    then 120 more (two 16-key blocks per key split: the online softmax runs
    across blocks), continued by decode steps, against the oracle token by
    token."""
    from oracle import pyoracle as po
    H, nh = ATTN_SHAPES["s397"]
    at = po.HostAttn(61, H, nh, 2, 256, 64, o_fmt=1)
    max_seq = 200
    dev = _dev_attn(be, at, max_seq)
    kc, vc = [a[0] for a in at.new_cache(max_seq)]
    rng = np.random.default_rng(62)
    base = 0
    for rows in (37, 120):
        print(f"[gqa prefill] rows {rows} from {base}", flush=True)
        X = _x(rng, rows, H)
        want = np.stack([po.oracle_attn_step(oracle, at, X[r], base + r, kc, vc) for r in range(rows)])
        got = dev.prefill(X, base)
        for r in range(rows):
            assert_close_rms(got[r], want[r], 1e-3, f"gqa prefill row {base + r}")
        base += rows
    for pos in range(base, base + 3):
        print(f"[gqa prefill] decode at {pos}", flush=True)
        x = _x(rng, 1, H)[0]
        want = po.oracle_attn_step(oracle, at, x, pos, kc, vc)
        assert_close_rms(dev.decode(x, pos), want, 1e-3, f"gqa decode after prefill pos {pos}")


@pytest.mark.parametrize("device_io", [False, True], ids=["host_io", "device_io"])
def test_gqa_slots(be, oracle, device_io):
    """coli_cuda_gqa_slots_q4_f16[_device]: three sequences at different
    lengths in one batch, a few rounds."""
    from oracle import pyoracle as po
    H, nh = ATTN_SHAPES["s35"]
    at = po.HostAttn(71, H, nh, 2, 256, 64, o_fmt=4)
    max_seq, nslots = 48, 3
    dev = _dev_attn(be, at, max_seq, slots=nslots)
    KC, VC = at.new_cache(max_seq, nslots)
    rng = np.random.default_rng(72)
    nextpos = [0, 0, 0]
    # slot 1 first runs ahead by 20 tokens through the slot call itself
    schedule = [[1] * 1 for _ in range(20)] + [[0, 1, 2], [2, 0], [1, 2, 0]]
    for rnd, batch in enumerate(schedule):
        X = _x(rng, len(batch), H)
        pos = []
        for s in batch:
            pos.append(nextpos[s])
            nextpos[s] += 1
        want = np.stack([po.oracle_attn_step(oracle, at, X[r], pos[r], KC[s], VC[s]) for r, s in enumerate(batch)])
        got = dev.slots_step(X, batch, pos, device_io=device_io)
        if rnd >= 19:
            print(f"[gqa slots] device_io={device_io} slots {batch} pos {pos}", flush=True)
        assert_close_rms(got, want, 1e-3, f"gqa slots {batch} {pos}")


def test_gqa_rejects_bad_arguments(be):
    from oracle import pyoracle as po
    from shiftwing_amd import HipError
    at = po.HostAttn(81, 512, 4, 2, 256, 64)
    dev = _dev_attn(be, at, 8, slots=2)
    x = np.zeros((1, 512), np.float32)
    with pytest.raises(HipError, match="invalid slot"):
        dev.slots_step(x, [0], [8])
    with pytest.raises(HipError, match="invalid argument"):
        dev.prefill(np.zeros((4, 512), np.float32), 6)


@pytest.mark.parametrize("dk,dv,K", [(64, 64, 3), (128, 96, 5)], ids=["dk64_dv64_K3", "dk128_dv96_K5"])
def test_gdn_other_shapes(be, oracle, dk, dv, K):
    """Shapes off the Qwen3.5 ones: key_dim 64 (the upper lane half of the
    recurrence holds no key rows), value_dim 96 (three 32-column waves), conv
    kernels of 3 and 5 taps (5 takes the ring path through memory), decode
    steps then a block of 3."""
    from oracle import pyoracle as po
    g = po.HostGdn(91, 512, 2, 4, dk, dv, K)
    dev = _dev_gdn(be, g)
    cs, st = [a[0] for a in g.new_state()]
    rng = np.random.default_rng(92)
    for pos in range(7):
        x = _x(rng, 1, 512)[0]
        a, b = po.oracle_gdn_gates(oracle, g, x)
        want = po.oracle_gdn_step(oracle, g, x, a, b, pos, cs, st)
        assert_close_rms(dev.decode(x, a, b, pos), want, 1e-3, f"gdn dk{dk} dv{dv} K{K} pos {pos}")
    X = _x(rng, 3, 512)
    AB = [po.oracle_gdn_gates(oracle, g, X[t]) for t in range(3)]
    A = np.stack([ab[0] for ab in AB])
    Bv = np.stack([ab[1] for ab in AB])
    want = np.stack([po.oracle_gdn_step(oracle, g, X[t], A[t], Bv[t], 7 + t, cs, st) for t in range(3)])
    assert_close_rms(dev.block(X, A, Bv, 7), want, 1e-3, f"gdn dk{dk} dv{dv} K{K} block")
    dcs, dst = dev.read_state()
    _close_state(dst[0], st, "recurrent state")
    _close_state(dcs[0], cs, "conv state")


@pytest.mark.parametrize("nh,nkv,hd,rd", [(8, 2, 128, 32), (4, 1, 64, 64)], ids=["hd128", "hd64"])
def test_gqa_other_head_dims(be, oracle, nh, nkv, hd, rd):
    """head_dim 128 and 64 (the other two attention instantiations), 4 query
    heads on one kv head, a full-width rotation: decode 0..23 then a prefill of
    10 rows."""
    from oracle import pyoracle as po
    at = po.HostAttn(93, 512, nh, nkv, hd, rd, o_fmt=4)
    dev = _dev_attn(be, at, 40)
    kc, vc = [a[0] for a in at.new_cache(40)]
    rng = np.random.default_rng(94)
    for pos in range(24):
        x = _x(rng, 1, 512)[0]
        want = po.oracle_attn_step(oracle, at, x, pos, kc, vc)
        assert_close_rms(dev.decode(x, pos), want, 1e-3, f"gqa hd{hd} pos {pos}")
    X = _x(rng, 10, 512)
    want = np.stack([po.oracle_attn_step(oracle, at, X[r], 24 + r, kc, vc) for r in range(10)])
    got = dev.prefill(X, 24)
    for r in range(10):
        assert_close_rms(got[r], want[r], 1e-3, f"gqa hd{hd} prefill row {24 + r}")
