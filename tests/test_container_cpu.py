"""The converted-snapshot loader's host side, without a GPU: indexing the
safetensors files of a directory (c/st.h), the reference's name prefixes and
format detection (load_qmat_mode, c/qwen.c:2224-2257: the .qtype tag, else the
payload and scale sizes; the .q3 sidecar of c/tools/requantize_expert_q2.py),
and its errors, which return -1 with a message where the reference exits."""
import ctypes as C
import os

import numpy as np
import pytest

import st_writer
from conftest import ROOT

SHAPE = (512, 16, 4, 256, 128)  # H, E, K, I, Ish


def _lib():
    from shiftwing_amd import abi
    return abi.load()


def _open(lib, d):
    c = C.c_void_p()
    rc = lib.coli_cuda_container_open(C.byref(c), d.encode())
    return rc, c


def _shape(lib, c, layer, use_q3):
    from shiftwing_amd import ColiMoeShape
    s = ColiMoeShape(0, 0, 7, 0, 0, 0, 0)
    rc = lib.coli_cuda_container_moe_shape(c, layer, use_q3, C.byref(s))
    return rc, s


@pytest.fixture(scope="module")
def layers(oracle):
    H, E, K, I, Ish = SHAPE
    return (oracle.host_layer(5, 3, H, E, K, I, Ish, 4), oracle.host_layer(5, 3, H, E, K, I, Ish, 3))


@pytest.mark.parametrize("prefix", ["", "model.", "model.language_model."])
def test_container_shapes_and_formats(tmp_path, layers, prefix):
    hl4, hl3 = layers
    lib = _lib()
    t = st_writer.moe_layer_tensors(hl4, 3, prefix, q3=hl3)
    st_writer.write_split(str(tmp_path), t, parts=3)
    rc, c = _open(lib, str(tmp_path))
    assert rc == 0, lib.coli_cuda_last_error()
    try:
        assert lib.coli_cuda_container_tensors(c) == len(t)
        H, E, K, I, Ish = SHAPE
        for use_q3, fmt in ((0, 4), (1, 3)):
            rc, s = _shape(lib, c, 3, use_q3)
            assert rc == 0, lib.coli_cuda_last_error()
            assert (s.hidden, s.experts, s.topk, s.intermediate, s.shared_intermediate, s.expert_format,
                    s.group_size) == (H, E, 7, I, Ish, fmt, 128)
        rc, s = _shape(lib, c, 2, 0)  # no such layer
        assert rc == -1 and "layer 2" in lib.coli_cuda_last_error().decode()
    finally:
        lib.coli_cuda_container_close(c)


def test_container_formats_without_tags(tmp_path, layers):
    """Without .qtype tags the sizes decide (c/qwen.c:2237-2254): the shared
    rows are int8 (payload rows x cols, one scale per row), the experts int4."""
    hl4, _ = layers
    lib = _lib()
    st_writer.write_split(str(tmp_path), st_writer.moe_layer_tensors(hl4, 0, qtype_tags=False), parts=1)
    rc, c = _open(lib, str(tmp_path))
    assert rc == 0, lib.coli_cuda_last_error()
    rc, s = _shape(lib, c, 0, 0)
    assert rc == 0 and s.expert_format == 4 and s.group_size == 128
    lib.coli_cuda_container_close(c)


def test_container_errors(tmp_path, layers):
    hl4, _ = layers
    lib = _lib()
    # no safetensors file
    rc, _ = _open(lib, str(tmp_path))
    assert rc == -1 and "no .safetensors" in lib.coli_cuda_last_error().decode()
    # a header that is not JSON
    bad = tmp_path / "bad"
    bad.mkdir()
    with open(bad / "x.safetensors", "wb") as f:
        f.write((7).to_bytes(8, "little") + b"{nope!!")
    rc, _ = _open(lib, str(bad))
    assert rc == -1 and "x.safetensors" in lib.coli_cuda_last_error().decode()
    # data offsets past the end of the file
    bad2 = tmp_path / "bad2"
    bad2.mkdir()
    st_writer.write(str(bad2 / "y.safetensors"), {"a": np.zeros(4, np.float32)})
    raw = open(bad2 / "y.safetensors", "rb").read()
    open(bad2 / "y.safetensors", "wb").write(raw[:-4])
    rc, _ = _open(lib, str(bad2))
    assert rc == -1 and "does not fit" in lib.coli_cuda_last_error().decode()
    # a quantized expert without .qs
    t = st_writer.moe_layer_tensors(hl4, 0)
    del t["layers.0.mlp.experts.0.gate_proj.weight.qs"]
    d3 = tmp_path / "noqs"
    st_writer.write_split(str(d3), t, parts=1)
    rc, c = _open(lib, str(d3))
    assert rc == 0
    rc, _ = _shape(lib, c, 0, 0)
    assert rc == -1 and ".qs" in lib.coli_cuda_last_error().decode()
    # an unknown qtype tag
    t = st_writer.moe_layer_tensors(hl4, 0)
    t["layers.0.mlp.experts.0.gate_proj.weight.qtype"] = np.array([5], np.uint8)
    d4 = tmp_path / "tag"
    st_writer.write_split(str(d4), t, parts=1)
    rc, c2 = _open(lib, str(d4))
    rc, _ = _shape(lib, c2, 0, 0)
    assert rc == -1 and "qtype" in lib.coli_cuda_last_error().decode()
    lib.coli_cuda_container_close(c)
    lib.coli_cuda_container_close(c2)
    # the .q3 sidecar asked for but absent
    st_writer.write_split(str(tmp_path / "noq3"), st_writer.moe_layer_tensors(hl4, 0), parts=1)
    rc, c3 = _open(lib, str(tmp_path / "noq3"))
    rc, _ = _shape(lib, c3, 0, 1)
    assert rc == -1 and ".q3" in lib.coli_cuda_last_error().decode()
    lib.coli_cuda_container_close(c3)


def _pick(rng, values):
    return values[int(rng.integers(0, len(values)))]


def _corrupt(raw: bytes, rng) -> bytes:
    """One damaged copy of a container file: truncated, a header byte
    changed, the header length changed, or a number in the header changed."""
    hlen = int.from_bytes(raw[:8], "little")
    kind = int(rng.integers(0, 4))
    if kind == 0:
        return raw[:int(rng.integers(0, len(raw)))]
    if kind == 1:
        b = bytearray(raw)
        for _ in range(int(rng.integers(1, 4))):
            b[8 + int(rng.integers(0, hlen))] = int(rng.choice(list(b'{}[]":,0123456789-e. \x00\xff')))
        return bytes(b)
    if kind == 2:
        n = _pick(rng, [0, 1, hlen - 1, hlen + 1, len(raw) - 8, len(raw), 2**31, 2**63 - 1, 2**64 - 1])
        return n.to_bytes(8, "little") + raw[8:]
    head = raw[8:8 + hlen].decode()
    digits = [i for i, ch in enumerate(head) if ch.isdigit()]
    i = int(rng.choice(digits))
    j = i
    while j < len(head) and head[j].isdigit():
        j += 1
    new = str(_pick(rng, [0, 1, 7, 2**31 - 1, 2**31, 2**32 + 3, 2**62, 10**30, -1]))
    head = head[:i] + new + head[j:]
    h = head.encode()
    return len(h).to_bytes(8, "little") + h + raw[8 + hlen:]


def test_container_survives_corrupt_files(tmp_path, layers):
    """Damaged files open with an error or, where the damage is harmless, load
    their shapes; nothing reads outside what the file holds (the sanitizer
    run of this test makes an out-of-bounds read fail it)."""
    hl4, hl3 = layers
    lib = _lib()
    src = tmp_path / "src"
    src.mkdir()
    st_writer.write(str(src / "m.safetensors"), st_writer.moe_layer_tensors(hl4, 0, q3=hl3))
    raw = open(src / "m.safetensors", "rb").read()
    rng = np.random.default_rng(23)
    opened = failed = 0
    for k in range(240):
        d = tmp_path / f"c{k}"
        d.mkdir()
        with open(d / "m.safetensors", "wb") as f:
            f.write(_corrupt(raw, rng))
        rc, c = _open(lib, str(d))
        if rc != 0:
            assert rc == -1 and lib.coli_cuda_last_error(), k
            failed += 1
            continue
        opened += 1
        assert lib.coli_cuda_container_tensors(c) >= 0
        for use_q3 in (0, 1):
            rc, s = _shape(lib, c, 0, use_q3)
            assert rc in (0, -1), k
            if rc == 0:
                assert s.hidden > 0 and s.experts > 0 and s.expert_format in (2, 3, 4), k
        lib.coli_cuda_container_close(c)
        os.remove(d / "m.safetensors")
    assert failed > 0 and opened > 0, (failed, opened)


def _reference():
    from oracle.pyoracle import Reference
    try:
        return Reference()
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")


def _int2_tensors(rng, layer, E, H, I, prefix="", suffix="", gs=128):
    """int2 routed experts (.qtype 2): rows of cols/4 bytes, 4 codes per byte,
    value 2*code-3 (c/qwen.c:1717-1724, 2244-2246), one scale per group."""
    t = {}
    for e in range(E):
        for nm, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
            base = f"{prefix}layers.{layer}.mlp.experts.{e}.{nm}_proj.weight{suffix}"
            t[base] = rng.integers(0, 256, (rows, cols // 4), dtype=np.uint8)
            t[base + ".qs"] = np.abs(rng.standard_normal((rows, cols // gs))).astype(np.float32) * 0.01
            t[base + ".qtype"] = np.array([2], np.uint8)
    return t


def test_container_matches_the_reference_loader(tmp_path, layers, oracle):
    """One snapshot directory read two ways: by the reference's own st.h index
    and load_qmat_mode (c/st.h:211-297, c/qwen.c:2198-2257, compiled in place
    in oracle/_ref) and by coli_cuda_container_moe_shape.  Formats, group sizes,
    row bytes and group counts agree, and the reference reads back exactly the
    payload bytes and scales of the host layer that coli_cuda_moe_layer_load
    is checked against on the GPU (test_gpu_container.py), for the main int4
    payload, the .q3 sidecar, the int8 shared expert and the float router."""
    ref = _reference()
    hl4, hl3 = layers
    H, E, K, I, Ish = SHAPE
    pre = "model.language_model."
    st_writer.write_split(str(tmp_path), st_writer.moe_layer_tensors(hl4, 3, pre, q3=hl3), parts=3)
    lib = _lib()
    rc, c = _open(lib, str(tmp_path))
    assert rc == 0, lib.coli_cuda_last_error()
    try:
        for side, hl in ((0, hl4), (1, hl3)):
            rc, s = _shape(lib, c, 3, side)
            assert rc == 0, lib.coli_cuda_last_error()
            for e in (0, 5, E - 1):
                for nm, rows, cols, q, sc in (("gate", I, H, hl.gq, hl.gsc), ("up", I, H, hl.uq, hl.usc),
                                              ("down", H, I, hl.dq, hl.dsc)):
                    info, pay, scl = ref.load_qmat(str(tmp_path), f"layers.3.mlp.experts.{e}.{nm}_proj.weight",
                                                   rows, cols, use_q3=side == 1)
                    assert info["fmt"] == s.expert_format and info["gs"] == s.group_size, (side, e, nm, info)
                    assert info["rb"] == q.shape[2] and info["ng"] == sc.shape[2], (side, e, nm, info)
                    assert np.array_equal(pay, q[e]), (side, e, nm)
                    assert np.array_equal(scl.view(np.uint32), sc[e].reshape(-1).view(np.uint32)), (side, e, nm)
        for nm, m, rows, cols in (("gate", hl4.shared_gate, Ish, H), ("up", hl4.shared_up, Ish, H),
                                  ("down", hl4.shared_down, H, Ish)):
            info, pay, scl = ref.load_qmat(str(tmp_path), f"layers.3.mlp.shared_expert.{nm}_proj.weight", rows, cols)
            assert info["fmt"] == 1 and info["rb"] == cols, info
            assert np.array_equal(pay.view(np.int8), np.asarray(m.q).reshape(rows, cols).view(np.int8))
            assert np.array_equal(scl, np.asarray(m.s, np.float32))
        info, pay, _ = ref.load_qmat(str(tmp_path), "layers.3.mlp.gate.weight", E, H)
        assert info["fmt"] == 0 and np.array_equal(pay, hl4.router_w)
        assert (s.hidden, s.experts, s.intermediate, s.shared_intermediate) == (H, E, I, Ish)
    finally:
        lib.coli_cuda_container_close(c)


def test_container_int2_and_group_sizes_as_the_reference_reads_them(tmp_path, oracle):
    """int2 experts and other group sizes are classified as the reference
    classifies them: int2 experts from .qtype 2 main payloads and from .q2
    sidecars (EXPERT_Q2=1, which falls back to the main payload for an expert
    without one, c/qwen.c:2207-2214), which coli_cuda_moe_layer_load widens to
    int4 records, and int4 experts in groups of 64, which it refuses by name
    (the GPU container tests load the one and check the refusal of the
    other)."""
    ref = _reference()
    H, E, K, I, Ish = SHAPE
    rng = np.random.default_rng(2)
    lib = _lib()
    hl = oracle.host_layer(6, 1, H, E, K, I, Ish, 4)
    # int2 main payloads
    t = st_writer.moe_layer_tensors(hl, 1)
    t.update(_int2_tensors(rng, 1, E, H, I))
    st_writer.write_split(str(tmp_path / "q2main"), t, parts=2)
    # int4 main payloads with .q2 sidecars for every expert but the last
    t = st_writer.moe_layer_tensors(hl, 1)
    side = _int2_tensors(rng, 1, E, H, I, suffix=".q2")
    t.update({k: v for k, v in side.items() if f".experts.{E - 1}." not in k})
    st_writer.write_split(str(tmp_path / "q2side"), t, parts=2)
    # int4 in groups of 64
    hl64 = oracle.host_layer(6, 1, H, E, K, I, Ish, 4, gs=64)
    st_writer.write_split(str(tmp_path / "g64"), st_writer.moe_layer_tensors(hl64, 1), parts=1)
    cases = [("q2main", 0, 0, 2, 128), ("q2side", 2, 1, 2, 128), ("q2side", 0, 0, 4, 128), ("g64", 0, 0, 4, 64)]
    for d, sidecar, use_q2, fmt, gs in cases:
        rc, c = _open(lib, str(tmp_path / d))
        assert rc == 0, lib.coli_cuda_last_error()
        rc, s = _shape(lib, c, 1, sidecar)
        assert rc == 0, lib.coli_cuda_last_error()
        lib.coli_cuda_container_close(c)
        assert (s.expert_format, s.group_size) == (fmt, gs), (d, sidecar)
        for e in (0, E - 1):
            info, _, _ = ref.load_qmat(str(tmp_path / d), f"layers.1.mlp.experts.{e}.gate_proj.weight", I, H,
                                       use_q2=bool(use_q2))
            want = 4 if (d == "q2side" and use_q2 and e == E - 1) else fmt
            assert (info["fmt"], info["gs"]) == (want, gs), (d, sidecar, e, info)
