"""Host-side pieces that run without a GPU: the C-ABI library loads and
exports every prototype of include/shiftwing_moe.h, its argument checks fail
with the reference's error convention (return -1, message in
coli_cuda_last_error, c/backend_cuda.cu:47-70) before touching the device,
and the benchmark's byte arithmetic equals the closed-form per-expert sizes."""
import ctypes as C
import os
import re
import subprocess
import sys

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "shiftwing_moe.h")


def _lib():
    from shiftwing_amd import abi
    return abi.load()


def _declared_names():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return sorted(set(re.findall(r"\b(coli_cuda_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib()
    names = _declared_names()
    assert len(names) >= 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_parser_covers_every_prototype():
    from shiftwing_amd import abi
    assert sorted(abi.parse_header()) == _declared_names()


def test_reference_prototypes_are_declared():
    """The MoE-path entry points of c/backend_cuda.h that the drop-in keeps
    with identical prototypes."""
    names = set(_declared_names())
    for n in ["create", "destroy", "last_error", "device_name", "compute_capability", "device_limits",
              "async_alloc_enabled", "memory_info", "malloc", "free", "malloc_host", "free_host",
              "host_register", "host_unregister", "upload", "download", "copy", "memset", "sync",
              "profile_reset", "profile_snapshot", "sigmoid", "silu_mul", "axpy", "sigmoid_axpy",
              "f32_to_f16", "f32_gemm", "q8_gemv", "q8_gemm", "q4_gemv", "q4_gemm", "q4_gemv_f16",
              "q3_gemv", "q3_gemv_f16", "grouped_q4_mlp_f16", "grouped_q3_mlp_f16",
              "grouped_q4_mlp_batch_f16", "grouped_q3_mlp_batch_f16", "shared_q4_mlp_batch_f16",
              "shared_q8_mlp_batch", "shared_q8_mlp_batch_device_scale", "shared_q4_mlp_f16"]:
        assert "coli_cuda_" + n in names, n


def test_argument_errors_follow_reference_convention():
    lib = _lib()
    h = C.c_void_p()
    assert lib.coli_cuda_moe_layer_create(None, C.byref(h), None) == -1
    assert b"null argument" in lib.coli_cuda_last_error()
    assert lib.coli_cuda_moe_set_router_mode(None, 0) == -1
    assert lib.coli_cuda_moe_set_decode_kernels(None, 1) == -1
    assert lib.coli_cuda_moe_forward(None, None, None, None, 1, None, None) == -1
    assert lib.coli_cuda_moe_route_stats_full(None, None, None) == -1


def test_context_creation_without_device_fails_cleanly():
    """No GPU here: create must return -1 with a message, not crash."""
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    lib = _lib()
    ctx = C.c_void_p()
    assert lib.coli_cuda_create(C.byref(ctx), 0) == -1
    assert lib.coli_cuda_last_error()


def test_product_path_has_no_oracle_dependency():
    """The shipped package never imports the oracle (test infrastructure)."""
    pkg = os.path.join(ROOT, "shiftwing_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "pyoracle" not in text and "moe_oracle" not in text, f


def test_missing_library_fails_loudly(tmp_path):
    from shiftwing_amd import abi
    saved = abi._LIB
    abi._LIB = None
    try:
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            abi.load(str(tmp_path / "absent.so"))
    finally:
        abi._LIB = saved


# ------------------------------------------------------------ byte arithmetic
def test_algorithmic_bytes_match_closed_form():
    """Per token-layer bytes: S35 18,632,704 and S397 72,130,560 (weights +
    scales of K routed experts, shared int8 expert, router f32, shared gate)."""
    sys.path.insert(0, ROOT)
    import bench
    s35 = bench.WORKLOADS["s35"]
    s397 = bench.WORKLOADS["s397"]
    assert sum(bench.kernel_bytes(*s35[:6])) == 18_632_704
    assert sum(bench.kernel_bytes(*s397[:6])) == 72_130_560
    # per expert: S35 1,671,168 B, S397 5,111,808 B
    H, E, K, I, Ish, fmt = s397[:6]
    assert bench.kernel_bytes(H, E, 1, I, Ish, fmt)[1] + bench.kernel_bytes(H, E, 1, I, Ish, fmt)[2] \
        - (H * Ish + 2 * Ish * 4 + H * 4) == 5_111_808
    H, E, K, I, Ish, fmt = s35[:6]
    assert bench.kernel_bytes(H, E, 1, I, Ish, fmt)[1] + bench.kernel_bytes(H, E, 1, I, Ish, fmt)[2] \
        - (H * Ish + 2 * Ish * 4 + H * 4) == 1_671_168


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_graft_entry_points_exist():
    sys.path.insert(0, ROOT)
    import __graft_entry__ as ge
    assert callable(ge.build) and callable(ge.smoke)


REF_C = "/root/reference/c"
LIB_SO = os.path.join(ROOT, "shiftwing_amd", "libshiftwing_moe.so")


def _defined_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def _undefined_symbols(path):
    out = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


@pytest.mark.skipif(not os.path.isdir(REF_C), reason="the reference tree is not present")
def test_reference_engine_links_against_this_library():
    """The drop-in link: the reference engine c/qwen.c built with -DCOLI_CUDA
    (its CUDA=1 configuration, c/Makefile:62-69, 124-125) links against
    libshiftwing_moe.so in place of backend_cuda.o, and so do the reference's
    GPU test and the glue harness.  Every coli_cuda_* symbol they import is
    defined by this library and declared in include/shiftwing_moe.h."""
    if not os.path.exists(LIB_SO):
        pytest.skip("libshiftwing_moe.so is not built")
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref-hip"], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    ours = _defined_symbols(LIB_SO)
    declared = set(_declared_names())
    for exe in ("qwen_hip", "test_backend_cuda", "libref_hip.so"):
        path = os.path.join(ROOT, "oracle", "_ref", exe)
        assert os.path.exists(path), path
        wanted = {s for s in _undefined_symbols(path) if s.startswith("coli_cuda_")}
        assert wanted, exe
        assert wanted <= ours, (exe, sorted(wanted - ours))
        assert wanted <= declared, (exe, sorted(wanted - declared))
    # every coli_cuda_ name the reference engine source calls
    src = open(os.path.join(REF_C, "qwen.c")).read()
    called = set(re.findall(r"\b(coli_cuda_\w+)\s*\(", src))
    assert called <= ours, sorted(called - ours)
