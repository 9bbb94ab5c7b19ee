"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

- The library's host side: context set-up without a device, argument checks,
  the header-bound prototypes and the safetensors loader's parser (including
  the corrupted-file test).  shiftwing_amd/build.py builds the same sources
  with -Xarch_host -fsanitize=address,undefined into shiftwing_amd/_san/; a
  child Python loads clang's ASan runtime first (LD_PRELOAD) and the
  sanitized library through SHIFTWING_MOE_LIB.
- The checker (oracle/moe_oracle.c): `make -C oracle san` builds it with gcc's
  sanitizers into oracle/_san/; a child Python runs the oracle's tests with
  gcc's runtime preloaded and SHIFTWING_ORACLE_LIB pointing at it.

Each child stops at the first report (UBSan without recovery, ASan's default)
and its pytest run must pass.  Kernels are never launched here."""
import glob
import os
import subprocess
import sys

import pytest

from conftest import ROOT


def _child(env_extra, args, timeout=600):
    env = dict(os.environ)
    env.update(env_extra)
    env["ASAN_OPTIONS"] = "detect_leaks=0"  # the interpreter keeps its objects to the end
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *args],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=timeout)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    return out


def test_library_host_code_under_asan_ubsan():
    from shiftwing_amd import build
    rt = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("clang's ASan runtime is not installed")
    if build.sources_newer_than(build.SAN_LIB):
        build.build(sanitize=True)
    probe = ("import ctypes; ctypes.CDLL(None)['__asan_init']; "
             "from shiftwing_amd import abi; abi.load(); print('asan ok')")
    env = {"LD_PRELOAD": rt[-1], "SHIFTWING_MOE_LIB": build.SAN_LIB}
    # the runtime is in the process and the sanitized build is what loads
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env={**os.environ, **env,
                       "ASAN_OPTIONS": "detect_leaks=0"}, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "asan ok" in r.stdout, r.stdout + r.stderr
    _child(env, ["tests/test_container_cpu.py", "tests/test_host_cpu.py", "-k",
                 "container or exports or argument_errors or context_creation or prototypes"])


def test_oracle_under_asan_ubsan():
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(rt) or not os.path.exists(rt):
        pytest.skip("gcc's ASan runtime is not installed")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "san"], check=True)
    lib = os.path.join(ROOT, "oracle", "_san", "liboracle.so")
    env = {"LD_PRELOAD": rt, "SHIFTWING_ORACLE_LIB": lib}
    probe = ("import ctypes; ctypes.CDLL(None)['__asan_init']; "
             "from oracle.pyoracle import Oracle; print(Oracle().lib._name)")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env={**os.environ, **env,
                       "ASAN_OPTIONS": "detect_leaks=0"}, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == lib, r.stdout + r.stderr
    _child(env, ["tests/test_oracle_cpu.py"])
