"""Compiles the gfx950 HIP sources into shiftwing_amd/libshiftwing_moe.so.

hipcc --offload-arch=gfx950, -ffp-contract=off (every fused multiply-add in
the kernels is written explicitly, so the rounding of the bit-exact paths is
the one in the source), packed FP32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SOURCES = ["context.hip", "backend.hip", "moe.hip", "moe_decode.hip", "moe_stack.hip", "head.hip", "mixer.hip", "container.cpp"]
LIB = os.path.join(HERE, "libshiftwing_moe.so")
# the same sources with the host code under AddressSanitizer and
# UndefinedBehaviorSanitizer (clang's runtime, linked shared: a process loads
# it first, LD_PRELOAD for Python), at -O1; for the CPU tests, which launch
# no kernel
SAN_LIB = os.path.join(HERE, "_san", "libshiftwing_moe.so")
SAN_FLAGS = [
    "-O1", "-g",
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
    "-shared-libsan",
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def build(verbose: bool = False, sanitize: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    out = SAN_LIB if sanitize else LIB
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    flags = [f for f in FLAGS if f != "-O3"] + SAN_FLAGS if sanitize else FLAGS
    cmd = [HIPCC, *flags, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libshiftwing_moe.so")
    os.replace(tmp, out)
    return out


def sources_newer_than(path: str) -> bool:
    """True when a source or header is newer than the built file (or it is absent)."""
    if not os.path.exists(path):
        return True
    t = os.path.getmtime(path)
    deps = [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [os.path.join(ROOT, "include", "shiftwing_moe.h")]
    return any(os.path.getmtime(d) > t for d in deps)


if __name__ == "__main__":
    print(build(verbose=True, sanitize="--sanitize" in sys.argv))
