"""ctypes binding of the C ABI in include/shiftwing_moe.h.

The prototypes are read from the header itself, so the Python side cannot
drift from the C declarations.  Loading fails loudly when the HIP library has
not been built: there is no CPU fallback behind this module.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "include", "shiftwing_moe.h")
# SHIFTWING_MOE_LIB names another build of the same library (the host-only
# sanitizer build that the CPU tests load)
LIB_PATH = os.environ.get("SHIFTWING_MOE_LIB") or os.path.join(HERE, "libshiftwing_moe.so")


class ColiMoeShape(C.Structure):
    _fields_ = [("hidden", C.c_int), ("experts", C.c_int), ("topk", C.c_int),
                ("intermediate", C.c_int), ("shared_intermediate", C.c_int),
                ("expert_format", C.c_int), ("group_size", C.c_int)]


_SCALARS = {
    "int": C.c_int, "float": C.c_float, "size_t": C.c_size_t, "void": None,
    "unsigned long long": C.c_ulonglong, "double": C.c_double,
}


def _ctype(decl: str):
    """ctypes type of one C parameter or return declaration (name stripped)."""
    d = re.sub(r"\bconst\b", "", decl).strip()
    if "[" in d:  # double stage_ms[8]
        return C.c_void_p
    stars = d.count("*")
    base = d.replace("*", " ").split()
    if stars == 0:
        return _SCALARS[" ".join(base)]
    if stars == 1 and " ".join(base[:1]) == "char" and len(base) == 1:
        return C.c_char_p
    return C.c_void_p


def parse_header(path: str = HEADER):
    """{name: (restype, [argtypes])} for every coli_cuda_* declaration."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(coli_cuda_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        ret = " ".join(ret.split())
        restype = C.c_char_p if ret.replace(" ", "") in ("constchar*",) else _ctype(ret.replace("extern", ""))
        argtypes = []
        a = " ".join(args.split())
        if a and a != "void":
            for p in a.split(","):
                p = p.strip()
                # drop the parameter name (last identifier, possibly with [N])
                p = re.sub(r"\b\w+\s*(\[\d*\])?$", lambda mm: ("[]" if mm.group(1) else ""), p).strip()
                argtypes.append(_ctype(p))
        out[name] = (restype, argtypes)
    return out


_LIB = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libshiftwing_moe.so and attach prototypes; raise if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m shiftwing_amd.build` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    lib = C.CDLL(path)
    for name, (res, args) in parse_header().items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib
