"""ctypes access to the CPU checker (liboracle.so) and the compiled reference
(oracle/_ref/libref_*.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product package never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SHIFTWING_ORACLE_LIB names another build of the checker (the sanitizer build)
ORACLE_SO = os.environ.get("SHIFTWING_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)


class OrQMat(C.Structure):
    _fields_ = [("fmt", C.c_int), ("O", C.c_int), ("I", C.c_int), ("gs", C.c_int),
                ("rb", C.c_int), ("ng", C.c_int), ("f", f32p), ("s", f32p),
                ("q", C.c_void_p)]


class OrLayer(C.Structure):
    _fields_ = [("H", C.c_int), ("E", C.c_int), ("K", C.c_int), ("I", C.c_int),
                ("I_sh", C.c_int), ("router", OrQMat), ("shared_gate", OrQMat),
                ("shared_up", OrQMat), ("shared_down", OrQMat),
                ("shared_scale", OrQMat), ("gate", C.POINTER(OrQMat)),
                ("up", C.POINTER(OrQMat)), ("down", C.POINTER(OrQMat))]


class OrTrace(C.Structure):
    _fields_ = [("logits", f32p), ("idx", i32p), ("weight", f32p),
                ("shared", f32p), ("sgate", f32p)]


def ptr(a: np.ndarray | None, typ=C.c_void_p):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return C.cast(a.ctypes.data, typ)


def build(ref: bool = False) -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref and os.path.isdir("/root/reference/c"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _declare(lib, prefix: str):
    P = prefix
    for name, res, args in [
        ("dot_q8f", C.c_float, [C.c_void_p, f32p, C.c_int]),
        ("qrow_i8", C.c_float, [f32p, C.c_void_p, C.c_int]),
        ("dot_i8i8", C.c_int32, [C.c_void_p, C.c_void_p, C.c_int]),
        ("dot_q4_group", C.c_float, [C.c_void_p, f32p, C.c_int]),
        ("dot_q3_group", C.c_float, [C.c_void_p, f32p, C.c_int]),
        ("dot_q2_group", C.c_float, [C.c_void_p, f32p, C.c_int]),
        ("expf", C.c_float, [C.c_float]),
        ("siluf", C.c_float, [C.c_float]),
        ("qmat_mul", None, [f32p, f32p, C.POINTER(OrQMat), C.c_int]),
        ("qmat_mul_batch", None, [f32p, f32p, C.c_int, C.c_int, C.POINTER(OrQMat), C.c_int]),
        ("router_topk", None, [f32p, C.c_int, C.c_int, i32p, f32p]),
        ("mlp_one", None, [f32p, f32p, C.POINTER(OrQMat), C.POINTER(OrQMat),
                            C.POINTER(OrQMat), C.c_int]),
    ]:
        fn = getattr(lib, P + name)
        fn.restype = res
        fn.argtypes = args
    dotname = "ref_dot" if P == "ref_" else "or_dot_f32"
    getattr(lib, dotname).restype = C.c_float
    getattr(lib, dotname).argtypes = [f32p, f32p, C.c_int]


class Oracle:
    """The restatement (liboracle.so)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build()
        self.lib = C.CDLL(path)
        L = self.lib
        _declare(L, "or_")
        L.or_sigmoidf.restype = C.c_float
        L.or_sigmoidf.argtypes = [C.c_float]
        L.or_q3_value.restype = C.c_int
        L.or_q3_value.argtypes = [C.c_void_p, C.c_int]
        L.or_qmat_dot_row.restype = C.c_float
        L.or_qmat_dot_row.argtypes = [C.POINTER(OrQMat), C.c_int, f32p]
        L.or_mlp_batch.restype = None
        L.or_mlp_batch.argtypes = [f32p, f32p, C.c_int, C.c_int, C.POINTER(OrQMat),
                                   C.POINTER(OrQMat), C.POINTER(OrQMat), C.c_int]
        L.or_moe_forward.restype = None
        L.or_moe_forward.argtypes = [C.POINTER(OrLayer), f32p, f32p, C.POINTER(OrTrace)]
        L.or_moe_prefill_grouped.restype = None
        L.or_moe_prefill_grouped.argtypes = [C.POINTER(OrLayer), f32p, C.c_int, f32p,
                                             C.POINTER(OrTrace)]
        L.or_bucket.restype = C.c_int
        L.or_bucket.argtypes = [i32p, C.c_int, C.c_int, C.c_int, i32p, i32p, i32p]
        L.or_synth_router.restype = None
        L.or_synth_router.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, f32p, f32p]
        L.or_synth_shared_q8.restype = None
        L.or_synth_shared_q8.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int,
                                         C.c_void_p, f32p, C.c_void_p, f32p,
                                         C.c_void_p, f32p]
        L.or_synth_expert.restype = None
        L.or_synth_expert.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, C.c_int, C.c_void_p, f32p, C.c_void_p,
                                      f32p, C.c_void_p, f32p]
        L.or_synth_x.restype = None
        L.or_synth_x.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, f32p]
        L.or_synth_bytes.restype = None
        L.or_synth_bytes.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int,
                                     C.c_void_p, C.c_uint64]
        for nm in ("or_sigmoid_batch", "or_expf_batch"):
            getattr(L, nm).restype = None
            getattr(L, nm).argtypes = [f32p, f32p, C.c_int64]
        L.or_rmsnorm_zero.restype = None
        L.or_rmsnorm_zero.argtypes = [f32p, f32p, f32p, C.c_int, C.c_float]
        L.or_siluf.restype = C.c_float
        L.or_siluf.argtypes = [C.c_float]
        L.or_set_threads.restype = None
        L.or_set_threads.argtypes = [C.c_int]
        L.or_get_threads.restype = C.c_int
        L.or_get_threads.argtypes = []

    # -- building blocks ------------------------------------------------------
    def dot(self, a, b):
        return self.lib.or_dot_f32(ptr(a, f32p), ptr(b, f32p), a.size)

    def router_topk(self, logit: np.ndarray, K: int):
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        self.lib.or_router_topk(ptr(logit, f32p), logit.size, K, ptr(idx, i32p), ptr(w, f32p))
        return idx, w

    def qmat_mul(self, x: np.ndarray, m: "HostQMat", allow_idot: int = 1):
        y = np.zeros(m.O, np.float32)
        self.lib.or_qmat_mul(ptr(y, f32p), ptr(x, f32p), C.byref(m.st), allow_idot)
        return y

    def qmat_mul_batch(self, x: np.ndarray, m: "HostQMat", allow_idot: int = 1):
        B, ldx = x.shape
        y = np.zeros((B, m.O), np.float32)
        self.lib.or_qmat_mul_batch(ptr(y, f32p), ptr(x, f32p), B, ldx, C.byref(m.st), allow_idot)
        return y

    def qrow_i8(self, x: np.ndarray):
        q = np.zeros(x.size, np.int8)
        s = self.lib.or_qrow_i8(ptr(x, f32p), ptr(q), x.size)
        return q, np.float32(s)

    def bucket(self, idx: np.ndarray, E: int):
        T, K = idx.shape
        idx = np.ascontiguousarray(idx, np.int32)
        off = np.zeros(E + 1, np.int32)
        tok = np.zeros(T * K, np.int32)
        slot = np.zeros(T * K, np.int32)
        n = self.lib.or_bucket(ptr(idx, i32p), T, K, E, ptr(off, i32p), ptr(tok, i32p),
                               ptr(slot, i32p))
        return off, tok[:n], slot[:n]

    def moe_forward(self, layer: "HostLayer", x: np.ndarray, trace: bool = False):
        H, E, K = layer.H, layer.E, layer.K
        out = np.zeros(H, np.float32)
        tr = None
        if trace:
            t = dict(logits=np.zeros(E, np.float32), idx=np.zeros(K, np.int32),
                     weight=np.zeros(K, np.float32), shared=np.zeros(H, np.float32),
                     sgate=np.zeros(1, np.float32))
            tr = OrTrace(ptr(t["logits"], f32p), ptr(t["idx"], i32p), ptr(t["weight"], f32p),
                         ptr(t["shared"], f32p), ptr(t["sgate"], f32p))
        self.lib.or_moe_forward(C.byref(layer.st), ptr(x, f32p), ptr(out, f32p),
                                C.byref(tr) if tr is not None else None)
        return (out, t) if trace else out

    def moe_prefill(self, layer: "HostLayer", x: np.ndarray, trace: bool = False):
        T, H = x.shape
        E, K = layer.E, layer.K
        out = np.zeros((T, H), np.float32)
        tr = None
        if trace:
            t = dict(logits=np.zeros((T, E), np.float32), idx=np.zeros((T, K), np.int32),
                     weight=np.zeros((T, K), np.float32), shared=np.zeros((T, H), np.float32),
                     sgate=np.zeros(T, np.float32))
            tr = OrTrace(ptr(t["logits"], f32p), ptr(t["idx"], i32p), ptr(t["weight"], f32p),
                         ptr(t["shared"], f32p), ptr(t["sgate"], f32p))
        self.lib.or_moe_prefill_grouped(C.byref(layer.st), ptr(x, f32p), T, ptr(out, f32p),
                                        C.byref(tr) if tr is not None else None)
        return (out, t) if trace else out

    def synth_x(self, seed: int, layer: int, step: int, H: int):
        x = np.zeros(H, np.float32)
        self.lib.or_synth_x(seed, layer, step, H, ptr(x, f32p))
        return x

    def set_threads(self, n: int):
        self.lib.or_set_threads(n)

    def rmsnorm_zero(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        for r in range(x.shape[0] if x.ndim == 2 else 1):
            xr = x[r] if x.ndim == 2 else x
            orow = out[r] if x.ndim == 2 else out
            self.lib.or_rmsnorm_zero(ptr(orow, f32p), ptr(xr, f32p), ptr(w, f32p), xr.size, eps)
        return out

    def sigmoid_batch(self, x: np.ndarray) -> np.ndarray:
        y = np.empty_like(x)
        self.lib.or_sigmoid_batch(ptr(x, f32p), ptr(y, f32p), x.size)
        return y

    def host_layer(self, seed, layer, H, E, K, I, I_sh, fmt, gs=128):
        return HostLayer(self, seed, layer, H, E, K, I, I_sh, fmt, gs)


def ref_lib_candidates():
    """Compiled-reference builds, best match for this host first."""
    flags = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("flags"):
                    flags = line
                    break
    except OSError:
        pass
    names = []
    if "avx512f" in flags and "avx512bw" in flags and "avx512_vnni" in flags:
        names += ["libref_native.so", "libref_v4.so"]
    if "avx2" in flags and " fma" in flags:
        names += ["libref_v3.so"]
    return [os.path.join(REF_DIR, n) for n in names if os.path.exists(os.path.join(REF_DIR, n))]


class Reference:
    """The reference's own CPU MoE code compiled in place (oracle/_ref)."""

    def __init__(self, path: str | None = None):
        if path is None:
            cands = ref_lib_candidates()
            if not cands:
                raise FileNotFoundError("oracle/_ref has no build usable on this CPU")
            path = cands[0]
        self.path = path
        self.lib = C.CDLL(path)
        L = self.lib
        _declare(L, "ref_")
        L.ref_layer_create.restype = C.c_void_p
        L.ref_layer_create.argtypes = [C.POINTER(OrLayer)]
        L.ref_layer_destroy.restype = None
        L.ref_layer_destroy.argtypes = [C.c_void_p]
        L.ref_moe_forward.restype = None
        L.ref_moe_forward.argtypes = [C.c_void_p, f32p, f32p]
        L.ref_moe_prefill_grouped.restype = None
        L.ref_moe_prefill_grouped.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        L.ref_rmsnorm_zero.restype = None
        L.ref_rmsnorm_zero.argtypes = [f32p, f32p, f32p, C.c_int, C.c_float]
        L.ref_set_threads.restype = None
        L.ref_set_threads.argtypes = [C.c_int]
        L.ref_omp_threads.restype = C.c_int

    def route_gather_all(self, idx: np.ndarray, weight: np.ndarray, E: int):
        """moe_prefill_route_gather for experts 0..E-1: (offsets, tokens,
        weights, gathered rows) in the reference's order."""
        T, K = idx.shape
        idx = np.ascontiguousarray(idx, np.int32)
        weight = np.ascontiguousarray(weight, np.float32)
        off = np.zeros(E + 1, np.int32)
        tok = np.zeros(T * K, np.int32)
        wt = np.zeros(T * K, np.float32)
        xb = np.zeros(T * K, np.float32)
        L = self.lib
        L.ref_route_gather_all.restype = C.c_int
        L.ref_route_gather_all.argtypes = [i32p, f32p, C.c_int, C.c_int, C.c_int, i32p, i32p, f32p, f32p]
        n = L.ref_route_gather_all(ptr(idx, i32p), ptr(weight, f32p), T, K, E, ptr(off, i32p), ptr(tok, i32p),
                                   ptr(wt, f32p), ptr(xb, f32p))
        return off, tok[:n], wt[:n], xb[:n]

    def dot(self, a, b):
        return self.lib.ref_dot(ptr(a, f32p), ptr(b, f32p), a.size)

    def router_topk(self, logit: np.ndarray, K: int):
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        self.lib.ref_router_topk(ptr(logit, f32p), logit.size, K, ptr(idx, i32p), ptr(w, f32p))
        return idx, w

    def qmat_mul(self, x, m: "HostQMat", allow_idot: int = 1):
        y = np.zeros(m.O, np.float32)
        self.lib.ref_qmat_mul(ptr(y, f32p), ptr(x, f32p), C.byref(m.st), allow_idot)
        return y

    def qmat_mul_batch(self, x, m: "HostQMat", allow_idot: int = 1):
        B, ldx = x.shape
        y = np.zeros((B, m.O), np.float32)
        self.lib.ref_qmat_mul_batch(ptr(y, f32p), ptr(x, f32p), B, ldx, C.byref(m.st),
                                    allow_idot)
        return y

    def qrow_i8(self, x: np.ndarray):
        q = np.zeros(x.size, np.int8)
        s = self.lib.ref_qrow_i8(ptr(x, f32p), ptr(q), x.size)
        return q, np.float32(s)

    def rmsnorm_zero(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.ref_rmsnorm_zero(ptr(out, f32p), ptr(x, f32p), ptr(w, f32p), x.size, eps)
        return out

    def load_qmat(self, snapshot_dir: str, base: str, rows: int, cols: int, use_q3: bool = False,
                  use_q2: bool = False):
        """The reference's load_qmat_mode (c/qwen.c:2224-2257) over a snapshot
        directory indexed by st_init (c/st.h:211): ({fmt, gs, rb, ng, drb},
        payload, scales).  payload: rows x rb bytes (uint8) for fmt 1-4, rows x
        cols floats for fmt 0; scales: rows x ng floats (rows for fmt 1)."""
        L = self.lib
        L.ref_load_qmat.restype = C.c_int
        L.ref_load_qmat.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, i32p,
                                    C.c_void_p, C.c_size_t, f32p, C.c_size_t]
        info = np.zeros(5, np.int32)
        cap = rows * max(cols, 64) * 4
        payload = np.zeros(cap, np.uint8)
        scales = np.zeros(rows * (cols + 7), np.float32)
        rc = L.ref_load_qmat(snapshot_dir.encode(), base.encode(), rows, cols, int(use_q3), int(use_q2),
                             ptr(info, i32p), payload.ctypes.data, payload.size, ptr(scales, f32p), scales.size)
        if rc != 0:
            raise RuntimeError(f"ref_load_qmat {base}: capacity")
        fmt, gs, rb, ng, drb = (int(v) for v in info)
        d = dict(fmt=fmt, gs=gs, rb=rb, ng=ng, drb=drb)
        if fmt == 0:
            return d, payload[:rows * cols * 4].view(np.float32).reshape(rows, cols), None
        nsc = rows if fmt == 1 else rows * ng
        return d, payload[:rows * rb].reshape(rows, rb), scales[:nsc].copy()

    def layer(self, host_layer: "HostLayer"):
        return RefLayer(self, host_layer)

    def set_threads(self, n: int):
        self.lib.ref_set_threads(n)


class RefLayer:
    def __init__(self, ref: Reference, hl: "HostLayer"):
        self.ref = ref
        self.hl = hl
        self.h = ref.lib.ref_layer_create(C.byref(hl.st))

    def forward(self, x: np.ndarray):
        out = np.zeros(self.hl.H, np.float32)
        self.ref.lib.ref_moe_forward(self.h, ptr(x, f32p), ptr(out, f32p))
        return out

    def prefill(self, x: np.ndarray):
        T = x.shape[0]
        out = np.zeros((T, self.hl.H), np.float32)
        self.ref.lib.ref_moe_prefill_grouped(self.h, ptr(x, f32p), T, ptr(out, f32p))
        return out

    def __del__(self):
        try:
            self.ref.lib.ref_layer_destroy(self.h)
        except Exception:
            pass


# -- host-side layer containers ------------------------------------------------

def row_bytes(fmt: int, cols: int, gs: int) -> int:
    """Container row bytes: int4 ng*gs/2, int3 ng*gs*3/8, int2 ng*gs/4, int8
    cols (c/qwen.c:2242-2254)."""
    if fmt == 1:
        return cols
    ng = (cols + gs - 1) // gs
    return ng * gs // 2 if fmt == 4 else ng * gs // 4 if fmt == 2 else ng * gs * 3 // 8


class HostQMat:
    """Owns numpy buffers and the matching OrQMat struct."""

    def __init__(self, fmt: int, O: int, I: int, gs: int = 0, q=None, s=None, f=None):
        self.fmt, self.O, self.I, self.gs = fmt, O, I, gs
        self.ng = (I + gs - 1) // gs if fmt in (2, 3, 4) else 0
        self.rb = row_bytes(fmt, I, gs) if fmt in (1, 2, 3, 4) else 0
        self.q, self.s, self.f = q, s, f
        self.st = OrQMat(fmt, O, I, gs, self.rb, self.ng,
                         ptr(f, f32p) if f is not None else None,
                         ptr(s, f32p) if s is not None else None,
                         ptr(q) if q is not None else None)


class HostLayer:
    """One synthetic MoE layer materialised on the host from sw_synth.h."""

    def __init__(self, oracle: Oracle, seed: int, layer: int, H: int, E: int, K: int,
                 I: int, I_sh: int, fmt: int, gs: int = 128, router=None):
        self.H, self.E, self.K, self.I, self.I_sh, self.fmt, self.gs = H, E, K, I, I_sh, fmt, gs
        L = oracle.lib
        self.router_w = np.zeros((E, H), np.float32)
        self.shared_gate_row = np.zeros(H, np.float32)
        L.or_synth_router(seed, layer, E, H, ptr(self.router_w, f32p),
                          ptr(self.shared_gate_row, f32p))
        if router is not None:
            self.router_w[...] = router
        sg_q = np.zeros((I_sh, H), np.int8); sg_s = np.zeros(I_sh, np.float32)
        su_q = np.zeros((I_sh, H), np.int8); su_s = np.zeros(I_sh, np.float32)
        sd_q = np.zeros((H, I_sh), np.int8); sd_s = np.zeros(H, np.float32)
        L.or_synth_shared_q8(seed, layer, H, I_sh, ptr(sg_q), ptr(sg_s, f32p), ptr(su_q),
                             ptr(su_s, f32p), ptr(sd_q), ptr(sd_s, f32p))
        self.router = HostQMat(0, E, H, f=self.router_w)
        self.shared_scale = HostQMat(0, 1, H, f=self.shared_gate_row)
        self.shared_gate = HostQMat(1, I_sh, H, q=sg_q, s=sg_s)
        self.shared_up = HostQMat(1, I_sh, H, q=su_q, s=su_s)
        self.shared_down = HostQMat(1, H, I_sh, q=sd_q, s=sd_s)
        rbh, rbi = row_bytes(fmt, H, gs), row_bytes(fmt, I, gs)
        ngh, ngi = (H + gs - 1) // gs, (I + gs - 1) // gs
        self.gq = np.zeros((E, I, rbh), np.uint8); self.gsc = np.zeros((E, I, ngh), np.float32)
        self.uq = np.zeros((E, I, rbh), np.uint8); self.usc = np.zeros((E, I, ngh), np.float32)
        self.dq = np.zeros((E, H, rbi), np.uint8); self.dsc = np.zeros((E, H, ngi), np.float32)
        for e in range(E):
            L.or_synth_expert(seed, layer, e, fmt, H, I, gs, ptr(self.gq[e]),
                              ptr(self.gsc[e], f32p), ptr(self.uq[e]), ptr(self.usc[e], f32p),
                              ptr(self.dq[e]), ptr(self.dsc[e], f32p))
        self.gate = [HostQMat(fmt, I, H, gs, q=self.gq[e], s=self.gsc[e]) for e in range(E)]
        self.up = [HostQMat(fmt, I, H, gs, q=self.uq[e], s=self.usc[e]) for e in range(E)]
        self.down = [HostQMat(fmt, H, I, gs, q=self.dq[e], s=self.dsc[e]) for e in range(E)]
        self._g = (OrQMat * E)(*[m.st for m in self.gate])
        self._u = (OrQMat * E)(*[m.st for m in self.up])
        self._d = (OrQMat * E)(*[m.st for m in self.down])
        self.st = OrLayer(H, E, K, I, I_sh, self.router.st, self.shared_gate.st,
                          self.shared_up.st, self.shared_down.st, self.shared_scale.st,
                          self._g, self._u, self._d)

    def set_router_column(self, col: int, values: np.ndarray):
        """Overwrite one router column in place (the Zipf bias feature)."""
        self.router_w[:, col] = values


# -- the mixer layers either side of the MoE block ----------------------------

class OrGdn(C.Structure):
    _fields_ = [("H", C.c_int), ("kh", C.c_int), ("vh", C.c_int), ("dk", C.c_int),
                ("dv", C.c_int), ("K", C.c_int), ("eps", C.c_float), ("qkv", OrQMat),
                ("z", OrQMat), ("a", OrQMat), ("b", OrQMat), ("out", OrQMat),
                ("conv", f32p), ("A_log", f32p), ("dt_bias", f32p), ("norm", f32p)]


class OrAttn(C.Structure):
    _fields_ = [("H", C.c_int), ("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int),
                ("rd", C.c_int), ("theta", C.c_float), ("eps", C.c_float), ("q", OrQMat),
                ("k", OrQMat), ("v", OrQMat), ("o", OrQMat), ("q_norm", f32p),
                ("k_norm", f32p)]


def random_q4(rng: np.random.Generator, O: int, I: int, gs: int = 128, scale: float = 0.005):
    """An int4 container matrix: uniform random nibbles, |N(0, scale)| group scales."""
    rb = row_bytes(4, I, gs)
    q = rng.integers(0, 256, size=(O, rb), dtype=np.uint8)
    s = np.abs(rng.normal(0.0, scale, size=(O, (I + gs - 1) // gs))).astype(np.float32)
    return HostQMat(4, O, I, gs, q=q, s=s)


def random_q8(rng: np.random.Generator, O: int, I: int, scale: float = 0.0004):
    q = rng.integers(-127, 128, size=(O, I), dtype=np.int8)
    s = np.abs(rng.normal(0.0, scale, size=O)).astype(np.float32)
    return HostQMat(1, O, I, q=q, s=s)


class HostGdn:
    """A Gated DeltaNet layer (GdnW, c/qwen.c:95-104) with random weights:
    int4 qkv / z / out projections, fp32 a / b gate rows."""

    def __init__(self, seed: int, H: int, kh: int, vh: int, dk: int, dv: int, K: int = 4,
                 gs: int = 128, eps: float = 1e-6):
        rng = np.random.default_rng(seed)
        self.H, self.kh, self.vh, self.dk, self.dv, self.K, self.gs, self.eps = H, kh, vh, dk, dv, K, gs, eps
        self.kd, self.vd = kh * dk, vh * dv
        self.cd = 2 * self.kd + self.vd
        self.qkv = random_q4(rng, self.cd, H, gs)
        self.z = random_q4(rng, self.vd, H, gs)
        self.out = random_q4(rng, H, self.vd, gs, scale=0.004)
        self.wa = rng.normal(0.0, 0.02, size=(vh, H)).astype(np.float32)
        self.wb = rng.normal(0.0, 0.02, size=(vh, H)).astype(np.float32)
        self.a = HostQMat(0, vh, H, f=self.wa)
        self.b = HostQMat(0, vh, H, f=self.wb)
        self.conv = rng.normal(0.0, 0.5, size=(self.cd, K)).astype(np.float32)
        self.A_log = rng.normal(0.0, 0.5, size=vh).astype(np.float32)
        self.dt_bias = rng.normal(0.0, 0.5, size=vh).astype(np.float32)
        self.norm = (1.0 + rng.normal(0.0, 0.1, size=dv)).astype(np.float32)
        self.st = OrGdn(H, kh, vh, dk, dv, K, eps, self.qkv.st, self.z.st, self.a.st, self.b.st,
                        self.out.st, ptr(self.conv, f32p), ptr(self.A_log, f32p),
                        ptr(self.dt_bias, f32p), ptr(self.norm, f32p))

    def new_state(self, slots: int = 1):
        """(conv_state [slots][K][channels], recurrent state [slots][vh][dk][dv]), zero."""
        return (np.zeros((slots, self.K, self.cd), np.float32),
                np.zeros((slots, self.vh, self.dk, self.dv), np.float32))


class HostAttn:
    """A gated GQA attention layer (AttnW, c/qwen.c:105-114) with random
    weights: int4 q (query | gate per head) / k / v, o in int8 (fmt 1) or int4."""

    def __init__(self, seed: int, H: int, nh: int, nkv: int, hd: int, rd: int,
                 o_fmt: int = 1, theta: float = 1e7, gs: int = 128, eps: float = 1e-6):
        rng = np.random.default_rng(seed)
        self.H, self.nh, self.nkv, self.hd, self.rd = H, nh, nkv, hd, rd
        self.theta, self.gs, self.eps, self.o_fmt = theta, gs, eps, o_fmt
        self.kvrows, self.ctxn = nkv * hd, nh * hd
        self.q = random_q4(rng, 2 * nh * hd, H, gs)
        self.k = random_q4(rng, self.kvrows, H, gs)
        self.v = random_q4(rng, self.kvrows, H, gs)
        self.o = (random_q8(rng, H, self.ctxn) if o_fmt == 1
                  else random_q4(rng, H, self.ctxn, gs, scale=0.004))
        self.q_norm = rng.normal(0.0, 0.1, size=hd).astype(np.float32)
        self.k_norm = rng.normal(0.0, 0.1, size=hd).astype(np.float32)
        self.st = OrAttn(H, nh, nkv, hd, rd, theta, eps, self.q.st, self.k.st, self.v.st,
                         self.o.st, ptr(self.q_norm, f32p), ptr(self.k_norm, f32p))

    def new_cache(self, max_seq: int, slots: int = 1):
        return (np.zeros((slots, max_seq, self.kvrows), np.float32),
                np.zeros((slots, max_seq, self.kvrows), np.float32))


def _declare_mixers(L, prefix: str):
    if prefix == "or_":
        L.or_gdn_gates.restype = None
        L.or_gdn_gates.argtypes = [C.POINTER(OrGdn), f32p, f32p, f32p]
        L.or_gdn_forward.restype = None
        L.or_gdn_forward.argtypes = [C.POINTER(OrGdn), f32p, f32p, f32p, C.c_int, f32p, f32p, f32p]
        L.or_attn_forward.restype = None
        L.or_attn_forward.argtypes = [C.POINTER(OrAttn), f32p, C.c_int, f32p, f32p, f32p]
    else:
        L.ref_gdn_create.restype = C.c_void_p
        L.ref_gdn_create.argtypes = [C.POINTER(OrGdn), f32p, f32p]
        L.ref_gdn_forward.restype = None
        L.ref_gdn_forward.argtypes = [C.c_void_p, f32p, C.c_int, f32p, f32p, f32p]
        L.ref_gdn_block.restype = None
        L.ref_gdn_block.argtypes = [C.c_void_p, f32p, C.c_int, C.c_int, f32p]
        L.ref_attn_create.restype = C.c_void_p
        L.ref_attn_create.argtypes = [C.POINTER(OrAttn), f32p, f32p, C.c_int]
        L.ref_attn_forward.restype = None
        L.ref_attn_forward.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        L.ref_attn_prefill.restype = None
        L.ref_attn_prefill.argtypes = [C.c_void_p, f32p, C.c_int, C.c_int, f32p]
        L.ref_mixer_destroy.restype = None
        L.ref_mixer_destroy.argtypes = [C.c_void_p]


def oracle_gdn_gates(orc: "Oracle", g: HostGdn, x: np.ndarray):
    _declare_mixers(orc.lib, "or_")
    x = np.ascontiguousarray(x, np.float32)
    a = np.zeros(g.vh, np.float32)
    b = np.zeros(g.vh, np.float32)
    orc.lib.or_gdn_gates(C.byref(g.st), ptr(x, f32p), ptr(a, f32p), ptr(b, f32p))
    return a, b


def oracle_gdn_step(orc: "Oracle", g: HostGdn, x, a, b, pos: int, conv_state, state):
    """One token through the restatement; conv_state [K][channels] and state
    [vh][dk][dv] (views of one slot) advance in place."""
    _declare_mixers(orc.lib, "or_")
    x = np.ascontiguousarray(x, np.float32)
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.zeros(g.H, np.float32)
    orc.lib.or_gdn_forward(C.byref(g.st), ptr(x, f32p), ptr(a, f32p), ptr(b, f32p), pos,
                           ptr(conv_state, f32p), ptr(state, f32p), ptr(out, f32p))
    return out


def oracle_attn_step(orc: "Oracle", at: HostAttn, x, pos: int, k_cache, v_cache):
    """One token through the restatement; k_cache / v_cache [max_seq][nkv*hd]
    (views of one slot) receive position pos."""
    _declare_mixers(orc.lib, "or_")
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(at.H, np.float32)
    orc.lib.or_attn_forward(C.byref(at.st), ptr(x, f32p), pos, ptr(k_cache, f32p),
                            ptr(v_cache, f32p), ptr(out, f32p))
    return out


class RefMixer:
    """A reference GdnW or AttnW layer (ref_harness.c) over caller buffers
    that this object keeps alive."""

    def __init__(self, lib, layer, *, max_seq: int = 0):
        _declare_mixers(lib, "ref_")
        self.lib, self.layer = lib, layer
        if isinstance(layer, HostGdn):
            self.conv_state, self.state = [a[0].copy() for a in layer.new_state()]
            self.h = lib.ref_gdn_create(C.byref(layer.st), ptr(self.conv_state, f32p),
                                        ptr(self.state, f32p))
        else:
            self.k_cache, self.v_cache = [a[0].copy() for a in layer.new_cache(max_seq)]
            self.h = lib.ref_attn_create(C.byref(layer.st), ptr(self.k_cache, f32p),
                                         ptr(self.v_cache, f32p), max_seq)

    def gdn(self, x, pos: int):
        """(out, a, b) of gdn_forward at position pos."""
        g = self.layer
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(g.H, np.float32)
        a = np.zeros(g.vh, np.float32)
        b = np.zeros(g.vh, np.float32)
        self.lib.ref_gdn_forward(self.h, ptr(x, f32p), pos, ptr(out, f32p), ptr(a, f32p), ptr(b, f32p))
        return out, a, b

    def gdn_block(self, x, base: int):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.shape[0], self.layer.H), np.float32)
        self.lib.ref_gdn_block(self.h, ptr(x, f32p), x.shape[0], base, ptr(out, f32p))
        return out

    def attn(self, x, pos: int):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(self.layer.H, np.float32)
        self.lib.ref_attn_forward(self.h, ptr(x, f32p), pos, ptr(out, f32p))
        return out

    def attn_prefill(self, x, base: int):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.shape[0], self.layer.H), np.float32)
        self.lib.ref_attn_prefill(self.h, ptr(x, f32p), x.shape[0], base, ptr(out, f32p))
        return out

    def close(self):
        if getattr(self, "h", None):
            self.lib.ref_mixer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
