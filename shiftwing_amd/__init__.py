"""shiftwing MoE path on MI355X (gfx950): host-side access to the C ABI.

The product is libshiftwing_moe.so (shiftwing_amd/csrc, declared in
include/shiftwing_moe.h).  This module is the Python mirror of how the
reference's host engine drives its backend (c/qwen.c: create a context,
upload activations, call the MoE entry points, download, sync): a context
object, device buffers, and an HBM-resident MoE layer.  Every compute call
goes to the HIP library; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .abi import ColiMoeShape, load

__all__ = ["Backend", "Container", "DeviceBuffer", "MoeLayer", "ColiMoeShape", "HipError", "load"]


class HipError(RuntimeError):
    pass


class DeviceBuffer:
    """A device allocation made through coli_cuda_malloc."""

    def __init__(self, backend: "Backend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        backend.check(backend.lib.coli_cuda_malloc(backend.ctx, C.byref(p), max(self.nbytes, 1)),
                      "coli_cuda_malloc")
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.backend.lib.coli_cuda_free(self.backend.ctx, C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def p(self):
        return C.c_void_p(self.ptr)


class Backend:
    """One ColiCuda context (one device, one stream)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        ctx = C.c_void_p()
        self.check(self.lib.coli_cuda_create(C.byref(ctx), device), "coli_cuda_create")
        self.ctx = ctx

    def last_error(self) -> str:
        return self.lib.coli_cuda_last_error().decode()

    def check(self, rc: int, what: str = "call"):
        if rc != 0:
            raise HipError(f"{what}: {self.lib.coli_cuda_last_error().decode()}")

    # -- memory ---------------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        b = self.alloc(a.nbytes)
        self.check(self.lib.coli_cuda_upload(self.ctx, b.p, a.ctypes.data_as(C.c_void_p), a.nbytes),
                   "coli_cuda_upload")
        b.keep = a  # the copy is stream-ordered; keep the source alive
        return b

    def download(self, b: DeviceBuffer, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.check(self.lib.coli_cuda_download(self.ctx, out.ctypes.data_as(C.c_void_p), b.p, out.nbytes),
                   "coli_cuda_download")
        self.sync()
        return out

    def sync(self):
        self.check(self.lib.coli_cuda_sync(self.ctx), "coli_cuda_sync")

    def memory_info(self):
        f, t = C.c_size_t(), C.c_size_t()
        self.check(self.lib.coli_cuda_memory_info(self.ctx, C.byref(f), C.byref(t)), "coli_cuda_memory_info")
        return f.value, t.value

    def device_name(self) -> str:
        return self.lib.coli_cuda_device_name(self.ctx).decode()

    def set_decode_kernels(self, mode):
        """Kernels for single-token steps: 1 or True (default) the persistent
        decode kernel, 2 the three per-layer decode kernels, 0 or False the
        many-token kernels."""
        m = int(mode) if not isinstance(mode, bool) else (1 if mode else 0)
        self.check(self.lib.coli_cuda_moe_set_decode_kernels(self.ctx, m), "coli_cuda_moe_set_decode_kernels")

    def close(self):
        if self.ctx:
            self.lib.coli_cuda_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Container:
    """A converted snapshot directory (coli_cuda_container_*): the reference's
    safetensors files, indexed once; layers are loaded from it with
    MoeLayer.load."""

    def __init__(self, snapshot_dir: str):
        self.lib = load()
        h = C.c_void_p()
        if self.lib.coli_cuda_container_open(C.byref(h), snapshot_dir.encode()) != 0:
            raise HipError(f"coli_cuda_container_open: {self.lib.coli_cuda_last_error().decode()}")
        self.h = h

    def tensors(self) -> int:
        return self.lib.coli_cuda_container_tensors(self.h)

    def moe_shape(self, layer: int, topk: int = 0, sidecar: int = 0) -> ColiMoeShape:
        """sidecar: 0 main payload, 1 (or True) the .q3 sidecar, 2 the .q2 sidecar."""
        s = ColiMoeShape(0, 0, topk, 0, 0, 0, 0)
        if self.lib.coli_cuda_container_moe_shape(self.h, layer, int(sidecar), C.byref(s)) != 0:
            raise HipError(f"coli_cuda_container_moe_shape: {self.lib.coli_cuda_last_error().decode()}")
        return s

    def close(self):
        if self.h:
            self.lib.coli_cuda_container_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeLayer:
    """An HBM-resident MoE layer (coli_cuda_moe_layer_*)."""

    @classmethod
    def load(cls, be: Backend, container: Container, layer: int, topk: int, sidecar: int = 0) -> "MoeLayer":
        """The layer `layer` of a converted snapshot (coli_cuda_moe_layer_load);
        sidecar as in Container.moe_shape."""
        shape = container.moe_shape(layer, topk, sidecar)
        h = C.c_void_p()
        be.check(be.lib.coli_cuda_moe_layer_load(be.ctx, container.h, layer, topk, int(sidecar), C.byref(h)),
                 "coli_cuda_moe_layer_load")
        self = cls.__new__(cls)
        self.be, self.shape, self.h = be, shape, h
        return self

    def __init__(self, be: Backend, hidden: int, experts: int, topk: int, intermediate: int,
                 shared_intermediate: int, expert_format: int, group_size: int = 128):
        self.be = be
        self.shape = ColiMoeShape(hidden, experts, topk, intermediate, shared_intermediate,
                                  expert_format, group_size)
        h = C.c_void_p()
        be.check(be.lib.coli_cuda_moe_layer_create(be.ctx, C.byref(h), C.byref(self.shape)),
                 "coli_cuda_moe_layer_create")
        self.h = h

    @property
    def H(self):
        return self.shape.hidden

    @property
    def K(self):
        return self.shape.topk

    def nbytes(self) -> int:
        return self.be.lib.coli_cuda_moe_layer_bytes(self.h)

    def synthesize(self, seed: int, layer_index: int):
        self.be.check(self.be.lib.coli_cuda_moe_layer_synthesize(self.be.ctx, self.h, C.c_ulonglong(seed),
                                                                  layer_index),
                      "coli_cuda_moe_layer_synthesize")

    def router_ptr(self) -> int:
        return self.be.lib.coli_cuda_moe_layer_router(self.h)

    def set_router_mode(self, mode: int):
        self.be.check(self.be.lib.coli_cuda_moe_set_router_mode(self.h, mode), "set_router_mode")

    def set_router(self, router: DeviceBuffer, shared_gate: DeviceBuffer):
        self.be.check(self.be.lib.coli_cuda_moe_layer_set_router(self.be.ctx, self.h, router.p, shared_gate.p),
                      "coli_cuda_moe_layer_set_router")

    def set_shared_q8(self, gq, gs, uq, us, dq, ds):
        self.be.check(self.be.lib.coli_cuda_moe_layer_set_shared_q8(
            self.be.ctx, self.h, gq.p, gs.p, uq.p, us.p, dq.p, ds.p), "coli_cuda_moe_layer_set_shared_q8")

    def set_expert(self, e: int, gq, gs, uq, us, dq, ds):
        self.be.check(self.be.lib.coli_cuda_moe_layer_set_expert(
            self.be.ctx, self.h, e, gq.p, gs.p, uq.p, us.p, dq.p, ds.p), "coli_cuda_moe_layer_set_expert")

    def forward(self, y: DeviceBuffer, x: DeviceBuffer, tokens: int, idx: DeviceBuffer | None = None,
                weight: DeviceBuffer | None = None):
        self.be.check(self.be.lib.coli_cuda_moe_forward(
            self.be.ctx, self.h, y.p, x.p, tokens, idx.p if idx else None, weight.p if weight else None),
            "coli_cuda_moe_forward")

    def route(self, x: DeviceBuffer, tokens: int, idx: DeviceBuffer, weight: DeviceBuffer):
        self.be.check(self.be.lib.coli_cuda_moe_route(self.be.ctx, self.h, x.p, tokens, idx.p, weight.p),
                      "coli_cuda_moe_route")

    def route_stats(self):
        t, f = C.c_ulonglong(), C.c_ulonglong()
        self.be.check(self.be.lib.coli_cuda_moe_route_stats(self.be.ctx, self.h, C.byref(t), C.byref(f)),
                      "coli_cuda_moe_route_stats")
        return t.value, f.value

    def route_stats_full(self):
        """(tokens, not certified by the bounds, needing every expert's chain)."""
        out = (C.c_ulonglong * 3)()
        self.be.check(self.be.lib.coli_cuda_moe_route_stats_full(self.be.ctx, self.h, out),
                      "coli_cuda_moe_route_stats_full")
        return tuple(int(v) for v in out)

    def forward_host(self, x: np.ndarray):
        """Convenience: host x [T,H] -> (y [T,H], idx [T,K], weight [T,K])."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.H)
        T = x.shape[0]
        dx = self.be.upload(x)
        dy = self.be.alloc(x.nbytes)
        di = self.be.alloc(T * self.K * 4)
        dw = self.be.alloc(T * self.K * 4)
        self.forward(dy, dx, T, di, dw)
        y = self.be.download(dy, (T, self.H), np.float32)
        idx = self.be.download(di, (T, self.K), np.int32)
        w = self.be.download(dw, (T, self.K), np.float32)
        return y, idx, w

    def close(self):
        if self.h:
            self.be.lib.coli_cuda_moe_layer_destroy(self.be.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
