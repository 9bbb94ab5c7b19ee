"""The hybrid decoder's mixer layers on the device, driven the way the
reference's host engine drives them (c/qwen.c:868-1075): weights and state
uploaded once, then one C-ABI call per step.

DeviceGdn mirrors cuda_gdn_prepare_locked / cuda_gdn_try (c/qwen.c:869-892,
893-911) over coli_cuda_gdn_{decode,block,slots,slots_device}_q4_f16;
DeviceAttn mirrors cuda_attn_prepare_locked / cuda_attn_try (c/qwen.c:922-943,
957-991) over coli_cuda_gqa_{decode,prefill,slots,slots_device}_q4_f16.
Every step runs in libshiftwing_moe.so; nothing here computes.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

__all__ = ["DeviceGdn", "DeviceAttn"]


def _f(a):
    return np.ascontiguousarray(a, np.float32)


def _hp(a):
    """host pointer of a contiguous numpy array"""
    return C.c_void_p(a.ctypes.data)


class _Mat:
    """A quantized matrix resident on the device: fmt 4 (int4 groups) or 1 (int8 rows)."""

    def __init__(self, be, fmt, q, s, gs=0):
        self.fmt, self.gs = fmt, gs
        q = np.ascontiguousarray(q)
        self.rows, self.rb = q.shape
        s = _f(s)
        self.ng = s.shape[1] if s.ndim == 2 else 0
        self.q, self.s = be.upload(q), be.upload(s)


class DeviceGdn:
    """A Gated DeltaNet layer (GdnW, c/qwen.c:95-104) with `slots` independent
    recurrent/convolution states on the device (slot 0 is the single-sequence
    state the decode and block calls use)."""

    def __init__(self, be, *, hidden, key_heads, value_heads, key_dim, value_dim, conv_kernel, group_size, eps,
                 qkv, z, out, conv, A_log, dt_bias, norm, slots=1):
        self.be = be
        self.H, self.kh, self.vh, self.dk, self.dv = hidden, key_heads, value_heads, key_dim, value_dim
        self.K, self.gs, self.eps, self.slots = conv_kernel, group_size, float(eps), slots
        self.cd = 2 * key_heads * key_dim + value_heads * value_dim
        self.qkv, self.z, self.out = (_Mat(be, 4, m[0], m[1], group_size) for m in (qkv, z, out))
        self.conv, self.A_log, self.dt_bias, self.norm = (be.upload(_f(a)) for a in (conv, A_log, dt_bias, norm))
        self.conv_state = be.alloc(slots * conv_kernel * self.cd * 4)
        self.state = be.alloc(slots * value_heads * key_dim * value_dim * 4)
        self.reset()

    def reset(self):
        be = self.be
        be.check(be.lib.coli_cuda_memset(be.ctx, self.conv_state.p, 0, self.conv_state.nbytes), "memset")
        be.check(be.lib.coli_cuda_memset(be.ctx, self.state.p, 0, self.state.nbytes), "memset")
        be.sync()

    def _weights(self):
        return (self.qkv.q.p, self.qkv.s.p, self.qkv.rb, self.qkv.ng, self.z.q.p, self.z.s.p, self.z.rb, self.z.ng,
                self.out.q.p, self.out.s.p, self.out.rb, self.out.ng, self.conv.p, self.A_log.p, self.dt_bias.p,
                self.norm.p, self.conv_state.p, self.state.p)

    def _dims(self):
        return (self.H, self.kh, self.vh, self.dk, self.dv, self.K, self.gs, C.c_float(self.eps))

    def decode(self, x, a, b, pos):
        """coli_cuda_gdn_decode_q4_f16: one token at position pos (host I/O)."""
        x, a, b = _f(x), _f(a), _f(b)
        y = np.zeros(self.H, np.float32)
        be = self.be
        be.check(be.lib.coli_cuda_gdn_decode_q4_f16(be.ctx, _hp(y), _hp(x), _hp(a), _hp(b), *self._weights(), pos,
                                                     *self._dims()), "coli_cuda_gdn_decode_q4_f16")
        return y

    def block(self, x, a, b, pos):
        """coli_cuda_gdn_block_q4_f16: T <= 8 consecutive tokens from position pos."""
        x, a, b = _f(x), _f(a), _f(b)
        y = np.zeros((x.shape[0], self.H), np.float32)
        be = self.be
        be.check(be.lib.coli_cuda_gdn_block_q4_f16(be.ctx, _hp(y), _hp(x), _hp(a), _hp(b), x.shape[0],
                                                    *self._weights(), pos, *self._dims()),
                 "coli_cuda_gdn_block_q4_f16")
        return y

    def slots_step(self, x, a, b, slot, pos, device_io=False):
        """coli_cuda_gdn_slots_q4_f16[_device]: row r advances slot[r] at
        position pos[r]."""
        x, a, b = _f(x), _f(a), _f(b)
        slot = np.ascontiguousarray(slot, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        B = x.shape[0]
        be = self.be
        args = (self.slots, *self._dims())
        if not device_io:
            y = np.zeros((B, self.H), np.float32)
            be.check(be.lib.coli_cuda_gdn_slots_q4_f16(be.ctx, _hp(y), _hp(x), _hp(a), _hp(b), B, _hp(slot),
                                                        _hp(pos), *self._weights(), *args),
                     "coli_cuda_gdn_slots_q4_f16")
            return y
        dx, da, db = be.upload(x), be.upload(a), be.upload(b)
        dy = be.alloc(B * self.H * 4)
        be.check(be.lib.coli_cuda_gdn_slots_q4_f16_device(be.ctx, dy.p, dx.p, da.p, db.p, B, _hp(slot), _hp(pos),
                                                           *self._weights(), *args),
                 "coli_cuda_gdn_slots_q4_f16_device")
        return be.download(dy, (B, self.H), np.float32)

    def read_state(self):
        """(conv_state [slots][K][channels], state [slots][vh][dk][dv])"""
        cs = self.be.download(self.conv_state, (self.slots, self.K, self.cd), np.float32)
        st = self.be.download(self.state, (self.slots, self.vh, self.dk, self.dv), np.float32)
        return cs, st


class DeviceAttn:
    """A gated GQA attention layer (AttnW, c/qwen.c:105-114) with fp32 KV
    caches of max_seq positions for `slots` sequences on the device."""

    def __init__(self, be, *, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta, eps,
                 q, k, v, o, o_fmt, q_norm, k_norm, max_seq, slots=1):
        self.be = be
        self.H, self.nh, self.nkv, self.hd, self.rd = hidden, query_heads, kv_heads, head_dim, rotary_dim
        self.gs, self.theta, self.eps, self.max_seq, self.slots = group_size, float(theta), float(eps), max_seq, slots
        self.kvrows = kv_heads * head_dim
        self.q, self.k, self.v = (_Mat(be, 4, m[0], m[1], group_size) for m in (q, k, v))
        self.o = _Mat(be, o_fmt, o[0], o[1], group_size)
        self.q_norm, self.k_norm = be.upload(_f(q_norm)), be.upload(_f(k_norm))
        self.k_cache = be.alloc(slots * max_seq * self.kvrows * 4)
        self.v_cache = be.alloc(slots * max_seq * self.kvrows * 4)
        be.check(be.lib.coli_cuda_memset(be.ctx, self.k_cache.p, 0, self.k_cache.nbytes), "memset")
        be.check(be.lib.coli_cuda_memset(be.ctx, self.v_cache.p, 0, self.v_cache.nbytes), "memset")
        be.sync()

    def _weights(self):
        return (self.q.q.p, self.q.s.p, self.q.rb, self.q.ng, self.k.q.p, self.k.s.p, self.k.rb, self.k.ng,
                self.v.q.p, self.v.s.p, self.v.rb, self.v.ng, self.o.q.p, self.o.s.p, self.o.fmt, self.o.rb,
                self.o.ng, self.q_norm.p, self.k_norm.p, self.k_cache.p, self.v_cache.p)

    def _tail(self):
        return (self.H, self.nh, self.nkv, self.hd, self.rd, self.gs, C.c_float(self.theta), C.c_float(self.eps))

    def decode(self, x, pos):
        """coli_cuda_gqa_decode_q4_f16: one token at position pos (slot 0)."""
        x = _f(x)
        y = np.zeros(self.H, np.float32)
        be = self.be
        be.check(be.lib.coli_cuda_gqa_decode_q4_f16(be.ctx, _hp(y), _hp(x), *self._weights(), pos, *self._tail()),
                 "coli_cuda_gqa_decode_q4_f16")
        return y

    def prefill(self, x, base):
        """coli_cuda_gqa_prefill_q4_f16: rows base .. base + len(x) - 1 (slot 0)."""
        x = _f(x)
        y = np.zeros((x.shape[0], self.H), np.float32)
        be = self.be
        be.check(be.lib.coli_cuda_gqa_prefill_q4_f16(be.ctx, _hp(y), _hp(x), x.shape[0], base, *self._weights(),
                                                      self.max_seq, *self._tail()),
                 "coli_cuda_gqa_prefill_q4_f16")
        return y

    def slots_step(self, x, slot, pos, device_io=False):
        """coli_cuda_gqa_slots_q4_f16[_device]: row r appends to slot[r] at pos[r]."""
        x = _f(x)
        slot = np.ascontiguousarray(slot, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        B = x.shape[0]
        be = self.be
        tail = (self.slots, self.max_seq, *self._tail())
        if not device_io:
            y = np.zeros((B, self.H), np.float32)
            be.check(be.lib.coli_cuda_gqa_slots_q4_f16(be.ctx, _hp(y), _hp(x), B, _hp(slot), _hp(pos),
                                                        *self._weights(), *tail),
                     "coli_cuda_gqa_slots_q4_f16")
            return y
        dx = be.upload(x)
        dy = be.alloc(B * self.H * 4)
        be.check(be.lib.coli_cuda_gqa_slots_q4_f16_device(be.ctx, dy.p, dx.p, B, _hp(slot), _hp(pos),
                                                           *self._weights(), *tail),
                 "coli_cuda_gqa_slots_q4_f16_device")
        return be.download(dy, (B, self.H), np.float32)

    def read_cache(self):
        shape = (self.slots, self.max_seq, self.kvrows)
        return (self.be.download(self.k_cache, shape, np.float32),
                self.be.download(self.v_cache, shape, np.float32))
