"""Writes safetensors files in the reference's container conventions (test
helper): an 8-byte little-endian header length, a JSON header
{name: {dtype, shape, data_offsets}} padded with spaces to 8 bytes, then the
data (c/st.h reads this layout)."""
from __future__ import annotations

import json
import os

import numpy as np

_DT = {np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8", np.dtype(np.float32): "F32",
       np.dtype(np.float16): "F16"}


def bf16(a: np.ndarray) -> "Raw":
    """f32 -> bfloat16 (round to nearest even) as a raw tensor."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return Raw("BF16", a.shape, u.tobytes())


def bf16_values(a: np.ndarray) -> np.ndarray:
    """The f32 values a bf16 tensor written by bf16() decodes to."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return u.astype(np.uint32).view(np.float32)


class Raw:
    def __init__(self, dtype: str, shape, data: bytes):
        self.dtype, self.shape, self.data = dtype, list(shape), data


def write(path: str, tensors: dict) -> None:
    header, blobs, off = {}, [], 0
    for name, v in tensors.items():
        if isinstance(v, Raw):
            dt, shape, data = v.dtype, v.shape, v.data
        else:
            a = np.ascontiguousarray(v)
            dt, shape, data = _DT[a.dtype], list(a.shape), a.tobytes()
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def moe_layer_tensors(hl, layer: int, prefix: str = "", q3: "object | None" = None,
                      router_bf16: bool = False, qtype_tags: bool = True, q2: "object | None" = None) -> dict:
    """The MoE tensors of one layer as c/tools/convert_qwen.py writes them
    (c/qwen.c:2443-2457, 2330-2346): router and gate row as float, the shared
    expert as int8 rows + .qs [rows] + .qtype 8, routed experts as packed
    codes + .qs [rows, groups] + .qtype 4 (or 3).  `q3`: a second host layer
    whose int3 experts go into the .q3 sidecar (c/tools/requantize_expert_q2.py);
    `q2`: one whose int2 experts go into .q2 sidecars (the EXPERT_Q2=1 lookup,
    c/qwen.c:2207-2212)."""
    p = f"{prefix}layers.{layer}.mlp."
    t = {}
    t[p + "gate.weight"] = bf16(hl.router_w) if router_bf16 else hl.router_w
    t[p + "shared_expert_gate.weight"] = hl.shared_gate_row.reshape(1, -1)
    for nm, m in (("gate", hl.shared_gate), ("up", hl.shared_up), ("down", hl.shared_down)):
        base = f"{p}shared_expert.{nm}_proj.weight"
        t[base] = m.q.view(np.uint8)
        t[base + ".qs"] = m.s
        if qtype_tags:
            t[base + ".qtype"] = np.array([8], np.uint8)
    tag = hl.fmt
    for e in range(hl.E):
        for nm, q, s in (("gate", hl.gq[e], hl.gsc[e]), ("up", hl.uq[e], hl.usc[e]), ("down", hl.dq[e], hl.dsc[e])):
            base = f"{p}experts.{e}.{nm}_proj.weight"
            t[base] = q
            t[base + ".qs"] = s
            if qtype_tags:
                t[base + ".qtype"] = np.array([tag], np.uint8)
    for side, sfx, tg in ((q3, ".q3", 3), (q2, ".q2", 2)):
        if side is None:
            continue
        for e in range(side.E):
            for nm, q, s in (("gate", side.gq[e], side.gsc[e]), ("up", side.uq[e], side.usc[e]),
                             ("down", side.dq[e], side.dsc[e])):
                base = f"{p}experts.{e}.{nm}_proj.weight{sfx}"
                t[base] = q
                t[base + ".qs"] = s
                t[base + ".qtype"] = np.array([tg], np.uint8)
    return t


def write_split(dirpath: str, tensors: dict, parts: int = 2) -> None:
    """Spread the tensors over `parts` files, as sharded snapshots are."""
    os.makedirs(dirpath, exist_ok=True)
    names = list(tensors)
    for i in range(parts):
        write(os.path.join(dirpath, f"model-{i + 1:05d}-of-{parts:05d}.safetensors"),
              {n: tensors[n] for n in names[i::parts]})
