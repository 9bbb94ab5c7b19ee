"""Writes the golden vectors under tests/golden/ from the compiled reference.

The reference's CPU MoE code (c/qwen.c) is compiled in place by
oracle/Makefile (`make -C oracle ref`) into oracle/_ref/; this script calls it
through oracle/pyoracle.py and stores inputs plus the reference's outputs as
.npz fixtures (no pickle).  The synthetic weights themselves are not stored:
they are regenerated from the seed by shiftwing_amd/csrc/sw_synth.h, so a
fixture holds (config, seed, x, outputs).

router.json is the reference's own fixture (c/fixtures/router.json, produced
with transformers by the reference authors), copied as data.

Run in the build container (needs /root/reference):
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.pyoracle import HostLayer, HostQMat, Oracle, Reference, build, row_bytes  # noqa: E402

REF_FIXTURE = "/root/reference/c/fixtures/router.json"

# (name, H, E, K, I, I_sh, fmt, gs, seed, layer, tokens)
LAYERS = [
    ("small_q4", 256, 16, 4, 128, 128, 4, 128, 11, 0, 7),
    ("small_q3", 256, 16, 4, 128, 128, 3, 128, 12, 1, 7),
    ("ragged_q4", 384, 32, 8, 257, 129, 4, 128, 13, 2, 5),
    ("ragged_q3", 384, 32, 8, 257, 129, 3, 128, 14, 3, 5),
    ("s35_q4", 2048, 256, 8, 512, 512, 4, 128, 35, 0, 3),
    ("s397_q3", 4096, 512, 10, 1024, 1024, 3, 128, 397, 0, 2),
    ("small_q2", 256, 16, 4, 128, 128, 2, 128, 15, 4, 7),
    ("ragged_q2", 384, 32, 8, 257, 129, 2, 128, 16, 5, 5),
]


def router_cases(rng):
    cases = []
    for _ in range(48):
        cases.append((rng.standard_normal(512).astype(np.float32) * 1.3, 10))
    for _ in range(16):
        cases.append((rng.standard_normal(256).astype(np.float32) * 1.3, 8))
    # exact ties: lowest index must win
    t = rng.standard_normal(64).astype(np.float32)
    t[[5, 9, 40]] = 3.0
    cases.append((t, 4))
    cases.append((np.zeros(32, np.float32), 6))
    # neighbours one ulp apart at the top
    u = rng.standard_normal(512).astype(np.float32)
    top = np.float32(4.0)
    u[100] = top
    u[7] = np.nextafter(top, np.float32(0))
    u[300] = np.nextafter(top, np.float32(10))
    u[301] = top
    cases.append((u, 10))
    # large spread: most probabilities underflow to zero
    v = (rng.standard_normal(512) * 60).astype(np.float32)
    cases.append((v, 10))
    return cases


def main():
    build(ref=True)
    o = Oracle()
    ref = Reference(os.path.join(os.path.dirname(HERE), "..", "oracle", "_ref", "libref_native.so"))
    shutil.copyfile(REF_FIXTURE, os.path.join(HERE, "router.json"))
    rng = np.random.default_rng(20261201)

    # router_topk
    logits, ks, idxs, ws, Es = [], [], [], [], []
    for lg, k in router_cases(rng):
        i, w = ref.router_topk(np.ascontiguousarray(lg), k)
        logits.append(np.pad(lg, (0, 512 - lg.size)))
        Es.append(lg.size)
        ks.append(k)
        idxs.append(np.pad(i, (0, 10 - k), constant_values=-1))
        ws.append(np.pad(w, (0, 10 - k)))
    np.savez(os.path.join(HERE, "router_topk.npz"), logits=np.stack(logits), E=np.array(Es),
             K=np.array(ks), idx=np.stack(idxs), weight=np.stack(ws))

    # single-matrix GEMV rows, fmt 1 (int8, IDOT and fp32-activation) / 3 / 4
    # (fmt 2 below)
    out = {}
    for fmt in (1, 3, 4):
        for I in (1, 31, 64, 128, 129, 257):
            O, gs = 5, 128
            rb = row_bytes(fmt, I, gs)
            if fmt == 1:
                q = rng.integers(-127, 128, (O, I), dtype=np.int8)
                s = np.abs(rng.standard_normal(O) * 0.01).astype(np.float32)
            else:
                q = rng.integers(0, 256, (O, rb), dtype=np.uint8)
                s = np.abs(rng.standard_normal((O, (I + gs - 1) // gs)) * 0.01).astype(np.float32)
                if fmt == 3:
                    s[1::2] *= -1  # mirrored int3 codebooks carry negative scales
            x = rng.standard_normal(I).astype(np.float32)
            m = HostQMat(fmt, O, I, gs, q=np.ascontiguousarray(q), s=np.ascontiguousarray(s))
            X = rng.standard_normal((6, I)).astype(np.float32)
            key = f"f{fmt}_I{I}"
            out[key + "_q"] = q
            out[key + "_s"] = s
            out[key + "_x"] = x
            out[key + "_y"] = ref.qmat_mul(x, m, 1)
            out[key + "_y_noidot"] = ref.qmat_mul(x, m, 0)
            out[key + "_X"] = X
            out[key + "_Y"] = ref.qmat_mul_batch(np.ascontiguousarray(X), m, 1)
    np.savez(os.path.join(HERE, "qmat.npz"), **out)

    # int2 rows (dot_q2_group), from a generator of their own so that the
    # fixtures above keep their bytes
    rng2 = np.random.default_rng(20261202)
    out2 = {}
    for I in (1, 3, 31, 64, 128, 129, 257):
        O, gs = 5, 128
        q = rng2.integers(0, 256, (O, row_bytes(2, I, gs)), dtype=np.uint8)
        s = np.abs(rng2.standard_normal((O, (I + gs - 1) // gs)) * 0.01).astype(np.float32)
        x = rng2.standard_normal(I).astype(np.float32)
        m = HostQMat(2, O, I, gs, q=np.ascontiguousarray(q), s=np.ascontiguousarray(s))
        key = f"f2_I{I}"
        out2[key + "_q"] = q
        out2[key + "_s"] = s
        out2[key + "_x"] = x
        out2[key + "_y"] = ref.qmat_mul(x, m, 1)
    np.savez(os.path.join(HERE, "qmat_q2.npz"), **out2)

    # whole layers: decode (moe_forward) per token and prefill (moe_prefill_grouped)
    for name, H, E, K, I, I_sh, fmt, gs, seed, layer, T in LAYERS:
        hl = HostLayer(o, seed, layer, H, E, K, I, I_sh, fmt, gs)
        rl = ref.layer(hl)
        X = np.stack([o.synth_x(seed, layer, t, H) for t in range(T)])
        dec = np.stack([rl.forward(X[t]) for t in range(T)])
        pre = rl.prefill(np.ascontiguousarray(X))
        # router indices/weights through the reference's own router GEMV + top-k
        logits = [ref.qmat_mul(X[t], hl.router, 0) for t in range(T)]
        routes = [ref.router_topk(lg, K) for lg in logits]
        np.savez(os.path.join(HERE, f"layer_{name}.npz"),
                 cfg=np.array([H, E, K, I, I_sh, fmt, gs, seed, layer, T]),
                 x=X, decode=dec, prefill=pre, logits=np.stack(logits),
                 idx=np.stack([r[0] for r in routes]),
                 weight=np.stack([r[1] for r in routes]))
        print(name, "done")


if __name__ == "__main__":
    main()
