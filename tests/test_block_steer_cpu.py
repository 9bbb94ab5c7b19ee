"""The steered inputs of test_gpu_moe_block.py decide the router on the last
bits of n (CPU only).  With rmsnorm_zero's sum of squares taken in another
order (numpy's pairwise float32 sum, as a parallel device reduction would),
n differs and router_topk picks other experts for some steered tokens: so the
GPU test's index check fails for a block whose norm is not the reference's
serial chain (c/qwen.c:1780-1784), not only its bit check of n."""
import numpy as np

import test_gpu_moe_block as tb


def _alt_norm(x, w, eps):
    ms = np.float32(np.sum(x * x, dtype=np.float32))
    r = np.float32(1) / np.sqrt(np.float32(ms / np.float32(x.size) + np.float32(eps)))
    return ((x * r).astype(np.float32) * (np.float32(1) + w)).astype(np.float32)


def test_steered_block_inputs_flip_routes_under_a_parallel_norm(oracle):
    flips = differ = total = 0
    for shape, T, reps in [(tb.S35, 7, 1), (tb.S397, 1, 4)]:
        H, E, K, I, Ish, fmt = shape
        seed = 44 + T
        hl = oracle.host_layer(seed, 1, H, E, K, I, Ish, fmt)
        rng = np.random.default_rng(seed)
        w = (rng.standard_normal(H) * 0.1).astype(np.float32)
        for rep in range(reps):
            for t in range(T):
                steer = tb.STEER[(rep + t) % len(tb.STEER)]
                x = tb._residual_with_tie(oracle, hl, oracle.synth_x(seed, 1, rep * T + t, H), w, steer,
                                          2.5 + 0.5 * (t % 3))
                n = oracle.rmsnorm_zero(x, w, tb.EPS)
                n_alt = _alt_norm(x, w, tb.EPS)
                _, a = oracle.moe_forward(hl, n, trace=True)
                _, b = oracle.moe_forward(hl, n_alt, trace=True)
                total += 1
                differ += not np.array_equal(n, n_alt)
                flips += not np.array_equal(a["idx"], b["idx"])
    assert differ >= total - 2, (differ, total)
    assert flips > 0, "no steered token's routes depend on the norm's summation order"
