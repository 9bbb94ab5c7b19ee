"""Zipf(s) expert hit frequencies realised through the router GEMV.

The batched decode workloads route tokens with expert hit frequencies that
follow Zipf(s = 1.1).  The skew is put into the router itself, so every token
still goes through the exact fp32 router and `router_topk`: one activation
feature is held at 1 (x[t, H-1] = 1) and router column H-1 holds
beta * log p_{pi(e)}, where p_k ~ k^-s is the Zipf law over E ranks and pi a
seeded permutation per layer (different experts are hot in different layers).
The remaining H-1 features give every logit N(0, (H-1) * 0.02^2) noise, so
beta sets how strongly the rank order wins over the noise; `calibrate_beta`
picks the beta whose top-K hit frequencies fit the exponent s.
"""
from __future__ import annotations

import numpy as np

ROUTER_STD = 0.02  # router weights ~N(0, 0.02), activations ~N(0, 1)


def zipf_probs(E: int, s: float = 1.1) -> np.ndarray:
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    return p / p.sum()


def zipf_rank_of_expert(E: int, seed: int, layer: int) -> np.ndarray:
    """rank[e] (0-based) of expert e in layer `layer`: a seeded permutation."""
    return np.random.default_rng([seed, layer, 0x5A1F]).permutation(E)


def zipf_column(E: int, beta: float, seed: int, layer: int, s: float = 1.1) -> np.ndarray:
    """Router column H-1 (f32 [E]) for layer `layer`."""
    lp = np.log(zipf_probs(E, s))
    return (beta * lp[zipf_rank_of_expert(E, seed, layer)]).astype(np.float32)


def fitted_exponent(hits_by_rank: np.ndarray) -> float:
    """Least-squares slope of log(hits) against log(rank) over the ranks that
    were hit at least once, negated (Zipf(s) gives s)."""
    h = np.asarray(hits_by_rank, np.float64)
    r = np.arange(1, h.size + 1, dtype=np.float64)
    m = h > 0
    if m.sum() < 2:
        return float("nan")
    slope = np.polyfit(np.log(r[m]), np.log(h[m]), 1)[0]
    return float(-slope)


def simulate_hits(H: int, E: int, K: int, beta: float, tokens: int, seed: int, s: float = 1.1) -> np.ndarray:
    """Top-K hit counts per Zipf rank for `tokens` tokens whose logits are the
    rank bias plus N(0, (H-1) * ROUTER_STD^2) noise (the router GEMV over
    N(0,1) activations)."""
    rng = np.random.default_rng(seed)
    bias = beta * np.log(zipf_probs(E, s))  # indexed by rank
    sigma = ROUTER_STD * np.sqrt(H - 1)
    hits = np.zeros(E, np.int64)
    for t0 in range(0, tokens, 1024):
        n = min(1024, tokens - t0)
        logits = bias[None, :] + sigma * rng.standard_normal((n, E))
        top = np.argpartition(-logits, K - 1, axis=1)[:, :K]
        np.add.at(hits, top.ravel(), 1)
    return hits


def calibrate_beta(H: int, E: int, K: int, s: float = 1.1, tokens: int = 8192, seed: int = 11) -> tuple[float, float]:
    """Bisection on beta so that the simulated top-K hit frequencies fit the
    exponent s.  Returns (beta, fitted exponent)."""
    lo, hi = 0.0, 64.0
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        if fitted_exponent(simulate_hits(H, E, K, mid, tokens, seed, s)) < s:
            lo = mid
        else:
            hi = mid
    beta = 0.5 * (lo + hi)
    return beta, fitted_exponent(simulate_hits(H, E, K, beta, tokens, seed, s))


def apply_to_layer(be, layer, beta: float, seed: int, layer_index: int, s: float = 1.1) -> np.ndarray:
    """Write the Zipf column into the device router of `layer` (router column
    H-1, in place).  Returns the column."""
    import ctypes as C
    E, H = layer.shape.experts, layer.shape.hidden
    col = zipf_column(E, beta, seed, layer_index, s)
    base = layer.router_ptr()
    w = np.empty((E, H), np.float32)
    be.check(be.lib.coli_cuda_download(be.ctx, w.ctypes.data_as(C.c_void_p), C.c_void_p(base), w.nbytes),
             "coli_cuda_download")
    be.sync()
    w[:, H - 1] = col
    be.check(be.lib.coli_cuda_upload(be.ctx, C.c_void_p(base), w.ctypes.data_as(C.c_void_p), w.nbytes),
             "coli_cuda_upload")
    be.sync()
    return col
