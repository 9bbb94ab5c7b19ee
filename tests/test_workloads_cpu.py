"""Host-side workload logic of the batched and prefill benchmarks (CPU only):
the Zipf(1.1) routing feature and the per-stage byte/flop model."""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT

sys.path.insert(0, ROOT)


def test_fitted_exponent_recovers_exact_zipf():
    from shiftwing_amd import zipf
    for s in (0.8, 1.1, 1.5):
        h = 1e6 * np.arange(1, 513, dtype=np.float64) ** -s
        assert abs(zipf.fitted_exponent(h) - s) < 1e-9
    # ranks with no hits are left out of the fit
    h = 1e6 * np.arange(1, 65, dtype=np.float64) ** -1.1
    h[40:] = 0
    assert abs(zipf.fitted_exponent(h) - 1.1) < 1e-9


def test_zipf_probs_and_column_order():
    from shiftwing_amd import zipf
    E = 512
    p = zipf.zipf_probs(E)
    assert abs(p.sum() - 1.0) < 1e-12 and np.all(np.diff(p) < 0)
    col = zipf.zipf_column(E, 0.5, 397, 3)
    rank = zipf.zipf_rank_of_expert(E, 397, 3)
    assert sorted(rank.tolist()) == list(range(E))
    # the expert holding rank 0 has the largest bias, rank E-1 the smallest
    assert int(np.argmax(col)) == int(np.where(rank == 0)[0][0])
    assert int(np.argmin(col)) == int(np.where(rank == E - 1)[0][0])
    assert np.isclose(col.max(), 0.5 * np.log(p[0]), rtol=1e-6)
    # different layers have different hot experts
    assert not np.array_equal(rank, zipf.zipf_rank_of_expert(E, 397, 4))


@pytest.mark.parametrize("H,E,K", [(4096, 512, 10), (2048, 256, 8)])
def test_calibrated_beta_fits_exponent(H, E, K):
    from shiftwing_amd import zipf
    beta, fit = zipf.calibrate_beta(H, E, K)
    assert abs(fit - 1.1) < 0.01
    # the fitted exponent grows with beta, so the bisection is well posed
    lo = zipf.fitted_exponent(zipf.simulate_hits(H, E, K, 0.5 * beta, 4096, 3))
    hi = zipf.fitted_exponent(zipf.simulate_hits(H, E, K, 2.0 * beta, 4096, 3))
    assert lo < 1.1 < hi
    # no bias: every expert equally likely, exponent near 0
    assert abs(zipf.fitted_exponent(zipf.simulate_hits(H, E, K, 0.0, 4096, 3))) < 0.1


def test_stage_model_matches_closed_form():
    """Per-stage bytes sum to U*expert + shared + router + gate row + T*H*8
    and flops to T*(K*6HI + 6HI_sh + 2EH): per token, three H x I products
    (2 flops a weight) for each of the K routed experts and the shared one,
    and the E x H router."""
    import bench
    H, E, K, I, Ish, fmt = 4096, 512, 10, 1024, 1024, 3
    for T, U in [(1, 10), (8, 61.5), (512, 512)]:
        names, nb, fl = bench.stage_model(H, E, K, I, Ish, fmt, T, U)
        assert len(names) == len(nb) == len(fl) == 7
        assert sum(nb) == pytest.approx(U * 5_111_808 + 12_607_488 + 8_388_608 + 16_384 + T * H * 8)
        assert sum(fl) == T * (K * 6 * H * I + 6 * H * Ish + 2 * E * H)
    H, E, K, I, Ish, fmt = 2048, 256, 8, 512, 512, 4
    names, nb, fl = bench.stage_model(H, E, K, I, Ish, fmt, 1, 8)
    assert sum(nb) == 18_632_704 + H * 8
    assert sum(fl) == 512 * 0 + (K * 6 * H * I + 6 * H * Ish + 2 * E * H)


def test_bench_many_workloads_declared():
    import bench
    assert set(bench.MANY) == {"s397-batch", "prefill-s35", "prefill-s397"}
    for name, (base, nl, T, zipf_on, desc) in bench.MANY.items():
        assert base in bench.WORKLOADS and desc.startswith("config")
        assert (T is None) == (name == "s397-batch")
