"""The matrix-core ceiling probe bench.py reports beside its rooflines (libod_probe.so, od_probe_mfma)."""
import pytest

pytestmark = pytest.mark.gpu


def test_probe_runs_and_reports_a_plausible_clock():
    import bench

    ceil = bench.mfma_ceiling(modes=(0, 2, 4), iters=2000)
    for k, c in ceil.items():
        assert 0 < c["frac_of_peak"] < 1.2, (k, c)
        assert 500 < c["clock_mhz"] < 3500, (k, c)
